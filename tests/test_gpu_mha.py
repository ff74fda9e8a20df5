"""Parity of the fused self-attention layer (``atx_mha_fwd``) against the
float64 oracle's module forward (``oracle.attention.mha_forward``, which
restates stratego/networks/attention.py:152-204).

Inputs and weights are drawn on the CPU from seeded generators and rounded to
the kernel's 16-bit dtype; the oracle runs in float64 on the same values.
Tolerance: the contract's 16-bit figure, ``max|y - ref| <= 2e-2``, plus a
normwise ``max|y - ref| <= 2e-2 * max|ref|``, since the layer rounds Q, K, V and
the attention output to 16 bits where the reference's bf16 modules do.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import MultiHeadAttention, _lib, ops
from oracle.attention import mha_forward as oracle_mha
from tests._cases import randn, to_np64

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


def layer(e, dtype, seed, bias=False):
    g = torch.Generator().manual_seed(seed)
    bound = e**-0.5  # nn.Linear's default init range
    ws = [((torch.rand(e, e, generator=g) * 2 - 1) * bound).to(dtype) for _ in range(4)]
    bs = [((torch.rand(e, generator=g) * 2 - 1) * bound).to(dtype) for _ in range(4)] if bias else [None] * 4
    return ws, bs


def run_case(cuda, b, l, h, dtype=torch.bfloat16, causal=False, bias=False, seed=0, x_view=False, packed=False, d=64):
    e = d * h
    _announce(f"mha b={b} l={l} h={h}x{d} {dtype} causal={causal} bias={bias} view={x_view} packed={packed}")
    x = randn((b, l, e), seed, dtype)
    ws, bs = layer(e, dtype, seed + 1, bias)
    if x_view:  # rows of a wider buffer, NaN after the sequence and in the padding columns
        big = torch.full((b, l + 5, e + 64), float("nan"), dtype=dtype)
        big[:, :l, :e] = x
        xd = big.to(cuda)[:, :l, :e]
    else:
        xd = x.to(cuda)
    wd = [w.to(cuda) for w in ws]
    if packed:
        wd = [ops.mha_pack_weight(w) for w in wd]
    bd = [t.to(cuda) if t is not None else None for t in bs]
    y = ops.mha_forward(xd, *wd, num_heads=h, b_q=bd[0], b_k=bd[1], b_v=bd[2], b_o=bd[3], causal=causal, packed=packed)
    torch.cuda.synchronize()
    names = ("q_proj", "k_proj", "v_proj", "out_proj")
    weights = {f"{n}.weight": to_np64(w) for n, w in zip(names, ws)}
    if bias:
        weights.update({f"{n}.bias": to_np64(t) for n, t in zip(names, bs)})
    ref = oracle_mha(to_np64(x), None, weights, h, causal=causal)
    got = to_np64(y)
    assert np.isfinite(got).all(), "non-finite output"
    err = float(np.max(np.abs(got - ref)))
    assert err <= 2e-2, f"max-abs {err:.3e}"
    assert err <= 2e-2 * float(np.max(np.abs(ref))), f"normwise {err:.3e} vs {np.max(np.abs(ref)):.3e}"
    return err


def test_move_net_layer(cuda):
    """C3 layer shape: L=100, E=384, 6 x 64, bf16."""
    run_case(cuda, 32, 100, 6, seed=1)


@pytest.mark.parametrize("h", [2, 4, 6, 8])
def test_heads(cuda, h):
    run_case(cuda, 4, 100, h, seed=10 + h)


@pytest.mark.parametrize("l", [1, 2, 15, 16, 17, 33, 40, 64, 97, 112, 128])
def test_seq_lengths(cuda, l):
    run_case(cuda, 3, l, 4, seed=20 + l)


@pytest.mark.parametrize("h,l", [(8, 48), (8, 64), (8, 80), (6, 48), (6, 64), (6, 128), (2, 128)])
def test_output_projection_forms(cuda, h, l):
    """Shapes either side of the kernel's switch between keeping Y in
    registers across heads and parking each head's output in y: 8 heads at
    48 (parked), 64 and 80 (registers); 6 heads at 48 (registers), 64
    (parked, measured faster) and 128 (parked: the accumulators and the
    second O buffer do not fit); 2 heads at 128 (registers)."""
    run_case(cuda, 3, l, h, seed=90 + h + l)


@pytest.mark.parametrize("l", [1, 17, 40, 100])
def test_causal(cuda, l):
    """Setup network: causal self-attention (40 pieces)."""
    run_case(cuda, 4, l, 6, causal=True, seed=40 + l)


def test_biases_and_fp16(cuda):
    run_case(cuda, 4, 100, 6, bias=True, seed=50)
    run_case(cuda, 4, 100, 6, dtype=torch.float16, seed=51)
    run_case(cuda, 4, 40, 8, dtype=torch.float16, bias=True, causal=True, seed=52)


def test_strided_input_and_guard_values(cuda):
    """x as a view into a wider buffer holding NaN past the sequence and in the
    columns beyond E: nothing outside the view is read."""
    run_case(cuda, 4, 100, 6, x_view=True, seed=60)


def test_rows_past_the_sequence_are_not_written(cuda):
    _announce("mha output guard rows")
    b, l, h = 3, 40, 6
    e = 64 * h
    x = randn((b, l, e), 61, torch.bfloat16).to(cuda)
    ws, _ = layer(e, torch.bfloat16, 62)
    out_big = torch.full((b, l + 8, e), 7.0, dtype=torch.bfloat16, device=cuda)
    ops.mha_forward(x, *[w.to(cuda) for w in ws], num_heads=h, out=out_big[:, :l])
    torch.cuda.synchronize()
    assert (out_big[:, l:] == 7.0).all()


def test_matches_the_unfused_module_path(cuda):
    """The fused layer equals MultiHeadAttention's unfused GPU path
    (hipBLASLt projections + the attention kernel) to bf16 rounding."""
    _announce("mha vs unfused module")
    torch.manual_seed(7)
    m = MultiHeadAttention(384, 6).to(cuda, torch.bfloat16).eval()
    x = randn((16, 100, 384), 70, torch.bfloat16).to(cuda)
    with torch.no_grad():
        m.fuse_layer = False
        unfused = m(x)
        m.fuse_layer = True
        fused = m(x)  # the module's inference path is the one-launch layer
        direct = ops.mha_forward(x, m.q_proj.weight, m.k_proj.weight, m.v_proj.weight, m.out_proj.weight, num_heads=6)
    assert torch.equal(fused, direct)
    err = (fused.float() - unfused.float()).abs().max().item()
    assert err <= 2e-2 * unfused.float().abs().max().item(), err


def test_module_with_autograd_keeps_the_unfused_path(cuda):
    """With autograd the module runs projections + attention kernel (which
    has a backward); the result matches the fused inference output."""
    torch.manual_seed(8)
    m = MultiHeadAttention(384, 6, causal=True).to(cuda, torch.bfloat16)
    x = randn((4, 40, 384), 71, torch.bfloat16).to(cuda).requires_grad_(True)
    y = m(x)
    y.float().sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    with torch.no_grad():
        yf = m(x)
    assert (y.detach().float() - yf.float()).abs().max().item() <= 2e-2 * yf.float().abs().max().item()


def test_deterministic(cuda):
    x = randn((64, 100, 384), 80, torch.bfloat16).to(cuda)
    ws = [w.to(cuda) for w in layer(384, torch.bfloat16, 81)[0]]
    a = ops.mha_forward(x, *ws, num_heads=6)
    b = ops.mha_forward(x, *ws, num_heads=6)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_rejects_unsupported(cuda):
    x = torch.zeros(2, 10, 384, device=cuda)
    w = torch.zeros(384, 384, device=cuda)
    with pytest.raises(NotImplementedError):
        ops.mha_forward(x, w, w, w, w, num_heads=6)  # fp32
    xb, wb = x.bfloat16(), w.bfloat16()
    with pytest.raises(NotImplementedError):
        ops.mha_forward(xb, wb, wb, wb, wb, num_heads=3)  # head_dim 128


@pytest.mark.parametrize("heads,short,long", [(6, 8, 16), (8, 16, 24), (8, 8, 40)])
def test_module_takes_the_fused_layer_only_where_it_is_faster(cuda, monkeypatch, heads, short, long):
    """Below FUSED_MIN_SEQ the module runs the unfused path (measured faster
    there); from it on, the one-launch layer."""
    from ataraxos_amd import attention as attn_mod

    _announce(f"mha dispatch h={heads}")
    assert short < attn_mod.FUSED_MIN_SEQ[heads] <= long
    calls = []
    real = ops.mha_forward
    monkeypatch.setattr(attn_mod.ops, "mha_forward", lambda *a, **k: calls.append(a[0].shape[1]) or real(*a, **k))
    m = MultiHeadAttention(64 * heads, heads, causal=True).to(cuda, torch.bfloat16).eval()
    with torch.no_grad():
        for seq in (short, long):
            x = randn((2, seq, 64 * heads), 90 + seq, torch.bfloat16).to(cuda)
            m.fuse_layer = False
            ref = m(x)
            m.fuse_layer = True
            got = m(x)
            assert (got.float() - ref.float()).abs().max().item() <= 2e-2 * ref.float().abs().max().item()
    assert calls == [long]


# ---- packed weights (atx_mha_pack_weight + atx_mha_fwd_packed) ---------------


@pytest.mark.parametrize("e,dtype", [(128, torch.bfloat16), (384, torch.bfloat16), (512, torch.float16), (96, torch.bfloat16)])
def test_pack_weight_layout(cuda, e, dtype):
    """The packed order is the header's formula: element
    ((rt * (e / 32) + kt) * 64 + 16 g + m) * 8 + i holds w[16 rt + m, 32 kt + 8 g + i],
    restated as a view/permute of w (row tile, row, k-step, group, element)."""
    _announce(f"pack weight e={e} {dtype}")
    w = randn((e, e), 300 + e, dtype)
    ref = w.view(e // 16, 16, e // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(e, e)
    got = ops.mha_pack_weight(w.to(cuda)).cpu()
    assert torch.equal(got, ref)
    # spot checks of the formula itself, element by element
    flat = got.reshape(-1)
    for rt, kt, g_, m, i in [(0, 0, 0, 0, 0), (1, 2, 3, 5, 7), (e // 16 - 1, e // 32 - 1, 3, 15, 7)]:
        assert flat[((rt * (e // 32) + kt) * 64 + 16 * g_ + m) * 8 + i] == w[16 * rt + m, 32 * kt + 8 * g_ + i]


def _random_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        h = int(rng.choice([2, 4, 6, 8]))
        l = int(rng.integers(1, 129))
        if not ops.mha_forward_supported(64 * h, h, l, torch.bfloat16):
            continue
        dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
        cases.append((int(rng.integers(1, 6)), l, h, dtype, bool(rng.random() < 0.5), bool(rng.random() < 0.3)))
    return cases


@pytest.mark.parametrize("b,l,h,dtype,causal,bias", _random_cases(24, 2024))
def test_packed_random_shapes_against_the_oracle(cuda, b, l, h, dtype, causal, bias):
    """The module's path (packed weights) against the float64 oracle on a
    seeded sweep of supported shapes: every head count, lengths 1..128,
    causal or not, biases, bf16 and fp16."""
    run_case(cuda, b, l, h, dtype=dtype, causal=causal, bias=bias, seed=500 + l + 7 * h, packed=True)


@pytest.mark.parametrize(
    "b,l,h,dtype,causal,bias",
    [
        (8, 100, 6, torch.bfloat16, False, False),
        (4, 100, 8, torch.bfloat16, False, False),
        (4, 40, 8, torch.bfloat16, True, False),
        (4, 64, 4, torch.float16, False, True),
        (3, 128, 2, torch.bfloat16, True, True),
        (3, 17, 6, torch.bfloat16, False, False),
        (5, 1, 4, torch.bfloat16, False, False),
        (3, 112, 8, torch.float16, True, True),
    ],
)
def test_packed_equals_row_major(cuda, b, l, h, dtype, causal, bias):
    """atx_mha_fwd_packed reads the same weights in another order and does the
    same arithmetic: bit-identical to atx_mha_fwd, which the float64 oracle
    pins (the tests above)."""
    e = 64 * h
    _announce(f"mha packed b={b} l={l} h={h} {dtype} causal={causal} bias={bias}")
    x = randn((b, l, e), 400 + l + h, dtype).to(cuda)
    ws, bs = layer(e, dtype, 401 + l + h, bias)
    wd = [w.to(cuda) for w in ws]
    bd = [t.to(cuda) if t is not None else None for t in bs]
    kw = dict(num_heads=h, b_q=bd[0], b_k=bd[1], b_v=bd[2], b_o=bd[3], causal=causal)
    plain = ops.mha_forward(x, *wd, **kw)
    packed = ops.mha_forward(x, *[ops.mha_pack_weight(w) for w in wd], packed=True, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(plain.float()).all()
    assert torch.equal(plain, packed)


def test_module_repacks_after_a_weight_update(cuda):
    """The module's fused path rearranges the weights on every call, so it
    follows in-place updates (an optimizer step, load_state_dict, the EMA
    swap's ``param.data.copy_`` of ema.py:67,80, which moves no version
    counter) and replaced parameters."""
    _announce("mha module weight updates")
    torch.manual_seed(9)
    m = MultiHeadAttention(384, 6).to(cuda, torch.bfloat16).eval()
    x = randn((4, 100, 384), 72, torch.bfloat16).to(cuda)

    def direct():
        return ops.mha_forward(x, m.q_proj.weight, m.k_proj.weight, m.v_proj.weight, m.out_proj.weight, num_heads=6)

    with torch.no_grad():
        y0 = m(x)
        assert torch.equal(y0, direct())
        m.k_proj.weight.mul_(1.5)  # in place: version counter moves
        y1 = m(x)
        assert not torch.equal(y1, y0)
        assert torch.equal(y1, direct())
        m.load_state_dict({k: v * 0.5 for k, v in m.state_dict().items()})
        y2 = m(x)
        assert torch.equal(y2, direct())
        m.v_proj.weight = torch.nn.Parameter(torch.flip(m.v_proj.weight, dims=[0]))  # replaced
        y3 = m(x)
        assert torch.equal(y3, direct())
        assert not torch.equal(y3, y2)
        # EMA apply / restore: shadow values copied in through .data
        shadow = {n: (p.detach() * 0.75).flip(0) for n, p in m.named_parameters()}
        versions = [p._version for p in m.parameters()]
        for n, p in m.named_parameters():
            p.data.copy_(shadow[n])
        assert [p._version for p in m.parameters()] == versions  # invisible to a version check
        y4 = m(x)
        assert torch.equal(y4, direct())
        assert not torch.equal(y4, y3)
        m.fuse_layer = False
        unfused = m(x)
        m.fuse_layer = True
    err = (y4.float() - unfused.float()).abs().max().item()
    assert err <= 2e-2 * unfused.float().abs().max().item(), err


def test_workspace_entry_point_equals_row_major(cuda):
    """atx_mha_fwd_ws (weights rearranged into the caller's workspace on every
    call, then the packed kernel) is bit-identical to atx_mha_fwd; a
    workspace too small or overlapping an operand is refused."""
    _announce("mha workspace entry point")
    for (b, l, h, causal, bias) in [(8, 100, 6, False, False), (4, 40, 8, True, True), (3, 17, 2, False, True)]:
        e = 64 * h
        x = randn((b, l, e), 500 + l, torch.bfloat16).to(cuda)
        ws, bs = layer(e, torch.bfloat16, 501 + l, bias)
        wd = [w.to(cuda) for w in ws]
        bd = [t.to(cuda) if t is not None else None for t in bs]
        kw = dict(num_heads=h, b_q=bd[0], b_k=bd[1], b_v=bd[2], b_o=bd[3], causal=causal)
        plain = ops.mha_forward(x, *wd, **kw)
        work = torch.full((ops.mha_workspace_bytes(e) + 256,), 0xFF, dtype=torch.uint8, device=cuda)
        got = ops.mha_forward(x, *wd, repack=True, workspace=work, **kw)
        torch.cuda.synchronize()
        assert torch.equal(plain, got), (b, l, h)
    assert _lib.load().atx_mha_workspace_bytes(384) == ops.mha_workspace_bytes(384) == 4 * 384 * 384 * 2
    with pytest.raises(ValueError, match="workspace"):
        ops.mha_forward(x, *wd, repack=True, workspace=work[: ops.mha_workspace_bytes(e) - 1], **kw)


def test_module_built_under_inference_mode(cuda):
    """Parameters created under inference_mode (no version counter): in-place
    changes take effect on the next call."""
    _announce("mha module under inference_mode")
    x = randn((4, 100, 384), 73, torch.bfloat16).to(cuda)
    with torch.inference_mode():
        torch.manual_seed(10)
        m = MultiHeadAttention(384, 6).to(cuda, torch.bfloat16).eval()
        assert m.q_proj.weight.is_inference()
        y0 = m(x)
        m.q_proj.weight.mul_(-1.0)
        y1 = m(x)
        direct = ops.mha_forward(x, m.q_proj.weight, m.k_proj.weight, m.v_proj.weight, m.out_proj.weight, num_heads=6)
    assert not torch.equal(y0, y1)
    assert torch.equal(y1, direct)


@pytest.mark.parametrize(
    "b,l,dtype,causal,bias,packed,x_view",
    [
        (1, 100, torch.bfloat16, False, False, True, False),
        (3, 65, torch.bfloat16, False, True, True, False),
        (300, 100, torch.bfloat16, False, False, True, False),
        (513, 101, torch.float16, False, True, False, False),
        (257, 80, torch.bfloat16, True, False, True, True),
        (40, 97, torch.float16, True, True, True, False),
        (600, 96, torch.bfloat16, False, False, False, True),
        (2, 81, torch.bfloat16, False, False, False, False),
    ],
)
def test_persistent_form_equals_the_one_workgroup_per_sample_form(cuda, monkeypatch, b, l, dtype, causal, bias, packed, x_view):
    """6 heads at 65-101 positions run the persistent producer/consumer kernel
    (one workgroup per CU looping over samples).  It does the arithmetic of
    the one-workgroup-per-sample kernel, which the float64 oracle pins above,
    in the same order: the outputs are bit-identical.  Batches past the CU
    count make workgroups run 2-3 samples; NaN guards around a strided x and
    around y check that nothing outside the views is read or written."""
    e = 384
    _announce(f"mha persistent form b={b} l={l} {dtype} causal={causal} bias={bias} packed={packed} view={x_view}")
    x = randn((b, l, e), 700 + l + b, dtype)
    if x_view:
        big = torch.full((b, l + 3, e + 64), float("nan"), dtype=dtype)
        big[:, :l, :e] = x
        xd = big.to(cuda)[:, :l, :e]
    else:
        xd = x.to(cuda)
    ws, bs = layer(e, dtype, 701 + l, bias)
    wd = [w.to(cuda) for w in ws]
    if packed:
        wd = [ops.mha_pack_weight(w) for w in wd]
    bd = [t.to(cuda) if t is not None else None for t in bs]
    kw = dict(num_heads=6, b_q=bd[0], b_k=bd[1], b_v=bd[2], b_o=bd[3], causal=causal, packed=packed)
    outs = []
    for form in ("1", "0"):
        monkeypatch.setenv("ATX_MHA_PERSISTENT", form)
        guard = torch.full((b, l + 2, e), 3.0, dtype=dtype, device=cuda)
        ops.mha_forward(xd, *wd, out=guard[:, :l], **kw)
        torch.cuda.synchronize()
        assert (guard[:, l:] == 3.0).all(), "rows past the sequence were written"
        outs.append(guard[:, :l].clone())
    assert torch.isfinite(outs[0].float()).all()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize(
    "b,l,dtype,causal,bias,packed,x_view",
    [
        (4, 101, torch.bfloat16, False, False, True, False),
        (3, 101, torch.bfloat16, False, True, False, False),
        (3, 100, torch.float16, False, False, True, True),
        (5, 1, torch.bfloat16, False, False, True, False),
        (3, 17, torch.bfloat16, True, False, False, False),
        (2, 40, torch.float16, True, True, True, False),
        (3, 64, torch.bfloat16, False, False, True, False),
        (2, 128, torch.bfloat16, True, True, True, False),
    ],
)
def test_head_dim_48_reference_move_layer(cuda, b, l, dtype, causal, bias, packed, x_view):
    """The reference Move network's layer, MultiHeadAttention(384, 8) with
    head_dim 48 (constants.py:149-150, move_net.py:142-149) at its 101
    tokens and other lengths, against the float64 oracle (scale 1/sqrt(48))."""
    run_case(cuda, b, l, 8, dtype=dtype, causal=causal, bias=bias, seed=800 + l, x_view=x_view, packed=packed, d=48)


def test_head_dim_48_module_takes_the_fused_layer(cuda, monkeypatch):
    """MultiHeadAttention(384, 8) in inference at L=101 runs the one-launch
    layer (no separate q/k/v projection), and equals the unfused module path
    within the 16-bit tolerance."""
    _announce("mha module 8x48 fused path")
    torch.manual_seed(11)
    m = MultiHeadAttention(384, 8).to(cuda, torch.bfloat16).eval()
    x = randn((6, 101, 384), 74, torch.bfloat16).to(cuda)
    calls = []
    real = ops.mha_forward
    monkeypatch.setattr(ops, "mha_forward", lambda *a, **k: calls.append(1) or real(*a, **k))
    with torch.no_grad():
        fused = m(x)
        m.fuse_layer = False
        unfused = m(x)
    torch.cuda.synchronize()
    assert calls, "the module did not take the fused layer"
    names = ("q_proj", "k_proj", "v_proj", "out_proj")
    weights = {f"{n}.weight": to_np64(getattr(m, n).weight) for n in names}
    ref = oracle_mha(to_np64(x), None, weights, 8)
    for y in (fused, unfused):
        err = float(np.max(np.abs(to_np64(y) - ref)))
        assert err <= 2e-2 * max(1.0, float(np.max(np.abs(ref)))), err


def test_head_dim_48_full_batch_sampled_rows(cuda):
    """B=4096 at the reference Move network's shape (L=101, 8 x 48), one
    launch; sampled rows against the float64 oracle on those rows alone."""
    b, l, e = 4096, 101, 384
    _announce(f"mha 8x48 full batch b={b} l={l}")
    x = randn((b, l, e), 810, torch.bfloat16)
    ws, _ = layer(e, torch.bfloat16, 811)
    xd = x.to(cuda)
    y = ops.mha_forward(xd, *[ops.mha_pack_weight(w.to(cuda)) for w in ws], num_heads=8, packed=True)
    torch.cuda.synchronize()
    rows = [0, 1, 255, 256, 2047, 4095] + list(range(77, 4000, 613))
    names = ("q_proj", "k_proj", "v_proj", "out_proj")
    weights = {f"{n}.weight": to_np64(w) for n, w in zip(names, ws)}
    ref = oracle_mha(to_np64(x[rows]), None, weights, 8)
    got = to_np64(y[rows])
    err = float(np.max(np.abs(got - ref)))
    assert np.isfinite(got).all()
    assert err <= 2e-2, err


def test_persistent_layer_that_gives_up_a_wait_writes_nan(cuda, monkeypatch):
    """The persistent layer's waves wait on each other through bounded polls.
    If a wait ever gave up (a broken schedule), the workgroup overwrites its
    samples' Y with NaN instead of leaving plausible wrong numbers.  Forced
    here from the host: ATX_MHA_WS_SPIN=1 lets every wait poll once, so the
    consumers' first wait (for the producers' first store) gives up; every
    wave still runs to its end.  512 samples make workgroups run two each;
    rows past the sequence stay unwritten."""
    b, l, e = 512, 100, 384
    _announce("mha persistent form, waits limited to one poll")
    monkeypatch.setenv("ATX_MHA_PERSISTENT", "1")
    x = randn((b, l, e), 77, torch.bfloat16).to(cuda)
    ws, _ = layer(e, torch.bfloat16, 78, False)
    pk = [ops.mha_pack_weight(w.to(cuda)) for w in ws]
    good = ops.mha_forward(x, *pk, num_heads=6, packed=True)
    monkeypatch.setenv("ATX_MHA_WS_SPIN", "1")
    guard = torch.full((b, l + 2, e), 3.0, dtype=torch.bfloat16, device=cuda)
    ops.mha_forward(x, *pk, num_heads=6, packed=True, out=guard[:, :l])
    torch.cuda.synchronize()
    assert torch.isnan(guard[:, :l].float()).all()
    assert (guard[:, l:] == 3.0).all(), "rows past the sequence were written"
    monkeypatch.delenv("ATX_MHA_WS_SPIN")
    again = ops.mha_forward(x, *pk, num_heads=6, packed=True)
    assert torch.isfinite(good.float()).all() and torch.equal(good, again)
