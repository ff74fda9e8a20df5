"""Parity of the HIP attention backward (``atx_attn_bwd``) against the
float64 oracle's gradients.

Every case draws seeded inputs on the CPU, runs the HIP forward (whose bf16
output is what training keeps) and then ``atx_attn_bwd`` through the C ABI
(``ataraxos_amd.ops.attention_backward``), and compares dQ, dK, dV with
``oracle.attention.attention_backward`` run in float64 on the same
bf16/fp16-rounded inputs.

Tolerance.  The contract's figure for 16-bit results is 2e-2 max-abs on
outputs of unit scale.  Gradients scale with the upstream gradient, so each
one is held to ``max|g - ref| <= 2e-2 * max|ref|`` (normwise relative), plus
``||g - ref||_F <= 1e-2 * ||ref||_F``.  fp32 gradients (fp32 products
throughout) are held to ``1e-4 * max|ref|`` and ``2e-5`` in Frobenius norm;
where they vanish exactly, ``max|ref|`` is floored at 4e-2, i.e. an absolute
4e-6: dQ = scale * P * (dP - delta) with dP and delta = sum_d O dO each an
fp32 sum of 64 unit-scale products, whose rounding is ~64 * 6e-8.  Where the exact gradient vanishes
(``S_kv = 1`` makes dQ and dK 0 in exact arithmetic) ``max|ref|`` is floored at
1e-4, i.e. an absolute 2e-6.  NaNs (rows that see no key) must coincide
exactly, and gradients of padded keys must be exactly 0.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import ops
from oracle.attention import attention_backward as oracle_backward
from tests._cases import randn, to_np64

pytestmark = pytest.mark.gpu

REL_MAX = 2e-2
REL_FRO = 1e-2
ZERO_FLOOR = 1e-4


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


FP32_REL_MAX = 1e-4
FP32_REL_FRO = 2e-5
FP32_ZERO_FLOOR = 4e-2


def assert_grad_close(got: torch.Tensor, ref: np.ndarray, what: str) -> float:
    fp32 = got.dtype == torch.float32
    rel_max, rel_fro = (FP32_REL_MAX, FP32_REL_FRO) if fp32 else (REL_MAX, REL_FRO)
    floor = FP32_ZERO_FLOOR if fp32 else ZERO_FLOOR
    g = to_np64(got)
    assert g.shape == ref.shape, f"{what}: shape {g.shape} vs {ref.shape}"
    nan_g, nan_r = np.isnan(g), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN pattern differs ({nan_g.sum()} vs {nan_r.sum()})"
    g, r = g[~nan_r], ref[~nan_r]
    if r.size == 0:
        return 0.0
    scale = max(float(np.max(np.abs(r))), floor)
    err = float(np.max(np.abs(g - r)))
    assert err <= rel_max * scale, f"{what}: max-abs {err:.3e} > {rel_max} * {scale:.3e}"
    if scale > floor:
        fro = float(np.linalg.norm(g - r) / np.linalg.norm(r))
        assert fro <= rel_fro, f"{what}: relative Frobenius error {fro:.3e} > {rel_fro}"
    return err / scale


def inputs(b, sq, skv, h, d, dtype, seed, std=1.0, hkv=None):
    hkv = h if hkv is None else hkv
    q = randn((b, sq, h, d), seed, dtype, std)
    k = randn((b, skv, hkv, d), seed + 1, dtype, std)
    v = randn((b, skv, hkv, d), seed + 2, dtype)
    g = randn((b, sq, h, d), seed + 3, dtype)
    return q, k, v, g


def _on_gpu(pad, cuda, view):
    """The padding mask on the GPU; with ``view``, as columns 1 .. skv of a
    wider mask whose other columns are True, so that its rows start at odd
    addresses with an odd stride (the kernels' byte-load path)."""
    if not view:
        return pad.to(cuda)
    b, skv = pad.shape
    big = torch.ones(b, skv + 3, dtype=torch.bool)
    big[:, 1 : skv + 1] = pad
    return big.to(cuda)[:, 1 : skv + 1]


def run_case(cuda, b, sq, skv, h, d, dtype, causal=False, pad_p=None, seed=0, std=1.0, scale=None, pad_view=False,
             hkv=None):
    _announce(f"bwd b={b} sq={sq} skv={skv} h={h}/{hkv or h} d={d} {dtype} causal={causal} pad={pad_p} std={std}")
    q, k, v, g = inputs(b, sq, skv, h, d, dtype, seed, std, hkv)
    pad = None
    if pad_p is not None:
        gen = torch.Generator().manual_seed(seed + 4)
        pad = torch.rand(b, skv, generator=gen) < pad_p
    qd, kd, vd, gd = (t.to(cuda) for t in (q, k, v, g))
    padd = None if pad is None else _on_gpu(pad, cuda, pad_view)
    out = ops.attention_forward(qd, kd, vd, causal=causal, scale=scale, key_padding_mask=padd)
    dq, dk, dv = ops.attention_backward(qd, kd, vd, out, gd, causal=causal, scale=scale, key_padding_mask=padd)
    torch.cuda.synchronize()
    ref = oracle_backward(to_np64(q), to_np64(k), to_np64(v), to_np64(g), causal=causal, scale=scale,
                          key_pad=None if pad is None else pad.numpy())
    errs = [assert_grad_close(a, r, f"{n} b={b} sq={sq} skv={skv} d={d} {dtype}") for n, a, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref)]
    if pad is not None:
        # exactly 0, except in a dv slice a row that sees no key made NaN
        # (whose pattern was matched against the oracle above)
        padded = pad.to(cuda)[:, :, None, None].expand_as(dk)
        assert (dk[padded] == 0).all(), "padded keys must get exactly 0 in dk"
        assert ((dv[padded] == 0) | dv[padded].isnan()).all(), "padded keys must get exactly 0 in dv"
    return errs


# --- the shapes of the reference's networks ---------------------------------


def test_move_net_layer_bf16(cuda):
    """C3 shape (L=100, 6 x 64, bf16) at B=64 against the float64 oracle."""
    run_case(cuda, 64, 100, 100, 6, 64, torch.bfloat16, seed=10)


def test_setup_net_causal_bf16(cuda):
    """Setup network: causal self-attention over 40 pieces."""
    run_case(cuda, 32, 40, 40, 8, 64, torch.bfloat16, causal=True, seed=11)


def test_belief_decoder_cross_with_padding(cuda):
    """Belief decoder: 40 queries over 100 encoder tokens with key padding."""
    run_case(cuda, 32, 40, 100, 8, 64, torch.bfloat16, pad_p=0.3, seed=12)


def test_belief_decoder_causal_self(cuda):
    run_case(cuda, 32, 40, 40, 8, 64, torch.bfloat16, causal=True, seed=13)


def test_move_net_full_batch_against_torch_fp32(cuda):
    """C3 at full size (B=4096): against torch fp32 autograd of the same math on
    the GPU (the float64 oracle would take minutes), and run-to-run bitwise
    determinism of the kernel."""
    _announce("bwd C3 full batch 4096x100x6x64 bf16")
    b, s, h, d = 4096, 100, 6, 64
    q, k, v, g = (t.to(cuda) for t in inputs(b, s, s, h, d, torch.bfloat16, seed=20))
    out = ops.attention_forward(q, k, v)
    dq, dk, dv = ops.attention_backward(q, k, v, out, g)
    again = ops.attention_backward(q, k, v, out, g)
    torch.cuda.synchronize()
    for a, bb in zip((dq, dk, dv), again):
        assert torch.equal(a, bb)
    qf, kf, vf = (t.float().transpose(1, 2).contiguous().requires_grad_(True) for t in (q, k, v))
    p = torch.softmax(torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * 0.125, dim=-1)
    o = torch.matmul(p, vf)
    want = torch.autograd.grad(o, (qf, kf, vf), g.float().transpose(1, 2))
    for name, a, w in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        w = w.transpose(1, 2)
        scale = w.abs().max().item()
        err = (a.float() - w).abs().max().item()
        assert err <= REL_MAX * scale, f"{name}: {err:.3e} > {REL_MAX} * {scale:.3e}"
        fro = ((a.float() - w).norm() / w.norm()).item()
        assert fro <= REL_FRO, f"{name}: relative Frobenius {fro:.3e}"


# --- coverage of the kernel's range ------------------------------------------


@pytest.mark.parametrize("d", [16, 32, 48, 64, 80, 96, 112, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_head_dims(cuda, d, dtype):
    run_case(cuda, 4, 100, 100, 3, d, dtype, seed=30 + d)


@pytest.mark.parametrize("s", [1, 2, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 97, 128, 129, 200, 256])
def test_seq_lengths(cuda, s):
    run_case(cuda, 3, s, s, 2, 64, torch.bfloat16, seed=40 + s)


@pytest.mark.parametrize("s", [1, 17, 40, 100, 256])
def test_causal(cuda, s):
    run_case(cuda, 3, s, s, 4, 64, torch.bfloat16, causal=True, seed=60 + s)


@pytest.mark.parametrize("sq,skv", [(1, 256), (256, 1), (40, 100), (100, 40), (17, 200), (200, 17), (33, 65)])
@pytest.mark.parametrize("causal", [False, True])
def test_cross_attention(cuda, sq, skv, causal):
    """S_q != S_kv, with the top-left causal mask of the reference."""
    run_case(cuda, 3, sq, skv, 4, 32, torch.bfloat16, causal=causal, seed=70 + sq + skv)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_key_padding(cuda, causal, dtype):
    run_case(cuda, 8, 64, 100, 4, 64, dtype, causal=causal, pad_p=0.4, seed=80)


def test_large_head_dim_long_sequence(cuda):
    """D=128 at the longest sequence whose tiles fit in LDS at once (S=128),
    and beyond it (S=200, 256), where the queries are staged in blocks."""
    assert not ops.attention_backward_plan(128, 128, 128, 2, 2, torch.bfloat16)["loop"]
    assert ops.attention_backward_plan(128, 129, 129, 2, 2, torch.bfloat16)["loop"]
    run_case(cuda, 2, 128, 128, 2, 128, torch.bfloat16, seed=90)
    run_case(cuda, 2, 200, 200, 2, 128, torch.bfloat16, causal=True, seed=93)
    run_case(cuda, 2, 256, 256, 2, 112, torch.float16, pad_p=0.3, seed=94)


def test_large_logits_are_stable(cuda):
    """Scores of magnitude ~100 (std 3 inputs): the recomputed softmax stays exact."""
    run_case(cuda, 4, 100, 100, 4, 64, torch.bfloat16, std=3.0, seed=91)


def test_scale_argument(cuda):
    run_case(cuda, 4, 50, 70, 4, 64, torch.bfloat16, scale=0.05, seed=92)


def test_rows_that_see_no_key(cuda):
    """Fully padded batch rows and, with causal, rows whose visible keys are all
    padded: dq and dk get 0 from them and that (batch, head)'s dv is NaN, as
    autograd through the reference's masked_fill + softmax gives."""
    _announce("bwd rows that see no key")
    b, s, h, d = 4, 40, 2, 64
    q, k, v, g = inputs(b, s, s, h, d, torch.bfloat16, seed=93)
    pad = torch.zeros(b, s, dtype=torch.bool)
    pad[1] = True  # every key of batch row 1
    pad[2, :5] = True  # with causal, query rows 0..4 of batch row 2 see nothing
    for causal in (False, True):
        qd, kd, vd, gd, pd = (t.to(cuda) for t in (q, k, v, g, pad))
        out = ops.attention_forward(qd, kd, vd, causal=causal, key_padding_mask=pd)
        got = ops.attention_backward(qd, kd, vd, out, gd, causal=causal, key_padding_mask=pd)
        torch.cuda.synchronize()
        ref = oracle_backward(to_np64(q), to_np64(k), to_np64(v), to_np64(g), causal=causal, key_pad=pad.numpy())
        for n, a, r in zip(("dq", "dk", "dv"), got, ref):
            assert_grad_close(a, r, f"{n} causal={causal}")
        assert (got[0][1] == 0).all() and (got[1][1] == 0).all() and torch.isnan(got[2][1]).all()


def test_strided_views_and_guard_rows(cuda):
    """Inputs as views of a packed [B, S+7, 3, H, D] buffer whose rows past the
    sequence hold NaN, and a non-contiguous upstream gradient: nothing past
    the sequence is read, strides are honoured."""
    _announce("bwd strided packed views")
    b, s, h, d = 6, 50, 4, 64
    base = randn((b, s + 7, 3, h, d), 94, torch.bfloat16)
    base[:, s:] = float("nan")
    g_full = randn((b, h, s, d), 95, torch.bfloat16)
    based = base.to(cuda)
    qd, kd, vd = based[:, :s, 0], based[:, :s, 1], based[:, :s, 2]
    gd = g_full.to(cuda).transpose(1, 2)  # [B, S, H, D], non-contiguous
    out = ops.attention_forward(qd, kd, vd, causal=True)
    got = ops.attention_backward(qd, kd, vd, out, gd, causal=True)
    torch.cuda.synchronize()
    ref = oracle_backward(to_np64(base[:, :s, 0]), to_np64(base[:, :s, 1]), to_np64(base[:, :s, 2]),
                          to_np64(g_full.transpose(1, 2)), causal=True)
    for n, a, r in zip(("dq", "dk", "dv"), got, ref):
        assert_grad_close(a, r, n)


# --- autograd integration ----------------------------------------------------


def test_autograd_takes_the_hip_backward(cuda):
    """``ops.attention`` under autograd returns exactly what the kernel returns."""
    _announce("bwd autograd integration")
    q, k, v, g = (t.to(cuda) for t in inputs(4, 100, 100, 6, 64, torch.bfloat16, seed=96))
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qa, ka, va, causal=False)
    got = torch.autograd.grad(out, (qa, ka, va), g)
    want = ops.attention_backward(q, k, v, out.detach(), g)
    for a, w in zip(got, want):
        assert torch.equal(a, w)


def test_module_backward_matches_oracle(cuda):
    """``MultiHeadAttention`` in bf16 on the GPU: the input gradient through
    projections + HIP attention + HIP backward agrees with float64 autograd
    of the module's math on the same bf16 parameters."""
    _announce("bwd module bf16")
    from ataraxos_amd import MultiHeadAttention

    torch.manual_seed(5)
    m = MultiHeadAttention(384, 6).to(cuda, torch.bfloat16)
    x = randn((8, 100, 384), 97, torch.bfloat16).to(cuda).requires_grad_(True)
    g = randn((8, 100, 384), 98, torch.bfloat16).to(cuda)
    (gx,) = torch.autograd.grad(m(x), (x,), g)
    m64 = MultiHeadAttention(384, 6).double()
    m64.load_state_dict({k2: t.double().cpu() for k2, t in m.state_dict().items()})
    x64 = x.detach().double().cpu().requires_grad_(True)
    (want,) = torch.autograd.grad(m64(x64), (x64,), g.double().cpu())
    err = (gx.double().cpu() - want).abs().max().item()
    assert err <= REL_MAX * want.abs().max().item(), err


# --- grouped-query attention, fp32, long query sequences ----------------------


@pytest.mark.parametrize("hkv", [2, 4])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_gqa(cuda, hkv, dtype):
    """8 query heads over 2 or 4 KV heads (test_attention.py:119-133): dk, dv
    sum the gradients of each group (attention.py:210-220)."""
    run_case(cuda, 4, 100, 100, 8, 64, dtype, hkv=hkv, seed=600 + hkv)


@pytest.mark.parametrize("causal,pad", [(True, None), (False, 0.4), (True, 0.3)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gqa_masked(cuda, causal, pad, dtype):
    run_case(cuda, 3, 40, 72, 8, 32, dtype, causal=causal, pad_p=pad, hkv=2, seed=610)


@pytest.mark.parametrize("d", [16, 48, 64, 128])
def test_gqa_head_dims(cuda, d):
    run_case(cuda, 2, 33, 65, 4, d, torch.bfloat16, hkv=1, seed=620 + d)


@pytest.mark.parametrize(
    "b,sq,skv,h,d,causal,pad",
    [
        (4, 101, 101, 8, 48, False, None),  # Move network (constants.py:149-150, L=101)
        (4, 40, 40, 8, 64, True, None),     # Setup network
        (4, 100, 100, 8, 64, False, None),  # Belief encoder
        (4, 40, 100, 8, 64, False, 0.4),    # Belief decoder cross-attention
        (4, 100, 100, 6, 64, False, None),  # config 1's layer
    ],
)
def test_fp32_reference_shapes(cuda, b, sq, skv, h, d, causal, pad):
    """fp32 -- what the reference's trainers run (they never enter the AMP
    helper) -- at the shapes of its networks."""
    assert ops.attention_backward_supported(d, sq, skv, h, h, torch.float32)
    run_case(cuda, b, sq, skv, h, d, torch.float32, causal=causal, pad_p=pad, seed=630 + d + sq)


@pytest.mark.parametrize("d", [16, 32, 80, 96, 112, 128])
def test_fp32_head_dims(cuda, d):
    run_case(cuda, 2, 57, 90, 2, d, torch.float32, seed=640 + d)


@pytest.mark.parametrize("sq,skv", [(1, 1), (17, 256), (256, 17), (256, 256)])
@pytest.mark.parametrize("causal", [False, True])
def test_fp32_seq_lengths(cuda, sq, skv, causal):
    run_case(cuda, 2, sq, skv, 2, 64, torch.float32, causal=causal, seed=650 + sq + skv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("sq,skv,causal", [(300, 100, False), (520, 256, True), (257, 40, False)])
def test_long_query_sequences_in_blocks(cuda, dtype, sq, skv, causal):
    """More than 256 queries: the backward stages them in blocks and sums
    dK / dV over the blocks."""
    plan = ops.attention_backward_plan(64, sq, skv, 2, 2, dtype)
    assert plan["loop"] and plan["query_block"] < sq
    run_case(cuda, 2, sq, skv, 2, 64, dtype, causal=causal, seed=660 + sq)


def test_loop_variant_is_deterministic(cuda):
    q, k, v, g = (t.to(cuda) for t in inputs(4, 300, 100, 8, 64, torch.bfloat16, seed=670, hkv=2))
    out = ops.attention_forward(q, k, v)
    a = ops.attention_backward(q, k, v, out, g)
    b2 = ops.attention_backward(q, k, v, out, g)
    torch.cuda.synchronize()
    assert all(torch.equal(x, y) for x, y in zip(a, b2))


@pytest.mark.parametrize("dtype,hkv", [(torch.float32, 8), (torch.bfloat16, 2), (torch.float32, 2)])
def test_autograd_uses_the_hip_backward_for_fp32_and_gqa(cuda, dtype, hkv):
    """Under autograd, fp32 and GQA gradients are exactly the kernel's."""
    q, k, v, g = (t.to(cuda) for t in inputs(2, 40, 60, 8, 32, dtype, seed=680, hkv=hkv))
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = ops.attention(qa, ka, va, causal=True)
    got = torch.autograd.grad(out, (qa, ka, va), g)
    want = ops.attention_backward(q, k, v, out.detach(), g, causal=True)
    for a, w in zip(got, want):
        assert torch.equal(a, w)


def test_fp32_beyond_lds_falls_back_under_autograd(cuda):
    """fp32 with head_dim >= 80 and more than 128 keys (K and V rows do not fit
    in LDS; used by no network of the reference): attention_backward refuses
    it and autograd differentiates an fp32 recomputation."""
    assert not ops.attention_backward_supported(128, 50, 200, 2, 2, torch.float32)
    q = torch.randn(2, 50, 2, 128, device=cuda)
    k = torch.randn(2, 200, 2, 128, device=cuda)
    with pytest.raises(NotImplementedError):
        ops.attention_backward(q, k, k, q, q)
    qa, ka = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    ops.attention(qa, ka, ka).sum().backward()
    assert torch.isfinite(qa.grad).all() and torch.isfinite(ka.grad).all()


@pytest.mark.parametrize("skv,dtype,view", [(129, torch.bfloat16, False), (200, torch.float16, True), (256, torch.bfloat16, True)])
def test_key_padding_long_rows(cuda, skv, dtype, view):
    """Backward with key padding over 129..256 keys (every lane of the
    per-lane padding words), mask rows 4-byte aligned or at odd addresses."""
    run_case(cuda, 3, 48, skv, 4, 64, dtype, pad_p=0.5, seed=700 + skv, pad_view=view)
