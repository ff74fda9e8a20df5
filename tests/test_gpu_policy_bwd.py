"""Parity of the policy-head backward (``atx_kq_bwd``) against the float64
oracle's gradients (``oracle.policy.kq_backward``).

Inputs are drawn on the CPU from seeded generators; q, k are rounded to the
kernel's 16-bit dtype first, and the oracle runs in float64 on the same
values.  In probs mode the kernel is given the HIP forward's probabilities.

Tolerance (gradients scale with the upstream gradient, so it is relative to
each gradient's own size): ``max|g - ref| <= 2e-2 * max|ref|`` and
``||g - ref||_F <= 1e-2 * ||ref||_F``; where the exact gradient vanishes,
``max|ref|`` is floored at 1e-4.  A sample with no legal entry must get
exactly 0.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import KeyQueryPolicyHead, masked_policy_logits, masked_policy_softmax, ops
from oracle.policy import kq_backward
from tests._cases import legal_mask, randn, to_np64

pytestmark = pytest.mark.gpu

REL_MAX = 2e-2
REL_FRO = 1e-2
ZERO_FLOOR = 1e-4


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


# fp32 q, k (fp32 products): 1e-4 of the gradient's scale, 2e-5 Frobenius
FP32_REL_MAX = 1e-4
FP32_REL_FRO = 2e-5


def assert_grad_close(got: torch.Tensor, ref: np.ndarray, what: str) -> None:
    rel_max, rel_fro = (FP32_REL_MAX, FP32_REL_FRO) if got.dtype == torch.float32 else (REL_MAX, REL_FRO)
    g = to_np64(got)
    assert g.shape == ref.shape, f"{what}: shape {g.shape} vs {ref.shape}"
    assert np.isfinite(g).all(), f"{what}: non-finite values"
    scale = max(float(np.max(np.abs(ref))), ZERO_FLOOR)
    err = float(np.max(np.abs(g - ref)))
    assert err <= rel_max * scale, f"{what}: max-abs {err:.3e} > {rel_max} * {scale:.3e}"
    if scale > ZERO_FLOOR:
        fro = float(np.linalg.norm(g - ref) / np.linalg.norm(ref))
        assert fro <= rel_fro, f"{what}: relative Frobenius error {fro:.3e} > {rel_fro}"


def run_case(cuda, b, s, d, dtype, output, p_legal=0.02, seed=0, scale=None, empty_sample=False, mask_view=False,
             grad_view=False):
    _announce(f"kq bwd b={b} s={s} d={d} {dtype} {output} p={p_legal} empty={empty_sample} view={mask_view} "
              f"grad_view={grad_view}")
    q = randn((b, s, d), seed, dtype)
    k = randn((b, s, d), seed + 1, dtype)
    mask = None if p_legal is None else legal_mask(b, s, seed + 2, p_legal)
    if mask is not None and empty_sample:
        mask[b // 2] = False
    grad = randn((b, s * s), seed + 3, torch.float32)
    sc = scale if scale is not None else d**-0.5
    qd, kd, gd = q.to(cuda), k.to(cuda), grad.to(cuda)
    if grad_view:  # rows of a wider buffer, one NaN before each: 4-byte aligned, not 16
        big = torch.full((b, s * s + 1), float("nan"), dtype=torch.float32)
        big[:, 1:] = grad
        gd = big.to(cuda)[:, 1:]
    md = None
    if mask is not None:
        if mask_view:  # rows of a wider buffer: row stride s + 3, not a multiple of 4
            big = torch.zeros(b, s, s + 3, dtype=torch.bool)
            big[:, :, :s] = mask
            md = big.to(cuda)[:, :, :s]
        else:
            md = mask.to(cuda)
    probs = ops.kq_policy(qd, kd, md, scale=sc, output="probs") if output == "probs" else None
    dq, dk = ops.kq_policy_backward(qd, kd, gd, md, sc, output=output, probs=probs)
    torch.cuda.synchronize()
    ref = kq_backward(to_np64(q), to_np64(k), None if mask is None else mask.numpy(), sc, grad.numpy().astype(np.float64),
                      wrt=output)
    assert_grad_close(dq, ref[0], f"dq b={b} s={s} d={d} {output}")
    assert_grad_close(dk, ref[1], f"dk b={b} s={s} d={d} {output}")
    if empty_sample:
        assert (dq[b // 2] == 0).all() and (dk[b // 2] == 0).all()


@pytest.mark.parametrize("output", ["logits", "probs"])
def test_config2_shape(cuda, output):
    """C2 (S=100, d=64, Bernoulli(0.02) legal moves, bf16) at B=256."""
    run_case(cuda, 256, 100, 64, torch.bfloat16, output, seed=10)


@pytest.mark.parametrize("output", ["logits", "probs"])
def test_config2_full_batch_against_torch_fp32(cuda, output):
    """C2 at B=4096 against torch fp32 autograd of the reference head's ops
    (matmul, masked_fill(-1e10), softmax) on the GPU; bitwise repeatable."""
    _announce(f"kq bwd C2 full batch {output}")
    b, s, d = 4096, 100, 64
    q, k = randn((b, s, d), 20, torch.bfloat16).to(cuda), randn((b, s, d), 21, torch.bfloat16).to(cuda)
    mask = legal_mask(b, s, 22).to(cuda)
    g = randn((b, s * s), 23, torch.float32).to(cuda)
    probs = ops.kq_policy(q, k, mask, scale=0.125, output="probs") if output == "probs" else None
    got = ops.kq_policy_backward(q, k, g, mask, 0.125, output=output, probs=probs)
    again = ops.kq_policy_backward(q, k, g, mask, 0.125, output=output, probs=probs)
    torch.cuda.synchronize()
    assert torch.equal(got[0], again[0]) and torch.equal(got[1], again[1])
    qf, kf = q.float().requires_grad_(True), k.float().requires_grad_(True)
    logits = (torch.matmul(qf, kf.transpose(1, 2).contiguous()) * 0.125).masked_fill(~mask, -1e10).reshape(b, -1)
    out = torch.softmax(logits, dim=-1) if output == "probs" else logits
    want = torch.autograd.grad(out, (qf, kf), g)
    for name, a, w in zip(("dq", "dk"), got, want):
        scale = w.abs().max().item()
        err = (a.float() - w).abs().max().item()
        assert err <= REL_MAX * scale, f"{name}: {err:.3e} > {REL_MAX} * {scale:.3e}"
        assert ((a.float() - w).norm() / w.norm()).item() <= REL_FRO


@pytest.mark.parametrize("s", [1, 5, 17, 32, 33, 64, 65, 99, 100, 128])
@pytest.mark.parametrize("output", ["logits", "probs"])
def test_seq_lengths(cuda, s, output):
    run_case(cuda, 8, s, 64, torch.bfloat16, output, p_legal=0.3, seed=30 + s)


@pytest.mark.parametrize("d", [16, 32, 48, 64, 80, 96, 112, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dims(cuda, d, dtype):
    run_case(cuda, 8, 100, d, dtype, "logits", p_legal=0.1, seed=50 + d)


@pytest.mark.parametrize("s", [100, 101])
@pytest.mark.parametrize("output", ["logits", "probs"])
def test_no_mask(cuda, s, output):
    run_case(cuda, 8, s, 64, torch.bfloat16, output, p_legal=None, seed=60)


@pytest.mark.parametrize("s", [100, 101])
@pytest.mark.parametrize("output", ["logits", "probs"])
def test_sample_without_legal_moves_gets_zero(cuda, s, output):
    run_case(cuda, 8, s, 64, torch.bfloat16, output, seed=61, empty_sample=True)


@pytest.mark.parametrize("s", [17, 100, 101])
@pytest.mark.parametrize("output", ["logits", "probs"])
def test_mask_rows_of_a_wider_buffer(cuda, s, output):
    """Mask rows not 4-byte aligned: the byte-wise legality path (and, for
    the logits at S % 4 != 0, the flat one)."""
    run_case(cuda, 8, s, 64, torch.bfloat16, output, p_legal=0.3, seed=62, mask_view=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("s", [100, 101])
@pytest.mark.parametrize("output", ["logits", "probs"])
def test_gradient_rows_not_16_byte_aligned(cuda, dtype, s, output):
    """G rows 4-byte but not 16-byte aligned (a view one float into a wider
    buffer, NaN around it): the logits gradient reads the sample's entries
    flat, one per lane, the probabilities gradient piece by piece with 4-byte
    loads; nothing outside the view is read."""
    run_case(cuda, 8, s, 64, dtype, output, p_legal=0.2, seed=63 + s, grad_view=True)


def test_autograd_takes_the_hip_backward(cuda):
    """masked_policy_logits / masked_policy_softmax under autograd return
    exactly the kernel's gradients."""
    _announce("kq bwd autograd")
    b, s, d = 16, 100, 64
    q, k = randn((b, s, d), 70, torch.bfloat16).to(cuda), randn((b, s, d), 71, torch.bfloat16).to(cuda)
    mask = legal_mask(b, s, 72).to(cuda)
    g = randn((b, s * s), 73, torch.float32).to(cuda)
    for fn, output in ((masked_policy_logits, "logits"), (masked_policy_softmax, "probs")):
        qa, ka = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
        out = fn(qa, ka, mask, 0.125)
        got = torch.autograd.grad(out, (qa, ka), g)
        probs = out.detach() if output == "probs" else None
        want = ops.kq_policy_backward(q, k, g, mask, 0.125, output=output, probs=probs)
        for a, w in zip(got, want):
            assert torch.equal(a, w)


def test_policy_head_module_gradients(cuda):
    """KeyQueryPolicyHead in bf16 on the GPU: input gradient through the
    projections and the HIP forward/backward agrees with float64 autograd of
    the head's math on the same parameters."""
    _announce("kq bwd module")
    torch.manual_seed(3)
    head = KeyQueryPolicyHead(128, 64).to(cuda, torch.bfloat16)
    x = randn((8, 100, 128), 80, torch.bfloat16).to(cuda).requires_grad_(True)
    mask = legal_mask(8, 100, 81, 0.1).to(cuda)
    g = randn((8, 100 * 100), 82, torch.float32).to(cuda)
    out = head(x, mask)
    (gx,) = torch.autograd.grad(out.float(), (x,), g)
    h64 = KeyQueryPolicyHead(128, 64).double()
    h64.load_state_dict({n: t.double().cpu() for n, t in head.state_dict().items()})
    x64 = x.detach().double().cpu().requires_grad_(True)
    (want,) = torch.autograd.grad(h64(x64, mask.cpu()), (x64,), g.double().cpu())
    err = (gx.double().cpu() - want).abs().max().item()
    assert err <= REL_MAX * want.abs().max().item(), err


@pytest.mark.parametrize("d", [192, 384, 512])
@pytest.mark.parametrize("output", ["logits", "probs"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_wide_dims(cuda, d, output, dtype):
    """policy_d_model wider than 128, in 64-column slices: the reference's
    Move network builds KeyQueryPolicyHead(dim, dim) with dim 384
    (move_net.py:151, constants.py:149)."""
    assert ops.kq_policy_backward_supported(101, d, dtype)
    run_case(cuda, 6, 101, d, dtype, output, p_legal=0.05, seed=300 + d)


def test_reference_move_policy_head_gradients(cuda, monkeypatch):
    """KeyQueryPolicyHead(384, 384) at the Move network's 101 tokens, bf16:
    the gradients run through atx_kq_bwd (no torch fallback) and the input
    gradient agrees with float64 autograd of the head's math."""
    _announce("kq bwd reference move head 384")
    import ataraxos_amd.policy as pol

    calls = []
    real = ops.kq_policy_backward
    monkeypatch.setattr(pol.ops, "kq_policy_backward", lambda *a, **k: calls.append(a[0].shape) or real(*a, **k))
    monkeypatch.setattr(pol, "_logit_grads", lambda *a, **k: pytest.fail("torch fallback taken"))
    torch.manual_seed(4)
    head = KeyQueryPolicyHead(384, 384).to(cuda, torch.bfloat16)
    x = randn((4, 101, 384), 90, torch.bfloat16).to(cuda).requires_grad_(True)
    mask = legal_mask(4, 101, 91, 0.05).to(cuda)
    g = randn((4, 101 * 101), 92, torch.float32).to(cuda)
    out = head(x, mask)
    (gx,) = torch.autograd.grad(out.float(), (x,), g)
    assert calls == [torch.Size([4, 101, 384])]
    h64 = KeyQueryPolicyHead(384, 384).double()
    h64.load_state_dict({n: t.double().cpu() for n, t in head.state_dict().items()})
    x64 = x.detach().double().cpu().requires_grad_(True)
    (want,) = torch.autograd.grad(h64(x64, mask.cpu()), (x64,), g.double().cpu())
    err = (gx.double().cpu() - want).abs().max().item()
    assert err <= REL_MAX * want.abs().max().item(), err


@pytest.mark.parametrize("output", ["logits", "probs"])
@pytest.mark.parametrize("s,d", [(100, 64), (101, 384), (33, 16), (64, 48), (128, 128), (100, 400), (17, 96),
                                 (96, 32), (97, 48), (112, 64), (113, 16)])
def test_fp32(cuda, s, d, output):
    """fp32 q, k -- the precision the reference's Move trainer runs its policy
    head in -- through the fp32 kernel (fp32 products)."""
    assert ops.kq_policy_backward_supported(s, d, torch.float32)
    run_case(cuda, 4, s, d, torch.float32, output, p_legal=0.05, seed=400 + s + d)


def test_config2_fp32_full_batch(cuda):
    """C2's shape (B=4096, 100 x 100, d=64) in fp32: sampled rows against the
    oracle, and a sub-batch gives bit-identical rows."""
    b, s, d = 4096, 100, 64
    _announce("kq bwd C2 fp32 full batch")
    q, k = randn((b, s, d), 410, torch.float32), randn((b, s, d), 411, torch.float32)
    mask = legal_mask(b, s, 412, 0.02)
    grad = randn((b, s * s), 413, torch.float32)
    qd, kd, md, gd = q.to(cuda), k.to(cuda), mask.to(cuda), grad.to(cuda)
    dq, dk = ops.kq_policy_backward(qd, kd, gd, md, 0.125)
    idx = torch.tensor([0, 1, 2047, 4095, 1234, 3000])
    ref = kq_backward(to_np64(q[idx]), to_np64(k[idx]), mask[idx].numpy(), 0.125, grad[idx].double().numpy())
    assert_grad_close(dq[idx.to(cuda)], ref[0], "C2 fp32 dq")
    assert_grad_close(dk[idx.to(cuda)], ref[1], "C2 fp32 dk")
    sdq, sdk = ops.kq_policy_backward(qd[100:200], kd[100:200], gd[100:200], md[100:200], 0.125)
    torch.cuda.synchronize()
    assert torch.equal(sdq, dq[100:200]) and torch.equal(sdk, dk[100:200])


def test_fp32_reference_move_policy_head(cuda, monkeypatch):
    """KeyQueryPolicyHead(384, 384) in fp32 at 101 tokens: its gradients run
    through atx_kq_bwd, and the input gradient matches float64 autograd."""
    _announce("kq bwd reference move head 384 fp32")
    import ataraxos_amd.policy as pol

    monkeypatch.setattr(pol, "_logit_grads", lambda *a, **k: pytest.fail("torch fallback taken"))
    torch.manual_seed(5)
    head = KeyQueryPolicyHead(384, 384).to(cuda)
    x = randn((4, 101, 384), 93, torch.float32).to(cuda).requires_grad_(True)
    mask = legal_mask(4, 101, 94, 0.05).to(cuda)
    g = randn((4, 101 * 101), 95, torch.float32).to(cuda)
    (gx,) = torch.autograd.grad(head(x, mask), (x,), g)
    h64 = KeyQueryPolicyHead(384, 384).double()
    h64.load_state_dict({n: t.double().cpu() for n, t in head.state_dict().items()})
    x64 = x.detach().double().cpu().requires_grad_(True)
    (want,) = torch.autograd.grad(h64(x64, mask.cpu()), (x64,), g.double().cpu())
    err = (gx.double().cpu() - want).abs().max().item()
    assert err <= 1e-4 * want.abs().max().item(), err


def test_unsupported_dims_fall_back(cuda):
    """A 16-bit dim above 128 that is not a multiple of 64: refused by the
    kernel, differentiated by torch ops under autograd."""
    qb = torch.randn(4, 100, 144, device=cuda, dtype=torch.bfloat16)
    assert not ops.kq_policy_backward_supported(100, 144, torch.bfloat16)
    with pytest.raises(NotImplementedError):
        ops.kq_policy_backward(qb, qb, torch.zeros(4, 10000, device=cuda))
    qa = qb.clone().requires_grad_(True)
    masked_policy_logits(qa, qb, None).float().sum().backward()
    assert torch.isfinite(qa.grad.float()).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("output", ["logits", "probs"])
def test_result_does_not_depend_on_batch_position(cuda, dtype, output):
    """At 101 squares a sample's G, P and mask rows start at a different
    alignment in each batch position, and the kernel phases its loads to it.
    The same sample at five positions (every alignment mod 16) gets
    bit-identical gradients: the probabilities' sum runs in a fixed
    (row, column) order whatever the alignment."""
    b, s, d = 5, 101, 64
    _announce(f"kq bwd batch-position independence {dtype} {output}")
    q = randn((1, s, d), 80, dtype).expand(b, s, d).contiguous().to(cuda)
    k = randn((1, s, d), 81, dtype).expand(b, s, d).contiguous().to(cuda)
    mask = legal_mask(1, s, 82, 0.2).expand(b, s, s).contiguous().to(cuda)
    grad = randn((1, s * s), 83, torch.float32).expand(b, s * s).contiguous().to(cuda)
    probs = ops.kq_policy(q, k, mask, output="probs") if output == "probs" else None
    dq, dk = ops.kq_policy_backward(q, k, grad, mask, output=output, probs=probs)
    torch.cuda.synchronize()
    for i in range(1, b):
        assert torch.equal(dq[i], dq[0]) and torch.equal(dk[i], dk[0]), f"position {i} differs"
