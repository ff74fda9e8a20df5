"""The drop-in modules on the GPU: the HIP backend is the one that runs, and
matches the math path / oracle; the reference's GPU-side invariants hold."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from ataraxos_amd import KeyQueryPolicyHead, MultiHeadAttention, math_attention, ops
from oracle.attention import mha_forward
from tests._cases import LOWP_ABS_TOL

pytestmark = pytest.mark.gpu


def test_backend_is_hip_on_gpu(cuda):
    m = MultiHeadAttention(384, 6).to(cuda)
    assert m.backend == "hip"
    m.train()
    assert m.backend == "hip"  # dropout 0: the kernel still runs in training
    md = MultiHeadAttention(512, 8, dropout=0.2).to(cuda)  # head_dim 64: the kernels' own dropout
    assert md.eval().backend == "hip" and md.train().backend == "hip"
    m32 = MultiHeadAttention(256, 8, dropout=0.2).to(cuda)  # head_dim 32: no dropout kernels
    assert m32.eval().backend == "hip" and m32.train().backend == "math"


def test_fp32_module_matches_oracle(cuda):
    torch.manual_seed(0)
    m = MultiHeadAttention(384, 6, qkv_bias=True).eval()
    x = torch.randn(4, 100, 384)
    want = mha_forward(x.double().numpy(), None, {k: v.double().numpy() for k, v in m.state_dict().items()}, 6)
    got = m.to(cuda)(x.to(cuda)).detach().cpu().double().numpy()
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("e,h,causal,kv", [(384, 6, False, None), (384, 8, False, None), (512, 8, True, None),
                                          (512, 8, False, 2)])
def test_bf16_module_matches_math_path(cuda, e, h, causal, kv):
    torch.manual_seed(1)
    m = MultiHeadAttention(e, h, num_kv_heads=kv, causal=causal).to(cuda, torch.bfloat16).eval()
    x = torch.randn(8, 101, e, device=cuda).bfloat16()
    with torch.no_grad():
        got = m(x)
        b, s, _ = x.shape
        q = m.q_proj(x).view(b, s, h, e // h)
        k = m.k_proj(x).view(b, s, m.num_kv_heads, e // h)
        v = m.v_proj(x).view(b, s, m.num_kv_heads, e // h)
        ref = math_attention(q.float(), k.float(), v.float(), causal).reshape(b, s, e)
        ref = m.out_proj(ref.bfloat16())
    assert (got.float() - ref.float()).abs().max().item() <= LOWP_ABS_TOL


def test_cross_attention_on_gpu(cuda):
    m = MultiHeadAttention(128, 4, causal=True).to(cuda).eval()
    q, kv = torch.randn(2, 10, 128, device=cuda), torch.randn(2, 50, 128, device=cuda)
    out = m(q, key_value=kv)
    assert out.shape == (2, 10, 128) and torch.isfinite(out).all()
    assert not torch.allclose(m(q), m(q, key_value=q[:, :7]), atol=1e-5)


def test_bf16_forward_backward_finite(cuda):
    """stratego tests/test_attention.py:191-211."""
    m = MultiHeadAttention(64, 4).to(cuda, torch.bfloat16)
    x = torch.randn(2, 16, 64, device=cuda, dtype=torch.bfloat16, requires_grad=True)
    out = m(x)
    assert out.dtype == torch.bfloat16 and torch.isfinite(out).all()
    out.sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()


def test_gradients_match_math_path(cuda):
    torch.manual_seed(2)
    b, s, h, d = 2, 40, 4, 32
    q, k, v = (torch.randn(b, s, h, d, device=cuda, requires_grad=True) for _ in range(3))
    g = torch.randn(b, s, h, d, device=cuda)
    for causal in (False, True):
        out = ops.attention(q, k, v, causal=causal)
        got = torch.autograd.grad(out, (q, k, v), g)
        ref = math_attention(q, k, v, causal)
        want = torch.autograd.grad(ref, (q, k, v), g)
        for a, w in zip(got, want):
            assert (a - w).abs().max().item() <= 1e-4 * w.abs().max().item()


def test_causal_first_token_independent_on_gpu(cuda):
    m = MultiHeadAttention(64, 4, causal=True).to(cuda).eval()
    x1 = torch.randn(1, 10, 64, device=cuda)
    x2 = x1.clone()
    x2[0, 5:] = torch.randn(5, 64, device=cuda)
    assert torch.allclose(m(x1)[0, :5], m(x2)[0, :5], atol=1e-6)


def test_unsupported_head_dim_raises_instead_of_falling_back(cuda):
    m = MultiHeadAttention(64, 8).to(cuda)  # head_dim 8
    with pytest.raises(RuntimeError, match="does not cover"):
        m(torch.randn(1, 4, 64, device=cuda))


def test_policy_head_on_gpu(cuda):
    torch.manual_seed(3)
    head = KeyQueryPolicyHead(384, 64).eval()
    x = torch.randn(4, 100, 384)
    mask = torch.rand(4, 100, 100) < 0.05
    mask[:, 0, 0] = True
    with torch.no_grad():
        want = head(x, mask)
        hg = head.to(cuda)
        got = hg(x.to(cuda), mask.to(cuda)).cpu()
        probs = hg.policy(x.to(cuda), mask.to(cuda)).cpu()
    legal = mask.reshape(4, -1)
    assert (got[~legal] == -1e10).all()
    assert (got[legal] - want[legal]).abs().max().item() <= 1e-5 * want[legal].abs().max().item()
    np.testing.assert_allclose(probs.double().numpy(), torch.softmax(want.double(), -1).numpy(), atol=1e-6)


def test_policy_gradients_match_math_path(cuda):
    torch.manual_seed(4)
    b, s, d = 3, 100, 64
    q = torch.randn(b, s, d, device=cuda, requires_grad=True)
    k = torch.randn(b, s, d, device=cuda, requires_grad=True)
    mask = torch.rand(b, s, s, device=cuda) < 0.1
    g = torch.randn(b, s * s, device=cuda)
    from ataraxos_amd import masked_policy_logits, masked_policy_softmax

    for fused, ref_fn in [
        (masked_policy_logits, lambda: (torch.matmul(q, k.transpose(1, 2)) / 8).masked_fill(~mask, -1e10).reshape(b, -1)),
        (masked_policy_softmax, lambda: torch.softmax((torch.matmul(q, k.transpose(1, 2)) / 8).masked_fill(~mask, -1e10).reshape(b, -1), -1)),
    ]:
        got = torch.autograd.grad(fused(q, k, mask), (q, k), g)
        want = torch.autograd.grad(ref_fn(), (q, k), g)
        for a, w in zip(got, want):
            assert (a - w).abs().max().item() <= 1e-4 * max(w.abs().max().item(), 1e-6)
