"""Interface parity of the drop-in modules on the CPU (``math`` backend).

Mirrors the reference's own module tests (stratego tests/test_attention.py,
tests/test_move_net.py:67-92) and checks values against the float64 oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from ataraxos_amd import KeyQueryPolicyHead, MultiHeadAttention, ops
from oracle.attention import mha_forward
from oracle.policy import kq_logits


def weights_of(mod: nn.Module) -> dict:
    return {k: v.detach().double().numpy() for k, v in mod.state_dict().items()}


# --- constructor / attributes / state_dict --------------------------------


def test_constructor_validation_matches_reference():
    with pytest.raises(ValueError, match="divisible by num_heads"):
        MultiHeadAttention(100, 8)
    with pytest.raises(ValueError, match="divisible by num_kv_heads"):
        MultiHeadAttention(512, 8, num_kv_heads=3)


def test_attributes_and_submodules():
    m = MultiHeadAttention(512, 8, num_kv_heads=2, dropout=0.2, causal=True)
    assert (m.embed_dim, m.num_heads, m.num_kv_heads, m.head_dim, m.dropout, m.causal) == (512, 8, 2, 64, 0.2, True)
    assert m.k_proj.out_features == 128 and m.q_proj.out_features == 512
    assert list(m.state_dict()) == ["q_proj.weight", "k_proj.weight", "v_proj.weight", "out_proj.weight"]
    mb = MultiHeadAttention(64, 4, qkv_bias=True)
    assert [k for k in mb.state_dict() if k.endswith("bias")] == ["q_proj.bias", "k_proj.bias", "v_proj.bias", "out_proj.bias"]


def test_parameter_initialisation_order_matches_reference():
    """Same RNG draws as q, k, v, out nn.Linear created in that order
    (attention.py:113-116), so seeded checkpoints line up."""
    torch.manual_seed(3)
    m = MultiHeadAttention(96, 4, num_kv_heads=2)
    torch.manual_seed(3)
    ref = [nn.Linear(96, 96, bias=False), nn.Linear(96, 48, bias=False), nn.Linear(96, 48, bias=False),
           nn.Linear(96, 96, bias=False)]
    for got, want in zip([m.q_proj, m.k_proj, m.v_proj, m.out_proj], ref):
        assert torch.equal(got.weight, want.weight)


def test_cpu_backend_is_math():
    assert MultiHeadAttention(64, 4).backend == "math"


# --- values against the oracle ---------------------------------------------


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("kv_heads", [None, 2])
def test_forward_matches_oracle(causal, kv_heads):
    torch.manual_seed(0)
    m = MultiHeadAttention(64, 4, num_kv_heads=kv_heads, causal=causal, qkv_bias=True).double().eval()
    x = torch.randn(2, 17, 64, dtype=torch.float64)
    want = mha_forward(x.numpy(), None, weights_of(m), 4, kv_heads, causal=causal)
    np.testing.assert_allclose(m(x).detach().numpy(), want, rtol=1e-10, atol=1e-12)


def test_cross_attention_matches_oracle_and_ignores_causal():
    torch.manual_seed(1)
    m = MultiHeadAttention(64, 4, causal=True).double().eval()
    x, kv = torch.randn(2, 10, 64, dtype=torch.float64), torch.randn(2, 30, 64, dtype=torch.float64)
    want = mha_forward(x.numpy(), kv.numpy(), weights_of(m), 4)
    np.testing.assert_allclose(m(x, key_value=kv).detach().numpy(), want, rtol=1e-10, atol=1e-12)


# --- the reference's invariants (stratego tests/test_attention.py) ---------


@pytest.mark.parametrize("e,h,causal,s", [(512, 8, False, 100), (512, 8, True, 92), (384, 8, False, 92)])
def test_output_shapes(e, h, causal, s):
    m = MultiHeadAttention(e, h, causal=causal)
    assert m(torch.randn(2, s, e)).shape == (2, s, e)


def test_causal_differs_and_first_token_independent():
    torch.manual_seed(0)
    mc, mn = MultiHeadAttention(64, 4, causal=True).eval(), MultiHeadAttention(64, 4).eval()
    mn.load_state_dict(mc.state_dict())
    x = torch.randn(2, 20, 64)
    assert not torch.allclose(mc(x), mn(x), atol=1e-5)
    x2 = x.clone()
    x2[:, 5:] = torch.randn(2, 15, 64)
    assert torch.allclose(mc(x)[:, 0], mc(x2)[:, 0], atol=1e-6)


def test_dropout_train_varies_eval_deterministic():
    m = MultiHeadAttention(64, 4, dropout=0.5)
    x = torch.randn(2, 16, 64)
    m.train()
    outs = [m(x) for _ in range(5)]
    assert any(not torch.allclose(outs[0], o, atol=1e-6) for o in outs[1:])
    m.eval()
    assert torch.allclose(m(x), m(x), atol=1e-6)


def test_gradients_flow():
    m = MultiHeadAttention(64, 4)
    x = torch.randn(2, 10, 64, requires_grad=True)
    m(x).sum().backward()
    assert x.grad is not None and x.grad.shape == x.shape and x.grad.abs().sum() > 0


@pytest.mark.parametrize("s", [1, 10, 100, 256])
def test_sequence_lengths_and_finiteness(s):
    out = MultiHeadAttention(64, 4)(torch.randn(2, s, 64))
    assert out.shape == (2, s, 64) and torch.isfinite(out).all()


def test_gqa_shapes():
    m = MultiHeadAttention(512, 8, num_kv_heads=2)
    assert m(torch.randn(2, 16, 512)).shape == (2, 16, 512)


# --- policy head ----------------------------------------------------------


def test_policy_head_matches_oracle_and_mask_invariant():
    torch.manual_seed(0)
    head = KeyQueryPolicyHead(64, 32).double().eval()
    assert head.scale == pytest.approx(32**0.5)
    x = torch.randn(2, 100, 64, dtype=torch.float64)
    mask = torch.zeros(2, 100, 100, dtype=torch.bool)
    mask[0, 3, 5] = True
    mask[1, 7, 2] = True
    out = head(x, legal_move_mask=mask)
    q, k = head._queries_keys(x)
    want = kq_logits(q.detach().numpy(), k.detach().numpy(), mask.numpy(), 1 / 32**0.5)
    np.testing.assert_allclose(out.detach().numpy(), want, rtol=1e-12, atol=1e-12)
    assert int((out <= -1e9).sum()) == 2 * 100 * 100 - 2
    probs = head.policy(x, mask)
    assert probs[0, 305] == 1.0 and probs[1, 702] == 1.0


def test_policy_head_submodules_and_default_dim():
    head = KeyQueryPolicyHead(384)
    assert head.wq.out_features == 384 and head.scale == pytest.approx(384**0.5)
    assert list(head.state_dict()) == ["policy_embedding.weight", "policy_embedding.bias", "wq.weight", "wk.weight"]


def test_gpu_ops_refuse_cpu_tensors():
    x = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.attention_forward(x, x, x)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.kq_policy(torch.zeros(1, 4, 8), torch.zeros(1, 4, 8))
