"""Pins ``oracle.attention`` (CPU, no GPU needed).

Independent references: torch's ``scaled_dot_product_attention`` and
``nn.MultiheadAttention`` on the CPU in float64 (library implementations that
share no code with the oracle), closed forms, and the invariants the
reference's own tests assert (stratego tests/test_attention.py:64-95,
tests/test_setup_net.py:96-111).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F  # noqa: N812

from oracle.attention import attention, expand_kv_heads, mha_forward

pytestmark = pytest.mark.filterwarnings("ignore::UserWarning")


def rnd(*shape, seed=0, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * scale


def sdpa_bshd(q, k, v, causal=False, key_pad=None, scale=None):
    """torch SDPA (float64, CPU) on BSHD numpy arrays."""
    tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(x)).transpose(1, 2) for x in (q, k, v))
    h, hkv = tq.shape[1], tk.shape[1]
    if hkv != h:
        tk = tk.repeat_interleave(h // hkv, dim=1)
        tv = tv.repeat_interleave(h // hkv, dim=1)
    mask = None
    if key_pad is not None:
        mask = ~torch.from_numpy(key_pad)[:, None, None, :]
    if causal:
        cm = torch.ones(q.shape[1], k.shape[1], dtype=torch.bool).tril()
        mask = cm if mask is None else (mask & cm)
    o = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=scale)
    return o.transpose(1, 2).numpy()


@pytest.mark.parametrize(
    "b,sq,skv,h,hkv,d",
    [(2, 100, 100, 6, 6, 64), (3, 101, 101, 8, 8, 48), (2, 10, 50, 4, 4, 32), (1, 1, 256, 4, 4, 16),
     (2, 33, 33, 8, 2, 32), (2, 7, 3, 6, 3, 64)],
)
def test_matches_torch_sdpa(b, sq, skv, h, hkv, d):
    q, k, v = rnd(b, sq, h, d, seed=1), rnd(b, skv, hkv, d, seed=2), rnd(b, skv, hkv, d, seed=3)
    np.testing.assert_allclose(attention(q, k, v), sdpa_bshd(q, k, v), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("sq,skv", [(40, 40), (100, 100), (10, 30), (1, 1)])
def test_causal_matches_torch_sdpa_top_left(sq, skv):
    """torch SDPA's causal mask is ``ones(L, S).tril()``: top-left aligned, as
    the reference's ``triu(ones(S_q, S_kv), 1)`` (attention.py:303-308)."""
    q, k, v = rnd(2, sq, 4, 32, seed=4), rnd(2, skv, 4, 32, seed=5), rnd(2, skv, 4, 32, seed=6)
    np.testing.assert_allclose(attention(q, k, v, causal=True), sdpa_bshd(q, k, v, causal=True), rtol=1e-12, atol=1e-12)


def test_key_padding_matches_torch_sdpa():
    q, k, v = rnd(3, 40, 8, 64, seed=7), rnd(3, 100, 8, 64, seed=8), rnd(3, 100, 8, 64, seed=9)
    pad = np.random.default_rng(10).random((3, 100)) < 0.6
    pad[:, 5] = False
    np.testing.assert_allclose(attention(q, k, v, key_pad=pad), sdpa_bshd(q, k, v, key_pad=pad), rtol=1e-12, atol=1e-12)


def test_scale_argument_matches_torch_sdpa():
    q, k, v = rnd(2, 20, 4, 32, seed=11), rnd(2, 20, 4, 32, seed=12), rnd(2, 20, 4, 32, seed=13)
    np.testing.assert_allclose(attention(q, k, v, scale=0.3), sdpa_bshd(q, k, v, scale=0.3), rtol=1e-12, atol=1e-12)


def test_module_forward_matches_torch_multihead_attention():
    """mha_forward against torch's own MultiheadAttention (packed in_proj,
    biases, key_padding_mask True = ignore), the module the Belief decoder
    uses (belief_net.py:105-114)."""
    e, h = 64, 4
    torch.manual_seed(0)
    ref = torch.nn.MultiheadAttention(e, h, batch_first=True, dtype=torch.float64)
    x = torch.randn(2, 12, e, dtype=torch.float64)
    mem = torch.randn(2, 30, e, dtype=torch.float64)
    pad = torch.rand(2, 30) < 0.5
    pad[:, 0] = False
    want, _ = ref(x, mem, mem, key_padding_mask=pad, need_weights=False)
    w, bias = ref.in_proj_weight.detach().numpy(), ref.in_proj_bias.detach().numpy()
    weights = {
        "q_proj.weight": w[:e], "k_proj.weight": w[e : 2 * e], "v_proj.weight": w[2 * e :],
        "q_proj.bias": bias[:e], "k_proj.bias": bias[e : 2 * e], "v_proj.bias": bias[2 * e :],
        "out_proj.weight": ref.out_proj.weight.detach().numpy(), "out_proj.bias": ref.out_proj.bias.detach().numpy(),
    }
    # key padding is an attention-level argument: project, attend, project.
    d = e // h
    q = (x.numpy() @ weights["q_proj.weight"].T + weights["q_proj.bias"]).reshape(2, 12, h, d)
    k = (mem.numpy() @ weights["k_proj.weight"].T + weights["k_proj.bias"]).reshape(2, 30, h, d)
    v = (mem.numpy() @ weights["v_proj.weight"].T + weights["v_proj.bias"]).reshape(2, 30, h, d)
    o = attention(q, k, v, key_pad=pad.numpy()).reshape(2, 12, e) @ weights["out_proj.weight"].T + weights["out_proj.bias"]
    np.testing.assert_allclose(o, want.detach().numpy(), rtol=1e-10, atol=1e-12)
    # and the unmasked module path through mha_forward
    want2, _ = ref(x, mem, mem, need_weights=False)
    np.testing.assert_allclose(mha_forward(x.numpy(), mem.numpy(), weights, h), want2.detach().numpy(), rtol=1e-10, atol=1e-12)


def test_self_attention_module_forward_causal_matches_torch():
    e, h = 32, 4
    torch.manual_seed(1)
    ref = torch.nn.MultiheadAttention(e, h, batch_first=True, bias=False, dtype=torch.float64)
    x = torch.randn(3, 9, e, dtype=torch.float64)
    causal = torch.ones(9, 9, dtype=torch.bool).triu(1)
    want, _ = ref(x, x, x, attn_mask=causal, need_weights=False)
    w = ref.in_proj_weight.detach().numpy()
    weights = {"q_proj.weight": w[:e], "k_proj.weight": w[e : 2 * e], "v_proj.weight": w[2 * e :],
               "out_proj.weight": ref.out_proj.weight.detach().numpy()}
    np.testing.assert_allclose(mha_forward(x.numpy(), None, weights, h, causal=True), want.detach().numpy(),
                               rtol=1e-10, atol=1e-12)
    # causal is ignored for cross-attention (attention.py:189)
    np.testing.assert_allclose(mha_forward(x.numpy(), x.numpy(), weights, h, causal=True),
                               mha_forward(x.numpy(), None, weights, h, causal=False), rtol=0, atol=0)


# --- closed forms -------------------------------------------------------------


def test_single_key_returns_value():
    q, k, v = rnd(2, 5, 3, 16, seed=1), rnd(2, 1, 3, 16, seed=2), rnd(2, 1, 3, 16, seed=3)
    np.testing.assert_allclose(attention(q, k, v), np.broadcast_to(v, (2, 5, 3, 16)), rtol=0, atol=1e-15)


def test_constant_keys_average_values():
    q, v = rnd(2, 7, 2, 8, seed=1), rnd(2, 11, 2, 8, seed=2)
    k = np.ones((2, 11, 2, 8))
    np.testing.assert_allclose(attention(q, k, v), np.broadcast_to(v.mean(axis=1, keepdims=True), q.shape), atol=1e-14)


def test_dominant_logit_selects_row():
    d = 16
    k = np.zeros((1, 6, 1, d))
    k[0, 4, 0, 0] = 1000.0
    q = np.zeros((1, 3, 1, d))
    q[0, :, 0, 0] = 1.0
    v = rnd(1, 6, 1, d, seed=5)
    np.testing.assert_allclose(attention(q, k, v), np.broadcast_to(v[:, 4:5], (1, 3, 1, d)), atol=1e-12)


def test_causal_first_row_is_first_value():
    q, k, v = rnd(2, 9, 3, 8, seed=1), rnd(2, 9, 3, 8, seed=2), rnd(2, 9, 3, 8, seed=3)
    np.testing.assert_allclose(attention(q, k, v, causal=True)[:, 0], v[:, 0], atol=1e-15)


def test_key_value_permutation_invariance_and_query_equivariance():
    q, k, v = rnd(2, 12, 2, 8, seed=1), rnd(2, 15, 2, 8, seed=2), rnd(2, 15, 2, 8, seed=3)
    perm_k = np.random.default_rng(0).permutation(15)
    perm_q = np.random.default_rng(1).permutation(12)
    base = attention(q, k, v)
    np.testing.assert_allclose(attention(q, k[:, perm_k], v[:, perm_k]), base, atol=1e-13)
    np.testing.assert_allclose(attention(q[:, perm_q], k, v), base[:, perm_q], atol=1e-13)


def test_gqa_equals_explicit_repeat_interleave():
    """attention.py:210-220: query head h reads KV head h // (H / H_kv)."""
    q, k, v = rnd(2, 5, 8, 4, seed=1), rnd(2, 6, 2, 4, seed=2), rnd(2, 6, 2, 4, seed=3)
    ke = np.repeat(k, 4, axis=2)
    ve = np.repeat(v, 4, axis=2)
    np.testing.assert_allclose(attention(q, k, v), attention(q, ke, ve), atol=0)
    x = np.arange(2 * 3).reshape(1, 2, 3, 1)  # [B, H_kv, S, D]
    assert expand_kv_heads(x, 6)[0, :, 0, 0].tolist() == [0, 0, 0, 3, 3, 3]


def test_fully_masked_row_is_nan():
    q, k, v = rnd(2, 3, 1, 8, seed=1), rnd(2, 4, 1, 8, seed=2), rnd(2, 4, 1, 8, seed=3)
    pad = np.zeros((2, 4), dtype=bool)
    pad[1] = True
    o = attention(q, k, v, key_pad=pad)
    assert np.isnan(o[1]).all() and np.isfinite(o[0]).all()
    t = torch.full((4,), float("-inf"))
    assert torch.isnan(torch.softmax(t, 0)).all()  # the torch behaviour this mirrors


# --- the reference's invariants ---------------------------------------------


def test_causal_prefix_independence():
    """Changing later tokens leaves earlier outputs unchanged
    (test_attention.py:83-95, test_setup_net.py:96-111)."""
    q, k, v = rnd(1, 10, 4, 16, seed=1), rnd(1, 10, 4, 16, seed=2), rnd(1, 10, 4, 16, seed=3)
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    q2[:, 5:], k2[:, 5:], v2[:, 5:] = rnd(1, 5, 4, 16, seed=9), rnd(1, 5, 4, 16, seed=10), rnd(1, 5, 4, 16, seed=11)
    a, b = attention(q, k, v, causal=True), attention(q2, k2, v2, causal=True)
    np.testing.assert_array_equal(a[:, :5], b[:, :5])
    assert not np.allclose(a[:, 5:], b[:, 5:])


def test_causal_differs_from_bidirectional():
    q, k, v = rnd(2, 20, 4, 16, seed=1), rnd(2, 20, 4, 16, seed=2), rnd(2, 20, 4, 16, seed=3)
    assert not np.allclose(attention(q, k, v, causal=True), attention(q, k, v))
