"""Pins the oracle's restatement of the kernels' dropout keep rule on the CPU:
MurmurHash3's fmix32 and splitmix64 against their published outputs, the
bijection property of the index hash, and the statistics the reference's
F.dropout promises (keep rate 1 - p within binomial bounds, no dependence on
position or on the neighbouring element, different streams for different
seeds and offsets)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.dropout import drop_hash, drop_key, fmix32, keep_mask, splitmix64


def test_fmix32_published_values():
    # MurmurHash3_x86_32 of the empty input is fmix32(seed): the published
    # test values for seeds 0, 1 and 0xffffffff
    assert int(fmix32(0)) == 0
    assert int(fmix32(1)) == 0x514E28B7
    assert int(fmix32(0xFFFFFFFF)) == 0x81F16F39


def test_splitmix64_published_values():
    # the first outputs of the splitmix64 generator from state 0 (Vigna)
    state, outs = 0, []
    for _ in range(3):
        outs.append(splitmix64(state))
        state = (state + 0x9E3779B97F4A7C15) & ((1 << 64) - 1)
    assert outs == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_index_hash_is_a_bijection_on_the_low_word():
    k0, k1, _, _ = drop_key(0.2, 123, 0)
    idx = np.arange(1 << 20, dtype=np.uint64) * np.uint64(4096) + np.uint64(7)
    assert np.unique(drop_hash(idx, k0, k1)).size == idx.size


@pytest.mark.parametrize("p", [0.1, 0.2, 0.5])
def test_keep_rate_and_independence(p):
    m = keep_mask(8, 8, 100, 100, p, seed=2024, offset=5)
    n = m.size
    rate = m.mean()
    sigma = np.sqrt(p * (1 - p) / n)
    assert abs(rate - (1 - p)) < 5 * sigma
    # no dependence on key position or query position
    by_key = m.mean(axis=(0, 1, 2))
    by_query = m.mean(axis=(0, 1, 3))
    s_pos = np.sqrt(p * (1 - p) / (n / 100))
    assert np.abs(by_key - (1 - p)).max() < 6 * s_pos
    assert np.abs(by_query - (1 - p)).max() < 6 * s_pos
    # neighbouring keys independent: P(both kept) = (1 - p)^2
    both = (m[..., 1:] & m[..., :-1]).mean()
    s_pair = np.sqrt((1 - p) ** 2 * (1 - (1 - p) ** 2) / m[..., 1:].size)
    assert abs(both - (1 - p) ** 2) < 6 * s_pair * 2


def test_streams_differ_by_seed_and_offset():
    a = keep_mask(2, 2, 50, 50, 0.3, seed=1, offset=0)
    b = keep_mask(2, 2, 50, 50, 0.3, seed=2, offset=0)
    c = keep_mask(2, 2, 50, 50, 0.3, seed=1, offset=1)
    assert (a != b).mean() > 0.3 and (a != c).mean() > 0.3
    assert np.array_equal(a, keep_mask(2, 2, 50, 50, 0.3, seed=1, offset=0))


def test_threshold_and_scale():
    assert drop_key(0.0, 1, 0)[2:] == (0, 1.0)
    k0, k1, t, s = drop_key(0.25, 1, 0)
    assert t == 1 << 30 and s == pytest.approx(4.0 / 3.0, rel=1e-7)


def _torch_dropout_attention(q, k, v, mult, causal, kpad):
    """float64 torch autograd through softmax -> (x mult) -> @ V: the
    reference's math path with F.dropout's mask made explicit."""
    import torch

    qh, kh, vh = (torch.tensor(t).transpose(1, 2).requires_grad_(True) for t in (q, k, v))
    s = torch.matmul(qh, kh.transpose(-2, -1)) / np.sqrt(q.shape[-1])
    if causal:
        s = s.masked_fill(torch.ones(s.shape[-2:], dtype=torch.bool).triu(1), float("-inf"))
    if kpad is not None:
        s = s.masked_fill(torch.tensor(kpad)[:, None, None, :], float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1) * torch.tensor(mult), vh).transpose(1, 2)
    return o, (qh, kh, vh)


@pytest.mark.parametrize("causal,padded", [(False, False), (True, False), (False, True)])
def test_oracle_dropout_attention_matches_torch_autograd(causal, padded):
    """The oracle's forward and hand-derived backward with dropout
    multipliers against torch float64 autograd on the same explicit mask."""
    import torch

    from oracle.attention import attention, attention_backward

    rng = np.random.default_rng(7)
    b, s, h, d = 2, 19, 3, 16
    q, k, v, g = (rng.standard_normal((b, s, h, d)) for _ in range(4))
    kpad = (rng.random((b, s)) < 0.2) if padded else None
    if kpad is not None:
        kpad[:, 0] = False
    p = 0.3
    keep = keep_mask(b, h, s, s, p, seed=11, offset=2)
    mult = keep / (1 - p)
    o_ref, leaves = _torch_dropout_attention(q, k, v, mult, causal, kpad)
    o_ref.backward(torch.tensor(g))
    want = [t.grad.transpose(1, 2).numpy() for t in leaves]
    o = attention(q, k, v, causal=causal, key_pad=kpad, drop=mult)
    np.testing.assert_allclose(o, o_ref.detach().numpy(), rtol=1e-12, atol=1e-12)
    got = attention_backward(q, k, v, g, causal=causal, key_pad=kpad, drop=mult)
    for x, y in zip(got, want):
        np.testing.assert_allclose(x, y, rtol=1e-10, atol=1e-12)


def test_oracle_dropout_backward_finite_differences():
    """Central differences of <O, G> pin the dropout backward independently
    of any autograd."""
    from oracle.attention import attention, attention_backward

    rng = np.random.default_rng(3)
    b, s, h, d = 1, 5, 2, 4
    q, k, v, g = (rng.standard_normal((b, s, h, d)) for _ in range(4))
    mult = keep_mask(b, h, s, s, 0.4, seed=5, offset=0) / 0.6
    dq, dk, dv = attention_backward(q, k, v, g, drop=mult)
    eps = 1e-6
    for x, dx in ((q, dq), (k, dk), (v, dv)):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            old = x[idx]
            x[idx] = old + eps
            fp = np.sum(attention(q, k, v, drop=mult) * g)
            x[idx] = old - eps
            fm = np.sum(attention(q, k, v, drop=mult) * g)
            x[idx] = old
            num[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(dx, num, rtol=1e-6, atol=1e-8)
