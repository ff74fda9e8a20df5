"""Planted mistakes: each plausible error in the oracle is rejected by at
least one of the pinning checks the CPU suite runs.

Each mutant below is a deliberately wrong variant of an oracle function (the
mistake is planted here, on the CPU, never in product code).  The test shows
that the independent reference the suite compares the oracle with disagrees
with the mutant, so the pinning checks would have caught that mistake.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F  # noqa: N812

from oracle.attention import attention, softmax_lastdim
from oracle.policy import kq_probs


def rnd(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape)


def sdpa(q, k, v, causal=False):
    tq, tk, tv = (torch.from_numpy(x).transpose(1, 2) for x in (q, k, v))
    h, hkv = tq.shape[1], tk.shape[1]
    tk, tv = tk.repeat_interleave(h // hkv, 1), tv.repeat_interleave(h // hkv, 1)
    return F.scaled_dot_product_attention(tq, tk, tv, is_causal=causal).transpose(1, 2).numpy()


def _bhsd(x):
    return x.transpose(0, 2, 1, 3)


def mutant_scale_before_sqrt(q, k, v):
    """Divides by D instead of sqrt(D)."""
    s = _bhsd(q) @ _bhsd(k).swapaxes(-1, -2) / q.shape[-1]
    return (softmax_lastdim(s) @ _bhsd(v)).transpose(0, 2, 1, 3)


def mutant_transposed_scores(q, k, v):
    """Softmax over the query axis instead of the key axis."""
    s = _bhsd(q) @ _bhsd(k).swapaxes(-1, -2) / np.sqrt(q.shape[-1])
    p = softmax_lastdim(s.swapaxes(-1, -2)).swapaxes(-1, -2)
    return (p @ _bhsd(v)).transpose(0, 2, 1, 3)


def mutant_bottom_right_causal(q, k, v):
    """Causal mask aligned bottom-right (the flash-attn convention for S_q != S_kv)."""
    sq, skv = q.shape[1], k.shape[1]
    s = _bhsd(q) @ _bhsd(k).swapaxes(-1, -2) / np.sqrt(q.shape[-1])
    s = np.where(np.triu(np.ones((sq, skv), bool), 1 + skv - sq), -np.inf, s)
    return (softmax_lastdim(s) @ _bhsd(v)).transpose(0, 2, 1, 3)


def mutant_gqa_tile(q, k, v):
    """Maps query head h to KV head h % H_kv (tile) instead of h // group."""
    h, hkv = q.shape[2], k.shape[2]
    return attention(q, np.tile(k, (1, 1, h // hkv, 1)), np.tile(v, (1, 1, h // hkv, 1)))


def mutant_to_major_probs(q, k, mask, scale):
    """Flattens the policy to-major (j*S + i)."""
    p = kq_probs(q, k, mask, scale).reshape(q.shape[0], q.shape[1], q.shape[1])
    return p.transpose(0, 2, 1).reshape(q.shape[0], -1)


def test_scale_mistake_is_caught():
    q, k, v = rnd(2, 20, 4, 64, seed=1), rnd(2, 20, 4, 64, seed=2), rnd(2, 20, 4, 64, seed=3)
    assert np.allclose(attention(q, k, v), sdpa(q, k, v))
    assert not np.allclose(mutant_scale_before_sqrt(q, k, v), sdpa(q, k, v), atol=1e-6)


def test_softmax_axis_mistake_is_caught():
    q, k, v = rnd(2, 20, 4, 16, seed=1), rnd(2, 20, 4, 16, seed=2), rnd(2, 20, 4, 16, seed=3)
    assert not np.allclose(mutant_transposed_scores(q, k, v), sdpa(q, k, v), atol=1e-6)


def test_causal_alignment_mistake_is_caught():
    q, k, v = rnd(2, 10, 4, 16, seed=1), rnd(2, 30, 4, 16, seed=2), rnd(2, 30, 4, 16, seed=3)
    assert np.allclose(attention(q, k, v, causal=True), sdpa(q, k, v, causal=True))
    assert not np.allclose(mutant_bottom_right_causal(q, k, v), sdpa(q, k, v, causal=True), atol=1e-6)


def test_gqa_mapping_mistake_is_caught():
    q, k, v = rnd(2, 9, 8, 16, seed=1), rnd(2, 9, 2, 16, seed=2), rnd(2, 9, 2, 16, seed=3)
    assert np.allclose(attention(q, k, v), sdpa(q, k, v))
    assert not np.allclose(mutant_gqa_tile(q, k, v), sdpa(q, k, v), atol=1e-6)


def test_flatten_order_mistake_is_caught():
    """The single-legal-move check pins the from-major index i*S + j."""
    mask = np.zeros((1, 100, 100), dtype=bool)
    mask[0, 3, 5] = True
    q, k = rnd(1, 100, 64, seed=1), rnd(1, 100, 64, seed=2)
    assert kq_probs(q, k, mask, 1 / 8)[0, 3 * 100 + 5] == 1.0
    assert mutant_to_major_probs(q, k, mask, 1 / 8)[0, 3 * 100 + 5] == 0.0
