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

from oracle.attention import attention, attention_backward, softmax_lastdim
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


# --- backward ----------------------------------------------------------------


def _bwd_parts(q, k, v, d_o):
    """P, dP and the BHSD operands of a small unmasked case."""
    qh, kh, vh, gh = (_bhsd(x) for x in (q, k, v, d_o))
    scale = 1 / np.sqrt(q.shape[-1])
    p = softmax_lastdim(qh @ kh.swapaxes(-1, -2) * scale)
    return qh, kh, vh, gh, p, gh @ vh.swapaxes(-1, -2), scale


def mutant_bwd_dropped_softmax_term(q, k, v, d_o):
    """dS = P * dP: the rowsum(dP * P) term of the softmax gradient dropped."""
    qh, kh, vh, gh, p, dp, scale = _bwd_parts(q, k, v, d_o)
    ds = p * dp
    return tuple(x.transpose(0, 2, 1, 3) for x in (ds @ kh * scale, ds.swapaxes(-1, -2) @ qh * scale,
                                                   p.swapaxes(-1, -2) @ gh))


def mutant_bwd_missing_scale(q, k, v, d_o):
    """dQ = dS K without the post-product scale."""
    dq, dk, dv = attention_backward(q, k, v, d_o)
    return dq * np.sqrt(q.shape[-1]), dk, dv


def mutant_bwd_untransposed_ds(q, k, v, d_o):
    """dK = dS Q instead of dS^T Q (same shape when S_q = S_kv)."""
    qh, kh, vh, gh, p, dp, scale = _bwd_parts(q, k, v, d_o)
    ds = p * (dp - np.sum(dp * p, axis=-1, keepdims=True))
    return tuple(x.transpose(0, 2, 1, 3) for x in (ds @ kh * scale, ds @ qh * scale, p.swapaxes(-1, -2) @ gh))


def mutant_bwd_gqa_first_head(q, k, v, d_o):
    """GQA: dk/dv taken from the first query head of each group instead of the sum."""
    h, hkv = q.shape[2], k.shape[2]
    dq, dk, dv = attention_backward(q, np.repeat(k, h // hkv, axis=2), np.repeat(v, h // hkv, axis=2), d_o)
    return dq, dk[:, :, :: h // hkv], dv[:, :, :: h // hkv]


def _fd_grads(q, k, v, d_o, eps=1e-6):
    """Central finite differences of <attention(q, k, v), dO> (the pinning check)."""
    out = []
    for which in range(3):
        x = [q, k, v]
        g = np.zeros_like(x[which])
        for idx in np.ndindex(*g.shape):
            p_, m_ = [a.copy() for a in x], [a.copy() for a in x]
            p_[which][idx] += eps
            m_[which][idx] -= eps
            g[idx] = (np.sum(attention(*p_) * d_o) - np.sum(attention(*m_) * d_o)) / (2 * eps)
        out.append(g)
    return out


def test_backward_mistakes_are_caught_by_finite_differences():
    q, k, v, d_o = rnd(1, 4, 2, 4, seed=1), rnd(1, 4, 2, 4, seed=2), rnd(1, 4, 2, 4, seed=3), rnd(1, 4, 2, 4, seed=4)
    fd = _fd_grads(q, k, v, d_o)
    for a, r in zip(attention_backward(q, k, v, d_o), fd):
        np.testing.assert_allclose(a, r, rtol=1e-6, atol=1e-8)
    for mutant in (mutant_bwd_dropped_softmax_term, mutant_bwd_missing_scale, mutant_bwd_untransposed_ds):
        got = mutant(q, k, v, d_o)
        assert not all(np.allclose(a, r, rtol=1e-4, atol=1e-6) for a, r in zip(got, fd)), mutant.__name__


def test_backward_gqa_mistake_is_caught_by_torch_autograd():
    q, k, v, d_o = rnd(2, 5, 8, 4, seed=1), rnd(2, 6, 2, 4, seed=2), rnd(2, 6, 2, 4, seed=3), rnd(2, 5, 8, 4, seed=4)
    tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (k, v))
    kh = tk.transpose(1, 2).repeat_interleave(4, 1)
    vh = tv.transpose(1, 2).repeat_interleave(4, 1)
    o = F.scaled_dot_product_attention(torch.from_numpy(q).transpose(1, 2), kh, vh).transpose(1, 2)
    o.backward(torch.from_numpy(d_o))
    ref = (tk.grad.numpy(), tv.grad.numpy())
    _, dk, dv = attention_backward(q, k, v, d_o)
    np.testing.assert_allclose(dk, ref[0], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dv, ref[1], rtol=1e-10, atol=1e-12)
    _, mk, mv = mutant_bwd_gqa_first_head(q, k, v, d_o)
    assert not np.allclose(mk, ref[0], atol=1e-6) and not np.allclose(mv, ref[1], atol=1e-6)


def test_policy_backward_mistakes_are_caught_by_torch_autograd():
    """Policy-head gradient mutants: the softmax term dropped (dL = P * G) and
    the mask not applied to the gradient.  torch autograd through the
    reference head's operations rejects both."""
    from oracle.policy import ILLEGAL_LOGIT, kq_backward

    b, s, d, scale = 2, 9, 8, 0.35
    q, k, g = rnd(b, s, d, seed=1), rnd(b, s, d, seed=2), rnd(b, s * s, seed=3)
    mask = np.random.default_rng(4).random((b, s, s)) < 0.4
    mask[:, 0, 0] = True
    tq, tk = (torch.from_numpy(x).requires_grad_(True) for x in (q, k))
    logits = (torch.matmul(tq, tk.transpose(1, 2)) * scale).masked_fill(~torch.from_numpy(mask), ILLEGAL_LOGIT)
    torch.softmax(logits.reshape(b, -1), dim=-1).backward(torch.from_numpy(g))
    ref = tq.grad.numpy()
    np.testing.assert_allclose(kq_backward(q, k, mask, scale, g, wrt="probs")[0], ref, rtol=1e-10, atol=1e-12)
    p = kq_probs(q, k, mask, scale)
    dl = np.where(mask, (p * g).reshape(b, s, s), 0.0)  # mutant: no "- sum(G * P)"
    assert not np.allclose(dl @ k * scale, ref, atol=1e-6)
    tq2 = torch.from_numpy(q).requires_grad_(True)
    logits2 = (torch.matmul(tq2, torch.from_numpy(k).transpose(1, 2)) * scale).masked_fill(~torch.from_numpy(mask), ILLEGAL_LOGIT)
    logits2.reshape(b, -1).backward(torch.from_numpy(g))
    unmasked = g.reshape(b, s, s) @ k * scale  # mutant: gradient reaches illegal entries
    np.testing.assert_allclose(kq_backward(q, k, mask, scale, g)[0], tq2.grad.numpy(), rtol=1e-10, atol=1e-12)
    assert not np.allclose(unmasked, tq2.grad.numpy(), atol=1e-6)


def test_dropout_mistakes_are_caught():
    """Dropout: renormalising over the kept weights (a softmax of the dropped
    scores), or a backward that leaves the mask out of dP, disagree with
    torch float64 autograd on the same explicit mask; a hash whose upper
    index word is ignored repeats the mask every 2^32 weights."""
    from oracle.dropout import drop_hash, drop_key, keep_mask

    b, s, h, d, p = 1, 12, 2, 8, 0.3
    q, k, v, g = (rnd(b, s, h, d, seed=i) for i in range(4))
    keep = keep_mask(b, h, s, s, p, seed=3, offset=0)
    mult = keep / (1 - p)
    tq, tk, tv = (torch.from_numpy(x).transpose(1, 2).requires_grad_(True) for x in (q, k, v))
    probs = torch.softmax(tq @ tk.transpose(-1, -2) / np.sqrt(d), dim=-1) * torch.from_numpy(mult)
    o = (probs @ tv).transpose(1, 2)
    o.backward(torch.from_numpy(g))
    want_o = o.detach().numpy()
    # renormalised over kept weights
    sc = _bhsd(q) @ _bhsd(k).swapaxes(-1, -2) / np.sqrt(d)
    renorm = (softmax_lastdim(np.where(keep, sc, -np.inf)) @ _bhsd(v)).transpose(0, 2, 1, 3)
    assert np.abs(renorm - want_o).max() > 1e-3
    np.testing.assert_allclose(attention(q, k, v, drop=mult), want_o, rtol=1e-12, atol=1e-12)
    # backward without the mask on dP: what attention_backward would give if
    # dropout only touched dV
    dq_mut = attention_backward(q, k, v, g)[0]
    assert np.abs(dq_mut - tq.grad.transpose(1, 2).numpy()).max() > 1e-3
    np.testing.assert_allclose(attention_backward(q, k, v, g, drop=mult)[0], tq.grad.transpose(1, 2).numpy(),
                               rtol=1e-10, atol=1e-12)
    # the upper index word matters
    k0, k1, _, _ = drop_key(p, 3, 0)
    lo = np.arange(4096, dtype=np.uint64)
    assert (drop_hash(lo, k0, k1) != drop_hash(lo + np.uint64(1 << 32), k0, k1)).mean() > 0.99
