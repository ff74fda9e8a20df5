"""Pins ``oracle.policy`` and ``oracle.decode`` (CPU).

Independent references: scipy's softmax over explicitly built masked
logits, torch SDPA for the decode step, closed forms, and the reference's
policy-head invariants (stratego tests/test_move_net.py:67-92,265-277).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F  # noqa: N812
from scipy.special import softmax as scipy_softmax

from oracle.decode import decode_step, full_recompute_last_row
from oracle.policy import ILLEGAL_LOGIT, kq_logits, kq_probs


def rnd(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape)


def mask_of(b, s, p, seed):
    m = np.random.default_rng(seed).random((b, s, s)) < p
    m[:, 0, 1] = True
    return m


def test_logits_against_explicit_loops():
    """Brute force on a tiny case: logit[b, i*S + j] = scale * <q_i, k_j>."""
    b, s, d = 2, 5, 3
    q, k = rnd(b, s, d, seed=1), rnd(b, s, d, seed=2)
    mask = mask_of(b, s, 0.5, 3)
    got = kq_logits(q, k, mask, 0.7)
    for bi in range(b):
        for i in range(s):
            for j in range(s):
                want = 0.7 * sum(q[bi, i, t] * k[bi, j, t] for t in range(d)) if mask[bi, i, j] else ILLEGAL_LOGIT
                assert got[bi, i * s + j] == pytest.approx(want, rel=1e-12, abs=1e-12)


def test_probs_match_scipy_softmax():
    b, s, d = 3, 100, 64
    q, k = rnd(b, s, d, seed=4), rnd(b, s, d, seed=5)
    mask = mask_of(b, s, 0.02, 6)
    logits = np.einsum("bid,bjd->bij", q, k) / 8.0
    logits = np.where(mask, logits, -1e10).reshape(b, -1)
    np.testing.assert_allclose(kq_probs(q, k, mask, 1 / 8), scipy_softmax(logits, axis=-1), rtol=1e-12, atol=1e-300)


def test_illegal_entries_exactly_zero_and_rows_sum_to_one():
    b, s, d = 4, 100, 64
    p = kq_probs(rnd(b, s, d, seed=7), rnd(b, s, d, seed=8), mask_of(b, s, 0.02, 9), 1 / 8)
    m = mask_of(b, s, 0.02, 9).reshape(b, -1)
    assert (p[~m] == 0.0).all()
    np.testing.assert_allclose(p.sum(axis=1), 1.0, rtol=1e-12)


def test_single_legal_entry_is_one():
    mask = np.zeros((1, 100, 100), dtype=bool)
    mask[0, 3, 5] = True
    p = kq_probs(rnd(1, 100, 64, seed=1), rnd(1, 100, 64, seed=2), mask, 1 / 8)
    assert p[0, 3 * 100 + 5] == 1.0 and (np.delete(p[0], 305) == 0).all()


def test_equal_logits_split_evenly_and_all_illegal_is_uniform():
    mask = mask_of(2, 10, 0.3, 1)
    p = kq_probs(np.zeros((2, 10, 4)), np.zeros((2, 10, 4)), mask, 1.0)
    for i in range(2):
        np.testing.assert_allclose(p[i][mask[i].reshape(-1)], 1.0 / mask[i].sum(), rtol=1e-14)
    p = kq_probs(rnd(1, 10, 4, seed=3), rnd(1, 10, 4, seed=4), np.zeros((1, 10, 10), bool), 1.0)
    np.testing.assert_allclose(p, 1.0 / 100, rtol=1e-14)


def test_reference_mask_count_invariant():
    """test_move_net.py:67-84: with one legal pair per sample, exactly
    2*S*S - 2 logits are <= -1e9; without a mask none is (:86-92)."""
    s = 100
    mask = np.zeros((2, s, s), dtype=bool)
    mask[0, 3, 5] = True
    mask[1, 7, 2] = True
    lo = kq_logits(rnd(2, s, 64, seed=1), rnd(2, s, 64, seed=2), mask, 1 / 8)
    assert int((lo <= -1e9).sum()) == 2 * s * s - 2
    assert (kq_logits(rnd(2, s, 64, seed=1), rnd(2, s, 64, seed=2), None, 1 / 8) > -1e9).all()


def test_from_major_flatten_and_asymmetry():
    """Entry i*S + j is from-square i to to-square j; q k^T is asymmetric
    (test_move_net.py:265-277)."""
    q, k = rnd(1, 6, 4, seed=1), rnd(1, 6, 4, seed=2)
    lo = kq_logits(q, k, None, 1.0).reshape(6, 6)
    assert lo[2, 4] == pytest.approx(float(q[0, 2] @ k[0, 4]))
    assert not np.allclose(lo, lo.T)


# --- decode ------------------------------------------------------------------


@pytest.mark.parametrize("t", [1, 2, 17, 40])
def test_decode_step_is_last_row_of_causal_recompute(t):
    b, h, d = 3, 8, 64
    qs, ks, vs = rnd(b, t, h, d, seed=1), rnd(b, t, h, d, seed=2), rnd(b, t, h, d, seed=3)
    step = decode_step(qs[:, -1], ks.transpose(0, 2, 1, 3), vs.transpose(0, 2, 1, 3))
    np.testing.assert_allclose(step, full_recompute_last_row(qs, ks, vs), rtol=1e-12, atol=1e-13)
    # and against torch SDPA's causal attention over the whole prefix
    tq, tk, tv = (torch.from_numpy(x).transpose(1, 2) for x in (qs, ks, vs))
    want = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True).transpose(1, 2)[:, -1].numpy()
    np.testing.assert_allclose(step, want, rtol=1e-12, atol=1e-13)


def test_decode_first_step_returns_value():
    v = rnd(2, 4, 1, 16, seed=5)
    out = decode_step(rnd(2, 4, 16, seed=6), rnd(2, 4, 1, 16, seed=7), v)
    np.testing.assert_allclose(out, v[:, :, 0], atol=1e-15)


# --- backward -----------------------------------------------------------------


def _torch_policy_grads(q, k, mask, scale, grad, wrt):
    """dq, dk by torch autograd (float64, CPU) through matmul, masked_fill(-1e10)
    and (``wrt="probs"``) softmax: the reference head's operations."""
    tq, tk = (torch.from_numpy(np.ascontiguousarray(x)).requires_grad_(True) for x in (q, k))
    logits = torch.matmul(tq, tk.transpose(-2, -1)) * scale
    if mask is not None:
        logits = logits.masked_fill(~torch.from_numpy(mask), ILLEGAL_LOGIT)
    out = logits.reshape(q.shape[0], -1)
    if wrt == "probs":
        out = torch.softmax(out, dim=-1)
    out.backward(torch.from_numpy(np.ascontiguousarray(grad)))
    return tq.grad.numpy(), tk.grad.numpy()


@pytest.mark.parametrize("wrt", ["logits", "probs"])
@pytest.mark.parametrize("masked", [False, True])
def test_backward_matches_torch_autograd(wrt, masked):
    from oracle.policy import kq_backward

    b, s, d = 3, 17, 16
    q, k = rnd(b, s, d, seed=1), rnd(b, s, d, seed=2)
    mask = mask_of(b, s, 0.2, seed=3) if masked else None
    if masked:
        mask[2] = False  # a sample with no legal move: uniform P, zero gradient
    g = rnd(b, s * s, seed=4)
    got = kq_backward(q, k, mask, 0.25, g, wrt=wrt)
    want = _torch_policy_grads(q, k, mask, 0.25, g, wrt)
    for a, w in zip(got, want):
        np.testing.assert_allclose(a, w, rtol=1e-10, atol=1e-12)
    if masked:
        assert np.all(got[0][2] == 0) and np.all(got[1][2] == 0)


@pytest.mark.parametrize("wrt", ["logits", "probs"])
def test_backward_central_finite_differences(wrt):
    """Each entry of dq, dk equals d<f(q, k), G>/dx by central differences of
    the (independently pinned) forward f = kq_logits or kq_probs."""
    from oracle.policy import kq_backward

    b, s, d, scale = 1, 4, 3, 0.7
    q, k = rnd(b, s, d, seed=5), rnd(b, s, d, seed=6)
    mask = mask_of(b, s, 0.5, seed=7)
    g = rnd(b, s * s, seed=8)
    f = kq_probs if wrt == "probs" else kq_logits
    grads = kq_backward(q, k, mask, scale, g, wrt=wrt)
    eps = 1e-6
    for which, gr in enumerate(grads):
        fd = np.zeros_like(gr)
        for idx in np.ndindex(*gr.shape):
            xs_p, xs_m = [q.copy(), k.copy()], [q.copy(), k.copy()]
            xs_p[which][idx] += eps
            xs_m[which][idx] -= eps
            fp = np.sum(np.where(f(*xs_p, mask, scale) > -1e9, f(*xs_p, mask, scale), 0.0) * g)
            fm = np.sum(np.where(f(*xs_m, mask, scale) > -1e9, f(*xs_m, mask, scale), 0.0) * g)
            fd[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(gr, fd, rtol=1e-6, atol=1e-8)
