"""Pins ``oracle.attention.attention_backward`` (CPU, no GPU needed).

Independent references: torch autograd through ``scaled_dot_product_attention``
and through an explicit softmax formulation on the CPU in float64 (library
code that shares nothing with the oracle), and central finite differences of
the oracle's forward, which is itself pinned against torch SDPA.  Planted
mistakes (a dropped softmax term, a missing scale, transposed operands, GQA
gradients not summed) are rejected in ``tests/test_oracle_mutations.py``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F  # noqa: N812

from oracle.attention import attention, attention_backward

pytestmark = pytest.mark.filterwarnings("ignore::UserWarning")


def rnd(*shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape)


def torch_grads(q, k, v, d_o, causal=False, key_pad=None, scale=None, explicit=False):
    """dq, dk, dv by torch autograd (float64, CPU) on BSHD numpy arrays."""
    tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(x)).requires_grad_(True) for x in (q, k, v))
    qh, kh, vh = (t.transpose(1, 2) for t in (tq, tk, tv))
    h, hkv = qh.shape[1], kh.shape[1]
    if hkv != h:
        kh = kh.repeat_interleave(h // hkv, dim=1)
        vh = vh.repeat_interleave(h // hkv, dim=1)
    sq, skv = q.shape[1], k.shape[1]
    keep = torch.ones(sq, skv, dtype=torch.bool)
    if causal:
        keep = keep.tril()
    keep = keep[None, None].expand(q.shape[0], 1, sq, skv)
    if key_pad is not None:
        keep = keep & ~torch.from_numpy(key_pad)[:, None, None, :]
    if explicit:
        sc = scale if scale is not None else 1.0 / np.sqrt(q.shape[-1])
        s = (qh @ kh.transpose(-1, -2)) * sc
        o = torch.softmax(s.masked_fill(~keep, float("-inf")), dim=-1) @ vh
    else:
        o = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=keep, scale=scale)
    o.transpose(1, 2).backward(torch.from_numpy(np.ascontiguousarray(d_o)))
    return tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()


@pytest.mark.parametrize(
    "b,sq,skv,h,hkv,d,causal,pad",
    [
        (2, 100, 100, 6, 6, 64, False, False),
        (2, 40, 40, 4, 4, 32, True, False),
        (2, 40, 100, 4, 4, 64, False, True),
        (2, 17, 9, 3, 3, 16, True, False),
        (2, 9, 17, 3, 3, 48, True, True),
        (2, 33, 33, 8, 2, 32, False, False),
        (1, 1, 1, 2, 2, 16, False, False),
    ],
)
def test_matches_torch_autograd_through_sdpa(b, sq, skv, h, hkv, d, causal, pad):
    q, k, v = rnd(b, sq, h, d, seed=1), rnd(b, skv, hkv, d, seed=2), rnd(b, skv, hkv, d, seed=3)
    d_o = rnd(b, sq, h, d, seed=4)
    key_pad = None
    if pad:
        key_pad = np.random.default_rng(5).random((b, skv)) < 0.3
        key_pad[:, 0] = False  # keep every row partly visible: SDPA and math differ on empty rows
    got = attention_backward(q, k, v, d_o, causal=causal, key_pad=key_pad)
    ref = torch_grads(q, k, v, d_o, causal=causal, key_pad=key_pad)
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        np.testing.assert_allclose(a, r, rtol=1e-10, atol=1e-11, err_msg=name)


def test_scale_argument_matches_torch():
    q, k, v, d_o = rnd(2, 12, 2, 16, seed=1), rnd(2, 12, 2, 16, seed=2), rnd(2, 12, 2, 16, seed=3), rnd(2, 12, 2, 16, seed=4)
    got = attention_backward(q, k, v, d_o, scale=0.3)
    ref = torch_grads(q, k, v, d_o, scale=0.3)
    for a, r in zip(got, ref):
        np.testing.assert_allclose(a, r, rtol=1e-10, atol=1e-11)


@pytest.mark.parametrize("causal,pad", [(False, False), (True, False), (False, True), (True, True)])
def test_central_finite_differences_of_the_forward(causal, pad):
    """Every gradient entry equals d<attention(x), dO>/dx by central
    differences of the (independently pinned) forward, step 1e-6."""
    b, sq, skv, h, d = 1, 3, 4, 2, 4
    q, k, v = rnd(b, sq, h, d, seed=11), rnd(b, skv, h, d, seed=12), rnd(b, skv, h, d, seed=13)
    d_o = rnd(b, sq, h, d, seed=14)
    key_pad = np.array([[False, True, False, False]]) if pad else None
    grads = attention_backward(q, k, v, d_o, causal=causal, key_pad=key_pad)
    eps = 1e-6
    inputs = [q, k, v]
    for which, g in enumerate(grads):
        fd = np.zeros_like(g)
        for idx in np.ndindex(*g.shape):
            plus = [x.copy() for x in inputs]
            minus = [x.copy() for x in inputs]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fp = np.sum(attention(*plus, causal=causal, key_pad=key_pad) * d_o)
            fm = np.sum(attention(*minus, causal=causal, key_pad=key_pad) * d_o)
            fd[idx] = (fp - fm) / (2 * eps)
        np.testing.assert_allclose(g, fd, rtol=1e-6, atol=1e-8, err_msg="dq dk dv".split()[which])
    if pad:
        # a padded key receives no gradient at all
        assert np.all(grads[1][:, 1] == 0) and np.all(grads[2][:, 1] == 0)


def test_fully_masked_row_matches_autograd_through_masked_fill():
    """An all-padded batch row under autograd through ``masked_fill`` +
    softmax + matmul (the reference math path's operations): its dq and dk
    are 0, its dv slice is NaN; the other batch row is finite and equal."""
    q, k, v, d_o = rnd(2, 3, 2, 8, seed=1), rnd(2, 4, 2, 8, seed=2), rnd(2, 4, 2, 8, seed=3), rnd(2, 3, 2, 8, seed=4)
    pad = np.zeros((2, 4), dtype=bool)
    pad[1] = True
    got = attention_backward(q, k, v, d_o, key_pad=pad)
    ref = torch_grads(q, k, v, d_o, key_pad=pad, explicit=True)
    for a, r in zip(got, ref):
        assert np.array_equal(np.isnan(a), np.isnan(r))
        assert np.isfinite(a[0]).all()
        np.testing.assert_allclose(a[0], r[0], rtol=1e-10, atol=1e-11)
    dq, dk, dv = got
    assert np.all(dq[1] == 0) and np.all(dk[1] == 0) and np.isnan(dv[1]).all()


def test_fully_masked_causal_rows_only_poison_their_head():
    """Causal plus padding of key 0: query row 0 sees no key.  Only dv of
    that (batch, head) goes NaN, matching autograd; dq row 0 is 0."""
    q, k, v, d_o = rnd(1, 4, 2, 8, seed=5), rnd(1, 4, 2, 8, seed=6), rnd(1, 4, 2, 8, seed=7), rnd(1, 4, 2, 8, seed=8)
    pad = np.array([[True, False, False, False]])
    got = attention_backward(q, k, v, d_o, causal=True, key_pad=pad)
    ref = torch_grads(q, k, v, d_o, causal=True, key_pad=pad, explicit=True)
    for a, r in zip(got, ref):
        assert np.array_equal(np.isnan(a), np.isnan(r))
        fin = ~np.isnan(r)
        np.testing.assert_allclose(a[fin], r[fin], rtol=1e-10, atol=1e-11)
    assert np.all(got[0][0, 0] == 0) and np.isnan(got[2]).all()


def test_gqa_gradients_sum_over_the_group():
    """With H_kv < H, dk/dv equal the per-head gradients of the explicitly
    expanded K/V summed over each group of H/H_kv query heads."""
    q, k, v, d_o = rnd(2, 5, 8, 4, seed=1), rnd(2, 6, 2, 4, seed=2), rnd(2, 6, 2, 4, seed=3), rnd(2, 5, 8, 4, seed=4)
    dq, dk, dv = attention_backward(q, k, v, d_o)
    dqe, dke, dve = attention_backward(q, np.repeat(k, 4, axis=2), np.repeat(v, 4, axis=2), d_o)
    np.testing.assert_allclose(dq, dqe, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dk, dke.reshape(2, 6, 2, 4, 4).sum(axis=3), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dv, dve.reshape(2, 6, 2, 4, 4).sum(axis=3), rtol=1e-12, atol=1e-13)
