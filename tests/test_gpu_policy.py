"""Parity of the fused key-query policy kernel against the float64 oracle."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import ops
from oracle.policy import kq_logits, kq_probs
from tests._cases import LOWP_ABS_TOL, legal_mask, randn, to_np64

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


def _run(cuda, b, s, d, dtype, p=0.02, seed=0, output="probs", with_mask=True):
    _announce(f"kq b={b} s={s} d={d} {dtype} {output} mask={with_mask}")
    q = randn((b, s, d), seed, dtype)
    k = randn((b, s, d), seed + 1, dtype)
    mask = legal_mask(b, s, seed + 2, p) if with_mask else None
    scale = 1.0 / np.sqrt(d)
    out = ops.kq_policy(q.to(cuda), k.to(cuda), None if mask is None else mask.to(cuda), scale=scale, output=output)
    torch.cuda.synchronize()
    fn = kq_probs if output == "probs" else kq_logits
    ref = fn(to_np64(q), to_np64(k), None if mask is None else mask.numpy(), scale)
    return out.cpu(), ref, mask


def _check_probs(out, ref, mask, dtype):
    o = out.double().numpy()
    if mask is not None:
        illegal = ~mask.reshape(mask.shape[0], -1).numpy()
        assert (o[illegal] == 0.0).all(), "illegal entries must be exactly 0"
    assert np.isfinite(o).all()
    np.testing.assert_allclose(o.sum(axis=1), 1.0, atol=1e-5)
    err = np.abs(o - ref).max()
    if dtype == torch.float32:
        assert err <= 1e-5 * np.abs(ref).max() + 1e-12
    else:
        assert err <= LOWP_ABS_TOL
    return err


def test_config2_full_size(cuda):
    """C2: B=4096, 100 squares, d=64, bf16, Bernoulli(0.02) legal mask."""
    out, ref, mask = _run(cuda, 4096, 100, 64, torch.bfloat16, seed=44)
    _check_probs(out, ref, mask, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("s", [1, 5, 16, 17, 64, 100, 101, 128])
def test_probs_shapes(cuda, dtype, s):
    out, ref, mask = _run(cuda, 6, s, 64, dtype, p=0.1, seed=s)
    _check_probs(out, ref, mask, dtype)


@pytest.mark.parametrize("d", [8, 32, 48, 64, 72, 384])
def test_policy_dims(cuda, d):
    """d=384 is the reference's default policy_d_model (= model dim)."""
    out, ref, mask = _run(cuda, 4, 100, d, torch.bfloat16, seed=d)
    _check_probs(out, ref, mask, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_logits_mode(cuda, dtype):
    out, ref, mask = _run(cuda, 8, 100, 64, dtype, p=0.3, seed=3, output="logits")
    o = out.double().numpy()
    illegal = ~mask.reshape(8, -1).numpy()
    assert (o[illegal] == np.float32(-1e10)).all()
    legal = ~illegal
    err = np.abs(o[legal] - ref[legal]).max()
    tol = 1e-5 * np.abs(ref[legal]).max() if dtype == torch.float32 else LOWP_ABS_TOL
    assert err <= tol
    # The reference's own invariant (tests/test_move_net.py:67-84).
    assert int((o <= -1e9).sum()) == int(illegal.sum())


def test_no_mask_probs_and_logits(cuda):
    out, ref, _ = _run(cuda, 4, 100, 64, torch.float32, seed=8, with_mask=False)
    _check_probs(out, ref, None, torch.float32)
    lo, lref, _ = _run(cuda, 4, 100, 64, torch.float32, seed=8, with_mask=False, output="logits")
    assert (lo > -1e9).all()  # tests/test_move_net.py:86-92
    np.testing.assert_allclose(lo.double().numpy(), lref, rtol=0, atol=1e-5 * np.abs(lref).max())


def test_single_legal_move_is_certain(cuda):
    b, s, d = 3, 100, 64
    q = randn((b, s, d), 1, torch.bfloat16).to(cuda)
    k = randn((b, s, d), 2, torch.bfloat16).to(cuda)
    mask = torch.zeros(b, s, s, dtype=torch.bool)
    mask[0, 3, 5] = True
    mask[1, 7, 2] = True
    mask[2, 99, 99] = True
    out = ops.kq_policy(q, k, mask.to(cuda)).cpu()
    assert out[0, 3 * s + 5] == 1.0 and out[1, 7 * s + 2] == 1.0 and out[2, 99 * s + 99] == 1.0
    assert int((out != 0).sum()) == 3


def test_all_illegal_is_uniform(cuda):
    b, s, d = 2, 100, 64
    q = randn((b, s, d), 1, torch.bfloat16).to(cuda)
    k = randn((b, s, d), 2, torch.bfloat16).to(cuda)
    mask = torch.zeros(b, s, s, dtype=torch.bool)
    mask[1, 0, 0] = True
    out = ops.kq_policy(q, k, mask.to(cuda)).cpu().double()
    np.testing.assert_allclose(out[0].numpy(), 1.0 / (s * s), rtol=1e-6)
    assert out[1, 0] == 1.0


def test_equal_logits_split_evenly(cuda):
    b, s, d = 2, 100, 64
    q = torch.zeros(b, s, d, dtype=torch.bfloat16, device=cuda)
    k = torch.zeros(b, s, d, dtype=torch.bfloat16, device=cuda)
    mask = legal_mask(b, s, 9, 0.05)
    out = ops.kq_policy(q, k, mask.to(cuda)).cpu().double()
    n = mask.reshape(b, -1).sum(dim=1).double()
    for i in range(b):
        legal = mask[i].reshape(-1)
        np.testing.assert_allclose(out[i][legal].numpy(), 1.0 / n[i].item(), rtol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 384])
@pytest.mark.parametrize("output", ["probs", "logits"])
def test_reference_move_head_shape(cuda, dtype, d, output):
    """101 squares (the reference Move network): the sample's mask bytes and
    output row start at every alignment mod 16 across 9 samples, which the
    kernel reads and writes in 4-entry groups phased to each base."""
    out, ref, mask = _run(cuda, 9, 101, d, dtype, p=0.1, seed=500 + d, output=output)
    if output == "probs":
        _check_probs(out, ref, mask, dtype)
    else:
        o = out.double().numpy()
        illegal = ~mask.reshape(9, -1).numpy()
        assert (o[illegal] == np.float32(-1e10)).all()
        err = np.abs(o[~illegal] - ref[~illegal]).max()
        assert err <= (1e-5 * np.abs(ref[~illegal]).max() if dtype == torch.float32 else LOWP_ABS_TOL)


@pytest.mark.parametrize("s", [100, 101])
@pytest.mark.parametrize("output", ["probs", "logits"])
def test_misaligned_mask_and_output_views(cuda, s, output):
    """A mask that starts 3 bytes into its buffer and an output that starts
    one float into its own (contiguous views, NaN around the output): the
    results match the aligned call bit for bit and nothing outside the
    output view is written."""
    b, d = 6, 64
    _announce(f"kq misaligned views s={s} {output}")
    q = randn((b, s, d), 70 + s, torch.bfloat16).to(cuda)
    k = randn((b, s, d), 71 + s, torch.bfloat16).to(cuda)
    mask = legal_mask(b, s, 72 + s, 0.1)
    mbig = torch.zeros(b * s * s + 3, dtype=torch.bool)
    mbig[3:] = mask.reshape(-1)
    mview = mbig.to(cuda)[3:].view(b, s, s)
    obig = torch.full((b * s * s + 2,), float("nan"), dtype=torch.float32, device=cuda)
    oview = obig[1:1 + b * s * s].view(b, s * s)
    ops.kq_policy(q, k, mview, output=output, out=oview)
    want = ops.kq_policy(q, k, mask.to(cuda), output=output)
    torch.cuda.synchronize()
    assert torch.isnan(obig[0]) and torch.isnan(obig[-1]), "written outside the output view"
    assert torch.equal(oview, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("s", [5, 17, 33, 127])
def test_wide_head_at_odd_square_counts(cuda, dtype, s):
    """d = 384 (rows staged in several slices) at square counts whose mask
    rows and outputs start unaligned, from one to eight tile rows."""
    out, ref, mask = _run(cuda, 6, s, 384, dtype, p=0.2, seed=600 + s)
    _check_probs(out, ref, mask, dtype)
