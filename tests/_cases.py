"""Seeded inputs and the comparison rules shared by the parity tests.

Inputs are always drawn on the CPU from a seeded ``torch.Generator`` and then
cast and moved, so the GPU and the oracle see identical values.

Tolerances:
* masked / illegal / padded entries: exactly 0 (probabilities) — checked with ``==``;
* fp32: normwise relative ``max|o - ref| / max|ref| <= 1e-5``;
* bf16 / fp16: ``max|o - ref| <= 2e-2``, where ``ref`` is the float64 oracle
  run on the bf16-rounded inputs.
"""

from __future__ import annotations

import numpy as np
import torch

FP32_REL_TOL = 1e-5
LOWP_ABS_TOL = 2e-2


def randn(shape, seed: int, dtype=torch.float32, std: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


def legal_mask(batch: int, seq: int, seed: int, p: float = 0.02) -> torch.Tensor:
    """Bernoulli(p) legal-move mask with at least one legal entry per sample."""
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand(batch, seq, seq, generator=g) < p
    empty = ~mask.flatten(1).any(dim=1)
    if empty.any():
        idx = torch.randint(0, seq * seq, (int(empty.sum()),), generator=g)
        flat = mask.view(batch, -1)
        flat[empty.nonzero().squeeze(1), idx] = True
    return mask


def to_np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


def assert_close(out: torch.Tensor, ref: np.ndarray, dtype: torch.dtype, what: str = "") -> float:
    """Apply the contract's tolerance for ``dtype``; NaNs must coincide.
    Returns the measured error."""
    o = to_np64(out)
    assert o.shape == ref.shape, f"{what}: shape {o.shape} vs {ref.shape}"
    nan_o, nan_r = np.isnan(o), np.isnan(ref)
    assert np.array_equal(nan_o, nan_r), f"{what}: NaN pattern differs ({nan_o.sum()} vs {nan_r.sum()})"
    o, r = o[~nan_r], ref[~nan_r]
    if o.size == 0:
        return 0.0
    err = float(np.max(np.abs(o - r)))
    if dtype == torch.float32:
        rel = err / max(float(np.max(np.abs(r))), 1e-30)
        assert rel <= FP32_REL_TOL, f"{what}: fp32 normwise relative error {rel:.3e} > {FP32_REL_TOL}"
        return rel
    assert err <= LOWP_ABS_TOL, f"{what}: {dtype} max-abs error {err:.3e} > {LOWP_ABS_TOL}"
    return err
