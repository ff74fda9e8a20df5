"""Incremental-decode oracle (float64, numpy).

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import numpy as np

from .attention import attention


def decode_step(q_t: np.ndarray, k_prefix: np.ndarray, v_prefix: np.ndarray, scale: float | None = None) -> np.ndarray:
    """Attention of the newest token over a prefix of ``t`` cached tokens.

    q_t ``[B, H, D]``; k_prefix / v_prefix ``[B, H_kv, t, D]`` -> ``[B, H, D]``.

    The reference has no cache: SetupNetwork re-runs the causal attention over
    the whole prefix for each new piece (stratego/training/selfplay.py:139-146,
    181) and reads the last position (selfplay.py:182).  Under the top-left
    causal mask of stratego/networks/attention.py:303-308 with S_q = S_kv = t,
    row ``t-1`` masks nothing, so that last row is plain attention of one
    query over all ``t`` keys, which is what this returns.
    """
    q = np.asarray(q_t)[:, None, :, :]  # [B, 1, H, D]
    k = np.asarray(k_prefix).transpose(0, 2, 1, 3)  # [B, t, H_kv, D]
    v = np.asarray(v_prefix).transpose(0, 2, 1, 3)
    return attention(q, k, v, causal=False, scale=scale)[:, 0]


def full_recompute_last_row(q_seq, k_seq, v_seq, scale: float | None = None) -> np.ndarray:
    """The reference's own route: causal attention over the whole prefix
    (``[B, t, H, D]`` inputs), keeping only the last query row."""
    return attention(q_seq, k_seq, v_seq, causal=True, scale=scale)[:, -1]
