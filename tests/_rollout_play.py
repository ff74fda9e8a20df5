"""Random self-play drivers shared by the oracle and GPU rollout tests."""

from __future__ import annotations

import numpy as np


def random_actions(mask: np.ndarray, rng: np.random.Generator, p_illegal: float = 0.1) -> np.ndarray:
    """One action per game: a uniformly random legal move from ``mask``
    ``[N, 100, 100]``, or with probability ``p_illegal`` (and always when no
    move is legal) a random integer in [-3, 10003), mostly illegal or out of
    range."""
    n = mask.shape[0]
    flat = mask.reshape(n, -1)
    scores = rng.random(flat.shape, dtype=np.float32)
    scores[~flat] = -1.0
    out = scores.argmax(axis=1).astype(np.int64)
    wild = (rng.random(n) < p_illegal) | ~flat.any(axis=1)
    out[wild] = rng.integers(-3, 10003, size=int(wild.sum()))
    return out


def perturb_trackers(st, rng: np.random.Generator) -> None:
    """Move an oracle state's counters and rings to the edges random play
    rarely reaches, keeping every value in its valid range: chase rings full
    (the overwrite path), counters one step from the draw limits, two-square
    counts at the limit, history rings at arbitrary heads."""
    n = st.n
    full = rng.random((n, 2)) < 0.5
    st.chase_len[:] = np.where(full, 64, rng.integers(0, 64, size=(n, 2)))
    st.chase_head[:] = np.where(full, rng.integers(0, 64, size=(n, 2)), 0)
    st.chase_hashes[:] = rng.integers(0, 1 << 62, size=st.chase_hashes.shape, dtype=np.int64)
    st.chase_last_src[:] = rng.integers(-1, 100, size=(n, 2))
    st.two_sq_count[:] = rng.integers(0, 5, size=(n, 2))
    st.since_attack[:] = rng.choice([0, 50, 98, 99], size=n)
    st.move_number[:] = rng.choice([10, 500, 3998, 3999], size=n)
    st.history_len[:] = rng.integers(0, 33, size=n)
    st.history_head[:] = rng.integers(0, 32, size=n)
