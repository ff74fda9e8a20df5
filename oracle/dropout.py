"""numpy restatement of the attention-dropout keep rule of the HIP kernels
(``drop_hash`` / ``make_drop_key`` in ``ataraxos_amd/csrc/atx_common.hpp``):
test infrastructure only (see ``oracle/__init__.py``).

The reference applies ``F.dropout`` to the softmax weights
(stratego/networks/attention.py:312-313; FA2's ``dropout_p``, :236-253): each
weight is zeroed with probability p and the survivors scaled by 1 / (1 - p).
Torch's own dropout draws from its Philox stream, which no other
implementation reproduces (FA2 has its own); the kernels draw from a
counter-based hash instead, and this file restates it so tests can
materialise the exact mask.  Its parity is pinned by MurmurHash3's published
fmix32 values, splitmix64's published outputs, and the keep rate and
independence statistics in tests/test_oracle_dropout.py.
"""

from __future__ import annotations

import numpy as np

M32 = np.uint64(0xFFFFFFFF)


def fmix32(h: np.ndarray) -> np.ndarray:
    """MurmurHash3's 32-bit finaliser on uint32 values."""
    h = np.asarray(h, dtype=np.uint64) & M32
    h ^= h >> np.uint64(16)
    h = (h * np.uint64(0x85EBCA6B)) & M32
    h ^= h >> np.uint64(13)
    h = (h * np.uint64(0xC2B2AE35)) & M32
    h ^= h >> np.uint64(16)
    return h.astype(np.uint32)


def splitmix64(z: int) -> int:
    """Vigna's splitmix64 step (one output for state z)."""
    m = (1 << 64) - 1
    z = (z + 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def drop_key(p: float, seed: int, offset: int) -> tuple[int, int, int, float]:
    """(k0, k1, thresh, scale) as make_drop_key derives them."""
    key = splitmix64((seed ^ splitmix64(offset)) & ((1 << 64) - 1))
    t = float(np.float32(p)) * 4294967296.0
    thresh = 0xFFFFFFFF if t >= 4294967295.0 else int(t)
    scale = float(np.float32(1.0) / (np.float32(1.0) - np.float32(p))) if p > 0 else 1.0
    return key & 0xFFFFFFFF, key >> 32, thresh, scale


def drop_hash(idx: np.ndarray, k0: int, k1: int) -> np.ndarray:
    idx = np.asarray(idx, dtype=np.uint64)
    lo = (idx & M32) ^ np.uint64(k0)
    hi = (idx >> np.uint64(32)) ^ np.uint64(k1)
    h = (lo * np.uint64(0x9E3779B1)) & M32
    h ^= (hi * np.uint64(0x85EBCA77)) & M32
    return fmix32(h)


def keep_mask(b: int, h: int, sq: int, skv: int, p: float, seed: int, offset: int) -> np.ndarray:
    """bool [b, h, sq, skv]: True where the weight survives."""
    k0, k1, thresh, _ = drop_key(p, seed, offset)
    idx = np.arange(b * h * sq * skv, dtype=np.uint64).reshape(b, h, sq, skv)
    return drop_hash(idx, k0, k1) >= np.uint32(thresh)
