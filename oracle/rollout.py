"""numpy state + ctypes front of ``oracle/rollout.c``, the CPU restatement of
the reference's batched Stratego simulator (csrc/stratego_buffer.cu / .cpp).

Test infrastructure only (see ``oracle/__init__.py``): tests and bench's CPU
leg use it to check the HIP rollout kernels.  ``build()`` compiles the C file
with gcc into ``oracle/_build/librollout_oracle.so``.

:class:`State` holds the same arrays, shapes and initial values as the
reference buffer's constructor (stratego_buffer.cpp:9-54) as numpy arrays.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "rollout.c"
LIB = HERE / "_build" / "librollout_oracle.so"

# name, dtype, shape after the game axis, initial value (stratego_buffer.cpp:24-53)
FIELDS = (
    ("owner", np.int8, (100,), -1),
    ("piece", np.int8, (100,), 0),
    ("player", np.int8, (), 0),
    ("move_number", np.int32, (), 0),
    ("since_attack", np.int32, (), 0),
    ("outcome", np.int8, (), -1),
    ("terminated", np.uint8, (), 0),
    ("flag_captured", np.uint8, (), 0),
    ("terminated_since", np.int32, (), 0),
    ("moved", np.uint8, (100,), 0),
    ("revealed", np.uint8, (100,), 0),
    ("history", np.int32, (32,), 0),
    ("history_head", np.int32, (), 0),
    ("history_len", np.int32, (), 0),
    ("two_sq_count", np.int32, (2,), 0),
    ("two_sq_lo", np.int32, (2,), -1),
    ("two_sq_hi", np.int32, (2,), -1),
    ("two_sq_violation", np.uint8, (), 0),
    ("chase_hashes", np.int64, (2, 64), 0),
    ("chase_head", np.int32, (2,), 0),
    ("chase_len", np.int32, (2,), 0),
    ("chase_last_src", np.int32, (2,), -1),
    ("chasing_violation", np.uint8, (), 0),
)
STATE_FIELDS = tuple(f[0] for f in FIELDS)


class _OrcState(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in STATE_FIELDS[:18]] + [("zobrist", ctypes.c_void_p)] + [
        (name, ctypes.c_void_p) for name in STATE_FIELDS[18:]
    ] + [("n", ctypes.c_int32)]


def build(force: bool = False) -> Path:
    """Compile rollout.c with gcc (-O2, no fast-math) if the library is
    missing or older than the source."""
    if force or not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
        LIB.parent.mkdir(exist_ok=True)
        tmp = LIB.with_suffix(".tmp.so")
        subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-o", str(tmp), str(SRC)], check=True)
        tmp.replace(LIB)
    return LIB


_lib = None


def _load():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(build()))
        ptr = ctypes.POINTER(_OrcState)
        lib.orc_apply.argtypes = [ptr, ctypes.c_void_p]
        lib.orc_legal_mask.argtypes = [ptr, ctypes.c_void_p]
        lib.orc_reset.argtypes = [ptr, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        lib.orc_infostate.argtypes = [ptr, ctypes.c_void_p]
        lib.orc_hash.argtypes = [ptr, ctypes.c_void_p]
        lib.orc_any_move.argtypes = [ptr, ctypes.c_void_p]
        for f in ("orc_apply", "orc_legal_mask", "orc_reset", "orc_infostate", "orc_hash", "orc_any_move"):
            getattr(lib, f).restype = None
        _lib = lib
    return _lib


class State:
    """The simulator state of ``n`` games as numpy arrays (attributes named as
    in :data:`STATE_FIELDS`) plus the Zobrist table ``[10, 10, 2, 13]``."""

    def __init__(self, n: int, zobrist: np.ndarray | None = None, seed: int = 0) -> None:
        self.n = n
        for name, dt, shape, init in FIELDS:
            setattr(self, name, np.full((n, *shape), init, dtype=dt))
        if zobrist is None:
            zobrist = np.random.default_rng(seed).integers(0, 1 << 62, size=(10, 10, 2, 13), dtype=np.int64)
        self.zobrist = np.ascontiguousarray(zobrist, dtype=np.int64)

    def copy(self) -> "State":
        other = State.__new__(State)
        other.n = self.n
        for name in STATE_FIELDS:
            setattr(other, name, getattr(self, name).copy())
        other.zobrist = self.zobrist.copy()
        return other

    def _c(self) -> _OrcState:
        s = _OrcState()
        for name in STATE_FIELDS:
            a = getattr(self, name)
            assert a.flags.c_contiguous
            setattr(s, name, a.ctypes.data)
        s.zobrist = self.zobrist.ctypes.data
        s.n = self.n
        return s

    def apply(self, actions) -> None:
        a = np.ascontiguousarray(actions, dtype=np.int64)
        assert a.shape == (self.n,)
        _load().orc_apply(ctypes.byref(self._c()), a.ctypes.data)

    def legal_mask(self) -> np.ndarray:
        out = np.empty((self.n, 100, 100), dtype=np.uint8)
        _load().orc_legal_mask(ctypes.byref(self._c()), out.ctypes.data)
        return out.astype(bool)

    def reset(self, setup_red, setup_blue, force_all: bool = False) -> None:
        r = np.ascontiguousarray(setup_red, dtype=np.int8).reshape(self.n, 100)
        b = np.ascontiguousarray(setup_blue, dtype=np.int8).reshape(self.n, 100)
        _load().orc_reset(ctypes.byref(self._c()), r.ctypes.data, b.ctypes.data, int(force_all))

    def infostate(self) -> np.ndarray:
        out = np.empty((self.n, 488, 10, 10), dtype=np.float32)
        _load().orc_infostate(ctypes.byref(self._c()), out.ctypes.data)
        return out

    def hash_board(self) -> np.ndarray:
        out = np.empty(self.n, dtype=np.int64)
        _load().orc_hash(ctypes.byref(self._c()), out.ctypes.data)
        return out

    def any_move(self) -> np.ndarray:
        out = np.empty(self.n, dtype=np.uint8)
        _load().orc_any_move(ctypes.byref(self._c()), out.ctypes.data)
        return out.astype(bool)


# PieceType counts per player (stratego/types.py piece_count): 40 pieces.
PIECE_COUNTS = {1: 1, 2: 8, 3: 5, 4: 4, 5: 4, 6: 4, 7: 3, 8: 2, 9: 1, 10: 1, 11: 1, 12: 6}


def random_setups(n: int, rng: np.random.Generator) -> tuple[np.ndarray, np.ndarray]:
    """``n`` random full setups per side as ``[n, 10, 10]`` int8 piece grids:
    Red in rows 0-3, Blue in rows 6-9 (stratego/constants.py:32-33), the 40
    pieces of :data:`PIECE_COUNTS` each."""
    pieces = np.repeat(np.array(list(PIECE_COUNTS), dtype=np.int8), list(PIECE_COUNTS.values()))
    red = np.zeros((n, 10, 10), dtype=np.int8)
    blue = np.zeros((n, 10, 10), dtype=np.int8)
    for g in range(n):
        red[g, 0:4] = rng.permutation(pieces).reshape(4, 10)
        blue[g, 6:10] = rng.permutation(pieces).reshape(4, 10)
    return red, blue


# oracle State attribute -> the reference buffer's tensor name (stratego_buffer.cpp:24-53)
BUFFER_NAMES = {
    "owner": "board_owner",
    "piece": "board_piece",
    "player": "current_player",
    "move_number": "move_number",
    "since_attack": "moves_since_attack",
    "outcome": "outcome",
    "terminated": "terminated",
    "flag_captured": "flag_captured",
    "terminated_since": "terminated_since",
    "moved": "moved_squares",
    "revealed": "revealed_squares",
    "history": "move_history",
    "history_head": "move_history_head",
    "history_len": "move_history_len",
    "two_sq_count": "two_square_count",
    "two_sq_lo": "two_square_pair_lo",
    "two_sq_hi": "two_square_pair_hi",
    "two_sq_violation": "two_square_violation",
    "chase_hashes": "chase_hashes",
    "chase_head": "chase_hash_head",
    "chase_len": "chase_hash_len",
    "chase_last_src": "chase_last_src",
    "chasing_violation": "chasing_violation",
}
