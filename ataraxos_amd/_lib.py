"""ctypes binding of ``libataraxos_attn.so`` (C ABI in ``include/ataraxos_attn.h``).

The structs below mirror the header field for field; ``tests/test_abi.py``
checks their layout against the C compiler's.  Loading is lazy: importing the
package never touches the GPU or the library, and every entry point raises
:class:`AtxError` (a ``RuntimeError``) when the library is missing, so a GPU
path can never silently run something else.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

ABI_VERSION = 3

OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_UNSUPPORTED = -2
ERR_LAUNCH = -3
ERR_ABI = -4

DTYPE_FP32 = 0
DTYPE_BF16 = 1
DTYPE_FP16 = 2

KQ_OUT_PROBS = 0
KQ_OUT_LOGITS = 1

LIB_NAME = "libataraxos_attn.so"

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float


class AttnParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("batch", _i32),
        ("seq_q", _i32),
        ("seq_kv", _i32),
        ("num_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("q", _ptr),
        ("q_stride_b", _i64),
        ("q_stride_s", _i64),
        ("q_stride_h", _i64),
        ("k", _ptr),
        ("k_stride_b", _i64),
        ("k_stride_s", _i64),
        ("k_stride_h", _i64),
        ("v", _ptr),
        ("v_stride_b", _i64),
        ("v_stride_s", _i64),
        ("v_stride_h", _i64),
        ("o", _ptr),
        ("o_stride_b", _i64),
        ("o_stride_s", _i64),
        ("o_stride_h", _i64),
        ("scale", _f32),
        ("causal", _i32),
        ("key_pad", _ptr),
        ("key_pad_stride_b", _i64),
        ("dropout_p", _f32),
        ("reserved_dropout", _i32),
        ("dropout_seed", _u64),
        ("dropout_offset", _u64),
    ]


class KqParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("batch", _i32),
        ("seq", _i32),
        ("dim", _i32),
        ("out_mode", _i32),
        ("q", _ptr),
        ("q_stride_b", _i64),
        ("q_stride_s", _i64),
        ("k", _ptr),
        ("k_stride_b", _i64),
        ("k_stride_s", _i64),
        ("mask", _ptr),
        ("mask_stride_b", _i64),
        ("mask_stride_s", _i64),
        ("out", _ptr),
        ("out_stride_b", _i64),
        ("scale", _f32),
    ]


class KqBwdParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("batch", _i32),
        ("seq", _i32),
        ("dim", _i32),
        ("out_mode", _i32),
        ("q", _ptr),
        ("q_stride_b", _i64),
        ("q_stride_s", _i64),
        ("k", _ptr),
        ("k_stride_b", _i64),
        ("k_stride_s", _i64),
        ("mask", _ptr),
        ("mask_stride_b", _i64),
        ("mask_stride_s", _i64),
        ("grad", _ptr),
        ("grad_stride_b", _i64),
        ("probs", _ptr),
        ("probs_stride_b", _i64),
        ("dq", _ptr),
        ("dq_stride_b", _i64),
        ("dq_stride_s", _i64),
        ("dk", _ptr),
        ("dk_stride_b", _i64),
        ("dk_stride_s", _i64),
        ("scale", _f32),
    ]


class MhaParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("batch", _i32),
        ("seq", _i32),
        ("embed_dim", _i32),
        ("num_heads", _i32),
        ("causal", _i32),
        ("reserved", _i32),
        ("x", _ptr),
        ("x_stride_b", _i64),
        ("x_stride_s", _i64),
        ("w_q", _ptr),
        ("w_k", _ptr),
        ("w_v", _ptr),
        ("w_o", _ptr),
        ("b_q", _ptr),
        ("b_k", _ptr),
        ("b_v", _ptr),
        ("b_o", _ptr),
        ("y", _ptr),
        ("y_stride_b", _i64),
        ("y_stride_s", _i64),
        ("scale", _f32),
        ("ln_weight", _ptr),
        ("ln_bias", _ptr),
        ("ln_eps", _f32),
        ("residual", _i32),
    ]


class DecodeParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("batch", _i32),
        ("num_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("kv_capacity", _i32),
        ("kv_len", _i32),
        ("kv_lens", _ptr),
        ("q", _ptr),
        ("q_stride_b", _i64),
        ("q_stride_h", _i64),
        ("k_cache", _ptr),
        ("k_stride_b", _i64),
        ("k_stride_h", _i64),
        ("k_stride_s", _i64),
        ("v_cache", _ptr),
        ("v_stride_b", _i64),
        ("v_stride_h", _i64),
        ("v_stride_s", _i64),
        ("k_new", _ptr),
        ("k_new_stride_b", _i64),
        ("k_new_stride_h", _i64),
        ("v_new", _ptr),
        ("v_new_stride_b", _i64),
        ("v_new_stride_h", _i64),
        ("o", _ptr),
        ("o_stride_b", _i64),
        ("o_stride_h", _i64),
        ("scale", _f32),
    ]


class AtxError(RuntimeError):
    """A failed call into ``libataraxos_attn.so``; ``code`` is the ATX_ERR_* value."""

    def __init__(self, message: str, code: int = ERR_LAUNCH) -> None:
        super().__init__(message)
        self.code = code


class AttnBwdParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("batch", _i32),
        ("seq_q", _i32),
        ("seq_kv", _i32),
        ("num_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
    ] + [
        (f"{name}{suffix}" if suffix == "" else f"{name.replace('d_o', 'do')}{suffix}", t)
        for name in ("q", "k", "v", "o", "d_o", "dq", "dk", "dv")
        for suffix, t in (("", _ptr), ("_stride_b", _i64), ("_stride_s", _i64), ("_stride_h", _i64))
    ] + [
        ("scale", _f32),
        ("causal", _i32),
        ("key_pad", _ptr),
        ("key_pad_stride_b", _i64),
        ("dropout_p", _f32),
        ("reserved_dropout", _i32),
        ("dropout_seed", _u64),
        ("dropout_offset", _u64),
    ]


class RolloutState(ctypes.Structure):
    """AtxRolloutState of include/ataraxos_rollout.h: the device arrays of N
    simulated games."""

    _fields_ = [("abi_version", _i32), ("n_games", _i32)] + [
        (name, _ptr)
        for name in (
            "board_owner", "board_piece", "current_player", "move_number", "moves_since_attack", "outcome",
            "terminated", "flag_captured", "terminated_since", "moved_squares", "revealed_squares",
            "move_history", "move_history_head", "move_history_len", "two_square_count",
            "two_square_pair_lo", "two_square_pair_hi", "two_square_violation", "zobrist_table",
            "chase_hashes", "chase_hash_head", "chase_hash_len", "chase_last_src", "chasing_violation",
        )
    ]


_state_ptr = ctypes.POINTER(RolloutState)

# Exported symbols, as declared in include/ataraxos_attn.h and
# include/ataraxos_rollout.h.
ENTRY_POINTS = {
    "atx_attn_fwd": (ctypes.c_int, [ctypes.POINTER(AttnParams), _ptr]),
    "atx_attn_bwd": (ctypes.c_int, [ctypes.POINTER(AttnBwdParams), _ptr]),
    "atx_kq_masked_softmax_fwd": (ctypes.c_int, [ctypes.POINTER(KqParams), _ptr]),
    "atx_kq_bwd": (ctypes.c_int, [ctypes.POINTER(KqBwdParams), _ptr]),
    "atx_mha_fwd": (ctypes.c_int, [ctypes.POINTER(MhaParams), _ptr]),
    "atx_mha_fwd_packed": (ctypes.c_int, [ctypes.POINTER(MhaParams), _ptr]),
    "atx_mha_pack_weight": (ctypes.c_int, [_i32, _i32, _ptr, _ptr, _ptr]),
    "atx_mha_workspace_bytes": (ctypes.c_int64, [_i32]),
    "atx_mha_fwd_ws": (ctypes.c_int, [ctypes.POINTER(MhaParams), _ptr, _i64, _ptr]),
    "atx_mha_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(MhaParams), _ptr]),
    "atx_attn_decode_fwd": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _ptr]),
    "atx_dropout_mask": (ctypes.c_int, [_i32, _i32, _i32, _i32, _f32, _u64, _u64, _ptr, _ptr]),
    # include/ataraxos_rollout.h
    "atx_rollout_apply": (ctypes.c_int, [_state_ptr, _ptr, _ptr]),
    "atx_rollout_legal_mask": (ctypes.c_int, [_state_ptr, _ptr, _ptr]),
    "atx_rollout_infostate": (ctypes.c_int, [_state_ptr, _ptr, _ptr]),
    "atx_rollout_reset": (ctypes.c_int, [_state_ptr, _ptr, _ptr, _i32, _ptr]),
    "atx_rollout_hash": (ctypes.c_int, [_state_ptr, _ptr, _ptr]),
    "atx_rollout_hello": (ctypes.c_int, [_ptr, _i32, _ptr]),
    "atx_last_error": (ctypes.c_char_p, []),
    "atx_abi_version": (ctypes.c_int, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.environ.get("ATARAXOS_AMD_LIB")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / LIB_NAME


def load() -> ctypes.CDLL:
    """Load the library once; raise :class:`AtxError` if it is absent or stale."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.exists():
            raise AtxError(
                f"{LIB_NAME} not found at {path}: build it with `python -m ataraxos_amd.build` "
                "(the HIP kernels have no substitute path)",
                ERR_LAUNCH,
            )
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in ENTRY_POINTS.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.atx_abi_version()
        if version != ABI_VERSION:
            raise AtxError(f"{path} has ABI version {version}, bindings expect {ABI_VERSION}", ERR_ABI)
        _lib = lib
        return lib


def available() -> bool:
    try:
        load()
        return True
    except (AtxError, OSError):
        return False


def last_error() -> str:
    raw = load().atx_last_error()
    return raw.decode() if raw else ""


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise AtxError(f"{what} failed ({rc}): {last_error()}", rc)


def call(name: str, params: ctypes.Structure, stream: int | None) -> int:
    """Invoke entry point ``name`` and return its raw code (no raising)."""
    fn = getattr(load(), name)
    return int(fn(ctypes.byref(params), ctypes.c_void_p(stream or 0)))
