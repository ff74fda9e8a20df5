"""``StrategoRolloutBuffer``: N Stratego games simulated on the GPU, the
producer of the legal-move masks (``[N, 100, 100]`` bool) and infostates
(``[N, 488, 10, 10]`` float32) that feed the policy head and the encoders.

Drop-in for the reference's CUDA extension class of the same name
(csrc/stratego_buffer.cpp:7-372, bound at :375-411): the same constructor,
methods, return shapes, dtypes and argument checks (``RuntimeError``, as
``TORCH_CHECK`` raises), the same state tensors.  The kernels are the HIP
entry points of include/ataraxos_rollout.h in ``libataraxos_attn.so``,
launched on the current stream of the buffer's device; a missing library
raises (there is no other implementation).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

BOARD = 10
SQUARES = 100
HISTORY = 32
CHASE_RING = 64
CHANNELS = 488

# (name, dtype, shape after the game axis, initial value): stratego_buffer.cpp:24-53
_FIELDS = (
    ("board_owner", torch.int8, (BOARD, BOARD), -1),
    ("board_piece", torch.int8, (BOARD, BOARD), 0),
    ("current_player", torch.int8, (), 0),
    ("move_number", torch.int32, (), 0),
    ("moves_since_attack", torch.int32, (), 0),
    ("outcome", torch.int8, (), -1),
    ("terminated", torch.bool, (), False),
    ("flag_captured", torch.bool, (), False),
    ("terminated_since", torch.int32, (), 0),
    ("moved_squares", torch.bool, (SQUARES,), False),
    ("revealed_squares", torch.bool, (SQUARES,), False),
    ("move_history", torch.int32, (HISTORY,), 0),
    ("move_history_head", torch.int32, (), 0),
    ("move_history_len", torch.int32, (), 0),
    ("two_square_count", torch.int32, (2,), 0),
    ("two_square_pair_lo", torch.int32, (2,), -1),
    ("two_square_pair_hi", torch.int32, (2,), -1),
    ("two_square_violation", torch.bool, (), False),
    ("chase_hashes", torch.int64, (2, CHASE_RING), 0),
    ("chase_hash_head", torch.int32, (2,), 0),
    ("chase_hash_len", torch.int32, (2,), 0),
    ("chase_last_src", torch.int32, (2,), -1),
    ("chasing_violation", torch.bool, (), False),
)


class StrategoRolloutBuffer:
    """``n_games`` games on ``cuda:device_id``.  Methods mirror
    stratego_buffer.cpp:375-411; each launches on the device's current stream
    and returns without synchronising (except ``board_strs`` and
    ``current_step``, which read the state back, as the reference's do)."""

    def __init__(self, n_games: int = 1, device_id: int = 0) -> None:
        self._lib = _lib.load()
        self._n = int(n_games)
        self._device_id = int(device_id)
        self._dev = torch.device("cuda", self._device_id)
        self._t: dict[str, torch.Tensor] = {
            name: torch.full((self._n, *shape), init, dtype=dt, device=self._dev) for name, dt, shape, init in _FIELDS
        }
        # random 62-bit Zobrist keys per (row, col, owner, piece), :43-46
        self._t["zobrist_table"] = torch.randint(0, 1 << 62, (BOARD, BOARD, 2, 13), dtype=torch.int64, device=self._dev)
        self._state = _lib.RolloutState()
        self._state.abi_version = _lib.ABI_VERSION
        self._state.n_games = self._n
        for name in self._t:
            setattr(self._state, name, self._t[name].data_ptr())

    # -- plumbing ----------------------------------------------------------
    def _stream(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(torch.cuda.current_stream(self._dev).cuda_stream or 0)

    def _run(self, name: str, *args) -> None:
        rc = getattr(self._lib, name)(ctypes.byref(self._state), *args, self._stream())
        _lib.check(int(rc), name)

    def raw_state(self) -> dict[str, torch.Tensor]:
        """The live state tensors by the reference's member names (without the
        trailing underscore), ``zobrist_table`` included.  Writes into them
        change the games; shapes and dtypes must not change."""
        return self._t

    # -- reference API -----------------------------------------------------
    @property
    def n_games(self) -> int:
        return self._n

    @property
    def device_id(self) -> int:
        return self._device_id

    def hello_world(self) -> torch.Tensor:
        """``int32 [1]`` = 42 from a kernel (the build check, :56-62)."""
        out = torch.zeros(1, dtype=torch.int32, device=self._dev)
        _lib.check(int(self._lib.atx_rollout_hello(ctypes.c_void_p(out.data_ptr()), 1, self._stream())),
                   "atx_rollout_hello")
        return out

    def apply_actions(self, actions: torch.Tensor) -> None:
        """Apply ``actions`` (int64 ``[N]``, ``src * 100 + dst``) to every
        game at once (:64-121)."""
        if actions.dim() != 1:
            raise RuntimeError("actions must be 1D (N,)")
        if actions.size(0) != self._n:
            raise RuntimeError(f"actions size mismatch: expected {self._n}, got {actions.size(0)}")
        if actions.dtype != torch.int64:
            raise RuntimeError("actions must be int64")
        a = actions.to(self._dev, torch.int64).contiguous()
        self._run("atx_rollout_apply", ctypes.c_void_p(a.data_ptr()))

    def compute_legal_action_mask(self, out: torch.Tensor | None = None) -> torch.Tensor:
        """``bool [N, 100, 100]``, ``mask[g, src, dst]`` legal for the side to
        move (:124-139).  ``out``: an optional preallocated mask to fill."""
        out = self._out(out, (self._n, SQUARES, SQUARES), torch.bool)
        self._run("atx_rollout_legal_mask", ctypes.c_void_p(out.data_ptr()))
        return out

    def compute_reward_pl0(self) -> torch.Tensor:
        """``float32 [N]``: +1 red win, -1 blue win, 0 otherwise (:141-151)."""
        reward = torch.zeros(self._n, dtype=torch.float32, device=self._dev)
        reward.masked_fill_(self._t["outcome"] == 0, 1.0)
        reward.masked_fill_(self._t["outcome"] == 1, -1.0)
        return reward

    def compute_infostate_tensor(self, out: torch.Tensor | None = None) -> torch.Tensor:
        """``float32 [N, 488, 10, 10]`` from the side to move's perspective
        (:154-178).  ``out``: an optional preallocated tensor to fill."""
        out = self._out(out, (self._n, CHANNELS, BOARD, BOARD), torch.float32)
        self._run("atx_rollout_infostate", ctypes.c_void_p(out.data_ptr()))
        return out

    def compute_two_square_rule_applies(self) -> torch.Tensor:
        return self._t["two_square_violation"].clone()

    def is_chasing_violation(self) -> torch.Tensor:
        return self._t["chasing_violation"].clone()

    def hash_board(self) -> torch.Tensor:
        """``int64 [N]`` Zobrist hash of every board (:192-206); the kernel
        writes every element, so the output is not cleared first."""
        out = torch.empty(self._n, dtype=torch.int64, device=self._dev)
        self._run("atx_rollout_hash", ctypes.c_void_p(out.data_ptr()))
        return out

    def get_terminated(self) -> torch.Tensor:
        return self._t["terminated"].clone()

    def get_outcomes(self) -> torch.Tensor:
        return self._t["outcome"].clone()

    def get_board_owner(self) -> torch.Tensor:
        return self._t["board_owner"].clone()

    def get_board_piece(self) -> torch.Tensor:
        return self._t["board_piece"].clone()

    def get_current_player(self) -> torch.Tensor:
        return self._t["current_player"].clone()

    def get_move_number(self) -> torch.Tensor:
        return self._t["move_number"].clone()

    def get_num_moves(self) -> torch.Tensor:
        return self._t["move_number"].clone()

    def get_num_moves_since_last_attack(self) -> torch.Tensor:
        return self._t["moves_since_attack"].clone()

    def get_flag_captured(self) -> torch.Tensor:
        return self._t["flag_captured"].clone()

    def get_has_legal_movement(self) -> torch.Tensor:
        """``bool [N]``: the side to move has a legal move (:214-217)."""
        return self.compute_legal_action_mask().view(self._n, -1).any(-1)

    def get_terminated_since(self) -> torch.Tensor:
        return self._t["terminated_since"].clone()

    def board_strs(self) -> list[str]:
        """One text board per game: ``. `` empty, else ``R``/``B`` and the
        piece number, padded to 3 characters; one line per row (:221-242)."""
        owner = self._t["board_owner"].cpu()
        piece = self._t["board_piece"].cpu()
        out = []
        for g in range(self._n):
            lines = []
            for r in range(BOARD):
                row = ""
                for c in range(BOARD):
                    o, p = int(owner[g, r, c]), int(piece[g, r, c])
                    row += ". " if o < 0 else ("R" if o == 0 else "B") + str(p) + (" " if p < 10 else "")
                lines.append(row + "\n")
            out.append("".join(lines))
        return out

    def reset_terminated(self, setup_red: torch.Tensor, setup_blue: torch.Tensor) -> None:
        """Restart every terminated game from ``setup_red`` / ``setup_blue``
        (int8 ``[N, 10, 10]`` piece grids) (:246-301)."""
        self._reset(setup_red, setup_blue, force_all=False)

    def reset_all(self, setup_red: torch.Tensor, setup_blue: torch.Tensor) -> None:
        """Restart every game (:304-307)."""
        self._reset(setup_red, setup_blue, force_all=True)

    def current_step(self) -> int:
        """Total moves over all games (:310-312)."""
        return int(self._t["move_number"].sum().item())

    # -- helpers -------------------------------------------------------------
    def _reset(self, setup_red: torch.Tensor, setup_blue: torch.Tensor, force_all: bool) -> None:
        for name, t in (("setup_red", setup_red), ("setup_blue", setup_blue)):
            if t.dim() != 3:
                raise RuntimeError(f"{name} must be (N, 10, 10)")
            if t.size(0) != self._n:
                raise RuntimeError(f"{name} N mismatch")
            if t.size(1) != BOARD or t.size(2) != BOARD:
                raise RuntimeError(f"{name} must be (N, 10, 10)")
            if t.dtype != torch.int8:
                raise RuntimeError(f"{name} must be int8")
        red = setup_red.to(self._dev, torch.int8).contiguous()
        blue = setup_blue.to(self._dev, torch.int8).contiguous()
        rc = self._lib.atx_rollout_reset(ctypes.byref(self._state), ctypes.c_void_p(red.data_ptr()),
                                         ctypes.c_void_p(blue.data_ptr()), 1 if force_all else 0, self._stream())
        _lib.check(int(rc), "atx_rollout_reset")

    def _out(self, out: torch.Tensor | None, shape: tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
        if out is None:
            return torch.empty(shape, dtype=dtype, device=self._dev)
        if tuple(out.shape) != shape or out.dtype != dtype or out.device != self._dev or not out.is_contiguous():
            raise RuntimeError(f"out must be a contiguous {dtype} tensor of shape {shape} on {self._dev}")
        if out.data_ptr() % 16:
            raise RuntimeError("out must be 16-byte aligned")
        return out
