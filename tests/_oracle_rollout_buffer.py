"""The reference buffer's API (csrc/stratego_buffer.cpp:375-411) over the
CPU oracle (``oracle.rollout.State``), so the scenarios of the reference's
own tests run against the oracle with the same calls as against the GPU
buffer.  Tensors are CPU torch tensors of the reference's dtypes."""

from __future__ import annotations

import numpy as np
import torch

from oracle.rollout import BUFFER_NAMES, State

_BOOL = {"terminated", "flag_captured", "moved", "revealed", "two_sq_violation", "chasing_violation"}


class OracleRolloutBuffer:
    def __init__(self, n_games: int = 1, device_id: int = 0, seed: int = 0) -> None:
        self.state = State(n_games, seed=seed)
        self.n_games, self.device_id = n_games, device_id

    def _get(self, name: str) -> torch.Tensor:
        a = getattr(self.state, name)
        t = torch.from_numpy(a.astype(bool) if name in _BOOL else a.copy())
        if name in ("owner", "piece"):
            t = t.view(self.n_games, 10, 10)
        return t

    def apply_actions(self, actions: torch.Tensor) -> None:
        if actions.dim() != 1:
            raise RuntimeError("actions must be 1D (N,)")
        if actions.size(0) != self.n_games:
            raise RuntimeError(f"actions size mismatch: expected {self.n_games}, got {actions.size(0)}")
        if actions.dtype != torch.int64:
            raise RuntimeError("actions must be int64")
        self.state.apply(actions.cpu().numpy())

    def compute_legal_action_mask(self) -> torch.Tensor:
        return torch.from_numpy(self.state.legal_mask())

    def compute_reward_pl0(self) -> torch.Tensor:
        o = self.state.outcome
        return torch.from_numpy(np.where(o == 0, 1.0, np.where(o == 1, -1.0, 0.0)).astype(np.float32))

    def compute_infostate_tensor(self) -> torch.Tensor:
        return torch.from_numpy(self.state.infostate())

    def compute_two_square_rule_applies(self) -> torch.Tensor:
        return self._get("two_sq_violation")

    def is_chasing_violation(self) -> torch.Tensor:
        return self._get("chasing_violation")

    def hash_board(self) -> torch.Tensor:
        return torch.from_numpy(self.state.hash_board())

    def get_terminated(self):
        return self._get("terminated")

    def get_outcomes(self):
        return self._get("outcome")

    def get_board_owner(self):
        return self._get("owner")

    def get_board_piece(self):
        return self._get("piece")

    def get_current_player(self):
        return self._get("player")

    def get_move_number(self):
        return self._get("move_number")

    def get_num_moves(self):
        return self._get("move_number")

    def get_num_moves_since_last_attack(self):
        return self._get("since_attack")

    def get_flag_captured(self):
        return self._get("flag_captured")

    def get_has_legal_movement(self):
        return self.compute_legal_action_mask().view(self.n_games, -1).any(-1)

    def get_terminated_since(self):
        return self._get("terminated_since")

    def board_strs(self) -> list[str]:
        out = []
        for g in range(self.n_games):
            s = ""
            for r in range(10):
                for c in range(10):
                    o, p = int(self.state.owner[g, r * 10 + c]), int(self.state.piece[g, r * 10 + c])
                    s += ". " if o < 0 else ("R" if o == 0 else "B") + str(p) + (" " if p < 10 else "")
                s += "\n"
            out.append(s)
        return out

    def reset_terminated(self, setup_red: torch.Tensor, setup_blue: torch.Tensor) -> None:
        self.state.reset(setup_red.numpy(), setup_blue.numpy())

    def reset_all(self, setup_red: torch.Tensor, setup_blue: torch.Tensor) -> None:
        self.state.reset(setup_red.numpy(), setup_blue.numpy(), force_all=True)

    def current_step(self) -> int:
        return int(self.state.move_number.sum())

    def raw_state(self) -> dict[str, np.ndarray]:
        return {BUFFER_NAMES[k]: getattr(self.state, k) for k in BUFFER_NAMES}
