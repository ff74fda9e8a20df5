"""Pins of the CPU restatement of the reference's Stratego simulator
(``oracle/rollout.c``), no GPU needed.

* The known-answer cases of the reference's own simulator tests
  (tests/_rollout_scenarios.py) run against the oracle.
* Two code paths of the oracle that must agree, on states from random play:
  the legal-move mask and the validation inside ``apply`` (every one of the
  10,000 actions of a game is applied to its own copy: the move number
  advances exactly where the mask is set); the mask's "any legal move" and
  the no-move loss check.
* Zobrist hash: XOR-linear over squares (a board's hash is the XOR of its
  one-piece boards' hashes), and the chase ring stores exactly the hash of
  the board after a threatening move.
* Infostate structure on random states, square by square, derived from the
  board rather than from the oracle's formula.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.rollout import State, random_setups
from tests._oracle_rollout_buffer import OracleRolloutBuffer
from tests._rollout_play import perturb_trackers, random_actions
from tests._rollout_scenarios import SCENARIOS


@pytest.mark.parametrize("name", sorted(SCENARIOS))
def test_reference_scenario(name):
    SCENARIOS[name](lambda n: OracleRolloutBuffer(n))


def played_states(n=24, steps=120, seed=0, perturb=False):
    """Snapshots of ``n`` games under random play (legal moves mostly, some
    illegal or out-of-range actions), restarting finished games."""
    rng = np.random.default_rng(seed)
    st = State(n, seed=seed)
    st.reset(*random_setups(n, rng), force_all=True)
    snaps = []
    for step in range(steps):
        if perturb and step % 10 == 5:
            perturb_trackers(st, rng)
        st.apply(random_actions(st.legal_mask(), rng))
        if step % 15 == 14:
            st.reset(*random_setups(n, rng))
        if step % 20 == 19:
            snaps.append(st.copy())
    return snaps


def single_game(st: State, g: int, copies: int) -> State:
    one = State(copies, zobrist=st.zobrist)
    for name in ("owner", "piece", "player", "move_number", "since_attack", "outcome", "terminated", "moved",
                 "revealed", "history", "history_head", "history_len", "two_sq_count", "two_sq_lo", "two_sq_hi",
                 "chase_hashes", "chase_head", "chase_len", "chase_last_src"):
        getattr(one, name)[:] = getattr(st, name)[g]
    return one


def test_mask_agrees_with_apply_validation():
    """mask[src, dst] == (apply accepts src*100 + dst), all 10,000 actions."""
    checked = 0
    for st in played_states(n=8, steps=100, seed=1):
        mask = st.legal_mask()
        for g in range(st.n):
            if st.terminated[g]:
                continue
            many = single_game(st, g, 10000)
            many.apply(np.arange(10000, dtype=np.int64))
            accepted = many.move_number != st.move_number[g]
            assert np.array_equal(accepted, mask[g].reshape(-1)), f"game {g}"
            checked += 1
    assert checked >= 10


def test_any_move_matches_mask():
    for st in played_states(seed=2):
        assert np.array_equal(st.any_move(), st.legal_mask().reshape(st.n, -1).any(axis=1))


def test_no_move_loss_and_draw_limits():
    """After every accepted move that ends a game without a flag capture, the
    side to move has no legal move or a draw limit was reached."""
    rng = np.random.default_rng(3)
    st = State(32, seed=3)
    st.reset(*random_setups(32, rng), force_all=True)
    ended = 0
    for _ in range(400):
        before = st.copy()
        st.apply(random_actions(st.legal_mask(), rng, p_illegal=0.0))
        newly = (st.terminated == 1) & (before.terminated == 0)
        for g in np.flatnonzero(newly):
            ended += 1
            if st.flag_captured[g]:
                assert st.outcome[g] == before.player[g]
            elif st.outcome[g] == 2:
                assert st.move_number[g] >= 4000 or st.since_attack[g] >= 100
            else:
                assert st.outcome[g] == before.player[g] and not st.any_move()[g]
        st.reset(*random_setups(32, rng))
    assert ended > 0


def test_hash_is_xor_of_one_piece_boards():
    for st in played_states(n=6, seed=4)[:2]:
        h = st.hash_board()
        for g in range(st.n):
            occupied = np.flatnonzero(st.owner[g] >= 0)
            parts = State(len(occupied), zobrist=st.zobrist)
            for i, s in enumerate(occupied):
                parts.owner[i, s], parts.piece[i, s] = st.owner[g, s], st.piece[g, s]
            acc = np.bitwise_xor.reduce(parts.hash_board()) if len(occupied) else np.int64(0)
            assert acc == h[g]
    assert State(3).hash_board().tolist() == [0, 0, 0]


def test_chase_ring_holds_the_board_hash():
    rng = np.random.default_rng(5)
    st = State(64, seed=5)
    st.reset(*random_setups(64, rng), force_all=True)
    seen = 0
    for _ in range(60):
        before = st.copy()
        st.apply(random_actions(st.legal_mask(), rng, p_illegal=0.0))
        h = st.hash_board()
        for g in range(64):
            me = before.player[g]
            if st.move_number[g] == before.move_number[g] or st.chase_last_src[g, me] < 0:
                continue
            k = st.chase_len[g, me] - 1 if st.chase_len[g, me] < 64 and before.chase_len[g, me] < 64 else (
                st.chase_head[g, me] - 1) % 64
            assert st.chase_hashes[g, me, k] == h[g]
            seen += 1
        st.reset(*random_setups(64, rng))
    assert seen > 50


def test_infostate_structure():
    for st in played_states(n=12, seed=6, perturb=True):
        x = st.infostate().reshape(st.n, 488, 100)
        for g in range(st.n):
            me = st.player[g]
            own = st.owner[g] == me
            opp = (st.owner[g] >= 0) & ~own
            rev = st.revealed[g] == 1
            assert np.array_equal(x[g, 0:12].sum(axis=0), own.astype(np.float32))
            np.testing.assert_allclose(x[g, 12:24].sum(axis=0), opp.astype(np.float32), rtol=1e-6)
            np.testing.assert_allclose(x[g, 24:36].sum(axis=0), own.astype(np.float32), rtol=1e-6)
            assert np.array_equal(x[g, 36] + x[g, 37], ((own | opp) & ~rev).astype(np.float32))
            assert np.array_equal(x[g, 38], (st.owner[g] < 0).astype(np.float32))
            assert np.all(x[g, 41] == np.float32(st.move_number[g]) / np.float32(4000))
            assert not x[g, 43:456].any()
            k = min(int(st.history_len[g]), 32)
            hist = x[g, 456:488]
            assert np.all((hist != 0).sum(axis=1)[:k] >= 1) and not hist[k:].any()
            # one +1 (at dst) and one -1 (at src) per recorded move; a slot
            # still holding the reset value 0 (src = dst = 0) shows only the +1
            head = int(st.history_head[g])
            moves = [int(st.history[g, (head - 1 - j) % 32]) for j in range(k)]
            assert hist.sum(axis=1)[:k].tolist() == [1.0 if a // 100 == a % 100 else 0.0 for a in moves]
