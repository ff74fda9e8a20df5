"""The known-answer cases of the reference's simulator tests, restated once
and run against any object with the reference buffer's API: the CPU oracle
(tests/test_rollout_oracle.py) and the HIP buffer (tests/test_gpu_rollout.py).

Each scenario cites the reference test it restates; positions, moves and
expected values are those of the reference's tests (tests/test_cuda_sim.py,
test_cuda_rules.py, test_cuda_infostate.py, test_cuda_api.py).  ``make(n)``
returns a fresh buffer of n games.
"""

from __future__ import annotations

import pytest
import torch

SPY, SCOUT, MINER, SERGEANT, MARSHAL, FLAG, BOMB = 1, 2, 3, 4, 10, 11, 12
RED, BLUE, EMPTY = 0, 1, -1
ONGOING, RED_WIN, BLUE_WIN, DRAW = -1, 0, 1, 2
UNIFORM = 1.0 / 12.0


def act(sr: int, sc: int, dr: int, dc: int) -> int:
    return (sr * 10 + sc) * 100 + dr * 10 + dc


def setup(red_pieces, blue_pieces, n: int = 1):
    red = torch.zeros((n, 10, 10), dtype=torch.int8)
    blue = torch.zeros((n, 10, 10), dtype=torch.int8)
    for r, c, p in red_pieces:
        red[:, r, c] = p
    for r, c, p in blue_pieces:
        blue[:, r, c] = p
    return red, blue


def acts(*a) -> torch.Tensor:
    return torch.tensor(list(a), dtype=torch.int64)


# test_cuda_rules.py:83-95
SHUTTLE_CYCLE = [act(8, 8, 8, 9), act(8, 9, 9, 9), act(9, 9, 9, 8), act(9, 8, 8, 8)]
SHUTTLE_OSC = [act(8, 8, 8, 9), act(8, 9, 8, 8)]


def alternate(buf, red_moves, blue_moves, n=1):
    """test_cuda_rules.py:98-104"""
    for i in range(max(len(red_moves), len(blue_moves))):
        if i < len(red_moves):
            buf.apply_actions(acts(*([red_moves[i]] * n)))
        if i < len(blue_moves):
            buf.apply_actions(acts(*([blue_moves[i]] * n)))


def b(x) -> bool:
    return bool(x.item()) if hasattr(x, "item") else bool(x)


# ---------------------------------------------------------------- sim tests
def sim_construction(make):
    """test_cuda_sim.py:108-112"""
    buf = make(4)
    assert buf.n_games == 4 and buf.device_id == 0


def sim_simple_move(make):
    """test_cuda_sim.py:114-130"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SPY)], []))
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    owner, piece = buf.get_board_owner(), buf.get_board_piece()
    assert owner[0, 4, 0].item() == RED and piece[0, 4, 0].item() == SPY
    assert owner[0, 3, 0].item() == EMPTY and piece[0, 3, 0].item() == 0


def sim_mask_shape_empty(make):
    """test_cuda_sim.py:132-139"""
    mask = make(4).compute_legal_action_mask()
    assert tuple(mask.shape) == (4, 100, 100) and mask.dtype == torch.bool
    assert not mask.any().item()


def sim_mask_with_pieces(make):
    """test_cuda_sim.py:141-153"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SPY)], []))
    mask = buf.compute_legal_action_mask()
    assert mask[0, 30, 20].item() is True and mask[0, 30, 40].item() is True and mask[0, 30, 31].item() is True
    assert mask[0, 30, 39].item() is False


def sim_spy_defeats_marshal(make):
    """test_cuda_sim.py:155-169"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SPY)], [(4, 0, MARSHAL)]))
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    owner, piece = buf.get_board_owner(), buf.get_board_piece()
    assert owner[0, 4, 0].item() == RED and piece[0, 4, 0].item() == SPY and owner[0, 3, 0].item() == EMPTY


def sim_miner_defeats_bomb(make):
    """test_cuda_sim.py:171-185"""
    buf = make(1)
    buf.reset_all(*setup([(3, 1, MINER)], [(4, 1, BOMB)]))
    buf.apply_actions(acts(act(3, 1, 4, 1)))
    owner, piece = buf.get_board_owner(), buf.get_board_piece()
    assert owner[0, 4, 1].item() == RED and piece[0, 4, 1].item() == MINER and owner[0, 3, 1].item() == EMPTY


def sim_equal_rank_both_die(make):
    """test_cuda_sim.py:187-202"""
    buf = make(1)
    buf.reset_all(*setup([(3, 4, SERGEANT)], [(4, 4, SERGEANT)]))
    buf.apply_actions(acts(act(3, 4, 4, 4)))
    owner, piece = buf.get_board_owner(), buf.get_board_piece()
    assert owner[0, 3, 4].item() == EMPTY and piece[0, 3, 4].item() == 0
    assert owner[0, 4, 4].item() == EMPTY and piece[0, 4, 4].item() == 0


def sim_flag_capture_wins(make):
    """test_cuda_sim.py:204-216"""
    buf = make(1)
    buf.reset_all(*setup([(3, 5, SPY)], [(4, 5, FLAG)]))
    buf.apply_actions(acts(act(3, 5, 4, 5)))
    assert buf.get_outcomes()[0].item() == RED_WIN and buf.get_terminated()[0].item() is True


def sim_initial_outcomes_terminated(make):
    """test_cuda_sim.py:218-232"""
    buf = make(4)
    outcome, term = buf.get_outcomes(), buf.get_terminated()
    assert tuple(outcome.shape) == (4,) and outcome.dtype == torch.int8 and (outcome == ONGOING).all().item()
    assert tuple(term.shape) == (4,) and term.dtype == torch.bool and not term.any().item()


def sim_current_step(make):
    """test_cuda_sim.py:234-251"""
    buf = make(2)
    buf.reset_all(*setup([(3, 0, SPY), (3, 1, SPY)], [(6, 0, FLAG), (6, 1, FLAG)], n=2))
    assert buf.current_step() == 0
    buf.apply_actions(acts(act(3, 0, 4, 0), act(3, 1, 4, 1)))
    assert buf.current_step() == 2


# -------------------------------------------------------------- rule tests
def rules_initial_no_violation(make):
    """test_cuda_rules.py:114-119, 224-229, 377-389"""
    buf = make(4)
    ts, ch, hb = buf.compute_two_square_rule_applies(), buf.is_chasing_violation(), buf.hash_board()
    assert tuple(ts.shape) == (4,) and tuple(ch.shape) == (4,) and tuple(hb.shape) == (4,)
    assert ts.dtype == torch.bool and ch.dtype == torch.bool and hb.dtype == torch.int64
    assert not ts.any().item() and not ch.any().item()


def _sergeant(make, n=1):
    buf = make(n)
    red, blue = setup([(3, 0, SERGEANT)], [(8, 8, SERGEANT)], n=n)
    buf.reset_all(red, blue)
    return buf, red, blue


def rules_single_move(make):
    """test_cuda_rules.py:121-126"""
    buf, _, _ = _sergeant(make)
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    assert not b(buf.compute_two_square_rule_applies()[0])


SHUTTLE_RED = [act(3, 0, 4, 0), act(4, 0, 3, 0), act(3, 0, 4, 0), act(4, 0, 3, 0), act(3, 0, 3, 1)]


def rules_three_crossings(make):
    """test_cuda_rules.py:128-139"""
    buf, _, _ = _sergeant(make)
    alternate(buf, SHUTTLE_RED[:3], SHUTTLE_CYCLE[:3])
    assert not b(buf.compute_two_square_rule_applies()[0])


def rules_four_crossings(make):
    """test_cuda_rules.py:141-153"""
    buf, _, _ = _sergeant(make)
    alternate(buf, SHUTTLE_RED[:4], SHUTTLE_CYCLE[:4])
    assert b(buf.compute_two_square_rule_applies()[0])


def rules_different_pair(make):
    """test_cuda_rules.py:155-166"""
    buf, _, _ = _sergeant(make)
    alternate(buf, [act(3, 0, 4, 0), act(4, 0, 4, 1), act(4, 1, 3, 1)], SHUTTLE_CYCLE[:3])
    assert not b(buf.compute_two_square_rule_applies()[0])


def rules_attack_resets_count(make):
    """test_cuda_rules.py:168-183"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, MARSHAL)], [(5, 0, SERGEANT), (8, 8, SERGEANT)]))
    alternate(buf, [act(3, 0, 4, 0), act(4, 0, 3, 0), act(3, 0, 4, 0), act(4, 0, 5, 0)], SHUTTLE_CYCLE[:4])
    assert not b(buf.compute_two_square_rule_applies()[0])


def rules_violation_sticky(make):
    """test_cuda_rules.py:185-198"""
    buf, _, _ = _sergeant(make)
    alternate(buf, SHUTTLE_RED[:5], SHUTTLE_CYCLE[:5])
    assert b(buf.compute_two_square_rule_applies()[0])


def rules_reset_clears_two_square(make):
    """test_cuda_rules.py:200-218"""
    buf, red, blue = _sergeant(make)
    alternate(buf, SHUTTLE_RED[:4], SHUTTLE_CYCLE[:4])
    assert b(buf.compute_two_square_rule_applies()[0])
    buf.reset_all(red, blue)
    assert not b(buf.compute_two_square_rule_applies()[0])


def rules_hash_consistent(make):
    """test_cuda_rules.py:231-243"""
    buf = make(2)
    buf.reset_all(*setup([(3, 0, SERGEANT)], [(6, 0, SERGEANT)], n=2))
    h1, h2 = buf.hash_board(), buf.hash_board()
    assert tuple(h1.shape) == (2,) and h1.dtype == torch.int64 and torch.equal(h1, h2)


def rules_hash_changes(make):
    """test_cuda_rules.py:245-252"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SERGEANT)], [(6, 0, SERGEANT)]))
    before = buf.hash_board()
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    assert before[0].item() != buf.hash_board()[0].item()


def rules_non_threatening(make):
    """test_cuda_rules.py:254-259"""
    buf, _, _ = _sergeant(make)
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    assert not b(buf.is_chasing_violation()[0])


def rules_single_threatening(make):
    """test_cuda_rules.py:261-269"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SERGEANT)], [(5, 0, SERGEANT), (8, 8, SERGEANT)]))
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    assert not b(buf.is_chasing_violation()[0])


CHASE_BLUE = [(5, 0, SERGEANT), (5, 1, SERGEANT), (2, 1, SERGEANT), (2, 0, SERGEANT), (8, 8, SERGEANT)]
CHASE_CYCLE = [act(3, 0, 4, 0), act(4, 0, 4, 1), act(4, 1, 3, 1), act(3, 1, 3, 0), act(3, 0, 4, 0)]


def rules_chasing_4cycle(make):
    """test_cuda_rules.py:271-307"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SERGEANT)], CHASE_BLUE))
    alternate(buf, CHASE_CYCLE, SHUTTLE_CYCLE[:4])
    assert b(buf.is_chasing_violation()[0])


def rules_chasing_exception(make):
    """test_cuda_rules.py:309-340"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SERGEANT)], [(5, 0, SERGEANT), (2, 0, SERGEANT), (8, 8, SERGEANT)]))
    alternate(buf, [act(3, 0, 4, 0), act(4, 0, 3, 0), act(3, 0, 4, 0)], SHUTTLE_OSC[:2])
    assert not b(buf.is_chasing_violation()[0])


def rules_reset_clears_chasing(make):
    """test_cuda_rules.py:342-373"""
    buf = make(1)
    red, blue = setup([(3, 0, SERGEANT)], CHASE_BLUE)
    buf.reset_all(red, blue)
    alternate(buf, CHASE_CYCLE, SHUTTLE_CYCLE[:4])
    assert b(buf.is_chasing_violation()[0])
    buf.reset_all(red, blue)
    assert not b(buf.is_chasing_violation()[0])


def rules_two_square_in_one_game(make):
    """test_cuda_rules.py:391-424"""
    buf, _, _ = _sergeant(make, n=2)
    red = [acts(act(3, 0, 4, 0), act(3, 0, 4, 0)), acts(act(4, 0, 3, 0), act(4, 0, 4, 1)),
           acts(act(3, 0, 4, 0), act(4, 1, 3, 1)), acts(act(4, 0, 3, 0), act(3, 1, 3, 0))]
    for i in range(4):
        buf.apply_actions(red[i])
        buf.apply_actions(acts(SHUTTLE_CYCLE[i], SHUTTLE_CYCLE[i]))
    v = buf.compute_two_square_rule_applies()
    assert b(v[0]) and not b(v[1])


# --------------------------------------------------------- infostate tests
def _spy_flag(make, n=1):
    buf = make(n)
    red, blue = setup([(3, 0, SPY)], [(6, 0, FLAG)], n=n)
    buf.reset_all(red, blue)
    return buf, red, blue


def info_shape(make):
    """test_cuda_infostate.py:98-107"""
    buf, _, _ = _spy_flag(make, 3)
    info = buf.compute_infostate_tensor()
    assert tuple(info.shape) == (3, 488, 10, 10) and info.dtype == torch.float32


def info_initial_channels(make):
    """test_cuda_infostate.py:109-141"""
    buf, _, _ = _spy_flag(make)
    info = buf.compute_infostate_tensor()
    assert info[0, 0, 3, 0].item() == pytest.approx(1.0)
    assert info[0, 10].sum().item() == pytest.approx(0.0)
    for ch in range(12, 24):
        assert info[0, ch, 6, 0].item() == pytest.approx(UNIFORM)
    assert info[0, 12:24, 6, 0].sum().item() == pytest.approx(1.0)
    assert info[0, 36, 3, 0].item() == pytest.approx(1.0)
    assert info[0, 37, 6, 0].item() == pytest.approx(1.0)
    assert info[0, 38, 0, 0].item() == pytest.approx(1.0) and info[0, 38, 3, 0].item() == pytest.approx(0.0)
    assert info[0, 43:456].abs().sum().item() == 0.0 and info[0, 456:488].abs().sum().item() == 0.0


def info_after_simple_move(make):
    """test_cuda_infostate.py:143-167"""
    buf, _, _ = _spy_flag(make)
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    info = buf.compute_infostate_tensor()
    assert info[0, 456, 4, 0].item() == 1.0 and info[0, 456, 3, 0].item() == -1.0
    assert info[0, 40, 4, 0].item() == 1.0 and info[0, 40, 3, 0].item() == 0.0
    assert info[0, 37, 4, 0].item() == 1.0
    assert info[0, 457:488].abs().sum().item() == 0.0


def info_after_attack(make):
    """test_cuda_infostate.py:169-196"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SPY)], [(4, 0, MARSHAL), (6, 9, SCOUT)]))
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    info = buf.compute_infostate_tensor()
    assert info[0, 37, 4, 0].item() == 0.0 and info[0, 12, 4, 0].item() == 1.0
    for ch in range(13, 24):
        assert info[0, ch, 4, 0].item() == 0.0
    assert info[0, 456, 4, 0].item() == 1.0 and info[0, 456, 3, 0].item() == -1.0


def info_scalar_channels(make):
    """test_cuda_infostate.py:198-218"""
    buf, _, _ = _spy_flag(make)
    info0 = buf.compute_infostate_tensor()
    assert info0[0, 41].sum().item() == 0.0 and info0[0, 42].sum().item() == 0.0
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    info1 = buf.compute_infostate_tensor()
    assert (info1[0, 41] == torch.tensor(1.0 / 4000.0, dtype=torch.float32)).all().item()
    assert (info1[0, 42] == torch.tensor(1.0 / 100.0, dtype=torch.float32)).all().item()


def info_history_two_moves(make):
    """test_cuda_infostate.py:220-245"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SCOUT)], [(6, 0, SCOUT)]))
    buf.apply_actions(acts(act(3, 0, 2, 0)))
    buf.apply_actions(acts(act(6, 0, 7, 0)))
    info = buf.compute_infostate_tensor()
    assert info[0, 456, 7, 0].item() == 1.0 and info[0, 456, 6, 0].item() == -1.0
    assert info[0, 457, 2, 0].item() == 1.0 and info[0, 457, 3, 0].item() == -1.0
    assert info[0, 458:488].abs().sum().item() == 0.0


def info_history_ring_overflow(make):
    """test_cuda_infostate.py:247-283"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SCOUT)], [(6, 0, SCOUT)]))
    for i in range(33):
        if i % 2 == 0:
            r, d = (3, 2) if i % 4 == 0 else (2, 3)
        else:
            r, d = (6, 7) if i % 4 == 1 else (7, 6)
        buf.apply_actions(acts(act(r, 0, d, 0)))
    info = buf.compute_infostate_tensor()
    assert (info[0, 456:488] != 0).any(dim=2).any(dim=1).sum().item() == 32
    assert info[0, 456, 2, 0].item() == 1.0 and info[0, 456, 3, 0].item() == -1.0
    assert info[0, 487, 7, 0].item() == 1.0 and info[0, 487, 6, 0].item() == -1.0


def info_reset_clears(make):
    """test_cuda_infostate.py:285-304"""
    buf, red, blue = _spy_flag(make)
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    assert buf.compute_infostate_tensor()[0, 456].abs().sum().item() > 0
    buf.reset_all(red, blue)
    info = buf.compute_infostate_tensor()
    assert info[0, 456:488].abs().sum().item() == 0.0
    assert info[0, 39].sum().item() == 0.0 and info[0, 40].sum().item() == 0.0 and info[0, 41].sum().item() == 0.0


# --------------------------------------------------------------- API tests
def api_initial_getters(make):
    """test_cuda_api.py:80-98, 133-138"""
    buf = make(3)
    for t, dt in ((buf.get_num_moves(), torch.int32), (buf.get_num_moves_since_last_attack(), torch.int32),
                  (buf.get_terminated_since(), torch.int32)):
        assert tuple(t.shape) == (3,) and t.dtype == dt and (t == 0).all().item()
    fc = buf.get_flag_captured()
    assert tuple(fc.shape) == (3,) and fc.dtype == torch.bool and not fc.any().item()


def api_flag_captured(make):
    """test_cuda_api.py:101-117, 140-147"""
    buf = make(1)
    buf.reset_all(*setup([(3, 5, SPY)], [(4, 5, FLAG)]))
    buf.apply_actions(acts(act(3, 5, 4, 5)))
    assert buf.get_flag_captured()[0].item() is True
    assert buf.get_terminated_since()[0].item() >= 1
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SPY)], []))
    buf.apply_actions(acts(act(3, 0, 4, 0)))
    assert not buf.get_flag_captured()[0].item()


def api_has_legal_movement(make):
    """test_cuda_api.py:119-131"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SPY)], []))
    hlm = buf.get_has_legal_movement()
    assert tuple(hlm.shape) == (1,) and hlm.dtype == torch.bool and hlm[0].item() is True
    assert not make(1).get_has_legal_movement()[0].item()


def api_board_strs(make):
    """test_cuda_api.py:149-162"""
    buf = make(1)
    buf.reset_all(*setup([(3, 0, SPY)], []))
    strs = buf.board_strs()
    assert len(strs) == 1 and isinstance(strs[0], str) and "R1" in strs[0]
    strs = make(2).board_strs()
    assert len(strs) == 2 and all(isinstance(s, str) for s in strs)


SCENARIOS = {f.__name__: f for f in (
    sim_construction, sim_simple_move, sim_mask_shape_empty, sim_mask_with_pieces, sim_spy_defeats_marshal,
    sim_miner_defeats_bomb, sim_equal_rank_both_die, sim_flag_capture_wins, sim_initial_outcomes_terminated,
    sim_current_step, rules_initial_no_violation, rules_single_move, rules_three_crossings, rules_four_crossings,
    rules_different_pair, rules_attack_resets_count, rules_violation_sticky, rules_reset_clears_two_square,
    rules_hash_consistent, rules_hash_changes, rules_non_threatening, rules_single_threatening,
    rules_chasing_4cycle, rules_chasing_exception, rules_reset_clears_chasing, rules_two_square_in_one_game,
    info_shape, info_initial_channels, info_after_simple_move, info_after_attack, info_scalar_channels,
    info_history_two_moves, info_history_ring_overflow, info_reset_clears, api_initial_getters, api_flag_captured,
    api_has_legal_movement, api_board_strs,
)}
