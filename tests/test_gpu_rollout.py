"""Parity of the HIP Stratego simulator (``StrategoRolloutBuffer`` over the
``atx_rollout_*`` entry points) with the CPU oracle (``oracle/rollout.c``).

Integer and byte work, so the bar is bit-exact: every state array after
every step, and the legal-move masks, infostates (float32, compared
bitwise) and hashes.  Cases:

* the reference's own simulator tests (tests/_rollout_scenarios.py);
* random play from random full setups: legal moves mostly, illegal and
  out-of-range actions mixed in, finished games restarted, and the trackers
  moved to their edges (full chase rings, counters one step from the draw
  limits) by writing oracle states into the buffer;
* the config-2 batch (4096 games) for the mask and infostate kernels, and
  game counts that do not fill the last workgroup;
* preallocated outputs full of garbage (every byte must be written), the
  argument checks, the build check kernel.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from ataraxos_amd import StrategoRolloutBuffer
from oracle.rollout import BUFFER_NAMES, State, random_setups
from tests._rollout_play import perturb_trackers, random_actions
from tests._rollout_scenarios import SCENARIOS, act, acts, setup

pytestmark = pytest.mark.gpu


def _announce(msg: str) -> None:
    print(f"\n[case] {msg}", flush=True)
    sys.stdout.flush()


def load_into(buf: StrategoRolloutBuffer, st: State) -> None:
    """Write an oracle state (and its Zobrist table) into the GPU buffer."""
    raw = buf.raw_state()
    for name, bname in BUFFER_NAMES.items():
        t = raw[bname]
        t.copy_(torch.from_numpy(getattr(st, name)).reshape(t.shape).to(t.dtype))
    raw["zobrist_table"].copy_(torch.from_numpy(st.zobrist))


def assert_same_state(buf: StrategoRolloutBuffer, st: State, what: str) -> None:
    raw = buf.raw_state()
    for name, bname in BUFFER_NAMES.items():
        want = getattr(st, name)
        got = raw[bname].cpu().numpy().reshape(want.shape).astype(want.dtype)
        if not np.array_equal(got, want):
            bad = np.argwhere(got != want)[:5].tolist()
            raise AssertionError(f"{what}: {bname} differs at {bad}")


def assert_same_outputs(buf: StrategoRolloutBuffer, st: State, what: str) -> None:
    mask = buf.compute_legal_action_mask().cpu().numpy()
    assert np.array_equal(mask, st.legal_mask()), f"{what}: legal mask"
    info = buf.compute_infostate_tensor().cpu().numpy()
    assert np.array_equal(info.view(np.uint32), st.infostate().view(np.uint32)), f"{what}: infostate"
    assert np.array_equal(buf.hash_board().cpu().numpy(), st.hash_board()), f"{what}: hash"
    assert np.array_equal(buf.get_has_legal_movement().cpu().numpy(), st.any_move()), f"{what}: any move"


@pytest.mark.parametrize("name", sorted(SCENARIOS))
def test_reference_scenario(cuda, name):
    _announce(f"rollout scenario {name}")
    SCENARIOS[name](lambda n: StrategoRolloutBuffer(n, 0))
    torch.cuda.synchronize()


@pytest.mark.parametrize("n,seed,perturb", [(300, 1, False), (97, 2, True), (5, 3, True)])
def test_random_play_matches_oracle(cuda, n, seed, perturb):
    """Bit-exact state after every step of random play."""
    _announce(f"rollout random play n={n} seed={seed} perturb={perturb}")
    rng = np.random.default_rng(seed)
    st = State(n, seed=seed)
    buf = StrategoRolloutBuffer(n, 0)
    load_into(buf, st)
    red, blue = random_setups(n, rng)
    st.reset(red, blue, force_all=True)
    buf.reset_all(torch.from_numpy(red), torch.from_numpy(blue))
    assert_same_state(buf, st, "after reset_all")
    for step in range(160):
        if perturb and step % 10 == 3:
            perturb_trackers(st, rng)
            load_into(buf, st)
        a = random_actions(st.legal_mask(), rng)
        st.apply(a)
        buf.apply_actions(torch.from_numpy(a))
        assert_same_state(buf, st, f"step {step}")
        if step % 16 == 15:
            assert_same_outputs(buf, st, f"step {step}")
            red, blue = random_setups(n, rng)
            st.reset(red, blue)
            buf.reset_terminated(torch.from_numpy(red), torch.from_numpy(blue))
            assert_same_state(buf, st, f"reset at step {step}")
    torch.cuda.synchronize()


def test_config2_batch_mask_and_infostate(cuda):
    """4096 games (the self-play batch of config 2) in played positions."""
    _announce("rollout 4096 games")
    n = 4096
    rng = np.random.default_rng(7)
    st = State(n, seed=7)
    st.reset(*random_setups(n, rng), force_all=True)
    for _ in range(30):
        st.apply(random_actions(st.legal_mask(), rng, p_illegal=0.0))
    buf = StrategoRolloutBuffer(n, 0)
    load_into(buf, st)
    assert_same_outputs(buf, st, "4096 games")
    a = random_actions(st.legal_mask(), rng)
    st.apply(a)
    buf.apply_actions(torch.from_numpy(a))
    assert_same_state(buf, st, "4096 games, one step")


def test_every_output_byte_is_written(cuda):
    _announce("rollout outputs over garbage")
    n = 33
    rng = np.random.default_rng(8)
    st = State(n, seed=8)
    st.reset(*random_setups(n, rng), force_all=True)
    buf = StrategoRolloutBuffer(n, 0)
    load_into(buf, st)
    mask = torch.full((n, 100, 100), 0xFF, dtype=torch.uint8, device=cuda).view(torch.bool)
    info = torch.full((n, 488, 10, 10), float("nan"), dtype=torch.float32, device=cuda)
    assert buf.compute_legal_action_mask(out=mask) is mask
    assert buf.compute_infostate_tensor(out=info) is info
    assert np.array_equal(mask.view(torch.uint8).cpu().numpy(), st.legal_mask().astype(np.uint8))
    assert np.array_equal(info.cpu().numpy().view(np.uint32), st.infostate().view(np.uint32))


def test_terminated_games_and_wild_actions_are_untouched(cuda):
    """A finished game ignores its action; out-of-range actions are no-ops."""
    _announce("rollout no-op actions")
    buf = StrategoRolloutBuffer(4, 0)
    buf.reset_all(*setup([(3, 5, 1), (3, 0, 4)], [(4, 5, 11), (8, 8, 4)], n=4))
    buf.apply_actions(acts(act(3, 5, 4, 5), -1, 10000, act(3, 0, 3, 0)))  # game 0 captures the flag
    before = {k: v.clone() for k, v in buf.raw_state().items()}
    buf.apply_actions(acts(act(8, 8, 8, 9), -7, 123456, act(3, 0, 5, 0)))
    after = buf.raw_state()
    for k in before:
        if k == "terminated_since":
            assert after[k].tolist() == [2, 0, 0, 0]
        else:
            assert torch.equal(before[k], after[k]), k


def test_argument_checks_and_hello(cuda):
    buf = StrategoRolloutBuffer(3, 0)
    with pytest.raises(RuntimeError, match="1D"):
        buf.apply_actions(torch.zeros(3, 1, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="size mismatch"):
        buf.apply_actions(torch.zeros(2, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="int64"):
        buf.apply_actions(torch.zeros(3, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="int8"):
        buf.reset_all(torch.zeros(3, 10, 10), torch.zeros(3, 10, 10, dtype=torch.int8))
    with pytest.raises(RuntimeError, match="N mismatch"):
        buf.reset_all(torch.zeros(2, 10, 10, dtype=torch.int8), torch.zeros(3, 10, 10, dtype=torch.int8))
    with pytest.raises(RuntimeError, match="out must be"):
        buf.compute_legal_action_mask(out=torch.empty(3, 100, 99, dtype=torch.bool, device=cuda))
    hw = buf.hello_world()
    assert hw.dtype == torch.int32 and hw.tolist() == [42]
    empty = StrategoRolloutBuffer(0, 0)
    empty.apply_actions(torch.zeros(0, dtype=torch.int64))
    assert tuple(empty.compute_infostate_tensor().shape) == (0, 488, 10, 10)
    assert empty.current_step() == 0
