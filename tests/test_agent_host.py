"""Host-only tests of the agent plumbing: the update clock (the reference's
cases, tests/test_algos_clock.py:23-127), the autoreset tracker
(ttrl/algos/base.py:190-253) and the Transition checks
(ttrl/algos/base.py:40-96).  No device."""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from ttrl_amd.algos.base import AutoresetTracker, Transition, leaf_array
from ttrl_amd.algos.clock import UpdateClock


def test_credit_comes_from_frames_not_calls():
    c = UpdateClock(train_freq=1, warmup=0)
    c.advance(4)
    assert c.owed == 4 and c.due


def test_advancing_to_one_frame_twice_accrues_once():
    c = UpdateClock(1, 0)
    c.advance(4)
    c.advance(4)
    assert c.owed == 4


def test_asking_never_accrues():
    c = UpdateClock(2, 0)
    c.advance(10)
    before = c.state_dict()
    for _ in range(3):
        assert c.due and c.owed == 5
    assert c.state_dict() == before


def test_warm_up_frames_earn_nothing_and_skip_earns_nothing():
    c = UpdateClock(1, 100)
    c.advance(100)
    assert c.owed == 0 and not c.due
    c.advance(103)
    assert c.owed == 3
    d = UpdateClock(1, 0)
    d.skip(50)
    assert d.owed == 0
    d.advance(53)
    assert d.owed == 3


def test_consume_keeps_the_remainder():
    c = UpdateClock(3, 0)
    c.advance(4)
    assert c.owed == 1
    c.consume(1)
    assert c.owed == 0
    c.advance(6)
    assert c.owed == 1  # 4/3 - 1 + 2/3 = 1


@pytest.mark.parametrize("train_freq,step", [(3, 1), (4, 3), (7, 5), (10, 8), (3, 2)])
def test_owed_equals_exact_arithmetic(train_freq, step):
    """The owed count is floor(credited frames / train_freq) - steps taken,
    exactly (checked with Fractions over many rounds)."""
    c = UpdateClock(train_freq, 5)
    credit = Fraction(0)
    last = 0
    for frame in range(step, 400, step):
        c.advance(frame)
        credit += Fraction(max(0, frame - max(last, 5)), train_freq)
        last = frame
        assert c.owed == int(credit)
        if c.due:
            k = c.owed
            c.consume(k)
            credit -= k


@pytest.mark.parametrize("n", [2, 3, 8])
def test_clocks_advanced_to_one_frame_hold_identical_credit(n):
    clocks = [UpdateClock(4, 0) for _ in range(n)]
    taken = [0] * n
    for frame in range(3, 300, 3):
        for i, c in enumerate(clocks):
            c.advance(frame)
            if c.due:
                taken[i] += c.owed
                c.consume(c.owed)
    assert len(set(taken)) == 1 and taken[0] == 297 // 4


def test_clock_state_round_trips_in_the_reference_form():
    c = UpdateClock(3, 5)
    c.advance(17)
    s = c.state_dict()
    assert s == {"frame": 17, "credit": 4.0}
    r = UpdateClock(3, 5)
    r.load_state_dict(s)
    assert r.owed == c.owed
    c.advance(19)
    r.advance(19)
    assert r.owed == c.owed and r.state_dict() == c.state_dict()


@pytest.mark.parametrize("train_freq,warmup", [(0, 0), (-1, 0), (1, -1)])
def test_bad_clock_settings_are_refused(train_freq, warmup):
    with pytest.raises(ValueError):
        UpdateClock(train_freq, warmup)


def _tr(done_term, done_trunc, lanes=3):
    obs = np.zeros((lanes, 2), np.float32)
    return Transition(obs, np.zeros(lanes), np.zeros(lanes, np.float32), np.asarray(done_term, bool),
                      np.asarray(done_trunc, bool), obs.copy())


def test_autoreset_drops_the_step_after_an_end():
    t = AutoresetTracker(3)
    assert t.valid(_tr([0, 1, 0], [0, 0, 0])).tolist() == [True, True, True]
    assert t.valid(_tr([0, 0, 0], [1, 0, 0])).tolist() == [True, False, True]
    assert t.valid(_tr([0, 0, 0], [0, 0, 0])).tolist() == [False, True, True]
    assert t.valid(_tr([0, 0, 0], [0, 0, 0])).tolist() == [True, True, True]


def test_autoreset_refuses_an_end_on_the_padding_step_and_wrong_lanes():
    t = AutoresetTracker(3)
    t.valid(_tr([1, 0, 0], [0, 0, 0]))
    with pytest.raises(ValueError, match="autoreset step"):
        t.valid(_tr([1, 0, 0], [0, 0, 0]))
    with pytest.raises(ValueError, match="lanes"):
        AutoresetTracker(2).valid(_tr([0, 0, 0], [0, 0, 0]))


def test_autoreset_state_checks_shape_and_starts_fresh():
    t = AutoresetTracker(3)
    t.valid(_tr([1, 0, 1], [0, 0, 0]))
    s = t.state_dict()
    assert s["pending"].tolist() == [True, False, True]
    r = AutoresetTracker(3)
    r.load_state_dict(s)
    assert not r.pending.any()
    with pytest.raises(ValueError):
        AutoresetTracker(2).load_state_dict(s)


def test_transition_checks_lanes_and_successor_shape():
    obs = np.zeros((2, 4), np.float32)
    with pytest.raises(ValueError, match="lanes"):
        Transition(obs, np.zeros(3), np.zeros(2), np.zeros(2, bool), np.zeros(2, bool), obs)
    with pytest.raises(ValueError, match="next_obs"):
        Transition(obs, np.zeros(2), np.zeros(2), np.zeros(2, bool), np.zeros(2, bool), np.zeros((2, 5)))
    tr = Transition({"obs": obs}, np.zeros(2), np.zeros(2), np.array([True, False]), np.array([False, True]),
                    {"obs": obs})
    assert tr.n_envs == 2 and tr.done.tolist() == [True, True]
    assert leaf_array(tr.obs, "obs") is not None
