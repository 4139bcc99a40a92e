"""The replay oracle (oracle/replay.py) pinned on the CPU.

The n-step read and the successor against a flat history of the same writes
(the independent-history check of the reference's
tests/buffers/test_replay_oracle.py:72-144, restated), the sampleable bound
at the seam, the uniform draw against the reference's generator calls made
explicitly, and the prioritized draw's distribution and weights against
their closed forms."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.replay import ReplayOracle


def _drive(oracle, n_writes, rng, p_end=0.3, lanes=1):
    """Writes whose observation encodes the flat write index; returns the
    flat history per lane."""
    hist = [[] for _ in range(lanes)]
    for _ in range(n_writes):
        for lane in range(lanes):
            t = len(hist[lane])
            x = rng.random()
            done = x < 0.6 * p_end
            trunc = (not done) and x < p_end
            reward = float(np.float32(rng.normal()))
            final = np.array([10_000.0 + t], np.float32) if (done or trunc) else None
            oracle.add(lane, np.array([float(t)], np.float32), int(rng.integers(0, 5)), reward, done, trunc, final)
            hist[lane].append(dict(reward=reward, done=done, end=done or trunc))
    return hist


def _expected(hist, t, n_step, gamma):
    g, disc, steps, done = 0.0, 1.0, 0, False
    succ = t + 1
    for k in range(n_step):
        h = hist[t + k]
        g += disc * np.float64(np.float32(h["reward"]))
        disc *= gamma
        steps += 1
        succ = t + k + 1
        if h["end"]:
            done = h["done"]
            succ = 10_000 + t + k
            break
    return g, done, steps, succ


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_n_step_read_and_successor_match_the_flat_history(seed):
    rng = np.random.default_rng(seed)
    cap, n_step, gamma = 17, 3, 0.9
    o = ReplayOracle((1,), np.float32, capacity=cap, n_step=n_step, gamma=gamma, seed=seed)
    hist = _drive(o, 60, rng)[0]
    start, count = o.sampleable()
    assert count[0] == cap - n_step
    written = len(hist)
    checked = 0
    for p in range(int(count[0])):
        col = int((start[0] + p) % cap)
        t = written - cap + p  # flat index of the transition at run position p
        g, end_cols, term, steps = o.walk(np.array([0]), np.array([col]))
        want_g, want_done, want_steps, want_succ = _expected(hist, t, n_step, gamma)
        assert g[0] == want_g and bool(term[0]) == want_done and steps[0] == want_steps
        assert int(o.successor(0, int(end_cols[0]))[0]) == want_succ
        assert int(o.obs[0, col, 0]) == t
        checked += 1
    assert checked == cap - n_step


def test_filling_bound_and_seam():
    o = ReplayOracle((1,), np.float32, capacity=10, n_step=3, seed=0)
    rng = np.random.default_rng(0)
    _drive(o, 3, rng, p_end=0.0)
    assert o.sampleable()[1][0] == 0
    _drive(o, 2, rng, p_end=0.0)
    assert o.sampleable()[1][0] == 2  # columns 0 and 1: col + n_step <= pos - 1
    _drive(o, 20, rng, p_end=0.0)
    start, count = o.sampleable()
    assert count[0] == 7 and start[0] == o.pos[0]


def test_uniform_draw_makes_the_reference_generator_calls():
    rng = np.random.default_rng(5)
    o = ReplayOracle((1,), np.float32, capacity=24, n_envs=3, n_step=2, seed=9)
    _drive(o, 11, rng, lanes=3)
    batch = o.sample(16)
    start, count = o.sampleable()
    g = np.random.default_rng(9)
    quota = g.multinomial(16, count / count.sum())
    lanes, offs = [], []
    for lane, k in enumerate(quota):
        if k:
            offs.append(g.integers(0, int(count[lane]), size=int(k)))
            lanes.append(np.full(int(k), lane))
    lanes = np.concatenate(lanes)
    assert np.array_equal(batch["lanes"], lanes)
    assert np.array_equal(batch["cols"], (start[lanes] + np.concatenate(offs)) % o.cols)
    assert batch["weights"] is None


def test_priority_draw_is_proportional_and_weights_follow_the_closed_form():
    rng = np.random.default_rng(3)
    o = ReplayOracle((1,), np.float32, capacity=30, n_envs=2, n_step=1, seed=4, alpha=0.6)
    _drive(o, 15, rng, p_end=0.0, lanes=2)
    start, count = o.sampleable()
    cols = [(start[l] + np.arange(count[l])) % o.cols for l in range(2)]
    pr = rng.uniform(0.1, 3.0, (2, int(count[0])))
    for l in range(2):
        o.update_priorities(np.full(len(cols[l]), l), cols[l], pr[l])
    w = (pr + 1e-6) ** 0.6
    assert np.allclose(o.weight[0, cols[0]], w[0])
    assert o.max_priority == pytest.approx(pr.max())
    hits = np.zeros_like(w)
    for _ in range(400):
        b = o.sample(64, beta=0.5)
        for lane, col in zip(b["lanes"], b["cols"]):
            hits[lane, int(np.flatnonzero(cols[lane] == col)[0])] += 1
        p = o.weight[b["lanes"], b["cols"]] / w.sum()
        want = (w.size * p) ** -0.5
        assert np.allclose(b["weights"], (want / want.max()).astype(np.float32))
    freq = hits / hits.sum()
    expect = w / w.sum()
    # 25600 draws: every column's frequency within 5 sigma of its probability.
    sigma = np.sqrt(expect * (1 - expect) / hits.sum())
    assert np.all(np.abs(freq - expect) < 5 * sigma + 1e-12)
    # A fresh write takes the largest priority seen so far.
    o.add(0, np.array([0.0], np.float32), 1, 0.0, False)
    assert o.weight[0, (o.pos[0] - 1) % o.cols] == pytest.approx((pr.max() + 1e-6) ** 0.6)
