"""Host<->device crossings of one learner update (the reference's crossing
budget, tests/engine/test_crossing_budget.py:22-37 and :71-92: one packed
metrics download per update): after the capture, an update from a host
batch queues the copy of each input of at least 256 KiB as soon as it is
staged (ttrl_h2d_enqueue, no wait: DQN's obs and next_obs frames), then
makes one ttrl_graph_step, which copies the rest of the staged batch in,
replays the graph, makes one device-to-host copy of the packed metrics and
waits once.  The metrics it returns equal a per-tensor read of the same
device buffers."""

from __future__ import annotations

import numpy as np
import pytest

from tests._dqn_helpers import build_learner
from tests._sac_helpers import build_sac

pytestmark = pytest.mark.gpu


class _Spy:
    def __init__(self, device):
        self.device = device
        self.names = []
        self._orig = device.call

    def __enter__(self):
        orig = self._orig

        def call(name, *args):
            self.names.append(name)
            return orig(name, *args)

        self.device.call = call
        return self

    def __exit__(self, *exc):
        del self.device.call


def test_dqn_update_from_a_host_batch_is_one_step_call(device):
    from ttrl_amd.workloads import dqn_batch

    learner, _, _ = build_learner(device, seed=1)
    try:
        learner.update(dqn_batch(10))  # capture
        for k in range(3):
            with _Spy(device) as spy:
                m = learner.update(dqn_batch(11 + k))
            assert spy.names == ["ttrl_h2d_enqueue", "ttrl_h2d_enqueue", "ttrl_graph_step"], spy.names
            blk = learner._metric_block.numpy()
            assert m["loss"] == float(blk[0]) and m["mean_q"] == float(blk[1])
            assert m["grad_norm"] == float(np.sqrt(float(blk[2])))
            assert np.array_equal(m["td_abs"], blk[4:])
            # the bound inputs hold exactly the staged batch
            b = dqn_batch(11 + k)
            obs = learner.inputs["obs.obs"].numpy()
            assert np.array_equal(obs, b["obs"])
            assert np.array_equal(learner.inputs["is_weights"].numpy().reshape(-1),
                                  np.asarray(b["is_weights"], np.float32).reshape(-1))
    finally:
        learner.close()


def test_dqn_partial_load_sends_only_what_was_loaded(device):
    """Inputs not loaded since the last update are not overwritten from the
    host image: a batch assembled on the device in place survives a later
    load of one input."""
    from ttrl_amd.workloads import dqn_batch

    learner, _, _ = build_learner(device, seed=2)
    try:
        learner.update(dqn_batch(20))
        dev_obs = np.random.default_rng(5).integers(0, 256, (32, 4, 84, 84), dtype=np.uint8)
        learner.inputs["obs.obs"].data.upload(dev_obs)  # a device-side write into the bound block
        w = np.full((32, 1), 0.5, np.float32)
        learner.step.load_input("is_weights", w)
        learner.step.flush_inputs()
        assert np.array_equal(learner.inputs["obs.obs"].numpy(), dev_obs)
        assert np.array_equal(learner.inputs["is_weights"].numpy(), w)
    finally:
        learner.close()


def test_sac_update_from_a_host_batch_is_one_call(device):
    from ttrl_amd.workloads import sac_batch

    learner, _, _ = build_sac(device, seed=3)
    try:
        learner.update(sac_batch(30))  # eager first update
        learner.update(sac_batch(31))  # capture, first replay
        for k in range(3):
            with _Spy(device) as spy:
                m = learner.update(sac_batch(32 + k))
            assert spy.names == ["ttrl_graph_step"], spy.names
            blk = learner._metric_block.numpy()
            B = 256
            assert m["critic_loss"] == float(blk[0]) and m["alpha"] == float(blk[1])
            assert m["actor_loss"] == float(blk[2]) and m["alpha_loss"] == float(blk[3])
            assert np.array_equal(m["q_target"], blk[8:8 + B])
            # td_abs at 8 + B, then the log-probabilities of obs (the metric) and next_obs
            assert np.array_equal(m["logp"], blk[8 + 2 * B:8 + 3 * B])
    finally:
        learner.close()
