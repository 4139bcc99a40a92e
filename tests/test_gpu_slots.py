"""Input slots on the GPU (TrainStep.enable_input_slots,
SACLearner.enable_input_slots): one graph captured per bound input block.

A learner whose batches are each written into an input slot and updated
there must end bit for bit where the same learner ends when each batch is
written into its one bound block and the update run: the same kernels and
plans run on the same floats, only the input block differs.  Compared:
every parameter, the Adam moments and the metric block; also when every
slot is written first and the updates then run back to back (a replay
draw of several batches at once)."""

from __future__ import annotations

import numpy as np
import pytest

from tests._dqn_helpers import build_learner
from tests._sac_helpers import build_sac

pytestmark = pytest.mark.gpu


def _same(a: dict, b: dict, what: str):
    assert a.keys() == b.keys()
    for k in a:
        assert np.array_equal(np.asarray(a[k]), np.asarray(b[k])), f"{what}: {k}"


def _adam_state(opt) -> dict:
    out = {f"m{i}": m.numpy() for i, m in enumerate(opt.m)}
    out.update({f"v{i}": v.numpy() for i, v in enumerate(opt.v)})
    return out


@pytest.mark.parametrize("ahead", [False, True])
def test_dqn_input_slots_match_one_bound_block(device, ahead):
    from ttrl_amd.workloads import dqn_batch

    ref, _, _ = build_learner(device, seed=7, step_mode="graph")
    got, _, _ = build_learner(device, seed=7, step_mode="graph")
    got.step.enable_input_slots(3)
    batches = [dqn_batch(70 + i) for i in range(7)]
    for learner in (ref, got):
        learner.load_batch(batches[0])
        learner.step.run()  # captures (every slot's graph for `got`), runs slot 0
    order = [1, 2, 0, 1, 2, 0]

    def write(i):
        got.load_batch(batches[i])
        got.step.flush_inputs()  # into slot 0's block
        k = order[i - 1]
        if k:
            got.step.slot_inputs(k)["_block"].copy_from(got.inputs["_block"])

    if ahead:
        for i in (1, 2):  # slots 1 and 2 first (slot 0 still holds batch 0 until batch 3)
            write(i)
    for i in range(1, 7):
        ref.load_batch(batches[i])
        ref.step.run()
        if not ahead or i > 2:
            write(i)
        got.step.replay_slot(order[i - 1])
    device.synchronize()
    _same(got.online.state_dict(), ref.online.state_dict(), "parameters")
    _same(_adam_state(got.optimizer), _adam_state(ref.optimizer), "Adam moments")
    assert np.array_equal(got._metric_block.numpy(), ref._metric_block.numpy())
    m_ref, m_got = ref.update(batches[3]), got.update(batches[3])  # the one-block path after slots
    for k in m_ref:
        assert np.array_equal(np.asarray(m_got[k]), np.asarray(m_ref[k])), k


def test_sac_input_slots_match_one_bound_block(device):
    from ttrl_amd.workloads import sac_batch

    ref, _, _ = build_sac(device, seed=5, step_mode="graph")
    got, _, _ = build_sac(device, seed=5, step_mode="graph")
    got.enable_input_slots(2)
    batches = [sac_batch(90 + i) for i in range(5)]
    for learner in (ref, got):
        learner.batch.load_batch(batches[0])
        learner._run()  # eager warm-up and capture (every slot's graph for `got`)
    for i in range(1, 5):
        ref.batch.load_batch(batches[i])
        ref._run()
        got.batch.load_batch(batches[i])
        got.batch.flush()
        k = i % 2
        if k:
            got.slot_block(k).copy_from(got.batch.block)
        got.replay_slot(k)
    device.synchronize()
    _same(got.nets.state_dict(), ref.nets.state_dict(), "networks")
    for name in ("critic_opt", "actor_opt"):
        _same(_adam_state(getattr(got, name)), _adam_state(getattr(ref, name)), name)
    assert np.array_equal(got._metric_block.numpy(), ref._metric_block.numpy())
