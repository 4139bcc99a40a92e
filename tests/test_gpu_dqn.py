"""Full DQN learner update on the GPU against the float64 oracle
(config: batch 32, 4x84x84 uint8 frames, 6 actions, double DQN, n-step 3,
prioritized weights, Huber delta 1, Adam lr 6.25e-5 eps 1.5e-4).

Tolerances: rel 1e-4 on Q-values, loss, mean_q, td_abs, every gradient
tensor, Adam-updated parameters (max abs error over each tensor relative to
its max |value|) and Adam deltas p1 - p0 (relative to the largest delta,
plus the float32 spacing of the parameter);
exact next actions wherever the top-two Q gap is decisive; ReLU gates
adopted from the device only where float64 puts the pre-activation within
1e-4 of the tensor's RMS of zero."""

from __future__ import annotations

import numpy as np
import pytest

from tests._dqn_helpers import build_learner, qnet_to_oracle
from tests._grads import check_deltas, check_grads, grad_state

pytestmark = pytest.mark.gpu

REL = 1e-4


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _update_recording(learner, batch):
    """Run one update while recording every layer's grouped outputs; returns
    (metrics, records of the last pass): the device's own activations of
    this update, so the oracle adopts exactly the gates the update used."""
    from ttrl_amd.engine import layers
    layers.RECORD = []
    try:
        m = learner.update(batch)
        recs = [[y.numpy() for y in ys] for ys in layers.RECORD[-5:]]
    finally:
        layers.RECORD = None
    return m, recs


@pytest.mark.parametrize("step_mode,defer", [("graph", True), ("eager", True), ("graph", False)])
def test_dqn_update_matches_oracle(device, step_mode, defer):
    """defer: the weight-gradient reductions, the Q head's gradients and the
    batch means formed by the Adam launch (gradient sources) rather than by
    launches of their own."""
    from oracle.dqn import dqn_update
    from oracle.nets import qnet_forward
    from ttrl_amd.workloads import dqn_batch

    learner, online, target = build_learner(device, seed=0, step_mode=step_mode, defer_grads=defer)
    batch = dqn_batch(11, batch=32)
    onet, tnet = qnet_to_oracle(online), qnet_to_oracle(target)
    m, recs = _update_recording(learner, batch)
    # recs: conv1, conv2, conv3, fc1 (ReLU outputs) and the Q layer, each over
    # the groups [online(s), online(s'), target(s')]
    _, acts = qnet_forward(onet, batch["obs"])
    gates = {}
    for i, name in enumerate(("conv0", "conv1", "conv2", "fc0")):
        r = recs[i][0]
        gates[name] = (r > 0).reshape(acts[i][1].shape)
    q_dev, q_next_dev = recs[4][0], recs[4][1]
    ref = dqn_update(onet, tnet, batch, double=True, delta=1.0, lr=6.25e-5, eps=1.5e-4, gates=gates,
                     device_next_actions=np.argmax(q_next_dev, 1))
    assert _rel(q_dev, ref["q"]) < REL
    assert sum(ref["gate_stats"].decided_mismatch.values()) == 0
    assert abs(m["loss"] - ref["loss"]) <= REL * abs(ref["loss"])
    assert abs(m["mean_q"] - ref["mean_q"]) <= REL * abs(ref["mean_q"])
    assert _rel(m["td_abs"], ref["td_abs"]) < REL
    assert abs(m["grad_norm"] - ref["grad_norm"]) <= REL * ref["grad_norm"]
    # every gradient tensor, each at rel 1e-4 of its own scale (the
    # reference checks every parameter gradient by name,
    # tests/hardware/test_algos_dqn_parity.py:147-152)
    # the update forms the pending gradients inside its Adam launch without
    # storing them; written on request from the same operands
    learner.optimizer.materialize_grads()
    check_grads(grad_state(learner.online), ref["grads"], REL, "dqn")
    new = learner.online.state_dict()
    for (k, got), want in zip(new.items(), ref["new_params"]):
        assert _rel(np.asarray(got).reshape(want.shape), want) < REL, k
    # the Adam step itself: p1 - p0 against the oracle's delta at rel 1e-4 of
    # the delta's scale (lr = 6.25e-5, eps = 1.5e-4: the delta is lr*g/(|g|+eps),
    # linear in g wherever |g| is below eps)
    check_deltas(list(online.values()), list(new.values()), ref["new_params"], REL, "dqn")
    learner.close()


def test_dqn_graph_replays_are_deterministic(device):
    """Two learners from the same state, same batches: bit-identical params
    after 3 graph replays (the reference's replay-determinism tests)."""
    from ttrl_amd.workloads import dqn_batch

    outs = []
    for _ in range(2):
        learner, _, _ = build_learner(device, seed=3, step_mode="graph")
        for k in range(3):
            learner.update(dqn_batch(100 + k))
        outs.append(learner.online.state_dict())
        learner.close()
    for k in outs[0]:
        assert np.array_equal(outs[0][k], outs[1][k]), k


def test_dqn_graph_and_eager_agree(device):
    from ttrl_amd.workloads import dqn_batch

    res = {}
    for mode in ("graph", "eager"):
        learner, _, _ = build_learner(device, seed=4, step_mode=mode)
        ms = [learner.update(dqn_batch(200 + k)) for k in range(3)]
        res[mode] = (ms, learner.online.state_dict())
        learner.close()
    for a, b in zip(res["graph"][0], res["eager"][0]):
        assert a["loss"] == b["loss"]
    for k in res["graph"][1]:
        assert np.array_equal(res["graph"][1][k], res["eager"][1][k]), k


def test_dqn_traced_fwd_bwd_with_deferred_gradients_tracks_the_oracle(device):
    """The reference's trace mode (forward and backward captured, Adam
    eager) with the weight-gradient reductions and batch means left to the
    Adam launch: three updates, each checked against the float64 oracle from
    the device's own parameters and Adam moments before it (loss, mean_q,
    td_abs, grad_norm, every updated parameter at rel 1e-4), and the same
    metrics and parameters as graph mode bit for bit.  The replays after the
    first re-queue the captured backward's pending gradients, so each step
    forms this update's gradients, not the capture's."""
    from oracle.dqn import dqn_update
    from oracle.nets import qnet_forward
    from tests._dqn_helpers import adam_moments
    from ttrl_amd.workloads import dqn_batch

    from ttrl_amd.engine import layers

    learner, _, _ = build_learner(device, seed=6, step_mode="traced_fwd_bwd", defer_grads=True)
    graph, _, _ = build_learner(device, seed=6, step_mode="graph", defer_grads=True)
    assert learner.defer_grads
    outputs = None  # the captured forward's layer outputs, rewritten by every replay
    try:
        for k in range(3):
            batch = dqn_batch(300 + k, batch=32)
            p0 = learner.online.state_dict()
            t0 = learner.target.state_dict()
            S0, V0 = adam_moments(learner.optimizer, learner.online)
            t_step = learner.optimizer.t + 1
            layers.RECORD = []
            try:
                m = learner.update(batch)
                if outputs is None:
                    outputs = layers.RECORD[-5:]
            finally:
                layers.RECORD = None
            recs = [[y.numpy() for y in ys] for ys in outputs]
            gm = graph.update(batch)
            for key in ("loss", "mean_q", "grad_norm"):
                assert m[key] == gm[key], (k, key)
            assert np.array_equal(m["td_abs"], gm["td_abs"]), k
            onet, tnet = qnet_to_oracle(p0), qnet_to_oracle(t0)
            _, acts = qnet_forward(onet, batch["obs"])
            gates = {n: (recs[i][0] > 0).reshape(acts[i][1].shape)
                     for i, n in enumerate(("conv0", "conv1", "conv2", "fc0"))}
            ref = dqn_update(onet, tnet, batch, double=True, delta=1.0, lr=6.25e-5, eps=1.5e-4, gates=gates,
                             device_next_actions=np.argmax(recs[4][1], 1), adam_state=(S0, V0), t=t_step)
            for key in ("loss", "mean_q", "grad_norm"):
                assert abs(m[key] - ref[key]) <= REL * abs(ref[key]), (k, key, m[key], ref[key])
            assert _rel(m["td_abs"], ref["td_abs"]) < REL, k
            new = learner.online.state_dict()
            for (name, got), want in zip(new.items(), ref["new_params"]):
                assert _rel(np.asarray(got).reshape(want.shape), want) < REL, (k, name)
            for name, v in graph.online.state_dict().items():
                assert np.array_equal(new[name], v), (k, name)
    finally:
        learner.close()
        graph.close()
