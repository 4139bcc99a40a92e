"""Full SAC learner update on the GPU against the float64 oracle (config:
batch 256, 11-dim observations, 3-dim actions, twin critics
14 -> 256 -> 256 -> 1 with targets, actor 11 -> 256 -> 256 -> 2x3 tanh-squashed
Gaussian, learned temperature with target entropy -3, three Adams at lr 3e-4,
Polyak tau 0.005).

Tolerance rel 1e-4 (max abs error over a tensor relative to its max |value|)
on losses, q_target, logp, gradient norms, every gradient tensor of the
policy and both critics, the temperature gradient and every updated
parameter; ReLU
gates adopted from the device only inside the 1e-4 RMS band; Adam with
eps 1e-8 turns a gradient of either sign into a step of size lr, so updated
parameters whose oracle gradient lies below the fp32 resolution of its
tensor (|g| < 1e-5 max|g|) are compared with an absolute 2*lr allowance and
counted."""

from __future__ import annotations

import numpy as np
import pytest

from tests._grads import check_grads, grad_of, grad_state
from tests._sac_helpers import build_sac, record_gates, sac_to_oracle

pytestmark = pytest.mark.gpu

REL = 1e-4


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _check_params(got_state: dict, ref_flat, grads, lr, label):
    undecided = 0
    for (k, got), want, g in zip(got_state.items(), ref_flat, grads):
        got = np.asarray(got, np.float64).reshape(want.shape)
        g = np.asarray(g, np.float64).reshape(want.shape)
        tiny = np.abs(g) < 1e-5 * max(np.max(np.abs(g)), 1e-30)
        undecided += int(tiny.sum())
        err = np.abs(got - want)
        scale = max(np.max(np.abs(want)), 1e-30)
        assert np.all(err[~tiny] <= REL * scale), (label, k, float(np.max(err[~tiny]) / scale))
        assert np.all(err[tiny] <= 2.0 * lr + REL * scale), (label, k)
    return undecided


@pytest.mark.parametrize("step_mode,fused", [("graph", True), ("eager", True), ("graph", False), ("eager", False)])
def test_sac_update_matches_oracle(device, step_mode, fused):
    """fused: the update as the library's eight fused stages
    (ttrl_sac_fused_stage) rather than one launch per layer."""
    from oracle.sac import sac_update
    from ttrl_amd.engine import layers
    from ttrl_amd.workloads import sac_batch

    learner, pol, crit = build_sac(device, seed=0, step_mode=step_mode, fused=fused)
    assert (learner._fused is not None) == fused
    batch = sac_batch(7)
    P = sac_to_oracle(pol, crit, crit, 0.0)
    layers.RECORD = []
    try:
        m = learner.update(batch)
        gates = record_gates(layers.RECORD, 256)
    finally:
        layers.RECORD = None
    ref = sac_update(P, batch, gates=gates)
    assert sum(ref["gate_stats"].decided_mismatch.values()) == 0
    for key in ("critic_loss", "actor_loss", "alpha_loss", "alpha", "entropy", "mean_q_target",
                "critic_grad_norm", "actor_grad_norm"):
        assert abs(m[key] - ref[key]) <= REL * max(abs(ref[key]), 1e-6), (key, m[key], ref[key])
    assert _rel(m["q_target"], ref["q_target"]) < REL
    assert _rel(m["logp"], ref["logp"]) < REL
    # every gradient tensor at rel 1e-4 of its own scale: the policy's from
    # the actor region, the critics' from the critic region (the actor region
    # leaves the critic gradients alone), and d alpha_loss / d log_alpha
    check_grads(grad_state(learner.nets.policy), ref["policy_grads"], REL, "policy")
    check_grads(grad_state(learner.nets.critics), ref["critic_grads"], REL, "critics")
    g_alpha = float(grad_of(learner.log_alpha).reshape(-1)[0])
    assert abs(g_alpha - ref["d_log_alpha"]) <= REL * max(abs(ref["d_log_alpha"]), 1e-6)
    lr = 3e-4
    _check_params(learner.nets.policy.state_dict(), ref["new_policy"], ref["policy_grads"], lr, "policy")
    crit_flat = [x for c in ref["new_critics"] for pair in c for x in pair]
    _check_params(learner.nets.critics.state_dict(), crit_flat, ref["critic_grads"], lr, "critics")
    targ_flat = [x for c in ref["new_targets"] for pair in c for x in pair]
    got_t = learner.nets.targets.state_dict()
    for (k, got), want in zip(got_t.items(), targ_flat):
        assert _rel(np.asarray(got).reshape(want.shape), want) < REL, k
    la = float(learner.log_alpha.numpy().reshape(-1)[0])
    assert abs(la - ref["new_log_alpha"]) <= 2e-6
    learner.close()


def test_sac_graph_replays_match_eager(device):
    from ttrl_amd.workloads import sac_batch

    res = {}
    for mode in ("graph", "eager"):
        learner, _, _ = build_sac(device, seed=2, step_mode=mode)
        ms = [learner.update(sac_batch(50 + k)) for k in range(4)]
        res[mode] = (ms, learner.nets.state_dict(), learner.log_alpha.numpy())
        learner.close()
    for a, b in zip(res["graph"][0], res["eager"][0]):
        assert a["critic_loss"] == b["critic_loss"] and a["actor_loss"] == b["actor_loss"]
    for k in res["graph"][1]:
        assert np.array_equal(res["graph"][1][k], res["eager"][1][k]), k
    assert np.array_equal(res["graph"][2], res["eager"][2])
