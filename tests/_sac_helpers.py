"""Shared set-up of SAC parity tests."""

from __future__ import annotations

import numpy as np


def _pairs(state: dict):
    items = list(state.items())
    return [(np.asarray(items[i][1], np.float64), np.asarray(items[i + 1][1], np.float64).reshape(-1))
            for i in range(0, len(items), 2)]


def sac_to_oracle(policy_state: dict, critics_state: dict, targets_state: dict, log_alpha: float):
    from oracle.sac import SacParams

    pol = _pairs(policy_state)
    crit = _pairs(critics_state)
    targ = _pairs(targets_state)
    n = len(crit) // 2
    return SacParams(trunk=pol[:-2], mean=pol[-2], log_std=pol[-1], critics=[crit[:n], crit[n:]],
                     targets=[targ[:n], targ[n:]], log_alpha=float(log_alpha))


def build_sac(device, *, seed=0, step_mode="graph", batch=256, fused=True, prioritized=False):
    from ttrl_amd.algos.sac import SACConfig, SACLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_sac_state

    cfg = SACConfig(batch_size=batch, step_mode=step_mode, fused_update=fused, prioritized=prioritized)
    learner = SACLearner(ObsSpec.vector(11), ActionSpec.continuous(3), device, cfg=cfg, seed=seed)
    pol = he_uniform_sac_state(learner.nets.policy, seed + 10)
    crit = he_uniform_sac_state(learner.nets.critics, seed + 20)
    learner.nets.policy.load_state_dict(pol)
    learner.nets.critics.load_state_dict(crit)
    learner.nets.targets.load_state_dict(crit)
    return learner, pol, crit


def record_gates(records, B):
    """Device ReLU outputs in execution order -> oracle gate names: the
    policy over [obs; next_obs] (one record per layer), the target critics
    and the critics as four groups (target 0, target 1, critic 0, critic 1),
    then the critics on the actor's actions."""
    out = {}
    it = iter(records)
    for layer in range(2):
        y = next(it).numpy().reshape(2, B, -1)
        out[f"policy.{layer}"] = y[0] > 0
        out[f"policy_next.{layer}"] = y[1] > 0
    for layer in range(2):
        y = next(it).numpy().reshape(4, B, -1)
        for g, name in enumerate(("target0", "target1", "critic0", "critic1")):
            out[f"{name}.{layer}"] = y[g] > 0
    for layer in range(2):
        y = next(it).numpy().reshape(2, B, -1)
        out[f"critic0_pi.{layer}"] = y[0] > 0
        out[f"critic1_pi.{layer}"] = y[1] > 0
    return out
