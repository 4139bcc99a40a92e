"""Float64 restatement of one SAC learner update, in the reference's order
(ttrl/algos/sac/agent.py:218-238): critic region, critic Adam, actor region
(reading the just-updated critics), actor and temperature Adam, Polyak.

critic_loss   ttrl/algos/sac/losses.py:46-76 (soft target under no_grad,
              min over the target critics, 0.5 * sum_i mean(w (Q_i - y)^2))
actor_loss    ttrl/algos/sac/losses.py:79-84 (mean(alpha logp - min_i Q_i))
alpha_loss    ttrl/algos/sac/losses.py:87-94 (-mean(log_alpha (logp + H)))
min / clamp   relu identities: gradient to the second operand iff a > b,
              clamp passes gradient strictly inside (ttrl/engine/ops/select.py:26-63)
policy head   mean and log_std heads, log_std clamped to [-20, 2]
              (ttrl/nets/heads.py:25-93)
critic input  concat(s, a) (ttrl/nets/fusion.py:36-71)
Polyak        target <- (1 - tau) target + tau critic (ttrl/algos/sac/targets.py:45-52)
metrics       ttrl/algos/sac/step.py:115-130
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import adam, gaussian, fa, float_type
from oracle.nets import GateStats, mlp_backward, mlp_forward

LOG_STD_MIN = -20.0
LOG_STD_MAX = 2.0


@dataclass
class SacParams:
    trunk: list        # policy hidden layers [(W, b)] with ReLU
    mean: tuple        # (W, b)
    log_std: tuple     # (W, b)
    critics: list      # two critics, each [(W, b)] x3 (ReLU on the first two)
    targets: list      # same structure as critics
    log_alpha: float

    def policy_flat(self):
        out = []
        for w, b in self.trunk:
            out += [w, b]
        out += [self.mean[0], self.mean[1], self.log_std[0], self.log_std[1]]
        return out

    def critics_flat(self):
        out = []
        for c in self.critics:
            for w, b in c:
                out += [w, b]
        return out


def policy_forward(P: SacParams, obs, *, gates=None, stats=None, prefix="policy."):
    h, acts = mlp_forward(P.trunk, obs, relu_last=True, gates=gates, stats=stats, prefix=prefix)
    mean = h @ P.mean[0] + P.mean[1].reshape(1, -1)
    raw = h @ P.log_std[0] + P.log_std[1].reshape(1, -1)
    return mean, raw, np.clip(raw, LOG_STD_MIN, LOG_STD_MAX), h, acts


def critic_forward(layers, obs, action, *, gates=None, stats=None, prefix=""):
    x = np.concatenate([fa(obs), fa(action)], axis=1)
    return mlp_forward(layers, x, gates=gates, stats=stats, prefix=prefix)


def _adam_all(params, grads, lr, eps, betas):
    out = []
    for p, g in zip(params, grads):
        p1, _, _ = adam.fused_step(p, g, np.zeros_like(g), np.zeros_like(g), 1, lr, betas[0], betas[1], eps)
        out.append(p1)
    return out


def sac_update(P: SacParams, batch: dict, *, lr: float = 3e-4, eps: float = 1e-8, betas=(0.9, 0.999),
               tau: float = 0.005, target_entropy: float | None = None, learn_alpha: bool = True,
               prioritized: bool = False, gates=None) -> dict:
    stats = GateStats()
    obs = fa(batch["obs"])
    nxt = fa(batch["next_obs"])
    act = fa(batch["actions"])
    B, d = act.shape
    H = -float(d) if target_entropy is None else float(target_entropy)
    r = fa(batch["rewards"]).reshape(-1)
    done = fa(batch["dones"]).reshape(-1)
    disc = fa(batch["discounts"]).reshape(-1)
    w = fa(batch["is_weights"]).reshape(-1) if prioritized else np.ones(B, float_type())
    alpha = float(np.exp(P.log_alpha))

    # ---- critic region
    mean_n, _, ls_n, _, _ = policy_forward(P, nxt, gates=gates, stats=stats, prefix="policy_next.")
    a_next, logp_next, _ = gaussian.sample(mean_n, ls_n, batch["next_noise"])
    qt = [critic_forward(t, nxt, a_next, gates=gates, stats=stats, prefix=f"target{i}.")[0].reshape(-1)
          for i, t in enumerate(P.targets)]
    soft = np.minimum(qt[0], qt[1]) - alpha * logp_next
    y = r + disc * (1.0 - done) * soft
    q, cacheq = [], []
    for i, c in enumerate(P.critics):
        out, acts = critic_forward(c, obs, act, gates=gates, stats=stats, prefix=f"critic{i}.")
        q.append(out.reshape(-1))
        cacheq.append(acts)
    errs = [qi - y for qi in q]
    critic_loss = 0.5 * sum(float(np.mean(w * e * e)) for e in errs)
    critic_grads = []
    for i, c in enumerate(P.critics):
        g, _ = mlp_backward(c, cacheq[i], (w * errs[i] / B).reshape(-1, 1))
        critic_grads.append(g)
    flat_cg = [x for g in critic_grads for pair in g for x in pair]
    critic_grad_sq = float(sum(np.sum(g * g) for g in flat_cg))
    new_critic_flat = _adam_all(P.critics_flat(), flat_cg, lr, eps, betas)
    it = iter(new_critic_flat)
    new_critics = [[(next(it), next(it)) for _ in c] for c in P.critics]

    # ---- actor region (updated critics)
    mean, raw, ls, h, pacts = policy_forward(P, obs, gates=gates, stats=stats, prefix="policy.")
    a_pi, logp, _ = gaussian.sample(mean, ls, batch["noise"])
    qa, cachea = [], []
    for i, c in enumerate(new_critics):
        out, acts = critic_forward(c, obs, a_pi, gates=gates, stats=stats, prefix=f"critic{i}_pi.")
        qa.append(out.reshape(-1))
        cachea.append(acts)
    actor_loss = float(np.mean(alpha * logp - np.minimum(qa[0], qa[1])))
    second = qa[0] - qa[1] > 0
    dq = [np.where(second, 0.0, -1.0 / B), np.where(second, -1.0 / B, 0.0)]
    g_action = np.zeros_like(a_pi)
    obs_dim = obs.shape[1]
    for i, c in enumerate(new_critics):
        _, dx = mlp_backward(c, cachea[i], dq[i].reshape(-1, 1), need_dx=True)
        g_action += dx[:, obs_dim:]
    g_logp = np.full(B, alpha / B, float_type())
    gmean, gls = gaussian.sample_backward(mean, ls, batch["noise"], g_action, g_logp)
    gls = gls * ((raw > LOG_STD_MIN) & (raw < LOG_STD_MAX))
    dW_mean, db_mean = h.T @ gmean, gmean.sum(0)
    dW_ls, db_ls = h.T @ gls, gls.sum(0)
    dh = gmean @ P.mean[0].T + gls @ P.log_std[0].T
    # back through the trunk; its last ReLU gate applies to dh
    g = dh
    tg = []
    for j in range(len(P.trunk) - 1, -1, -1):
        h_in, _, m = pacts[j]
        g = g * m
        tg.append((h_in.T @ g, g.sum(0)))
        if j > 0:
            g = g @ P.trunk[j][0].T
    tg.reverse()
    policy_grads = [x for pair in tg for x in pair] + [dW_mean, db_mean, dW_ls, db_ls]
    actor_grad_sq = float(sum(np.sum(x * x) for x in policy_grads))
    new_policy = _adam_all(P.policy_flat(), policy_grads, lr, eps, betas)
    alpha_loss = -float(P.log_alpha * np.mean(logp + H)) if learn_alpha else 0.0
    d_log_alpha = -float(np.mean(logp + H))
    new_log_alpha = P.log_alpha
    if learn_alpha:
        new_log_alpha = float(_adam_all([np.array([[P.log_alpha]])], [np.array([[d_log_alpha]])],
                                        lr, eps, betas)[0].reshape(-1)[0])

    # ---- Polyak
    new_targets = [[((1 - tau) * tw + tau * cw, (1 - tau) * tb + tau * cb)
                    for (tw, tb), (cw, cb) in zip(t, c)] for t, c in zip(P.targets, new_critics)]

    return {
        "q_target": y, "logp_next": logp_next, "a_next": a_next, "q": q, "critic_loss": critic_loss,
        "critic_grads": flat_cg, "critic_grad_sq": critic_grad_sq, "new_critics": new_critics,
        "mean": mean, "log_std": ls, "action": a_pi, "logp": logp, "q_pi": qa,
        "actor_loss": actor_loss, "policy_grads": policy_grads, "actor_grad_sq": actor_grad_sq,
        "new_policy": new_policy, "alpha_loss": alpha_loss, "d_log_alpha": d_log_alpha,
        "new_log_alpha": new_log_alpha, "new_targets": new_targets, "alpha": alpha,
        "entropy": float(-np.mean(logp)), "mean_q_target": float(np.mean(y)),
        "critic_grad_norm": float(np.sqrt(critic_grad_sq)), "actor_grad_norm": float(np.sqrt(actor_grad_sq)),
        "gate_stats": stats,
    }
