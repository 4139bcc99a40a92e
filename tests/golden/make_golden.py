"""Writes the committed golden fixtures of this directory.

    python tests/golden/make_golden.py

known_answers.json  literal known answers from the reference's own tests:
                    conv_out_size cases and the ragged-stride refusal
                    (tests/engine/test_geometry_and_scalars.py:16-30), the
                    Nature-CNN geometry 84 -> 20 -> 9 -> 7 (ttrl/nets/towers.py:37-40),
                    the fused Adam scalars' textbook identity at t in {1, 10,
                    100000} with that test's inputs (:33-50), and the GAE
                    padding answer [2, 1, 0, 1] (tests/buffers/test_rollout.py:58-68)
conv_small.npz      a padded, strided convolution: inputs and the oracle's
                    forward, dX, dW, db
gae_128x8.npz       a 128-step, 8-lane rollout with padding: inputs and the
                    oracle's float32 advantages and returns (bit-exact target)
ppo_b64.npz         one PPO minibatch: inputs and the oracle's loss parts,
                    new log-probs and gradients
dqn_b4_36.npz       one DQN update of the Nature CNN on 4x36x36 frames at
                    batch 4: the batch, the seed and SHA-256 of the generated
                    parameters, and the oracle's loss, mean_q, td_abs, next
                    actions, grad_sq and per-tensor Adam deltas

Every array is produced by the float64 oracle under `oracle/` from seeded
numpy inputs; nothing here runs the reference.  Re-running the script
reproduces every array exactly (tests/test_golden.py checks the oracle
against them).
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import adam, conv, dqn, ppo  # noqa: E402
from oracle.nets import QNet  # noqa: E402

DQN_SEED = 1234
DQN_SHAPES = [((32, 4, 8, 8), 4), ((64, 32, 4, 4), 2), ((64, 64, 3, 3), 1)]
FC_SHAPES = [(64, 512), (512, 6)]


def known_answers() -> dict:
    lr, b1, b2, eps, m, v = 1e-4, 0.9, 0.999, 1e-8, 0.37, 0.0021
    adam_cases = []
    for t in (1, 10, 100_000):
        mhat, vhat = m / (1 - b1 ** t), v / (1 - b2 ** t)
        adam_cases.append({"lr": lr, "b1": b1, "b2": b2, "eps": eps, "t": t, "m": m, "v": v,
                           "S": m / (1 - b1), "V": v / (1 - b2),
                           "update": lr * mhat / (np.sqrt(vhat) + eps)})
    return {
        "conv_out_size": [{"size": 84, "kernel": 8, "stride": 4, "padding": 0, "out": 20},
                          {"size": 5, "kernel": 3, "stride": 1, "padding": 1, "out": 5}],
        "conv_out_size_ragged": [{"size": 6, "kernel": 3, "stride": 2, "padding": 0}],
        "nature_cnn_geometry": [84, 20, 9, 7],
        "nature_cnn_flatten": 3136,
        "adam_fused_scalars": adam_cases,
        "gae_padding": {"gamma": 1.0, "lam": 1.0, "rewards": [1, 1, 1, 1], "valid": [1, 1, 0, 1],
                        "advantages": [2.0, 1.0, 0.0, 1.0]},
    }


def conv_small() -> dict:
    rng = np.random.default_rng(7)
    B, C, H, W, O, k, s, p = 2, 6, 11, 11, 5, 3, 2, 1
    x = rng.standard_normal((B, H, W, C)).astype(np.float32)
    w = (rng.standard_normal((O, C, k, k)) / np.sqrt(C * k * k)).astype(np.float32)
    b = (0.1 * rng.standard_normal(O)).astype(np.float32)
    y = conv.forward(x.astype(np.float64), w.astype(np.float64), b.astype(np.float64), s, p)
    dy = rng.standard_normal(y.shape).astype(np.float32)
    dx, dw, db = conv.backward(x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64), s, p)
    geom = np.array([B, C, H, W, O, k, s, p], np.int64)
    return dict(geom=geom, x=x, w=w, b=b, y=y, dy=dy, dx=dx, dw=dw, db=db)


def gae_rollout() -> dict:
    rng = np.random.default_rng(8)
    T, N = 128, 8
    r = rng.choice(np.array([-1.0, 0.0, 1.0], np.float32), (T, N), p=[0.05, 0.9, 0.05])
    v = rng.standard_normal((T, N)).astype(np.float32)
    d = (rng.random((T, N)) < 0.01).astype(np.float32)
    valid = (rng.random((T, N)) > 0.05).astype(np.float32)
    last = rng.standard_normal(N).astype(np.float32)
    adv, ret = ppo.gae(r, v, d, last, 0.99, 0.95, valid)
    return dict(rewards=r, values=v, dones=d, valid=valid, last_values=last, gamma=np.float64(0.99),
                lam=np.float64(0.95), advantages=adv, returns=ret)


def ppo_minibatch() -> dict:
    rng = np.random.default_rng(9)
    B, A = 64, 18
    z = rng.standard_normal((B, A)).astype(np.float32)
    a = rng.integers(0, A, B).astype(np.int32)
    old_lp = (ppo.log_softmax(z)[np.arange(B), a] + rng.normal(0, 0.15, B)).astype(np.float32)
    adv = rng.standard_normal(B).astype(np.float32)
    ret = rng.standard_normal(B).astype(np.float32)
    old_v = rng.standard_normal(B).astype(np.float32)
    v = (old_v + rng.normal(0, 0.2, B)).astype(np.float32)
    valid = (rng.random(B) > 0.2).astype(np.float32)
    cfg = dict(clip_eps=0.1, value_clip_eps=0.1, value_coef=0.5, entropy_coef=0.01)
    out = ppo.ppo_objective(z, a, old_lp, adv, ret, old_v, v, valid, **cfg)
    return dict(logits=z, actions=a, old_logp=old_lp, advantages=adv, returns=ret, old_values=old_v, values=v,
                valid=valid, cfg=np.array([cfg["clip_eps"], cfg["value_clip_eps"], cfg["value_coef"],
                                           cfg["entropy_coef"]]),
                loss=np.array([out["loss"], out["policy_loss"], out["value_loss"], out["entropy"]]),
                new_logp=out["new_logp"], dlogits=out["dlogits"], dvalues=out["dvalues"])


def dqn_params(seed: int):
    """He-uniform Nature-CNN parameters for 4x36x36 frames (weights, then
    bias U(+-1/sqrt(fan_in)), in layer order): float32 arrays."""
    rng = np.random.default_rng(seed)
    out = []
    for shape, _ in DQN_SHAPES:
        fan = int(np.prod(shape[1:]))
        out.append(rng.uniform(-np.sqrt(6 / fan), np.sqrt(6 / fan), shape).astype(np.float32))
        out.append(rng.uniform(-1 / np.sqrt(fan), 1 / np.sqrt(fan), shape[0]).astype(np.float32))
    for shape in FC_SHAPES:
        fan = shape[0]
        out.append(rng.uniform(-np.sqrt(6 / fan), np.sqrt(6 / fan), shape).astype(np.float32))
        out.append(rng.uniform(-1 / np.sqrt(fan), 1 / np.sqrt(fan), shape[1]).astype(np.float32))
    return out


def params_digest(params) -> str:
    h = hashlib.sha256()
    for p in params:
        h.update(np.ascontiguousarray(p, np.float32).tobytes())
    return h.hexdigest()


def qnet(params) -> QNet:
    convs = [(params[2 * i].astype(np.float64), params[2 * i + 1].astype(np.float64), s, 0)
             for i, (_, s) in enumerate(DQN_SHAPES)]
    fcs = [(params[6 + 2 * j].astype(np.float64), params[7 + 2 * j].astype(np.float64)) for j in range(2)]
    return QNet(convs, fcs, 1.0 / 255.0)


def dqn_small() -> dict:
    online = dqn_params(DQN_SEED)
    rng = np.random.default_rng(DQN_SEED + 1)
    target = [(p + 0.05 * np.abs(p).max() * rng.standard_normal(p.shape)).astype(np.float32) for p in online]
    B = 4
    brng = np.random.default_rng(DQN_SEED + 2)
    batch = {
        "obs": brng.integers(0, 256, (B, 4, 36, 36), dtype=np.uint8),
        "next_obs": brng.integers(0, 256, (B, 4, 36, 36), dtype=np.uint8),
        "actions": brng.integers(0, 6, B).astype(np.int64),
        "rewards": np.array([1.0, 0.0, -1.0, 0.0], np.float32),
        "dones": np.array([0.0, 0.0, 0.0, 1.0], np.float32),
        "discounts": np.full(B, 0.99 ** 3, np.float32),
        "is_weights": brng.uniform(0.4, 1.0, B).astype(np.float32),
    }
    out = dqn.dqn_update(qnet(online), qnet(target), batch)
    deltas = [np.asarray(n) - np.asarray(p, np.float64) for n, p in zip(out["new_params"], online)]
    res = {k: v for k, v in batch.items()}
    res.update(
        seed=np.int64(DQN_SEED),
        online_digest=np.array(params_digest(online)),
        target_digest=np.array(params_digest(target)),
        loss=np.float64(out["loss"]), mean_q=np.float64(out["mean_q"]), td_abs=out["td_abs"],
        next_actions=out["next_actions"].astype(np.int64), grad_sq=np.float64(out["grad_sq"]),
        q=out["q"],
    )
    for i, d in enumerate(deltas):
        res[f"delta{i}_head"] = d.reshape(-1)[:64]
        res[f"delta{i}_sum"] = np.float64(d.sum())
        res[f"delta{i}_abs"] = np.float64(np.abs(d).sum())
    return res


def build_all() -> dict:
    return {"conv_small.npz": conv_small(), "gae_128x8.npz": gae_rollout(), "ppo_b64.npz": ppo_minibatch(),
            "dqn_b4_36.npz": dqn_small()}


def main() -> None:
    (HERE / "known_answers.json").write_text(json.dumps(known_answers(), indent=1, sort_keys=True) + "\n")
    for name, arrays in build_all().items():
        np.savez_compressed(HERE / name, **arrays)
    print("wrote", ", ".join(["known_answers.json"] + sorted(build_all())))


if __name__ == "__main__":
    main()
