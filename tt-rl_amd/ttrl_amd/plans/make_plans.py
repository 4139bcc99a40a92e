"""Tune and write the packaged GEMM plan table (gfx950.tsv beside this file).

Runs every learner workload of this package once on GPU 0 with no table
loaded, so each GEMM signature is timed at its first call, then writes the
context's table.  Every later process loads the table at device open and runs
the same plans, so its split-K summation orders, and with them its bits,
match.  With --extend the packaged table is loaded first: only the signatures
it lacks (a newer build's) are timed, and every packaged entry is kept.
Usage (on a gfx950 machine):

    python -m ttrl_amd.plans.make_plans [--extend] [--out PATH]
"""

from __future__ import annotations

import argparse
import os
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def tune_all(dev) -> None:
    import numpy as np

    from ttrl_amd.algos.dqn import DQNConfig, DQNLearner
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner, RecurrentConfig, RecurrentPPOLearner
    from ttrl_amd.algos.sac import SACConfig, SACLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import dqn_batch, ppo_rollout, recurrent_ppo_rollout, sac_batch

    image = ObsSpec.image((4, 84, 84))
    for batch in (32,):
        for prioritized, defer in ((True, True), (False, True), (True, False)):
            cfg = DQNConfig(lr=6.25e-5, adam_eps=1.5e-4, batch_size=batch, prioritized=prioritized)
            dqn = DQNLearner(image, ActionSpec.discrete(6), dev, cfg=cfg, seed=0, n_envs=8, defer_grads=defer)
            for k in range(2):
                dqn.update(dqn_batch(k, batch=batch))
            rng = np.random.default_rng(0)
            for lanes in (1, 8, 16, 32):
                dqn._acting.decide(rng.integers(0, 256, (lanes, 4, 84, 84), dtype=np.uint8))
            dqn.close()
    sac = SACLearner(ObsSpec.vector(11), ActionSpec.continuous(3), dev, cfg=SACConfig(batch_size=256), seed=0,
                     n_envs=16)
    for k in range(3):
        sac.update(sac_batch(k))
    rng = np.random.default_rng(1)
    for lanes in (1, 16, 256):
        sac._acting.decide(rng.standard_normal((lanes, 11)).astype(np.float32),
                           noise=rng.standard_normal((lanes, 3)).astype(np.float32))
    sac.close()
    for A in (18, 6):
        ppo = PPOLearner(image, ActionSpec.discrete(A), dev, cfg=PPOConfig(minibatch_size=256, epochs=4, n_steps=128),
                         seed=0)
        ppo.update(ppo_rollout(1, 128, 8, A))
        ppo.close()
    rcfg = PPOConfig(minibatch_size=512, epochs=4, n_steps=128, recurrent=RecurrentConfig(hidden_size=512, seq_len=32))
    rppo = RecurrentPPOLearner(image, ActionSpec.discrete(18), dev, cfg=rcfg, seed=0)
    rppo.update(recurrent_ppo_rollout(2, 128, 16, 18, 32, 512))
    rppo.close()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", default=str(HERE / "gfx950.tsv"))
    ap.add_argument("--extend", action="store_true", help="keep the packaged table, time only what it lacks")
    args = ap.parse_args()
    # read when the device opens: the packaged table, or none (tune from scratch)
    os.environ["TTRL_PLANS"] = str(HERE / "gfx950.tsv") if args.extend else "none"
    from ttrl_amd.engine.device import open_device

    dev = open_device(0)
    tune_all(dev)
    dev.synchronize()
    dev.save_plans(args.out)
    n = len(Path(args.out).read_text().splitlines())
    print(f"wrote {n} plans to {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.path.insert(0, str(HERE.parents[1]))
    sys.exit(main())
