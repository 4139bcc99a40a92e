#!/usr/bin/env python3
"""Learner-update throughput on one MI355X: DQN updates/s at batch 32 (the
headline value) and SAC updates/s at batch 256, with roofline fractions and
a CPU baseline timed on this machine's host cores.

One step = one full learner update (forward, backward, Adam; for SAC also
the temperature step and the Polyak blend) replayed as one hipGraph, on a
fresh synthetic batch: --ring distinct batches are resident in HBM, each in
one of the learner's input slots (a bound input block with a graph captured
against it), and update i reads slot i mod ring where it lies, so no step
re-reads the previous step's inputs and neither a host transfer nor a device
copy is timed.  `copy_in_each_step` times the same updates with a device copy
of each batch into one bound block in front of every update, and `--mode
eager` runs that form without graphs.  Weights are seeded He-uniform; data is
synthetic (uint8 Atari-shaped frames, Hopper-shaped vectors).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
Prints one JSON line.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "tt-rl_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import numpy as np  # noqa: E402

PEAK_FP32_MFMA = 157.3e12
# HBM bytes per call of the DQN Adam step at batch 32, from rocprofv3 FETCH_SIZE and WRITE_SIZE
# passes over the step's kernel, each scaled by what the same counter reads for a 256 MiB
# device-to-device copy (profiles/dqn_adam_step_roofline_and_traffic.md), and the SHA-256 of the
# optimizer kernels' source the passes measured: a build from other source reports traffic null.
ADAM_STEP_TRAFFIC_BYTES = 45348659
ADAM_STEP_TRAFFIC_SOURCE = "e4f92d8030583bd49af478ed7481ecc0f111f223e09826a20ed8628f63f7b3a4"
ADAM_STEP_SOURCES = ("tt-rl_amd/csrc/optim.hip", "tt-rl_amd/csrc/common.hpp", "tt-rl_amd/csrc/adam_dev.hpp")
PEAK_HBM = 8.0e12


def _source_digest(paths) -> str:
    import hashlib

    h = hashlib.sha256()
    for rel in paths:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def adam_step_traffic():
    """(bytes, digest now): the committed traffic figure when the kernel
    source is the one it was measured on, else None."""
    digest = _source_digest(ADAM_STEP_SOURCES)
    return (ADAM_STEP_TRAFFIC_BYTES if digest == ADAM_STEP_TRAFFIC_SOURCE else None), digest

# Multiply-accumulates per sample of the Nature CNN at 4x84x84 (conv1..3, fc1, fc2).
NATURE_MACS = (20 * 20 * 32 * 4 * 64, 9 * 9 * 64 * 32 * 16, 7 * 7 * 64 * 64 * 9, 3136 * 512, 512 * 6)


def dqn_update_flops(batch: int = 32) -> float:
    """3 forwards + weight gradients of all layers + input gradients of all but conv1."""
    fwd = sum(NATURE_MACS)
    return 2.0 * batch * (3 * fwd + fwd + (fwd - NATURE_MACS[0]))


def sac_update_flops(batch: int = 256) -> float:
    pol = 11 * 256 + 256 * 256 + 2 * 256 * 3
    crit = 14 * 256 + 256 * 256 + 256
    crit_dw, crit_dx = crit, 256 * 256 + 256 + 3 * 256
    critic_region = pol + 2 * crit + 2 * crit + 2 * (crit_dw + 256 * 256 + 256)
    actor_region = pol + 2 * crit + 2 * crit_dx + pol + (pol - 11 * 256)
    return 2.0 * batch * (critic_region + actor_region)


def _fill_slots(dev, n, write, slot_block):
    """Slot r's block holds batch r: written into the bound block (slot 0)
    and copied into slot r; slot 0's own batch is written last."""
    for r in range(n - 1, -1, -1):
        write(r)
        if r:
            slot_block(r).copy_from(slot_block(0))
    dev.synchronize()


def _ring(dev, block, fill, n):
    from ttrl_amd.engine.tensor import DeviceArray

    ring = []
    for r in range(n):
        fill(r)
        slot = DeviceArray(dev, block.shape, np.uint8)
        slot.copy_from(block)
        ring.append(slot)
    dev.synchronize()
    return ring


def _time_steps(dev, step, steps, warmup):
    """step(i): update number i."""
    for i in range(warmup):
        step(i)
    dev.synchronize()
    dev.call("ttrl_timer_start")
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    ms = C.c_float(0.0)
    dev.call("ttrl_timer_stop", C.byref(ms))
    dev.synchronize()
    wall = time.perf_counter() - t0
    return wall, ms.value / 1e3


REPEATS = 5
REPEAT_MIN_UPDATES = 1000


def _spread(rates) -> dict:
    r = sorted(rates)
    return {"runs": len(r), "median": round(float(np.median(r)), 2), "min": round(r[0], 2), "max": round(r[-1], 2),
            "values": [round(x, 2) for x in rates]}


def _graph_legs(dev, steps, warmup, n, replay_slot, slot_block, run_slot):
    """(wall, gpu) of the headline loop: update i reads the resident batch
    of slot i mod n where it lies; then, beside it:
      repeats            the same loop REPEATS more times (at least
                         REPEAT_MIN_UPDATES updates each): median and spread;
      with_metric_read   update i as an agent that drew its batch on the
                         device pays for it: slot i mod n's graph and the
                         packed metric read-back in one call, one wait per
                         update (ttrl_graph_step with no input bytes);
      copy_in_each_step  a device copy of the batch into slot 0's block in
                         front of every update."""
    wall, gpu = _time_steps(dev, lambda i: replay_slot(i % n), steps, warmup)
    per = max(steps, REPEAT_MIN_UPDATES)
    reps = [per / _time_steps(dev, lambda i: replay_slot(i % n), per, 0)[0] for _ in range(REPEATS)]
    read = [per / _time_steps(dev, lambda i: run_slot(i % n), per, warmup if k == 0 else 0)[0]
            for k in range(REPEATS)]

    def copied(i):
        slot_block(0).copy_from(slot_block(1 + i % (n - 1)))
        replay_slot(0)

    cwall, cgpu = _time_steps(dev, copied, steps, warmup)
    legs = {"repeats": dict(_spread(reps), updates_per_run=per),
            "with_metric_read": dict(_spread(read), updates_per_run=per,
                                     note="resident batch, graph replay and the packed metric read-back in one "
                                          "call with one wait per update"),
            "copy_in_each_step": {"value": round(steps / cwall, 2), "ms_per_step": round(cwall / steps * 1e3, 5),
                                  "gpu_ms_per_step": cgpu / steps * 1e3}}
    return wall, gpu, legs


def bench_dqn(dev, steps, warmup, ring_n, mode="graph"):
    from ttrl_amd.algos.dqn import DQNConfig, DQNLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import dqn_batch, he_uniform_qnet_state

    cfg = DQNConfig(lr=6.25e-5, adam_eps=1.5e-4, batch_size=32, step_mode=mode, prioritized=True)
    learner = DQNLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(6), dev, cfg=cfg, seed=0)
    learner.online.load_state_dict(he_uniform_qnet_state(learner.online, 1))
    learner.target.copy_from(learner.online)
    block = learner.inputs["_block"]

    def write(r):
        learner.load_batch(dqn_batch(1000 + r))
        learner.step.flush_inputs()

    if mode == "eager":
        ring = _ring(dev, block, write, ring_n)
        learner.update()

        def step(i):
            block.copy_from(ring[i % ring_n])
            learner.step.run()

        wall, gpu = _time_steps(dev, step, steps, warmup)
        return learner, wall, gpu, 0, None
    learner.step.enable_input_slots(ring_n)
    slot_block = lambda k: learner.step.slot_inputs(k)["_block"]
    _fill_slots(dev, ring_n, write, slot_block)
    learner.update()  # captures one graph per input slot and runs the first update (slot 0)
    wall, gpu, legs = _graph_legs(dev, steps, warmup, ring_n, learner.step.replay_slot, slot_block,
                                  learner.step.run_slot)
    return learner, wall, gpu, learner.step._trace.nodes, legs


def bench_sac(dev, steps, warmup, ring_n, mode="graph"):
    from ttrl_amd.algos.sac import SACConfig, SACLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_sac_state, sac_batch

    learner = SACLearner(ObsSpec.vector(11), ActionSpec.continuous(3), dev, cfg=SACConfig(batch_size=256, step_mode=mode), seed=0)
    learner.nets.policy.load_state_dict(he_uniform_sac_state(learner.nets.policy, 2))
    crit = he_uniform_sac_state(learner.nets.critics, 3)
    learner.nets.critics.load_state_dict(crit)
    learner.nets.targets.load_state_dict(crit)
    block = learner.batch.block

    def write(r):
        learner.batch.load_batch(sac_batch(2000 + r))
        learner.batch.flush()

    if mode == "eager":
        ring = _ring(dev, block, write, ring_n)
        learner.update()

        def step(i):
            block.copy_from(ring[i % ring_n])
            learner._run()

        wall, gpu = _time_steps(dev, step, steps, warmup)
        return learner, wall, gpu, 0, None
    learner.enable_input_slots(ring_n)
    _fill_slots(dev, ring_n, write, learner.slot_block)
    learner.update()  # eager first update (slot 0), then one graph captured per input slot
    learner.update()  # first replay
    wall, gpu, legs = _graph_legs(dev, steps, warmup, ring_n, learner.replay_slot, learner.slot_block,
                                  learner.run_slot)
    return learner, wall, gpu, learner._graph.nodes, legs


def ppo_step_flops(batch: int = 256, actions: int = 18) -> float:
    """One PPO minibatch step on the shared Nature-CNN actor-critic:
    forward, weight gradients of every layer, input gradients of all but conv1."""
    fwd = sum(NATURE_MACS[:-1]) + 512 * (actions + 1)
    return 2.0 * batch * (2 * fwd + (fwd - NATURE_MACS[0]))


def bench_ppo(dev, updates=5, mode="graph"):
    """PPO updates over one resident rollout of 8 envs x 128 steps (1024
    uint8 4x84x84 frames): GAE, normalisation and 4 epochs x 4 minibatches
    of 256, each minibatch step one replay of the captured step graph."""
    from ttrl_amd.algos.ppo import PPOConfig, PPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state, ppo_rollout

    cfg = PPOConfig(minibatch_size=256, epochs=4, n_steps=128, step_mode=mode)
    learner = PPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(18), dev, cfg=cfg, seed=0)
    learner.net.load_state_dict(he_uniform_qnet_state(learner.net, 4))
    rollout = ppo_rollout(5000, 128, 8, 18)
    steps = learner.load_rollout(rollout)
    learner.run_update(steps)  # captures the step graph
    dev.synchronize()
    t0 = time.perf_counter()
    for _ in range(updates):
        learner.run_update(steps)
    dev.synchronize()
    dt = (time.perf_counter() - t0) / updates
    t1 = time.perf_counter()
    learner.update(rollout)
    host_dt = time.perf_counter() - t1
    flops = ppo_step_flops(256, 18)
    out = {"unit": "PPO minibatch steps/s", "value": round(steps / dt, 2), "batch": 256, "steps_per_update": steps,
           "ms_per_update": round(dt * 1e3, 3), "ms_per_step": round(dt / steps * 1e3, 4),
           "flops_per_step": flops, "roofline_frac": flops * steps / dt / PEAK_FP32_MFMA,
           "ms_per_update_with_upload": round(host_dt * 1e3, 3),
           "workload": "PPO update: 8 envs x 128 steps of uint8 4x84x84, GAE 0.99/0.95, 4 epochs x 4 minibatches "
                       "of 256, Nature-CNN -> 512 -> {18, 1}, clip 0.1, vclip 0.1, vf 0.5, ent 0.01, "
                       "grad clip 0.5, Adam 2.5e-4"}
    learner.close()
    return out


def bench_replay(dev, reps=200, cpu=True):
    """One batch of 32 sampled from the GPU-resident replay of 8 lanes of
    uint8 4x84x84 frames (n-step 3), assembled into a learner's input
    buffers: prioritized at 1M transitions (28 GB of frames in HBM), uniform
    at 100k.  Times the whole sample call (host generator draws, the lane-sum
    read of a prioritized draw, the uploads, the pick, the IS weights, the
    n-step assembly)."""
    import gc

    from ttrl_amd.buffers import PriorityConfig, ReplayBuffer
    from ttrl_amd.engine.tensor import DeviceArray
    from ttrl_amd.spaces import ActionSpec, ObsSpec

    spec, lanes, batch = ObsSpec.image((4, 84, 84)), 8, 32
    rng = np.random.default_rng(7)
    steps_per_call = 512
    frames = rng.integers(0, 256, (steps_per_call, lanes, 4, 84, 84), dtype=np.uint8)
    out = {}
    sink = {"obs": DeviceArray(dev, (batch, 4, 84, 84), np.uint8), "next_obs": DeviceArray(dev, (batch, 4, 84, 84),
            np.uint8), "actions_onehot": DeviceArray(dev, (batch, 6)), "rewards": DeviceArray(dev, (batch, 1)),
            "dones": DeviceArray(dev, (batch, 1)), "discounts": DeviceArray(dev, (batch, 1)),
            "weights": DeviceArray(dev, (batch, 1))}
    for name, capacity, prio in (("prioritized", 1_000_000, PriorityConfig()), ("uniform", 100_000, None)):
        buf = ReplayBuffer(spec, ActionSpec.discrete(6), dev, capacity=capacity, n_envs=lanes, n_step=3,
                           gamma=0.99, seed=0, priority=prio)
        t0 = time.perf_counter()
        for _ in range(buf.per_lane_capacity // steps_per_call + 1):
            buf.add_steps(frames, rng.integers(0, 6, (steps_per_call, lanes)),
                          rng.standard_normal((steps_per_call, lanes)).astype(np.float32),
                          np.zeros((steps_per_call, lanes), bool))
        if prio is not None:
            cols = np.arange(buf.per_lane_capacity)
            for lane in range(lanes):
                for c0 in range(0, cols.size, 1024):
                    cc = cols[c0:c0 + 1024]
                    buf.update_priorities(np.full(cc.size, lane), cc, rng.exponential(1.0, cc.size))
        dev.synchronize()
        fill_s = time.perf_counter() - t0
        beta = 0.4 if prio is not None else None
        for _ in range(10):
            buf.sample(batch, beta=beta, out=sink)
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            buf.sample(batch, beta=beta, out=sink)
        dev.synchronize()
        us = (time.perf_counter() - t0) / reps * 1e6
        out[name] = {"capacity": buf.capacity, "us_per_sample": round(us, 2), "fill_seconds": round(fill_s, 2)}
        del buf
        gc.collect()
    if cpu:
        out["cpu_prioritized_draw"] = cpu_replay_draw(1_000_000, lanes, batch)
    return out


def bench_agent(dev, steps=300, capacity=1_000_000, lanes=8):
    """DQN agent gradient steps at batch 32 over a 1M-transition prioritized
    replay (8 lanes of uint8 4x84x84 frames, n-step 3, resident in HBM): each
    step is the agent's own gradient step (ttrl/algos/dqn/agent.py:183-214):
    the prioritized draw on the device assembled straight into the update's
    bound inputs, the captured update with its packed metric read-back, and
    the write-back of the batch's TD errors into the priority table from the
    device.  Also times the draw alone (its call, which waits for the lane
    sums, plus a stream wait for its kernels)."""
    from ttrl_amd.algos.agents import DQNAgent
    from ttrl_amd.algos.dqn import DQNConfig
    from ttrl_amd.buffers import beta_at
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state

    cfg = DQNConfig(lr=6.25e-5, adam_eps=1.5e-4, batch_size=32, prioritized=True, buffer_capacity=capacity,
                    train_freq=1, learning_starts=0)
    agent = DQNAgent(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(6), dev, cfg=cfg, n_envs=lanes, seed=0)
    try:
        agent.online.load_state_dict(he_uniform_qnet_state(agent.online, 1))
        agent.target.copy_from(agent.online)
        rng = np.random.default_rng(11)
        per_call = 512
        frames = rng.integers(0, 256, (per_call, lanes, 4, 84, 84), dtype=np.uint8)
        buf = agent.buffer
        t0 = time.perf_counter()
        for _ in range(buf.per_lane_capacity // per_call + 1):
            buf.add_steps(frames, rng.integers(0, 6, (per_call, lanes)),
                          rng.choice(np.array([-1.0, 0.0, 1.0], np.float32), (per_call, lanes), p=[0.05, 0.9, 0.05]),
                          np.zeros((per_call, lanes), bool))
        cols = np.arange(buf.per_lane_capacity)
        for lane in range(lanes):
            for c0 in range(0, cols.size, 1024):
                cc = cols[c0:c0 + 1024]
                buf.update_priorities(np.full(cc.size, lane), cc, rng.exponential(1.0, cc.size))
        dev.synchronize()
        fill_s = time.perf_counter() - t0
        for _ in range(20):
            agent._gradient_step()
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            agent._gradient_step()
        dev.synchronize()
        step_s = (time.perf_counter() - t0) / steps
        beta = beta_at(agent.priority, agent.learner.update_count)
        t0 = time.perf_counter()
        for _ in range(steps):
            buf.sample(32, beta=beta, out=agent._out)
        dev.synchronize()
        draw_s = (time.perf_counter() - t0) / steps
        return {"gradient_steps_per_s": round(1.0 / step_s, 1), "us_per_step": round(step_s * 1e6, 2),
                "prioritized_draw_us": round(draw_s * 1e6, 2), "capacity": buf.capacity, "lanes": lanes,
                "batch": 32, "fill_seconds": round(fill_s, 2),
                "note": "DQNAgent._gradient_step: device prioritized draw into the bound inputs, captured update "
                        "with the packed metric read-back, device PER write-back"}
    finally:
        agent.close()


def cpu_replay_draw(capacity, lanes, batch, seconds=3.0):
    """The oracle's restatement of the reference's host prioritized draw
    (per-lane cumsum + searchsorted over float64 priorities) and n-step
    assembly, at the same capacity, with one-byte observations so the time is
    the draw's."""
    from oracle.replay import ReplayOracle

    o = ReplayOracle((1,), np.uint8, capacity=capacity, n_envs=lanes, n_step=3, seed=0, alpha=0.6)
    o.pos[:] = 0
    o.full[:] = True
    o.weight[:] = (np.random.default_rng(1).exponential(1.0, o.weight.shape) + 1e-6) ** 0.6
    o.sample(batch, beta=0.4)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds or n < 3:
        o.sample(batch, beta=0.4)
        n += 1
    ms = (time.perf_counter() - t0) / n * 1e3
    return {"capacity": o.cols * lanes, "ms_per_sample": round(ms, 3), "kind": "port",
            "sample": f"{n} prioritized draws of {batch} from the float64 numpy oracle"}


def rppo_step_flops(rows=512, hidden=512, features=512, actions=18) -> float:
    """One recurrent PPO minibatch step: the Nature-CNN trunk's forward,
    weight and input gradients (no input gradient at conv1), the GRU's input
    projection, recurrent GEMMs and their gradients over all timesteps, and
    both heads."""
    trunk = sum(NATURE_MACS[:4])
    per_row = 2 * trunk + (trunk - NATURE_MACS[0])
    per_row += 3 * hidden * (3 * features + 3 * hidden) + 3 * hidden * (actions + 1)
    return 2.0 * rows * per_row


def bench_rppo(dev, updates=3, mode="graph"):
    """Recurrent PPO updates over one resident rollout of 16 envs x 128 steps
    of uint8 4x84x84 frames: sequences of 32, GRU hidden 512, 4 epochs x 4
    minibatches of 512 rows (16 sequences), 18 actions."""
    from ttrl_amd.algos.ppo import PPOConfig, RecurrentConfig, RecurrentPPOLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state, recurrent_ppo_rollout

    cfg = PPOConfig(minibatch_size=512, epochs=4, n_steps=128, step_mode=mode,
                    recurrent=RecurrentConfig(hidden_size=512, seq_len=32))
    learner = RecurrentPPOLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(18), dev, cfg=cfg, seed=0)
    learner.net.load_state_dict(he_uniform_qnet_state(learner.net, 6))
    rollout = recurrent_ppo_rollout(6000, 128, 16, 18, 32, 512)
    steps = learner.load_rollout(rollout)
    learner.run_update(steps)
    dev.synchronize()
    t0 = time.perf_counter()
    for _ in range(updates):
        learner.run_update(steps)
    dev.synchronize()
    dt = (time.perf_counter() - t0) / updates
    flops = rppo_step_flops()
    out = {"unit": "recurrent PPO minibatch steps/s", "value": round(steps / dt, 2), "rows": 512,
           "steps_per_update": steps, "ms_per_update": round(dt * 1e3, 3), "ms_per_step": round(dt / steps * 1e3, 4),
           "flops_per_step": flops, "roofline_frac": flops * steps / dt / PEAK_FP32_MFMA,
           "workload": "recurrent PPO update: 16 envs x 128 steps of uint8 4x84x84, sequences of 32, "
                       "Nature-CNN -> 512 -> GRU(512) -> {18, 1}, 4 epochs x 4 minibatches of 16 sequences"}
    learner.close()
    return out


def dominant_kernel(dev, learner, reps=200):
    """The DQN update's HBM-bound launch (its other launches are MFMA GEMMs or
    latency-bound row kernels, reported per kernel with their MFMA fractions
    beside the update's own FLOP rate), its Adam step, as the update calls it
    (ttrl_adam_step_sources: k_adam_src over the 1,687,296-float parameter
    arena, forming the gradients the update left pending as it reads them and
    updating p, m and v with them without storing the gradients, then
    k_finish_sums: the update count, sum of g^2, loss and mean Q).  One forward and backward of the update's body run on
    the bound batch (not captured) leave those sources pending: the three
    convolutions' split-K partials and the two linear layers' outer products.
    The step is then timed alone on the library's stream with HIP events over
    `reps` calls, each forming the same gradients again and stepping.
    Algorithmic HBM bytes per call: 24 per parameter whose gradient is formed
    in the step (p, m, v read and written), 28 per other parameter (g read
    too), plus the outer products' inputs and output gradients read once;
    the split-K partials of the convolutions' weight gradients are this
    build's own intermediate, reported beside it, not counted."""
    from ttrl_amd import _lib
    from ttrl_amd.engine.pending import take_sources, take_sums

    opt = learner.optimizer
    opt.zero_grad()
    learner._step_fn(learner.inputs)
    sources = take_sources(opt.params)
    sums = take_sums(dev)
    d, arrays = opt._sources_desc(sources, sums)

    def launch():
        dev.call("ttrl_adam_step_sources", C.byref(d))

    for _ in range(10):
        launch()
    dev.synchronize()
    ms = C.c_float(0.0)
    dev.call("ttrl_timer_start")
    for _ in range(reps):
        launch()
    dev.call("ttrl_timer_stop", C.byref(ms))
    dev.synchronize()
    for p in sources:
        p.release()
    sec = ms.value / 1e3 / reps
    outer, partials, formed = 0, 0, 0
    for p in sources:
        s = p.source
        formed += s.rows * s.cols + (-(-s.cols // 4) * 4 if s.db else 0)
        if s.kind == _lib.GRAD_SPLITS:
            partials += 4 * s.splits * (s.rows + (1 if s.db else 0)) * s.cols
        else:
            outer += 4 * s.batch * (s.rows + s.cols)
    n = opt.arena.numel
    kinds = sorted(f"{p.source.rows}x{p.source.cols} {'split-K' if p.source.kind == _lib.GRAD_SPLITS else 'outer'}"
                   for p in sources)
    return {"name": f"ttrl_adam_step_sources: Adam over the {n:,}-float DQN arena forming {len(sources)} pending "
                    f"gradients ({', '.join(kinds)}), batch 32",
            "kernels": ["k_adam_src<false> (the sources' workgroups, then the plain float4s; the formed gradients "
                        "are not stored)", "k_finish_sums (update count, sum of g^2, loss and mean Q)"],
            "seconds": sec, "bytes": 24 * formed + 28 * (n - formed) + outer, "flops": 0.0,
            "formed_params": formed, "outer_operand_bytes": outer, "split_partial_bytes": partials,
            "store_formed_grads": bool(d.store_grads)}


def achievable_peaks(dev, copy_mib=512, reps=10):
    """The box's achievable rates beside the published peaks: a
    device-to-device copy of `copy_mib` MiB (bytes read plus bytes written
    per second, the median of `reps` copies timed one by one with the stream
    timer) and the FP32 matrix rate of back-to-back v_mfma_f32_16x16x4f32
    with no memory traffic (ttrl_mfma_rate, two 256-thread workgroups per
    CU), the median of five launches."""
    from ttrl_amd.engine.tensor import DeviceArray

    n = copy_mib * (1 << 20) // 4
    src, dst = DeviceArray(dev, (n,)), DeviceArray(dev, (n,))
    src.fill(1.0)
    dst.copy_from(src)
    dev.synchronize()
    ms = C.c_float(0.0)
    copies = []
    for _ in range(reps):
        dev.call("ttrl_timer_start")
        dst.copy_from(src)
        dev.call("ttrl_timer_stop", C.byref(ms))
        copies.append(2.0 * n * 4 / (ms.value / 1e3))
    del src, dst
    from ttrl_amd.engine.device import probe_profile

    cus = int(probe_profile(dev).compute_units or 256)
    wgs, iters = 2 * cus, 20000
    out = DeviceArray(dev, (wgs * 256,))
    flops = C.c_double(0.0)
    dev.call("ttrl_mfma_rate", wgs, iters, out.vp, C.byref(flops))  # warm-up
    dev.synchronize()
    rates = []
    for _ in range(5):
        dev.call("ttrl_timer_start")
        dev.call("ttrl_mfma_rate", wgs, iters, out.vp, C.byref(flops))
        dev.call("ttrl_timer_stop", C.byref(ms))
        rates.append(flops.value / (ms.value / 1e3))
    dev.synchronize()
    hbm, mfma = float(np.median(copies)), float(np.median(rates))
    return {"hbm_copy_gbps": round(hbm / 1e9, 1), "hbm_published_gbps": PEAK_HBM / 1e9,
            "hbm_frac_of_published": hbm / PEAK_HBM,
            "mfma_fp32_tflops": round(mfma / 1e12, 2), "mfma_fp32_published_tflops": PEAK_FP32_MFMA / 1e12,
            "mfma_frac_of_published": mfma / PEAK_FP32_MFMA,
            "copy": f"{copy_mib} MiB device-to-device, {reps} copies",
            "mfma": f"{wgs} workgroups x 256 threads x {iters} rounds of 8 independent v_mfma_f32_16x16x4f32"}


def pcie_inclusive(dev, learner, n=100):
    """Updates/s when every update starts from a host batch (numpy arrays in
    pageable memory): the host-to-device copy of the batch is inside the loop."""
    from ttrl_amd.workloads import dqn_batch

    batches = [dqn_batch(4000 + i) for i in range(8)]
    for i in range(5):
        learner.update(batches[i % 8])
    dev.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        learner.update(batches[i % 8])
    dev.synchronize()
    return n / (time.perf_counter() - t0)


def bench_act(dev, dqn, sac, steps=500, lanes_dqn=(1, 8, 16, 32), lanes_sac=(1, 16, 256)):
    """Acting steps/s of the learners' acting networks: one step = host
    observations (pageable numpy) staged into the step's mapped input block,
    the captured forward + fused head-and-decision kernel launched directly,
    the decisions read from its mapped output block (DQN: greedy actions
    before the host epsilon draw; SAC: squashed-Gaussian actions at
    host-drawn noise).  At 32 lanes the DQN step is the batch-32 Q-network
    forward of the deploy path, plus the observations' staging and the
    decisions' read."""
    out = {"dqn": [], "sac": []}
    rng = np.random.default_rng(17)
    for lanes in lanes_dqn:
        frames = [rng.integers(0, 256, (lanes, 4, 84, 84), dtype=np.uint8) for _ in range(8)]
        for i in range(20):
            dqn._acting.decide(frames[i % 8])
        t0 = time.perf_counter()
        for i in range(steps):
            dqn._acting.decide(frames[i % 8])
        dt = time.perf_counter() - t0
        out["dqn"].append({"lanes": lanes, "steps_per_s": round(steps / dt, 1), "us_per_step": round(dt / steps * 1e6, 2)})
    # Config 1 on the GPU: the batch-32 Q-network forward with its frames
    # resident in HBM (an acting graph at 32 lanes over device blocks,
    # replayed back to back, no host copies): forwards/s against the FP32
    # MFMA roofline.  The learner's own acting net keeps its blocks in mapped
    # host memory, which a step reads once; replayed back to back it would
    # read the frames over PCIe every time.
    from ttrl_amd.nets.acting import ActingNet, GreedyDecision

    resident = ActingNet(dqn.online, dqn.obs_spec, dev, width=32, lanes=32, decision=GreedyDecision(), mapped=False)
    try:
        resident.decide(rng.integers(0, 256, (32, 4, 84, 84), dtype=np.uint8))  # captures
        fw = resident._views[32].graphs[False]
        fw.replay_n(50)
        dev.synchronize()
        t0 = time.perf_counter()
        fw.replay_n(steps * 4)
        dev.synchronize()
        dt = (time.perf_counter() - t0) / (steps * 4)
    finally:
        resident.close()
    flops = 2.0 * 32 * sum(NATURE_MACS)
    out["dqn_forward_bs32"] = {"forwards_per_s": round(1.0 / dt, 1), "us_per_forward": round(dt * 1e6, 2),
                               "flops": flops, "roofline_frac": flops / dt / PEAK_FP32_MFMA}
    for lanes in lanes_sac:
        obs = [rng.standard_normal((lanes, 11)).astype(np.float32) for _ in range(8)]
        noise = [rng.standard_normal((lanes, 3)).astype(np.float32) for _ in range(8)]
        for i in range(20):
            sac._acting.decide(obs[i % 8], noise=noise[i % 8])
        t0 = time.perf_counter()
        for i in range(steps):
            sac._acting.decide(obs[i % 8], noise=noise[i % 8])
        dt = time.perf_counter() - t0
        out["sac"].append({"lanes": lanes, "steps_per_s": round(steps / dt, 1), "us_per_step": round(dt / steps * 1e6, 2)})
    return out


def _he(rng, shape, fan, dtype):
    b = np.sqrt(6.0 / fan)
    return rng.uniform(-b, b, shape).astype(dtype)


def _cpu_worker(spec: str) -> int:
    """One CPU measurement in this process, whose BLAS thread count the
    parent set in the environment: spec "kind,dtype,seconds", kind dqn (the
    oracle's DQN update, batch 32), sac (the oracle's SAC update, batch 256)
    or deploy (the oracle's restatement of the reference's numpy deploy
    forward, batch 32 frames).  Prints one JSON line."""
    import oracle
    from oracle import deploy
    from oracle.dqn import dqn_update
    from oracle.nets import QNet
    from oracle.sac import SacParams, sac_update
    from ttrl_amd.workloads import dqn_batch, sac_batch

    kind, dname, seconds = spec.split(",")
    dt = np.float32 if dname == "f32" else np.float64
    rng = np.random.default_rng(0)
    if kind == "dqn":
        net = QNet([(_he(rng, (32, 4, 8, 8), 256, dt), _he(rng, (32,), 256, dt), 4, 0),
                    (_he(rng, (64, 32, 4, 4), 512, dt), _he(rng, (64,), 512, dt), 2, 0),
                    (_he(rng, (64, 64, 3, 3), 576, dt), _he(rng, (64,), 576, dt), 1, 0)],
                   [(_he(rng, (3136, 512), 3136, dt), _he(rng, (512,), 3136, dt)),
                    (_he(rng, (512, 6), 512, dt), _he(rng, (6,), 512, dt))])
        target = net.copy()
        batches = [dqn_batch(3000 + i) for i in range(4)]
        step = lambda i: dqn_update(net, target, batches[i % 4])  # noqa: E731
    elif kind == "sac":
        def mlp(dims):
            return [(_he(rng, (a, b), a, dt), _he(rng, (b,), a, dt)) for a, b in zip(dims[:-1], dims[1:])]
        crit = [mlp((14, 256, 256, 1)) for _ in range(2)]
        P = SacParams(trunk=mlp((11, 256, 256)), mean=mlp((256, 3))[0], log_std=mlp((256, 3))[0], critics=crit,
                      targets=[[(w.copy(), b.copy()) for w, b in c] for c in crit], log_alpha=0.0)
        batches = [sac_batch(4000 + i) for i in range(4)]
        step = lambda i: sac_update(P, batches[i % 4])  # noqa: E731
    else:
        meta = {"obs_shape": [4, 84, 84], "trunk_layers": 1,
                "conv": [{"stride": 4, "padding": 0}, {"stride": 2, "padding": 0}, {"stride": 1, "padding": 0}]}
        arrays = {"conv.0.weight": _he(rng, (32, 4, 8, 8), 256, dt), "conv.0.bias": _he(rng, (32,), 256, dt),
                  "conv.1.weight": _he(rng, (64, 32, 4, 4), 512, dt), "conv.1.bias": _he(rng, (64,), 512, dt),
                  "conv.2.weight": _he(rng, (64, 64, 3, 3), 576, dt), "conv.2.bias": _he(rng, (64,), 576, dt),
                  "trunk.0.weight": _he(rng, (3136, 512), 3136, dt), "trunk.0.bias": _he(rng, (512,), 3136, dt),
                  "head.weight": _he(rng, (512, 6), 512, dt), "head.bias": _he(rng, (6,), 512, dt)}
        frames = rng.integers(0, 256, (32, 4, 84, 84), dtype=np.uint8)
        step = lambda i: deploy.head_rows(meta, arrays, frames)  # noqa: E731
    with oracle.precision(dt):
        step(0)  # warm caches and the BLAS pool
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < float(seconds) or n < 2:
            step(n)
            n += 1
        dt_s = time.perf_counter() - t0
    try:
        from threadpoolctl import threadpool_info
        blas = [{k: i.get(k) for k in ("internal_api", "version", "num_threads")} for i in threadpool_info()
                if i.get("user_api") == "blas"]
    except ImportError:
        blas = []
    print(json.dumps({"n": n, "seconds": dt_s, "rate": n / dt_s, "blas_runtime": blas}), flush=True)
    return 0


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _numpy_blas() -> dict:
    try:
        deps = np.show_config(mode="dicts")["Build Dependencies"]
        return {k: deps[k].get("name") + " " + str(deps[k].get("version")) for k in ("blas", "lapack") if k in deps}
    except Exception:  # the layout of show_config's dict is not a stable API
        return {}


def cpu_baseline(seconds: float):
    """The float64 numpy oracle of the same updates on this host, and the same
    arithmetic in float32 (the GPU path's type): the DQN update, the SAC
    update and the deploy forward, each on every core this process may use
    (threads capped by OMP_NUM_THREADS) and on one, each case in a child
    process so its BLAS starts with that thread count.  `value` is the DQN
    update in float32 on all those cores."""
    import subprocess

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    runs = []
    for kind, secs, unit in (("dqn", seconds / 2, "DQN updates/s"), ("sac", seconds / 4, "SAC updates/s"),
                             ("deploy", seconds / 4, "DQN forwards/s (batch 32)")):
        for dname in ("f32", "f64"):
            for t in (threads, 1):
                env = dict(os.environ)
                for var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS", "BLIS_NUM_THREADS"):
                    env[var] = str(t)
                proc = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--cpu-worker",
                                       f"{kind},{dname},{secs}"], env=env, capture_output=True, text=True,
                                      timeout=600)
                if proc.returncode != 0:
                    raise RuntimeError(f"cpu baseline worker {kind},{dname},{t} failed:\n{proc.stderr[-2000:]}")
                out = json.loads(proc.stdout.strip().splitlines()[-1])
                runs.append({"workload": kind, "dtype": dname, "threads": t, "value": round(out["rate"], 3),
                             "unit": unit, "sample": f"{out['n']} in {out['seconds']:.1f} s",
                             "blas_runtime": out["blas_runtime"]})
    head = next(r for r in runs if r["workload"] == "dqn" and r["dtype"] == "f32" and r["threads"] == threads)
    return {"value": head["value"], "unit": "DQN updates/s", "cores": threads, "kind": "port",
            "sample": f"{head['sample']}: DQN updates (batch 32, 4x84x84 uint8) of the numpy oracle in float32",
            "cpu": _cpu_model(), "logical_cpus": cores, "numpy_blas": _numpy_blas(), "runs": runs}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--ring", type=int, default=32,
                    help="distinct resident batches cycled through (one input slot each in graph mode)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--act-steps", type=int, default=500, help="acting steps timed per lane count (0: skip)")
    ap.add_argument("--ppo-updates", type=int, default=5, help="PPO updates timed (0: skip)")
    ap.add_argument("--replay-reps", type=int, default=200, help="replay samples timed (0: skip)")
    ap.add_argument("--agent-steps", type=int, default=300,
                    help="DQN agent gradient steps timed over a 1M prioritized replay (0: skip)")
    ap.add_argument("--mode", choices=("graph", "eager"), default="graph",
                    help="eager dispatches every kernel from the host (for profilers that cannot trace graphs)")
    ap.add_argument("--cpu-worker", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run five device-to-device copies of MIB MiB (the reference for scaling a "
                         "profiler's FETCH_SIZE / WRITE_SIZE counters to bytes)")
    args = ap.parse_args()
    if args.cpu_worker:
        return _cpu_worker(args.cpu_worker)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): this build has no multi-GPU path; "
              "replicas would shard as independent learners with a periodic parameter all-reduce.",
              file=sys.stderr)
        return 2
    from ttrl_amd.engine.device import open_device

    dev = open_device(0)
    dqn, wall, gpu, nodes, dqn_legs = bench_dqn(dev, args.steps, args.warmup, args.ring, args.mode)
    value = args.steps / wall
    flops = dqn_update_flops(32)
    sac, swall, sgpu, snodes, sac_legs = bench_sac(dev, args.steps, args.warmup, args.ring, args.mode)
    dqn_legs, sac_legs = dqn_legs or {}, sac_legs or {}
    sac_value = args.steps / swall
    sflops = sac_update_flops(256)
    dom = dominant_kernel(dev, dqn)
    achieved = dom["bytes"] / dom["seconds"]
    traffic, digest = adam_step_traffic()
    ppo = bench_ppo(dev, args.ppo_updates, args.mode) if args.ppo_updates > 0 else None
    rppo = bench_rppo(dev, max(1, args.ppo_updates // 2), args.mode) if args.ppo_updates > 0 else None
    replay = bench_replay(dev, args.replay_reps, not args.no_cpu_baseline) if args.replay_reps > 0 else None
    agent = bench_agent(dev, args.agent_steps) if args.agent_steps > 0 and args.mode == "graph" else None
    host_rate = pcie_inclusive(dev, dqn) if args.mode == "graph" else None
    act = bench_act(dev, dqn, sac, args.act_steps) if args.act_steps > 0 and args.mode == "graph" else None
    peaks = achievable_peaks(dev) if args.mode == "graph" else None
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)
    if act is not None and cpu is not None:
        act["cpu_deploy_forward"] = [r for r in cpu["runs"] if r["workload"] == "deploy"]
    line = {
        "metric": "DQN updates/s @bs32, SAC updates/s @bs256 on 1 MI355X; % of roofline",
        "value": round(value, 2),
        "unit": "DQN updates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded uint8 frames, resident in HBM, fresh batch per step)",
        "input_slots": args.ring if args.mode == "graph" else 1,
        "repeats": dqn_legs.get("repeats"),
        "with_metric_read": dqn_legs.get("with_metric_read"),
        "copy_in_each_step": dqn_legs.get("copy_in_each_step"),
        "mode": args.mode,
        "config": {"workload": "DQN learner update: double DQN, n-step 3, PER weights, Nature-CNN 4x84x84 -> 6, "
                               "Huber 1, Adam lr 6.25e-5 eps 1.5e-4", "batch": 32, "graph_nodes": nodes},
        "update_roofline": {"flops_per_update": flops, "achieved_tflops": flops * value / 1e12,
                            "frac": flops * value / PEAK_FP32_MFMA, "gpu_ms_per_step": gpu / args.steps * 1e3},
        "sac": {"value": round(sac_value, 2), "unit": "SAC updates/s", "batch": 256,
                "ms_per_step": round(swall / args.steps * 1e3, 5), "gpu_ms_per_step": sgpu / args.steps * 1e3,
                "graph_nodes": snodes, "flops_per_update": sflops, "roofline_frac": sflops * sac_value / PEAK_FP32_MFMA,
                "repeats": sac_legs.get("repeats"), "with_metric_read": sac_legs.get("with_metric_read"),
                "copy_in_each_step": sac_legs.get("copy_in_each_step")},
        "roofline": {"bound": "hbm", "kernel": dom["name"], "kernels": dom["kernels"], "achieved": achieved / 1e9,
                     "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": achieved / PEAK_HBM,
                     "traffic": traffic, "traffic_source_sha256": digest, "algorithmic_bytes": dom["bytes"],
                     "split_partial_bytes": dom["split_partial_bytes"], "formed_params": dom["formed_params"],
                     "avg_us": dom["seconds"] * 1e6,
                     "achievable_peak": None if peaks is None else peaks["hbm_copy_gbps"],
                     "frac_of_achievable": None if peaks is None else achieved / 1e9 / peaks["hbm_copy_gbps"]},
        "achievable": peaks,
        "pcie_inclusive": None if host_rate is None else {
            "value": round(host_rate, 2), "unit": "DQN updates/s",
            "note": "each update loads a host numpy batch (pageable) through the learner's update(batch)"},
        "ppo": ppo,
        "recurrent_ppo": rppo,
        "replay": replay,
        "agent": agent,
        "act": act,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    if args.copy_calibration > 0:
        from ttrl_amd.engine.tensor import DeviceArray
        n = args.copy_calibration * (1 << 20) // 4
        src, dst = DeviceArray(dev, (n,)), DeviceArray(dev, (n,))
        src.fill(1.0)
        for _ in range(5):
            dst.copy_from(src)
        dev.synchronize()
    dqn.close()
    sac.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
