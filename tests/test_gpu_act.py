"""The acting step on the GPU against the float64 oracle.

Kernels through the C-ABI: `ttrl_q_act` (Q head + first-index argmax),
`ttrl_gaussian_act` (Gaussian head + clamp + squashed sample) and
`ttrl_sac_head_sample` (the same launch in the SAC update, keeping u).  Then the
acting network at lane counts below the width it was built for
(ttrl/nets/acting.py:117-188, the cases of the reference's
tests/hardware/test_acting_width.py), and the agents' `act`
(ttrl/algos/dqn/agent.py:97-119, ttrl/algos/sac/agent.py:111-125).

Tolerances: Q values, means, log-stds, actions and log-densities within rel
1e-5 of the float64 oracle for the single-layer kernels (fp32 sums of at most
a few thousand terms) and rel 1e-4 for whole-network outputs (max abs error
over the tensor relative to its max |value|); argmax actions exact wherever
the top-two gap is decisive (within 1e-4 of the row's scale the device's
choice is adopted).  A narrow view and the full-width net agree within rel
1e-5 rather than bitwise: each batch size has its own GEMM plan, so the K
sums are associated differently.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tests._dqn_helpers import build_learner, qnet_to_oracle
from tests._sac_helpers import build_sac, sac_to_oracle

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _frames(lanes, seed):
    return np.random.default_rng(seed).integers(0, 256, (lanes, 4, 84, 84), dtype=np.uint8)


@pytest.mark.parametrize("B,K,A,bias", [(1, 512, 6, True), (5, 512, 6, True), (16, 3136, 18, True),
                                         (33, 100, 1, False), (7, 64, 32, True), (4, 512, 9, True)])
def test_q_act_kernel_matches_oracle(device, B, K, A, bias):
    from oracle.dqn import select_actions
    from ttrl_amd.engine.tensor import DeviceArray, to_device

    rng = np.random.default_rng(B * 1000 + K + A)
    h = np.maximum(rng.standard_normal((B, K)), 0).astype(np.float32)
    W = (rng.standard_normal((K, A)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(A).astype(np.float32) * 0.1
    if B >= 4:
        h[3] = 0.0  # an all-tie row when there is no bias: first index wins
    dh, dW = to_device(h, device), to_device(W, device)
    db = to_device(b, device) if bias else None
    q = DeviceArray(device, (B, A))
    act = DeviceArray(device, (B,), np.int32)
    for _ in range(2):
        device.call("ttrl_q_act", B, K, A, dh.ptr, dW.ptr, None if db is None else db.ptr, q.ptr, act.ptr)
    ref = h.astype(np.float64) @ W.astype(np.float64) + (b.astype(np.float64) if bias else 0.0)
    assert _rel(q.numpy(), ref) < 1e-5
    got = act.numpy().astype(np.int64)
    want, _ = select_actions(ref, got)
    assert np.array_equal(got, want)
    if B >= 4 and not bias:
        assert got[3] == 0


@pytest.mark.parametrize("B,K,d,det", [(1, 256, 3, False), (7, 256, 3, False), (16, 64, 1, False),
                                        (256, 256, 3, False), (9, 128, 16, False), (16, 256, 3, True)])
def test_gaussian_act_kernel_matches_oracle(device, B, K, d, det):
    from oracle import gaussian
    from ttrl_amd.engine.tensor import DeviceArray, to_device

    rng = np.random.default_rng(B + K * 7 + d)
    h = np.maximum(rng.standard_normal((B, K)), 0).astype(np.float32)
    Wm = (rng.standard_normal((K, d)) / np.sqrt(K)).astype(np.float32)
    Ws = (rng.standard_normal((K, d)) / np.sqrt(K)).astype(np.float32)
    bm = (rng.standard_normal(d) * 0.1).astype(np.float32)
    bs = (rng.standard_normal(d) * 0.1).astype(np.float32)
    # Clamp bounds [-5, 1] rather than the default [-20, 2]: at log_std = -20
    # the fp32 z = (u - mean) / sigma loses the noise to cancellation (as the
    # reference's own fp32 sample does), which a float64 oracle would flag.
    lo, hi = -5.0, 1.0
    bs[0] = 40.0  # drives column 0 of log_std into the upper clamp
    if d > 1:
        bs[1] = -60.0  # and column 1 into the lower one
    noise = rng.standard_normal((B, d)).astype(np.float32)
    lo_b = rng.uniform(-3, -1, d).astype(np.float32)
    hi_b = rng.uniform(1, 3, d).astype(np.float32)
    centre = ((hi_b + lo_b) * 0.5).astype(np.float32)
    half = ((hi_b - lo_b) * 0.5).astype(np.float32)
    log_det = float(np.sum(np.log(half.astype(np.float64))))
    dev = {k: to_device(v, device) for k, v in dict(h=h, Wm=Wm, Ws=Ws, bm=bm, bs=bs, noise=noise, c=centre,
                                                       hw=half).items()}
    head = DeviceArray(device, (B, 2 * d))
    action = DeviceArray(device, (B, d))
    logp = DeviceArray(device, (B,))
    device.call("ttrl_gaussian_act", B, K, d, dev["h"].ptr, dev["Wm"].ptr, dev["bm"].ptr, dev["Ws"].ptr,
                dev["bs"].ptr, C.c_float(lo), C.c_float(hi), dev["noise"].ptr, dev["c"].ptr, dev["hw"].ptr,
                C.c_float(log_det), int(det), head.ptr, action.ptr, logp.ptr)
    h64 = h.astype(np.float64)
    mean = h64 @ Wm.astype(np.float64) + bm
    log_std = np.clip(h64 @ Ws.astype(np.float64) + bs, lo, hi)
    assert _rel(head.numpy()[:, :d], mean) < 1e-5
    assert _rel(head.numpy()[:, d:], log_std) < 1e-5
    if det:
        assert _rel(action.numpy(), centre + half * np.tanh(mean)) < 1e-5
        assert np.all(logp.numpy() == 0.0)
    else:
        a_ref, lp_ref, _u = gaussian.sample(mean, log_std, noise, centre, half, log_det)
        assert _rel(action.numpy(), a_ref) < 1e-5
        assert _rel(logp.numpy(), lp_ref) < 1e-5


@pytest.mark.parametrize("rows,K,d", [(512, 256, 3), (37, 100, 1), (9, 128, 16)])
def test_sac_head_sample_matches_oracle_and_acting_launch(device, rows, K, d):
    """ttrl_sac_head_sample (the learner's policy head and sample) against
    the float64 oracle at rel 1e-5, with the pre-squash u the sample's
    backward takes; head, action and logp bit-identical to
    ttrl_gaussian_act's, the same kernel."""
    from oracle import gaussian
    from ttrl_amd import _lib
    from ttrl_amd.engine.tensor import DeviceArray, to_device

    rng = np.random.default_rng(rows * 3 + K + d)
    x = np.maximum(rng.standard_normal((rows, K)), 0).astype(np.float32)
    Wm = (rng.standard_normal((K, d)) / np.sqrt(K)).astype(np.float32)
    Ws = (rng.standard_normal((K, d)) / np.sqrt(K)).astype(np.float32)
    bm = (rng.standard_normal(d) * 0.1).astype(np.float32)
    bs = (rng.standard_normal(d) * 0.1).astype(np.float32)
    lo, hi = -5.0, 1.0
    bs[0] = 40.0  # log_std column 0 in the upper clamp
    noise = rng.standard_normal((rows, d)).astype(np.float32)
    centre = rng.uniform(-0.5, 0.5, d).astype(np.float32)
    half = rng.uniform(0.5, 2.0, d).astype(np.float32)
    log_det = float(np.sum(np.log(half.astype(np.float64))))
    dv = {k: to_device(v, device) for k, v in dict(x=x, Wm=Wm, Ws=Ws, bm=bm, bs=bs, noise=noise, c=centre,
                                                      hw=half).items()}
    out = {k: DeviceArray(device, shape) for k, shape in (("head", (rows, 2 * d)), ("action", (rows, d)),
                                                          ("logp", (rows,)), ("u", (rows, d)))}
    desc = _lib.SacHeadDesc()
    desc.rows, desc.K, desc.d = rows, K, d
    desc.x, desc.W1, desc.b1, desc.W2, desc.b2 = (dv[k].ptr for k in ("x", "Wm", "bm", "Ws", "bs"))
    desc.lo, desc.hi = lo, hi
    desc.noise, desc.centre, desc.half_width, desc.log_det = dv["noise"].ptr, dv["c"].ptr, dv["hw"].ptr, log_det
    desc.head, desc.action, desc.logp, desc.u = (out[k].ptr for k in ("head", "action", "logp", "u"))
    device.call("ttrl_sac_head_sample", C.byref(desc))
    x64 = x.astype(np.float64)
    mean = x64 @ Wm.astype(np.float64) + bm
    log_std = np.clip(x64 @ Ws.astype(np.float64) + bs, lo, hi)
    a_ref, lp_ref, u_ref = gaussian.sample(mean, log_std, noise, centre, half, log_det)
    got = {k: v.numpy() for k, v in out.items()}
    assert _rel(got["head"][:, :d], mean) < 1e-5
    assert _rel(got["head"][:, d:], log_std) < 1e-5
    assert _rel(got["action"], a_ref) < 1e-5
    assert _rel(got["logp"], lp_ref) < 1e-5
    assert _rel(got["u"], u_ref) < 1e-5
    act = {k: DeviceArray(device, out[k].shape) for k in ("head", "action", "logp")}
    device.call("ttrl_gaussian_act", rows, K, d, dv["x"].ptr, dv["Wm"].ptr, dv["bm"].ptr, dv["Ws"].ptr,
                dv["bs"].ptr, C.c_float(lo), C.c_float(hi), dv["noise"].ptr, dv["c"].ptr, dv["hw"].ptr,
                C.c_float(log_det), 0, act["head"].ptr, act["action"].ptr, act["logp"].ptr)
    for k in act:
        assert np.array_equal(act[k].numpy(), got[k]), k
    desc.d = 17
    with pytest.raises(ValueError, match="at most 16 action dimensions"):
        device.call("ttrl_sac_head_sample", C.byref(desc))


@pytest.mark.parametrize("mode", ["graph", "eager"])
def test_acting_net_matches_deploy_forward_and_full_width(device, mode):
    from oracle.nets import qnet_forward
    from oracle.dqn import select_actions
    from ttrl_amd.nets.acting import ActingNet, GreedyDecision
    from ttrl_amd.spaces import ObsSpec

    learner, online, _ = build_learner(device, seed=3, batch=8)
    onet = qnet_to_oracle(online)
    acting = ActingNet(learner.online, ObsSpec.image((4, 84, 84)), device, width=8, lanes=2,
                       decision=GreedyDecision(), mode=mode)
    try:
        for lanes, seed in ((2, 1), (8, 2), (1, 3), (2, 4)):
            frames = _frames(lanes, seed)
            out = acting.decide(frames)
            q_ref, _ = qnet_forward(onet, frames)
            assert out["q"].shape == (lanes, 6) and out["actions"].dtype == np.int32
            assert _rel(out["q"], q_ref) < 1e-4
            want, _ = select_actions(q_ref, out["actions"])
            assert np.array_equal(out["actions"].astype(np.int64), want)
            # The reference surface: the eager forward at the lane count.
            eager_q = acting(frames).numpy().reshape(lanes, 6)
            assert _rel(eager_q, out["q"]) < 1e-5
        # A narrow view against the full-width network on the same frames.
        frames = _frames(8, 9)
        wide = acting.decide(frames)["q"]
        narrow = acting.decide(frames[:2])["q"]
        assert _rel(narrow, wide[:2]) < 1e-5
    finally:
        acting.close()
        learner.close()


def test_acting_graph_sees_parameter_updates(device):
    from oracle.nets import qnet_forward
    from ttrl_amd.nets.acting import ActingNet, GreedyDecision
    from ttrl_amd.spaces import ObsSpec

    learner, online, _ = build_learner(device, seed=4, batch=8)
    acting = ActingNet(learner.online, ObsSpec.image((4, 84, 84)), device, width=8, lanes=2,
                       decision=GreedyDecision())
    try:
        frames = _frames(2, 5)
        before = acting.decide(frames)["q"]
        conv = learner.online.encoder.layers[0]
        conv.load_weight_numpy(conv.weight_numpy() * 0.5)
        after = acting.decide(frames)["q"]
        assert not np.array_equal(before, after)
        state = learner.online.state_dict()
        q_ref, _ = qnet_forward(qnet_to_oracle(state), frames)
        assert _rel(after, q_ref) < 1e-4
    finally:
        acting.close()
        learner.close()


def test_a_width_past_the_network_batch_is_refused(device):
    from ttrl_amd.nets.acting import ActingNet, GreedyDecision
    from ttrl_amd.spaces import ObsSpec

    learner, _, _ = build_learner(device, seed=5, batch=8)
    acting = ActingNet(learner.online, ObsSpec.image((4, 84, 84)), device, width=8, lanes=2,
                       decision=GreedyDecision())
    try:
        with pytest.raises(ValueError, match="at most 8 observations"):
            acting.decide(_frames(9, 6))
        with pytest.raises(ValueError, match="uint8"):
            acting.decide(_frames(2, 6).astype(np.float32))
    finally:
        acting.close()
        learner.close()


def test_dqn_act_is_epsilon_greedy_in_the_reference_order(device):
    from oracle.act import dqn_act, epsilon
    from ttrl_amd.algos.dqn import DQNConfig, DQNLearner
    from ttrl_amd.spaces import ActionSpec, ObsSpec
    from ttrl_amd.workloads import he_uniform_qnet_state

    cfg = DQNConfig(batch_size=16, eps_start=0.5, eps_end=0.1, eps_decay_frames=40, eval_epsilon=0.05)
    learner = DQNLearner(ObsSpec.image((4, 84, 84)), ActionSpec.discrete(6), device, cfg=cfg, seed=7, n_envs=4)
    try:
        state = he_uniform_qnet_state(learner.online, 70)
        learner.online.load_state_dict(state)
        onet = qnet_to_oracle(state)
        rng = np.random.default_rng(7)
        frames_seen = 0
        for step in range(12):
            frames = _frames(4, 100 + step)
            eps = epsilon(frames_seen, 0.5, 0.1, 40)
            assert abs(learner.epsilon() - eps) < 1e-12
            got = learner.act(frames)
            # The oracle consumes the same stream; adopt the device's greedy
            # choice only on near-ties.
            greedy_dev = learner._acting.decide(frames)["actions"]
            want, _q, _g, _ = dqn_act(onet, frames, eps=eps, rng=rng, device_greedy=greedy_dev)
            assert got.dtype == np.int64 and np.array_equal(got, want)
            frames_seen += 4
            assert learner.frame_count == frames_seen
        # Evaluation acting draws from its own stream and leaves the clock.
        eval_rng = np.random.default_rng(7).spawn(1)[0]
        frames = _frames(3, 999)
        got = learner.act(frames, deterministic=True)
        greedy_dev = learner._acting.decide(frames)["actions"]
        want, _q, _g, _ = dqn_act(onet, frames, eps=0.05, rng=eval_rng, device_greedy=greedy_dev)
        assert np.array_equal(got, want)
        assert learner.frame_count == frames_seen
    finally:
        learner.close()


def test_sac_act_matches_oracle(device):
    from oracle.act import sac_act

    learner, pol, crit = build_sac(device, seed=8, batch=32)
    try:
        P = sac_to_oracle(pol, crit, crit, 0.0)
        scale = learner.scale
        rng = np.random.default_rng(8)
        obs_rng = np.random.default_rng(80)
        learner.n_envs = 16
        learner._rng = np.random.default_rng(8)
        for lanes in (16, 5, 16):
            obs = obs_rng.standard_normal((lanes, 11)).astype(np.float32)
            got = learner.act(obs)
            a_ref, _lp, _m, _ls = sac_act(P, obs, rng=rng, centre=scale.centre, half_width=scale.half_width,
                                         log_det=scale.log_det)
            assert got.shape == (lanes, 3) and got.dtype == np.float32
            assert _rel(got, a_ref) < 1e-4
        obs = obs_rng.standard_normal((7, 11)).astype(np.float32)
        frames_before = learner.frame_count
        got = learner.act(obs, deterministic=True)
        a_ref, _lp, _m, _ls = sac_act(P, obs, deterministic=True, centre=scale.centre,
                                     half_width=scale.half_width, log_det=scale.log_det)
        assert _rel(got, a_ref) < 1e-4
        assert learner.frame_count == frames_before
        out = learner._acting.decide(obs, deterministic=True)
        assert np.all(out["logp"] == 0.0)
        # Stochastic log-density of the sample against the oracle's.
        noise = rng.standard_normal((7, 3))
        out = learner._acting.decide(obs, noise=noise)
        from oracle import gaussian
        from oracle.sac import policy_forward
        mean, _raw, log_std, _h, _a = policy_forward(P, obs.astype(np.float64))
        a_ref, lp_ref, _u = gaussian.sample(mean, log_std, noise.astype(np.float32), scale.centre,
                                            scale.half_width, scale.log_det)
        assert _rel(out["action"], a_ref) < 1e-4
        assert _rel(out["logp"], lp_ref) < 1e-4
    finally:
        learner.close()


def test_direct_replay_gives_the_graph_launch_bits(device):
    """An acting step replayed as direct launches of its kernels
    (ttrl_graph_set_direct, the ActingNet default) gives the same bits as
    the same captured graph launched whole, for a greedy Nature-CNN step and
    a squashed-Gaussian step; so does a step whose input and output blocks
    are device memory with copies either way, against the default's mapped
    host blocks the kernels read and write in place; a graph with a node
    other than a kernel is refused."""
    from ttrl_amd.engine.tensor import DeviceArray
    from ttrl_amd.engine.trace import capture
    from ttrl_amd.nets.acting import ActingNet, GreedyDecision
    from ttrl_amd.spaces import ObsSpec

    learner, _, _ = build_learner(device, seed=6, batch=8)
    acting = ActingNet(learner.online, ObsSpec.image((4, 84, 84)), device, width=8, lanes=3,
                       decision=GreedyDecision())
    try:
        for lanes, seed in ((3, 11), (8, 12)):
            frames = _frames(lanes, seed)
            direct = acting.decide(frames)
            w = acting._view(lanes)
            for g in w.graphs.values():
                g.set_direct(False)
            whole = acting.decide(frames)
            for g in w.graphs.values():
                g.set_direct(True)
            assert np.array_equal(direct["q"], whole["q"]) and np.array_equal(direct["actions"], whole["actions"])
        copied = ActingNet(learner.online, ObsSpec.image((4, 84, 84)), device, width=8, lanes=3,
                           decision=GreedyDecision(), direct=False, mapped=False)
        try:
            for lanes, seed in ((3, 13), (8, 14), (3, 15)):
                frames = _frames(lanes, seed)
                a, b = acting.decide(frames), copied.decide(frames)
                assert np.array_equal(a["q"], b["q"]) and np.array_equal(a["actions"], b["actions"])
        finally:
            copied.close()
    finally:
        acting.close()
        learner.close()

    sac, _, _ = build_sac(device, seed=9, batch=32)
    try:
        obs = np.random.default_rng(90).standard_normal((5, 11)).astype(np.float32)
        noise = np.random.default_rng(91).standard_normal((5, 3))
        direct = sac._acting.decide(obs, noise=noise)
        w = sac._acting._view(5)
        for g in w.graphs.values():
            g.set_direct(False)
        whole = sac._acting.decide(obs, noise=noise)
        for k in direct:
            assert np.array_equal(direct[k], whole[k]), k
    finally:
        sac.close()

    a = DeviceArray(device, (64,))
    b = DeviceArray(device, (64,))
    trace, _ = capture(device, lambda: b.copy_from(a))  # a copy node, not a kernel
    try:
        with pytest.raises(ValueError, match="nodes other than kernels"):
            trace.set_direct(True)
    finally:
        trace.close()
