"""PPO's device-side arithmetic behind the reference's interfaces.

compute_gae            RolloutBuffer.compute_gae (ttrl/buffers/rollout.py:195-226):
                       one lane per env, reverse scan, on the device
normalize_advantages   the minibatch advantage normalisation
                       (ttrl/buffers/rollout.py:269-270)
objective              the clipped-ratio objective with the categorical head's
                       log-prob and entropy (ttrl/algos/ppo/loss.py:42-83,
                       ttrl/algos/ppo/policy.py:64-76) as one fused tape node
                       whose backward writes d loss / d logits and d loss /
                       d values
clip_grad_norm         the global-norm clip (ttrl/algos/grads.py:13-43) over a
                       flat gradient arena, with no host read, so it can sit
                       inside a captured update

All of it runs on libttrl_hip; there is no host fallback.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.algos.state import TOWERS_PPO, assemble, from_reference_keys, to_reference_keys, validate
from ttrl_amd.engine.autograd import Tensor, _detached, _needs
from ttrl_amd.engine.optim import Adam
from ttrl_amd.engine.tensor import DeviceArray, arena_of, bound_block, to_device
from ttrl_amd.engine.trace import capture

__all__ = ["PPOConfig", "PPOLearner", "PPOLossConfig", "compute_gae", "normalize_advantages", "objective",
           "objective_packed", "clip_grad_norm", "clip_grad_norm_device"]


def _dev(x, device, dtype=np.float32) -> DeviceArray:
    if isinstance(x, Tensor):
        return x.data
    if isinstance(x, DeviceArray):
        return x
    return to_device(np.ascontiguousarray(np.asarray(x, dtype)), device, dtype)


def compute_gae(device, rewards, values, dones, last_values, gamma: float, lam: float, valid=None):
    """-> (advantages, returns) as [T, N] device arrays.

    rewards, values, dones (and valid) are time-major [T, N]; last_values is
    the critic's value after the last step, [N].  Host arrays are uploaded;
    device arrays are used in place.
    """
    r = _dev(rewards, device)
    if len(r.shape) != 2:
        raise ValueError(f"compute_gae: rewards must be [T, N], got shape {r.shape}")
    T, N = (int(d) for d in r.shape)
    arrays = {"values": _dev(values, device), "dones": _dev(dones, device)}
    if valid is not None:
        arrays["valid"] = _dev(valid, device)
    for name, a in arrays.items():
        if tuple(a.shape) != (T, N):
            raise ValueError(f"compute_gae: {name} has shape {a.shape}, expected {(T, N)}")
    lv = _dev(last_values, device)
    if lv.numel != N:
        raise ValueError(f"compute_gae: last_values must have {N} entries, got {lv.numel}")
    adv = DeviceArray(device, (T, N))
    ret = DeviceArray(device, (T, N))
    device.call("ttrl_gae", T, N, r.vp, arrays["values"].vp, arrays["dones"].vp,
                arrays["valid"].vp if "valid" in arrays else None, lv.vp, C.c_double(gamma), C.c_double(lam),
                adv.vp, ret.vp)
    return adv, ret


def normalize_advantages(device, advantages, valid=None, eps: float = 1e-8):
    """-> (normalised advantages, stats [mean, std]) as device arrays."""
    a = _dev(advantages, device)
    out = DeviceArray(device, a.shape)
    stats = DeviceArray(device, (2,))
    v = None if valid is None else _dev(valid, device)
    if v is not None and v.numel != a.numel:
        raise ValueError(f"normalize_advantages: valid has {v.numel} entries, advantages {a.numel}")
    device.call("ttrl_normalize_advantages", a.vp, None if v is None else v.vp, C.c_long(a.numel),
                C.c_float(eps), out.vp, stats.vp)
    return out, stats


@dataclass(frozen=True)
class PPOLossConfig:
    """The objective's coefficients (ttrl/algos/ppo/config.py:75-78)."""

    clip_eps: float = 0.1
    value_clip_eps: float = 0.1
    value_coef: float = 0.5
    entropy_coef: float = 0.01

    def __post_init__(self):
        if not self.clip_eps > 0.0:
            raise ValueError(f"PPOLossConfig: clip_eps must be > 0, got {self.clip_eps}")
        if not self.value_clip_eps > 0.0:
            raise ValueError(f"PPOLossConfig: value_clip_eps must be > 0, got {self.value_clip_eps}")


def objective(policy_out: Tensor, value: Tensor, batch, cfg: PPOLossConfig, valid=None):
    """`(loss, parts, new_logp)` for one minibatch, as ttrl/algos/ppo/loss.py:42-83.

    policy_out: logits [B, A]; value: [B, 1]; `batch` carries `actions`,
    `old_logp`, `advantages`, `returns` and `values` (host arrays or device
    arrays of B entries).  `valid` ([B], optional) gives the masked mean of
    the recurrent path (masked_mean, loss.py:27-39); without it every row
    counts.  `loss` is a (1, 1) tape node differentiable in policy_out and
    value; `parts` holds detached policy_loss, value_loss and entropy.
    """
    dev = policy_out.device
    if len(policy_out.shape) != 2:
        raise ValueError(f"objective: policy_out must be [B, A], got {policy_out.shape}")
    B, A = (int(d) for d in policy_out.shape)
    if value.data.numel != B:
        raise ValueError(f"objective: value has {value.data.numel} entries, expected {B}")

    def field(name, dtype=np.float32):
        x = batch[name] if isinstance(batch, dict) else getattr(batch, name)
        arr = _dev(np.asarray(x).reshape(-1) if not isinstance(x, (DeviceArray, Tensor)) else x, dev, dtype)
        if arr.numel != B:
            raise ValueError(f"objective: batch.{name} has {arr.numel} entries, expected {B}")
        return arr

    actions = field("actions", np.int32)
    old_logp, adv, ret, old_v = (field(n) for n in ("old_logp", "advantages", "returns", "values"))
    w = None if valid is None else _dev(valid, dev)
    out4 = DeviceArray(dev, (4,))
    new_logp = DeviceArray(dev, (B, 1))
    dlogits = DeviceArray(dev, (B, A))
    dvalue = DeviceArray(dev, tuple(int(d) for d in value.shape))
    dev.call("ttrl_ppo_loss", B, A, policy_out.data.vp, actions.vp, old_logp.vp, adv.vp, ret.vp, old_v.vp,
             value.data.vp, None if w is None else w.vp, C.c_float(cfg.clip_eps), C.c_float(cfg.value_clip_eps),
             C.c_float(cfg.value_coef), C.c_float(cfg.entropy_coef), out4.vp, new_logp.vp, dlogits.vp, dvalue.vp)
    loss_arr = out4.view(0, (1, 1))
    parts = {"policy_loss": Tensor(out4.view(1, (1, 1))), "value_loss": Tensor(out4.view(2, (1, 1))),
             "entropy": Tensor(out4.view(3, (1, 1)))}
    if not _needs(policy_out, value):
        return _detached(loss_arr), parts, Tensor(new_logp)
    loss = Tensor(loss_arr, True, (policy_out, value), "ppo_objective")

    def _backward(grad):
        from ttrl_amd.engine.ops import _kernels as K

        scale = None if grad.unit else grad.reshape((1, 1))
        for t, g in ((policy_out, dlogits), (value, dvalue)):
            if t.requires_grad:
                t._accumulate(g if scale is None else K.binary("mul", g, scale))

    loss._backward = _backward
    return loss, parts, Tensor(new_logp)


def objective_packed(head: Tensor, mb: dict, cfg, out5: DeviceArray, new_logp: DeviceArray,
                     valid: DeviceArray | None = None) -> Tensor:
    """The objective over the fused head's packed [logits | value] rows, as
    one tape node (ttrl/algos/ppo/loss.py:42-83).  `mb` holds the minibatch's
    device arrays `actions` (int32), `old_logp`, `advantages`, `returns`,
    `values`; out5 receives {loss, policy_loss, value_loss, entropy,
    approx_kl} and new_logp the rows' log-probs.  The loss is the (1, 1)
    view out5[0]."""
    dev = head.device
    B, N = (int(d) for d in head.shape)
    A = N - 1
    dhead = DeviceArray(dev, (B, N))
    dev.call("ttrl_ppo_loss_packed", B, A, head.data.vp, mb["actions"].vp, mb["old_logp"].vp,
             mb["advantages"].vp, mb["returns"].vp, mb["values"].vp, None if valid is None else valid.vp,
             C.c_float(cfg.clip_eps),
             C.c_float(cfg.value_clip_eps), C.c_float(cfg.value_coef), C.c_float(cfg.entropy_coef), out5.vp,
             new_logp.vp, dhead.vp)
    loss_arr = out5.view(0, (1, 1))
    if not _needs(head):
        return _detached(loss_arr)
    loss = Tensor(loss_arr, True, (head,), "ppo_objective")

    def _backward(grad):
        from ttrl_amd.engine.ops import _kernels as K

        head._accumulate(dhead if grad.unit else K.binary("mul", dhead, grad.reshape((1, 1))))

    loss._backward = _backward
    return loss


def clip_grad_norm_device(grad: DeviceArray, max_norm: float) -> DeviceArray:
    """Clip one flat gradient buffer in place; -> the norm before clipping,
    as a (1,) device array (readable after the update)."""
    if not max_norm > 0.0:
        raise ValueError(f"clip_grad_norm: max_norm must be > 0, got {max_norm}")
    dev = grad.dev
    sq = DeviceArray(dev, (1,))
    norm = DeviceArray(dev, (1,))
    dev.call("ttrl_clip_grad_norm", grad.vp, C.c_long(grad.numel), C.c_float(max_norm), sq.vp, norm.vp)
    return norm


def clip_grad_norm(params, max_norm: float) -> float:
    """Scale every gradient so their global L2 norm is at most `max_norm`;
    returns the norm before clipping (ttrl/algos/grads.py:26-43).  The
    parameters must be exactly one arena's, each holding this step's
    gradient in its slot."""
    params = list(params)
    arena = arena_of(params)
    if arena is None:
        raise ValueError("clip_grad_norm: the parameters must be exactly one ParamArena's tensors, in order")
    if any(p.grad is None for p in params):
        raise RuntimeError("clip_grad_norm: every parameter of the arena needs this step's gradient")
    from ttrl_amd.engine.pending import settle
    settle(params)
    norm = clip_grad_norm_device(arena.grad, max_norm)
    return float(norm.numpy()[0])


# ------------------------------------------------------------ the learner ---

@dataclass(frozen=True)
class RecurrentConfig:
    """The memory's settings (ttrl/algos/ppo/config.py:21-65)."""

    hidden_size: int = 128
    seq_len: int = 16

    def __post_init__(self):
        if self.hidden_size < 1:
            raise ValueError(f"RecurrentConfig: hidden_size must be >= 1, got {self.hidden_size}")
        if self.seq_len < 2:
            raise ValueError(f"RecurrentConfig: seq_len must be >= 2, got {self.seq_len}")


@dataclass(frozen=True)
class PPOConfig:
    """Learner-side fields of ttrl/algos/ppo/config.py:67-120, plus the Adam
    epsilon (the engine default 1e-8, ttrl/algos/ppo/agent.py:81)."""

    lr: float = 2.5e-4
    adam_eps: float = 1e-8
    gamma: float = 0.99
    lam: float = 0.95
    n_steps: int = 128
    minibatch_size: int = 32
    epochs: int = 4
    clip_eps: float = 0.1
    value_clip_eps: float = 0.1
    value_coef: float = 0.5
    entropy_coef: float = 0.01
    max_grad_norm: float = 0.5
    normalize_adv: bool = True
    anneal_lr: bool = False
    total_frames: int | None = None
    step_mode: str = "graph"
    encoder: str = "auto"
    recurrent: RecurrentConfig | None = None

    def __post_init__(self):
        if self.lr <= 0 or self.adam_eps <= 0:
            raise ValueError("PPOConfig: lr and adam_eps must be > 0")
        if self.recurrent is not None and self.minibatch_size % self.recurrent.seq_len:
            raise ValueError(f"PPOConfig: minibatch_size={self.minibatch_size} is not a multiple of "
                             f"seq_len={self.recurrent.seq_len}; a recurrent minibatch is a whole number of "
                             f"sequences")
        if not 0.0 < self.gamma <= 1.0 or not 0.0 <= self.lam <= 1.0:
            raise ValueError(f"PPOConfig: need 0 < gamma <= 1 and 0 <= lam <= 1, got {self.gamma}, {self.lam}")
        if self.n_steps < 1 or self.minibatch_size < 1 or self.epochs < 1:
            raise ValueError("PPOConfig: n_steps, minibatch_size and epochs must be >= 1")
        if not (self.clip_eps > 0 and self.value_clip_eps > 0 and self.max_grad_norm > 0):
            raise ValueError("PPOConfig: clip_eps, value_clip_eps and max_grad_norm must be > 0")
        if self.step_mode not in ("eager", "graph"):
            raise ValueError(f"PPOConfig: step_mode must be 'eager' or 'graph', got {self.step_mode!r}")
        if self.anneal_lr and not self.total_frames:
            raise ValueError("PPOConfig: anneal_lr needs total_frames")
        if self.anneal_lr and self.step_mode == "graph":
            raise ValueError("PPOConfig: the learning rate is a constant of the captured minibatch step; "
                             "anneal_lr needs step_mode='eager'")


class _Resident:
    """One rollout of T x N transitions resident in HBM, flattened time-major
    (row t * N + n, the reference's reshape order), with the shuffled index
    table of every minibatch of one update and the per-step metric ring."""

    def __init__(self, device, obs_spec, T: int, N: int, cfg: PPOConfig, extra=(), steps_per_epoch=None):
        rows = T * N
        self.T, self.N, self.rows = T, N, rows
        mb = cfg.minibatch_size
        per_epoch = rows // mb if steps_per_epoch is None else steps_per_epoch
        self.table_len = cfg.epochs * per_epoch * mb
        if obs_spec.kind == "image":
            frames = np.zeros((rows,) + tuple(obs_spec.shape), np.uint8)
        else:
            frames = np.zeros((rows, obs_spec.size), np.float32)
        z = np.zeros(rows, np.float32)
        specs = [("obs", frames), ("actions", np.zeros(rows, np.int32)), ("logp", z), ("values", z),
                 ("rewards", z), ("dones", z), ("valid", z), ("last_values", np.zeros(N, np.float32)),
                 ("idx", np.zeros(max(self.table_len, 1), np.int32))] + list(extra)
        self.host, self.block = bound_block(device, specs)
        self.image = np.zeros(self.block.nbytes, np.uint8)
        self.advantages = DeviceArray(device, (rows,))
        self.returns = DeviceArray(device, (rows,))
        self.adv_norm = DeviceArray(device, (rows,))
        self.slots = cfg.epochs * per_epoch
        self.ring = DeviceArray(device, (max(self.slots, 1), len(PPOLearner.METRICS)))

    def stage(self, name: str, array) -> None:
        view = self.host[name]
        arr = np.ascontiguousarray(array, dtype=view.dtype)
        if arr.size != view.numel:
            raise ValueError(f"PPO rollout field {name!r}: {arr.shape} does not fit {view.shape}")
        off = view.offset - self.block.offset
        self.image[off:off + arr.nbytes] = arr.reshape(-1).view(np.uint8)


class PPOLearner:
    """The PPO update (ttrl/algos/ppo/learn.py:46-112) on a shared-trunk
    actor-critic (ttrl/nets/build.py:95-117).

    `update(rollout)` uploads one rollout (time-major [T, N] fields plus the
    frames) into a resident HBM block in one copy, runs GAE and the advantage
    normalisation on the device, and then every minibatch step of every
    epoch: gather by index from the resident rollout, trunk forward, the
    fused [logits | value] head, the fused objective, backward, global-norm
    clip, Adam, and the step's metrics into a device ring.  In graph mode the
    minibatch step is one captured graph replayed epochs x minibatches times
    back to back (a device counter selects the minibatch); the metrics are
    read once per update.  The shuffles are the reference's: one
    `rng.permutation` of the valid rows per epoch from a generator seeded
    with `seed`, trailing partial minibatch dropped.
    """

    METRICS = ("loss", "policy_loss", "value_loss", "entropy", "approx_kl", "grad_norm")

    def __init__(self, obs_spec, action_spec, device, *, cfg: PPOConfig = PPOConfig(), seed: int | None = None):
        if action_spec.kind != "discrete":
            raise ValueError(f"PPOLearner supports discrete actions only, got {action_spec.kind!r}")
        self.cfg = cfg
        self.device = device
        self.obs_spec, self.action_spec = obs_spec, action_spec
        if seed is not None:
            np.random.seed(seed)
        self.net = self._build_net()
        self.params = list(self.net.parameters())
        self.optimizer = Adam(self.params, lr=cfg.lr, eps=cfg.adam_eps)
        # Each convolution's weight-gradient split-K partials wait in a
        # gradient bank of the device context; the step forms them all in one
        # launch when it settles the gradients before the clip.
        from ttrl_amd.engine.conv import Conv2d
        from ttrl_amd.nets.acting import _walk_modules

        convs = [m for _, m in _walk_modules(self.net) if isinstance(m, Conv2d)]
        for bank, conv in enumerate(convs[:4]):
            conv.defer_bank = bank
        self._rng = np.random.default_rng(seed)
        self.frame_count = 0
        self.update_count = 0
        mb = cfg.minibatch_size
        if obs_spec.kind == "image":
            obs = np.zeros((mb,) + tuple(obs_spec.shape), np.uint8)
        else:
            obs = np.zeros((mb, obs_spec.size), np.float32)
        z = np.zeros(mb, np.float32)
        self.mb, self.mb_block = bound_block(device, [
            ("obs", obs), ("actions", np.zeros(mb, np.int32)), ("old_logp", z), ("advantages", z),
            ("returns", z), ("values", z)] + self._mb_extra())
        self._counter = DeviceArray(device, (1,), np.int32)
        self._metrics = DeviceArray(device, (len(self.METRICS),))
        self._sq = DeviceArray(device, (1,))
        self._new_logp = DeviceArray(device, (mb, 1))
        self._res: _Resident | None = None
        self._graph = None
        self._pool = None

    def _build_net(self):
        from ttrl_amd.nets.build import build_actor_critic

        if self.cfg.recurrent is not None:
            raise ValueError("PPOLearner: a recurrent config needs RecurrentPPOLearner")
        return build_actor_critic(self.obs_spec, self.action_spec, self.device, batch=self.cfg.minibatch_size,
                                  encoder=self.cfg.encoder)

    def _mb_extra(self) -> list:
        return []

    # -- one minibatch step --------------------------------------------------

    def _gather(self) -> None:
        r, mb = self._res, self.mb
        pairs = [(r.host["obs"], mb["obs"]), (r.host["actions"], mb["actions"]), (r.host["logp"], mb["old_logp"]),
                 (r.adv_norm, mb["advantages"]), (r.returns, mb["returns"]), (r.host["values"], mb["values"])]
        row_bytes = (C.c_long * len(pairs))(*[d.nbytes // self.cfg.minibatch_size for _s, d in pairs])
        self.device.call("ttrl_gather_rows", self.cfg.minibatch_size, len(pairs), _lib.ptrs(s.ptr for s, _ in pairs),
                         _lib.ptrs(d.ptr for _, d in pairs), row_bytes, C.c_long(r.rows), r.host["idx"].vp,
                         C.c_long(r.table_len), self._counter.vp, self.cfg.minibatch_size)

    def _forward_backward(self) -> None:
        from ttrl_amd.nets.heads import policy_value_packed

        self._gather()
        net = self.net
        features = net.encoders["actor"](Tensor(self.mb["obs"]))
        head = policy_value_packed(net.heads["policy"], net.heads["value"], features)
        loss = objective_packed(head, self.mb, self.cfg, self._metrics.view(0, (5,)), self._new_logp)
        loss.backward()

    def _step(self) -> None:
        self._forward_backward()
        # clip_grad_norm and the Adam step with one read of the gradient, its
        # finishing launch also ending the step (the metric ring's row, the
        # step counter)
        r = self._res
        self.optimizer.step_clipped(self.cfg.max_grad_norm, self._sq.vp, C.c_void_p(self._metrics.ptr + 4 * 5),
                                    end=(self._counter.vp, self._metrics.vp, len(self.METRICS), r.ring.vp, r.slots))

    def _capture(self) -> None:
        dev = self.device
        self._pool = dev.create_pool()
        with dev.use_pool(self._pool):
            self.optimizer.zero_grad()
            self._forward_backward()  # warm-up: tunes plans and fills the pool; no parameter changes
            self.optimizer.zero_grad()
            dev.synchronize()
            self._graph, _ = capture(dev, self._step)

    def _release_graph(self) -> None:
        if self._graph is not None:
            self._graph.close()
            self._graph = None
        if self._pool is not None and not self.device.closed:
            self.device.release_pool(self._pool)
        self._pool = None

    # -- one update ----------------------------------------------------------

    def _resident(self, T: int, N: int) -> _Resident:
        r = self._res
        if r is None or (r.T, r.N) != (T, N):
            self._release_graph()
            self._res = r = _Resident(self.device, self.obs_spec, T, N, self.cfg)
        return r

    def load_rollout(self, rollout: dict) -> int:
        """Upload one rollout and its minibatch index table; -> minibatch
        steps this update will run.  Fields (time-major): obs [T, N, ...],
        actions, rewards, dones, values, logp [T, N], last_values [N]
        (the critic's value after the last step), optional valid [T, N]."""
        rewards = np.asarray(rollout["rewards"], np.float32)
        if rewards.ndim != 2:
            raise ValueError(f"PPOLearner: rollout fields must be time-major [T, N], got rewards {rewards.shape}")
        T, N = rewards.shape
        r = self._resident(T, N)
        cfg = self.cfg
        valid = rollout.get("valid")
        valid = np.ones((T, N), np.float32) if valid is None else np.asarray(valid, np.float32).reshape(T, N)
        keep = np.flatnonzero(valid.reshape(-1) > 0.0)
        total = int(keep.size)
        mb = cfg.minibatch_size
        n_full = total // mb
        if n_full == 0:
            raise ValueError(f"PPOLearner: {total} valid transitions but minibatch_size={mb}, which would yield "
                             f"zero minibatches (n_steps={T}, n_envs={N}). Lower minibatch_size or collect a "
                             f"longer rollout.")
        table = np.zeros(max(r.table_len, 1), np.int32)
        for e in range(cfg.epochs):
            perm = self._rng.permutation(total)
            table[e * n_full * mb:(e + 1) * n_full * mb] = keep[perm[:n_full * mb]]
        r.stage("obs", np.asarray(rollout["obs"]).reshape((T * N,) + r.host["obs"].shape[1:]))
        r.stage("actions", np.asarray(rollout["actions"]).reshape(-1).astype(np.int32))
        for name, key in (("logp", "logp"), ("values", "values"), ("rewards", "rewards"), ("dones", "dones")):
            r.stage(name, np.asarray(rollout[key], np.float32).reshape(-1))
        r.stage("valid", valid.reshape(-1))
        r.stage("last_values", np.asarray(rollout["last_values"], np.float32).reshape(-1))
        r.stage("idx", table)
        r.block.upload(r.image)
        return cfg.epochs * n_full

    def begin_update(self) -> None:
        """GAE and the advantage normalisation over the resident rollout,
        and the step counter back to the first minibatch (no host transfer)."""
        cfg, r, dev = self.cfg, self._res, self.device
        h = r.host
        dev.call("ttrl_gae", r.T, r.N, h["rewards"].vp, h["values"].vp, h["dones"].vp, h["valid"].vp,
                 h["last_values"].vp, C.c_double(cfg.gamma), C.c_double(cfg.lam), r.advantages.vp, r.returns.vp)
        if cfg.normalize_adv:
            dev.call("ttrl_normalize_advantages", r.advantages.vp, h["valid"].vp, C.c_long(r.rows),
                     C.c_float(1e-8), r.adv_norm.vp, None)
        else:
            r.adv_norm.copy_from(r.advantages)
        self._counter.fill(0)
        if cfg.step_mode == "graph" and self._graph is None:
            self._capture()

    def run_steps(self, n: int) -> None:
        """The next n minibatch steps of the current update."""
        if self.cfg.step_mode == "graph":
            self._graph.replay_n(n)
            for _ in range(n):
                self.optimizer._replayed()
        else:
            for _ in range(n):
                self.optimizer.zero_grad()
                self._step()

    def run_update(self, steps: int) -> None:
        """GAE, normalisation and `steps` minibatch steps over the resident
        rollout (no host transfer)."""
        self.begin_update()
        self.run_steps(steps)

    def update(self, rollout: dict) -> dict:
        """One rollout's update; -> the reference's metric keys averaged over
        the minibatch steps, plus lr and minibatches."""
        cfg = self.cfg
        if cfg.anneal_lr:
            self.optimizer.lr = cfg.lr * max(0.0, 1.0 - self.frame_count / cfg.total_frames)
        steps = self.load_rollout(rollout)
        self.run_update(steps)
        ring = self._res.ring.numpy()[:steps].astype(np.float64)
        self.update_count += 1
        out = {k: float(np.mean(ring[:, i])) for i, k in enumerate(self.METRICS)}
        out["lr"] = self.optimizer.lr
        out["minibatches"] = float(steps)
        return out

    # -- state -------------------------------------------------------------

    _WEIGHT_KEYS = ("net",)
    _RUN_KEYS = ("optimizer", "frame_count", "update_count", "rng_state")

    def state_dict(self, *, weights_only: bool = False) -> dict:
        """The reference agent's state tree (ttrl/algos/ppo/state.py:25-46)
        for the parts a learner holds; the agent loop's autoreset phase and
        partial rollout are not part of it."""
        return assemble(self.cfg, {"net": to_reference_keys(self.net.state_dict(), TOWERS_PPO, self.obs_spec.name)},
                        {"optimizer": self.optimizer.state_dict(), "frame_count": self.frame_count,
                         "update_count": self.update_count, "rng_state": self._rng.bit_generator.state},
                        weights_only=weights_only)

    def load_state_dict(self, state: dict, *, weights_only: bool = False) -> None:
        """In place, so a captured minibatch step keeps its buffers
        (ttrl/algos/ppo/state.py:49-72)."""
        load_run = validate(state, algo="PPO", config=self.cfg, weight_keys=self._WEIGHT_KEYS,
                            run_keys=self._RUN_KEYS, weights_only=weights_only)
        self.net.load_state_dict(from_reference_keys(state["net"], TOWERS_PPO, self.obs_spec.name))
        if not load_run:
            return
        self.optimizer.load_state_dict(state["optimizer"])
        self.frame_count = int(state["frame_count"])
        self.update_count = int(state["update_count"])
        self._rng.bit_generator.state = state["rng_state"]

    def close(self) -> None:
        self._release_graph()


class RecurrentPPOLearner(PPOLearner):
    """The recurrent PPO update (ttrl/algos/ppo/learn.py:74-90,
    ttrl/algos/ppo/recurrent.py:190-225, ttrl/buffers/seqbatch.py:40-120) on
    a shared trunk with a GRU memory (ttrl/nets/recurrent.py).

    The rollout additionally carries `starts` [T, N] (1 where the step opens
    an episode: the state entering it is reset) and `hidden` [T / seq_len,
    N, hidden_size] (the unmasked state entering each sequence's first step).
    A minibatch is `minibatch_size / seq_len` whole sequences, shuffled as
    units over (chunk, lane) with one permutation per epoch; rows are
    time-major (t * n_seq + sequence).  The loss reduces over valid slots;
    the advantages are normalised over the valid slots of the rollout.  The
    step graph gathers the rows and the sequences' initial states by index
    from the resident rollout, runs trunk, unroll and both heads, the
    objective, backward, clip and Adam.
    """

    def __init__(self, obs_spec, action_spec, device, *, cfg: PPOConfig, seed: int | None = None):
        if cfg.recurrent is None:
            raise ValueError("RecurrentPPOLearner needs cfg.recurrent")
        self.seq_len = cfg.recurrent.seq_len
        self.hidden_size = cfg.recurrent.hidden_size
        self.n_seq = cfg.minibatch_size // self.seq_len
        super().__init__(obs_spec, action_spec, device, cfg=cfg, seed=seed)
        self._h0 = Tensor(self.mb["h0"])
        self._starts = Tensor(self.mb["starts"])

    def _build_net(self):
        from ttrl_amd.nets.recurrent import build_recurrent_actor_critic

        return build_recurrent_actor_critic(self.obs_spec, self.action_spec, self.device,
                                            batch=self.cfg.minibatch_size, hidden_size=self.hidden_size,
                                            encoder=self.cfg.encoder)

    def _mb_extra(self) -> list:
        mb = self.cfg.minibatch_size
        return [("valid", np.zeros(mb, np.float32)), ("starts", np.zeros((self.seq_len, self.n_seq, 1), np.float32)),
                ("h0", np.zeros((self.n_seq, self.hidden_size), np.float32))]

    def _resident(self, T: int, N: int) -> _Resident:
        r = self._res
        if r is None or (r.T, r.N) != (T, N):
            if T % self.seq_len:
                raise ValueError(f"RecurrentPPOLearner: n_steps={T} is not a multiple of seq_len={self.seq_len}")
            self._release_graph()
            chunks = T // self.seq_len
            per_epoch = (chunks * N) // self.n_seq
            extra = [("starts", np.zeros(T * N, np.float32)),
                     ("hidden", np.zeros((chunks * N, self.hidden_size), np.float32)),
                     ("idx_h0", np.zeros(max(self.cfg.epochs * per_epoch * self.n_seq, 1), np.int32))]
            self._res = r = _Resident(self.device, self.obs_spec, T, N, self.cfg, extra, per_epoch)
            r.h0_len = self.cfg.epochs * per_epoch * self.n_seq
        return r

    def load_rollout(self, rollout: dict) -> int:
        rewards = np.asarray(rollout["rewards"], np.float32)
        if rewards.ndim != 2:
            raise ValueError(f"RecurrentPPOLearner: rollout fields must be time-major [T, N], got {rewards.shape}")
        T, N = rewards.shape
        r = self._resident(T, N)
        cfg, L, S = self.cfg, self.seq_len, self.n_seq
        chunks = T // L
        total = chunks * N
        n_full = total // S
        if n_full == 0:
            raise ValueError(f"RecurrentPPOLearner: the rollout holds {total} sequences of {L} steps and a "
                             f"minibatch of {cfg.minibatch_size} rows wants {S} of them, which would yield zero "
                             f"minibatches. Lower minibatch_size or seq_len, or collect a longer rollout.")
        valid = rollout.get("valid")
        valid = np.ones((T, N), np.float32) if valid is None else np.asarray(valid, np.float32).reshape(T, N)
        if not (valid > 0).any():
            raise ValueError("RecurrentPPOLearner: the rollout holds no valid transitions")
        hidden = np.asarray(rollout["hidden"], np.float32)
        if hidden.shape != (chunks, N, self.hidden_size):
            raise ValueError(f"RecurrentPPOLearner: hidden must be ({chunks}, {N}, {self.hidden_size}), "
                             f"got {hidden.shape}")
        rows_t = np.zeros(max(r.table_len, 1), np.int32)
        h0_t = np.zeros(max(r.h0_len, 1), np.int32)
        steps = np.arange(L)
        k = 0
        for _ in range(cfg.epochs):
            perm = self._rng.permutation(total)
            for start in range(0, n_full * S, S):
                ids = perm[start:start + S]
                ch, ln = ids // N, ids % N
                # time-major rows: (t, s) -> flat rollout row (ch_s * L + t) * N + ln_s
                rows = (ch[None, :] * L + steps[:, None]) * N + ln[None, :]
                rows_t[k * S * L:(k + 1) * S * L] = rows.reshape(-1)
                h0_t[k * S:(k + 1) * S] = ch * N + ln
                k += 1
        batch_valid = valid.reshape(-1)[rows_t[:k * S * L].reshape(k, S * L)]
        if not np.all(batch_valid.sum(axis=1) > 0):
            raise ValueError("RecurrentPPOLearner: a sequence minibatch holds no valid transitions")
        r.stage("obs", np.asarray(rollout["obs"]).reshape((T * N,) + r.host["obs"].shape[1:]))
        r.stage("actions", np.asarray(rollout["actions"]).reshape(-1).astype(np.int32))
        for name in ("logp", "values", "rewards", "dones"):
            r.stage(name, np.asarray(rollout[name], np.float32).reshape(-1))
        r.stage("valid", valid.reshape(-1))
        r.stage("starts", np.asarray(rollout["starts"], np.float32).reshape(-1))
        r.stage("hidden", hidden.reshape(chunks * N, self.hidden_size))
        r.stage("last_values", np.asarray(rollout["last_values"], np.float32).reshape(-1))
        r.stage("idx", rows_t)
        r.stage("idx_h0", h0_t)
        r.block.upload(r.image)
        return k

    def _gather(self) -> None:
        r, mb, dev = self._res, self.mb, self.device
        n = self.cfg.minibatch_size
        pairs = [(r.host["obs"], mb["obs"]), (r.host["actions"], mb["actions"]), (r.host["logp"], mb["old_logp"]),
                 (r.adv_norm, mb["advantages"]), (r.returns, mb["returns"]), (r.host["values"], mb["values"]),
                 (r.host["valid"], mb["valid"]), (r.host["starts"], mb["starts"])]
        row_bytes = (C.c_long * len(pairs))(*[d.nbytes // n for _s, d in pairs])
        dev.call("ttrl_gather_rows", n, len(pairs), _lib.ptrs(s.ptr for s, _ in pairs),
                 _lib.ptrs(d.ptr for _, d in pairs), row_bytes, C.c_long(r.rows), r.host["idx"].vp,
                 C.c_long(r.table_len), self._counter.vp, n)
        h_rows = r.host["hidden"].shape[0]
        hb = (C.c_long * 1)(self.hidden_size * 4)
        dev.call("ttrl_gather_rows", self.n_seq, 1, _lib.ptrs([r.host["hidden"].ptr]), _lib.ptrs([mb["h0"].ptr]), hb,
                 C.c_long(h_rows), r.host["idx_h0"].vp, C.c_long(r.h0_len), self._counter.vp, self.n_seq)

    def _forward_backward(self) -> None:
        self._gather()
        head = self.net.forward_packed(Tensor(self.mb["obs"]), self._h0, self._starts, seq_len=self.seq_len)
        loss = objective_packed(head, self.mb, self.cfg, self._metrics.view(0, (5,)), self._new_logp,
                                valid=self.mb["valid"])
        loss.backward()
