"""The DQN learner update (ttrl/algos/dqn/losses.py:44-140,
ttrl/algos/dqn/agent.py:151-214).

`step_inputs` names the bound buffers one update reads; `update_loss` is the
update body: online forward with tape, target and online forwards on s'
without tape, the fused TD/Huber head, backward, metrics.  `DQNLearner` owns
the networks, the Adam optimizer and the TrainStep; `update(batch)` loads
one replay batch and runs one gradient step (the body of the reference's
`_gradient_step` after sampling).

Image observations are bound as uint8 NCHW frames, the layout the
environment produces, so an update uploads 1 byte per pixel and no host
transpose; the first convolution reads them directly.
"""

from __future__ import annotations

from dataclasses import dataclass

import ctypes as C

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.algos.grads import grad_sq_device
from ttrl_amd.algos.state import TOWERS_DQN, assemble, from_reference_keys, to_reference_keys, validate
from ttrl_amd.buffers.replay import PriorityConfig
from ttrl_amd.engine.autograd import Tensor, no_grad
from ttrl_amd.engine.conv import Conv2d
from ttrl_amd.engine import layers as layers_mod
from ttrl_amd.engine.layers import Linear, ReLU
from ttrl_amd.engine.ops.fused import dqn_head_td_loss, dqn_tail_td_loss, dqn_td_loss, linear_node
from ttrl_amd.engine.optim import Adam
from ttrl_amd.engine.step import TrainStep
from ttrl_amd.engine.tensor import DeviceArray, bound_block
from ttrl_amd.nets.acting import ActingNet, GreedyDecision
from ttrl_amd.nets.build import build_q_net

__all__ = ["DQNConfig", "DQNLearner", "leaf_key", "step_inputs", "update_loss"]


@dataclass(frozen=True)
class DQNConfig:
    """The learner-side fields of ttrl/algos/dqn/config.py:19-151, plus the
    Adam epsilon, which the reference leaves at the engine default 1e-8."""

    lr: float = 1e-4
    adam_eps: float = 1e-8
    gamma: float = 0.99
    n_step: int = 3
    batch_size: int = 32
    double: bool = True
    huber_delta: float = 1.0
    target_sync_interval: int = 8000
    prioritized: bool = True
    step_mode: str = "graph"
    encoder: str = "auto"
    eps_start: float = 1.0
    eps_end: float = 0.01
    eps_decay_frames: int = 1_000_000
    eval_epsilon: float = 0.05
    act_mode: str = "graph"
    # the agent's replay and update clock (DQNAgent)
    buffer_capacity: int = 100_000
    train_freq: int = 4
    learning_starts: int = 1_000
    priority: PriorityConfig | None = None

    def __post_init__(self):
        if self.lr <= 0 or self.adam_eps <= 0:
            raise ValueError("DQNConfig: lr and adam_eps must be > 0")
        if self.batch_size < 1:
            raise ValueError(f"DQNConfig: batch_size must be >= 1, got {self.batch_size}")
        if self.huber_delta <= 0:
            raise ValueError(f"DQNConfig: huber_delta must be > 0, got {self.huber_delta}")
        if self.target_sync_interval < 1:
            raise ValueError("DQNConfig: target_sync_interval must be >= 1")
        if not 0.0 <= self.eps_end <= self.eps_start <= 1.0:
            raise ValueError(f"DQNConfig: the epsilon schedule must satisfy 0 <= eps_end <= eps_start <= 1, "
                             f"got eps_start={self.eps_start}, eps_end={self.eps_end}")
        if self.eps_decay_frames < 1:
            raise ValueError(f"DQNConfig: eps_decay_frames must be >= 1, got {self.eps_decay_frames}")
        if not 0.0 <= self.eval_epsilon <= 1.0:
            raise ValueError(f"DQNConfig: eval_epsilon must be in [0, 1], got {self.eval_epsilon}")
        if self.buffer_capacity < 1 or self.train_freq < 1 or self.learning_starts < 0:
            raise ValueError("DQNConfig: buffer_capacity and train_freq must be >= 1, learning_starts >= 0")
        if self.priority is not None and not self.prioritized:
            raise ValueError("DQNConfig: a priority config needs prioritized=True (the update reads IS weights)")

    def replay_priority(self) -> PriorityConfig | None:
        """The agent's replay prioritisation: `priority`, or the default
        settings when only `prioritized` is set."""
        if not self.prioritized:
            return None
        return self.priority if self.priority is not None else PriorityConfig()


def leaf_key(which: str, leaf: str) -> str:
    return f"{which}.{leaf}"


def _obs_host(spec, batch):
    if spec.kind == "image":
        return np.zeros((batch,) + tuple(spec.shape), np.uint8)
    return np.zeros((batch, spec.size), np.float32)


def step_inputs(obs_spec, device, *, batch: int, num_actions: int, mask_n: int = 0,
                prioritized: bool = False) -> dict:
    """The fixed device buffers one update reads, allocated once, back to
    back in one block (`inputs["_block"]`) so one copy refreshes a batch."""
    if mask_n:
        raise ValueError("step_inputs: legal-action masks are not supported by this learner")
    z = np.zeros((batch, 1), np.float32)
    specs = [
        (leaf_key("obs", obs_spec.name), _obs_host(obs_spec, batch)),
        (leaf_key("next_obs", obs_spec.name), _obs_host(obs_spec, batch)),
        ("rewards", z), ("dones", z), ("discounts", z),
        ("actions_onehot", np.zeros((batch, num_actions), np.float32)),
    ]
    if prioritized:
        specs.append(("is_weights", np.ones((batch, 1), np.float32)))
    arrays, whole = bound_block(device, specs)
    inputs = {name: Tensor(arr) for name, arr in arrays.items()}
    inputs["_block"] = whole
    return inputs


def _lockstep_layers(nets):
    """Encoder layers + Q head of same-structured EncoderHead Q networks, or None."""
    try:
        stacks = [list(n.encoder.layers) + [n.head.q] for n in nets]
    except AttributeError:
        return None
    first = stacks[0]
    for st in stacks[1:]:
        if len(st) != len(first) or any(type(a) is not type(b) for a, b in zip(st, first)):
            return None
    return stacks


def q_forward_multi(nets, inputs, tape_group: int | None = 0, *, skip_last: int = 0):
    """Q values of several same-shaped Q networks, one launch per layer.

    `nets[g]` is applied to `inputs[g]`; the evaluations share each layer's
    launch (per-group weight and activation pointers).  Only group
    `tape_group` records a tape (the online network on s); every other group
    is a constant of the step, as under no_grad in the reference.  The last
    `skip_last` layers (a ReLU counting as one) are not applied: the
    features they would consume are returned.
    """
    stacks = _lockstep_layers(nets)
    if stacks is None:
        raise ValueError("q_forward_multi: the networks do not share one layer structure")
    G = len(nets)
    if G > 4:
        raise ValueError("q_forward_multi: at most 4 networks per launch")
    xs = list(inputs)
    dev = xs[0].device
    layers0 = stacks[0][:len(stacks[0]) - int(skip_last)]
    i = 0
    while i < len(layers0):
        layer = layers0[i]
        fuse = i + 1 < len(layers0) and isinstance(layers0[i + 1], ReLU)
        group = [st[i] for st in stacks]
        if isinstance(layer, Conv2d):
            batch = layer._check_input(xs[0])
            for x, conv in zip(xs, group):
                conv._check_input(x)
            ys = [conv.out_array(dev) for conv in group]
            dev.call("ttrl_conv2d_forward_multi", C.byref(layer._c_geom(batch)), G,
                     _lib.ptrs(x.data.ptr for x in xs), _lib.ptrs(c.weight.data.ptr for c in group),
                     _lib.ptrs(None if c.bias is None else c.bias.data.ptr for c in group),
                     _lib.ptrs(y.ptr for y in ys), C.c_float(layer.input_scale), int(fuse))
            if layers_mod.RECORD is not None:  # every group's output of this layer, in launch order
                layers_mod.RECORD.append(list(ys))
            xs = [group[g].node(xs[g], ys[g], fuse) if g == tape_group else Tensor(ys[g]) for g in range(G)]
        elif isinstance(layer, Linear):
            M, K = (int(d) for d in xs[0].shape)
            N = layer.out_features
            weights = [lin.effective_weight() for lin in group]
            ys = [DeviceArray(dev, (M, N)) for _ in range(G)]
            dev.call("ttrl_linear_forward_multi", M, K, N, G, _lib.ptrs(x.data.ptr for x in xs),
                     _lib.ptrs(w.data.ptr for w in weights),
                     _lib.ptrs(None if lin.bias is None else lin.bias.data.ptr for lin in group),
                     _lib.ptrs(y.ptr for y in ys), int(fuse))
            if layers_mod.RECORD is not None:
                layers_mod.RECORD.append(list(ys))
            xs = [linear_node(xs[g], weights[g], group[g].bias, ys[g], relu=fuse) if g == tape_group
                  else Tensor(ys[g]) for g in range(G)]
        else:
            xs = [group[g](xs[g]) for g in range(G)]  # Flatten: a view; only the taped group records
            fuse = False
        i += 2 if fuse else 1
    return xs


def update_loss(online, target, inputs: dict, *, leaves, num_actions: int, mask_n: int = 0, double: bool = True,
                huber_delta: float = 1.0, prioritized: bool = False, grad_sq: bool = True,
                metrics_out: dict | None = None, defer: bool = False) -> dict:
    """One DQN update body: Huber loss against the n-step double-Q target,
    backward, metrics.  Reads only `inputs`; no host reads (capturable).

    The online forward on s (with tape), the online forward on s' and the
    target forward on s' (both constants of the step) run as one grouped
    launch per layer.  `metrics_out` may name the device arrays `loss`,
    `mean_q` and `td_abs` are written to.  defer=True leaves the Q head's
    gradients, the loss and mean Q to the optimizer step that follows
    (engine.pending); the caller's step must run before they are read."""
    (leaf,) = tuple(leaves)
    obs = inputs[leaf_key("obs", leaf)]
    next_obs = inputs[leaf_key("next_obs", leaf)]
    stacks = _lockstep_layers([online, target])
    nets = [online, online, target] if double else [online, target]
    feeds = [obs, next_obs, next_obs] if double else [obs, next_obs]
    if stacks is not None and _fused_tail_fits(stacks[0], obs):
        # The last two layers, the loss and the head's backward in one GEMM and one kernel.
        features = q_forward_multi(nets, feeds, skip_last=3)
        tails = [_lockstep_layers([n])[0][-3:] for n in nets]
        loss, extra, hs, qs = dqn_tail_td_loss(features, [t[0] for t in tails], [t[2] for t in tails],
                                               inputs["actions_onehot"], inputs["rewards"], inputs["dones"],
                                               inputs["discounts"], inputs["is_weights"] if prioritized else None,
                                               huber_delta, out=metrics_out, defer=defer)
        if layers_mod.RECORD is not None:  # the first layer's outputs, then the Q values, of every group
            layers_mod.RECORD.append(list(hs))
            layers_mod.RECORD.append(list(qs))
        return _finish_update(online, loss, extra, prioritized, grad_sq)
    if stacks is not None and _fused_head_fits(stacks[0], obs, len(nets)):
        # The Q head's last layer and the loss in one launch.
        features = q_forward_multi(nets, feeds, skip_last=1)
        heads = [_lockstep_layers([n])[0][-1] for n in nets]
        loss, extra, qs = dqn_head_td_loss(features, heads, inputs["actions_onehot"], inputs["rewards"],
                                           inputs["dones"], inputs["discounts"],
                                           inputs["is_weights"] if prioritized else None, huber_delta,
                                           out=metrics_out)
        if layers_mod.RECORD is not None:
            layers_mod.RECORD.append(list(qs))
        return _finish_update(online, loss, extra, prioritized, grad_sq)
    if stacks is not None:
        if double:
            q, selector, next_target_q = q_forward_multi(nets, feeds)
        else:
            q, next_target_q = q_forward_multi(nets, feeds)
            selector = next_target_q
    else:
        q = online(obs)
        with no_grad():
            next_target_q = target(next_obs)
            selector = online(next_obs) if double else next_target_q
    loss, extra = dqn_td_loss(q, selector, next_target_q, inputs["actions_onehot"], inputs["rewards"],
                              inputs["dones"], inputs["discounts"],
                              inputs["is_weights"] if prioritized else None, huber_delta, out=metrics_out)
    return _finish_update(online, loss, extra, prioritized, grad_sq)


def _fused_tail_fits(layers, obs) -> bool:
    """ttrl_dqn_tail applies to Q networks ending Linear -> ReLU -> Linear
    (at most 2048 hidden units, 32 actions) at a batch of at most 1024,
    the last layer's weight its own parameter."""
    if len(layers) < 3:
        return False
    fc1, act, fc2 = layers[-3:]
    if not (isinstance(fc1, Linear) and isinstance(act, ReLU) and isinstance(fc2, Linear)):
        return False
    if fc2.effective_weight() is not fc2.weight or not fc2.weight.requires_grad:
        return False
    return (int(fc1.out_features) <= 2048 and 0 < int(fc2.out_features) <= 32 and
            int(obs.shape[0]) <= 1024)


def _fused_head_fits(layers, obs, groups: int) -> bool:
    """The fused Q head (ttrl_dqn_head) applies to a last Linear layer with
    at most 32 actions whose weights for every group, padded to 8/16/32
    actions, fit a workgroup's 128 KiB of LDS."""
    head = layers[-1]
    A = head.out_features if isinstance(head, Linear) else 0
    if not 0 < A <= 32:
        return False
    ap = 8 if A <= 8 else (16 if A <= 16 else 32)
    rows = 16 // groups
    return groups * (head.in_features * ap + rows * A) * 4 <= 128 * 1024


def _finish_update(online, loss, extra, prioritized: bool, grad_sq: bool) -> dict:
    loss.backward()
    metrics = {"loss": loss, "mean_q": extra["mean_q"]}
    if prioritized:
        metrics["td_abs"] = extra["td_abs"]
    if grad_sq:
        total = grad_sq_device(online.parameters())
        if total is not None:
            metrics["grad_sq"] = Tensor(total)
    return metrics


class DQNLearner:
    """Online and target Q networks, Adam, one captured update, and the
    acting step either side of it (ttrl/algos/dqn/agent.py:89-119)."""

    def __init__(self, obs_spec, action_spec, device, *, cfg: DQNConfig = DQNConfig(), seed: int | None = None,
                 online_state: dict | None = None, target_state: dict | None = None, n_envs: int = 1,
                 defer_grads: bool = True):
        if action_spec.kind != "discrete":
            raise ValueError(f"DQN supports discrete actions only, got {action_spec.kind!r}")
        self.obs_spec = obs_spec
        self.action_spec = action_spec
        self.device = device
        self.cfg = cfg
        self.num_actions = int(action_spec.n)
        if seed is not None:
            np.random.seed(seed)
        self.online = build_q_net(obs_spec, action_spec, device, batch=cfg.batch_size, encoder=cfg.encoder)
        self.target = build_q_net(obs_spec, action_spec, device, batch=cfg.batch_size, encoder=cfg.encoder)
        if online_state is not None:
            self.online.load_state_dict(online_state)
        self.target.copy_from(self.online)
        if target_state is not None:
            self.target.load_state_dict(target_state)
        self.optimizer = Adam(list(self.online.parameters()), lr=cfg.lr, eps=cfg.adam_eps)
        # The update's weight-gradient reductions (convolution split-K sums,
        # the Q head's outer product) and batch means are formed by the Adam
        # launch that consumes them, one gradient bank per convolution; the
        # formed gradients update the parameters without a store nothing
        # reads (optimizer.materialize_grads() writes them on request).
        self.defer_grads = bool(defer_grads)
        self.optimizer.store_formed_grads = not self.defer_grads
        if self.defer_grads:
            convs = [m for m in getattr(getattr(self.online, "encoder", None), "layers", []) if isinstance(m, Conv2d)]
            for bank, conv in enumerate(convs[:4]):
                conv.defer_bank = bank
        # Every metric of an update in one device block, read back with one
        # copy: [loss, mean_q, grad_sq, -, td_abs[B]].
        B = cfg.batch_size
        self._metric_block = DeviceArray(device, (4 + B,))
        self._metric_block.fill(0.0)
        self._metrics_out = {"loss": self._metric_block.view(0, (1, 1)), "mean_q": self._metric_block.view(1, (1, 1)),
                             "td_abs": self._metric_block.view(4, (B, 1))}
        self.optimizer.grad_sq = self._metric_block.view(2, (1, 1))
        self.inputs = step_inputs(obs_spec, device, batch=cfg.batch_size, num_actions=self.num_actions,
                                  prioritized=cfg.prioritized)
        self.step = TrainStep(self._step_fn, self.inputs, device, optimizer=self.optimizer, mode=cfg.step_mode)
        self.update_count = 0
        self.n_envs = int(n_envs)
        self._acting = ActingNet(self.online, obs_spec, device, width=cfg.batch_size, lanes=self.n_envs,
                                 decision=GreedyDecision(), mode=cfg.act_mode)
        self.frame_count = 0
        self._rng = np.random.default_rng(seed)
        # A separate stream for evaluation acting, so evaluation does not
        # perturb the training exploration trajectory.
        self._eval_rng = np.random.default_rng(seed).spawn(1)[0]

    # -- state -------------------------------------------------------------

    _WEIGHT_KEYS = ("online", "target")
    _RUN_KEYS = ("optimizer", "frame_count", "update_count", "rng_state")

    def state_dict(self, *, weights_only: bool = False) -> dict:
        """The reference agent's state tree (ttrl/algos/dqn/agent.py:225-238)
        for the parts a learner holds; the agent loop's autoreset phase and
        update clock are not part of it."""
        leaf = self.obs_spec.name
        return assemble(self.cfg, {"online": to_reference_keys(self.online.state_dict(), TOWERS_DQN, leaf),
                                   "target": to_reference_keys(self.target.state_dict(), TOWERS_DQN, leaf)},
                        {"optimizer": self.optimizer.state_dict(), "frame_count": self.frame_count,
                         "update_count": self.update_count, "rng_state": self._rng.bit_generator.state},
                        weights_only=weights_only)

    def load_state_dict(self, state: dict, *, weights_only: bool = False) -> None:
        """In place, so a captured update keeps its buffers
        (ttrl/algos/dqn/agent.py:240-253)."""
        load_run = validate(state, algo="DQN", config=self.cfg, weight_keys=self._WEIGHT_KEYS,
                            run_keys=self._RUN_KEYS, weights_only=weights_only)
        leaf = self.obs_spec.name
        self.online.load_state_dict(from_reference_keys(state["online"], TOWERS_DQN, leaf))
        self.target.load_state_dict(from_reference_keys(state["target"], TOWERS_DQN, leaf))
        if not load_run:
            return
        self.optimizer.load_state_dict(state["optimizer"])
        self.frame_count = int(state["frame_count"])
        self.update_count = int(state["update_count"])
        self._rng.bit_generator.state = state["rng_state"]

    # -- acting ------------------------------------------------------------

    def epsilon(self) -> float:
        cfg = self.cfg
        frac = min(1.0, self.frame_count / cfg.eps_decay_frames)
        return cfg.eps_start + frac * (cfg.eps_end - cfg.eps_start)

    def act(self, obs, *, deterministic: bool = False, episode_starts=None) -> np.ndarray:
        """One action per lane: epsilon-greedy over the online network's
        greedy action, the random draws made on the host in the reference's
        order (ttrl/algos/dqn/agent.py:97-119).  `episode_starts` is part of
        the acting contract for a policy with memory; this one has none."""
        eps = self.cfg.eval_epsilon if deterministic else self.epsilon()
        rng = self._eval_rng if deterministic else self._rng
        greedy = self._acting.decide(obs)["actions"]
        batch = greedy.shape[0]
        draws = rng.random(batch)
        random_actions = rng.integers(0, self.num_actions, size=batch)
        actions = np.where(draws < eps, random_actions, greedy).astype(np.int64)
        if not deterministic:
            self.frame_count += batch
        return actions

    def _step_fn(self, inputs: dict) -> dict:
        metrics = update_loss(self.online, self.target, inputs, leaves=(self.obs_spec.name,),
                              num_actions=self.num_actions, double=self.cfg.double,
                              huber_delta=self.cfg.huber_delta, prioritized=self.cfg.prioritized, grad_sq=False,
                              metrics_out=self._metrics_out, defer=self.defer_grads)
        # Adam reduces sum(g^2) over the same gradients in its own launch.
        metrics["grad_sq"] = Tensor(self.optimizer.grad_sq)
        return metrics

    def load_batch(self, batch: dict) -> None:
        """Stage one replay batch for the bound buffers (written into the
        step's pinned host image; the next update sends it with one copy)."""
        leaf = self.obs_spec.name
        step = self.step
        step.load_input(leaf_key("obs", leaf), batch["obs"])
        step.load_input(leaf_key("next_obs", leaf), batch["next_obs"])
        B = self.cfg.batch_size
        step.load_input("rewards", np.asarray(batch["rewards"], np.float32).reshape(B, 1))
        step.load_input("dones", np.asarray(batch["dones"], np.float32).reshape(B, 1))
        step.load_input("discounts", np.asarray(batch["discounts"], np.float32).reshape(B, 1))
        onehot = np.zeros((B, self.num_actions), np.float32)
        onehot[np.arange(B), np.asarray(batch["actions"]).reshape(-1).astype(np.int64)] = 1.0
        step.load_input("actions_onehot", onehot)
        if self.cfg.prioritized:
            w = batch.get("is_weights")
            step.load_input("is_weights", np.ones((B, 1), np.float32) if w is None
                            else np.asarray(w, np.float32).reshape(B, 1))

    def update(self, batch: dict | None = None) -> dict:
        """One gradient step; returns the reference's metric keys."""
        if batch is not None:
            self.load_batch(batch)
        out = self.step.run()
        self.update_count += 1
        if self.update_count % self.cfg.target_sync_interval == 0:
            self.target.copy_from(self.online)
        grad_sq = float(np.asarray(out.get("grad_sq", 0.0)).reshape(-1)[0])
        metrics = {
            "loss": float(np.asarray(out["loss"]).reshape(-1)[0]),
            "mean_q": float(np.asarray(out["mean_q"]).reshape(-1)[0]),
            "grad_norm": float(np.sqrt(max(grad_sq, 0.0))),
        }
        if "td_abs" in out:
            metrics["td_abs"] = np.asarray(out["td_abs"]).reshape(-1)
        return metrics

    def close(self) -> None:
        try:
            self._acting.close()
        finally:
            self.step.close()
