"""The SAC learner update (ttrl/algos/sac/losses.py:25-94, step.py:28-130,
targets.py:21-96, agent.py:175-238).

One update, in the reference's order: critic region (soft target under
no_grad, twin-critic loss, backward), critic Adam, actor region (reading the
just-updated critics: reparameterised sample, actor loss, temperature loss,
backwards), policy and temperature Adam, Polyak blend of the targets.  In
"graph" mode the whole update, optimizers and blend included, is one
hipGraph; in "eager" mode the same kernels run one by one.

Fused pieces:
* `TwinQ` runs both critics of a `build_sac_nets` critic list as one grouped
  launch per layer (they live in one parameter arena at a fixed stride), with
  concat(s, a) folded into the first layer's loads;
* `squashed_sample` (ttrl_amd.algos.gaussian) is one kernel forward and one
  backward;
* the critic loss and the actor + temperature losses are one kernel each.
The critic weight gradients that the reference computes in the actor region
and then discards (its RegionOptimizers zero them) are not computed: the
critics enter the actor region with their parameters frozen.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.algos.gaussian import ActionScale, sampled_rows_tape, squashed_sample, squashed_sample_rows
from ttrl_amd.algos.state import TOWERS_SAC, assemble, from_reference_keys, to_reference_keys, validate
from ttrl_amd.buffers.replay import PriorityConfig
from ttrl_amd.nets.acting import ActingNet, SquashedDecision
from ttrl_amd.engine.autograd import Tensor, _needs, no_grad
from ttrl_amd.engine import layers as layers_mod
from ttrl_amd.engine.layers import Linear, ReLU
from ttrl_amd.engine.ops import _kernels as K
from ttrl_amd.engine.ops.fused import grad_targets, linear_node
from ttrl_amd.engine.optim import Adam, adam_multi, finish_steps
from ttrl_amd.engine.slots import InputSlots, check_slot_count, metric_ptrs
from ttrl_amd.engine.step import InputBinder, MetricReader
from ttrl_amd.engine.tensor import DeviceArray, ParamArena, bound_block
from ttrl_amd.engine.trace import capture
from ttrl_amd.nets.build import build_sac_nets
from ttrl_amd.nets.heads import GaussianHead, packed_linear_pair_rows, packed_tape

__all__ = ["SACConfig", "SACLearner", "TwinQ", "sac_critic_loss", "sac_actor_losses"]


@dataclass(frozen=True)
class SACConfig:
    """Learner-side fields of ttrl/algos/sac/config.py:15-183."""

    lr: float = 3e-4
    adam_eps: float = 1e-8
    gamma: float = 0.99
    tau: float = 0.005
    batch_size: int = 256
    learn_alpha: bool = True
    init_log_alpha: float = 0.0
    target_entropy: float | None = None
    prioritized: bool = False
    step_mode: str = "graph"
    # the update as the library's fused stages when the networks have the
    # standard shape (two hidden layers of one width); the per-layer path otherwise
    fused_update: bool = True
    critic_hidden: tuple = (256, 256)
    policy_hidden: tuple = (256, 256)
    act_mode: str = "graph"
    # the agent's replay and update clock (SACAgent)
    n_step: int = 1
    buffer_capacity: int = 100_000
    train_freq: int = 1
    learning_starts: int = 1_000
    priority: PriorityConfig | None = None

    def __post_init__(self):
        if self.lr <= 0 or self.adam_eps <= 0:
            raise ValueError("SACConfig: lr and adam_eps must be > 0")
        if self.n_step < 1 or self.buffer_capacity < 1 or self.train_freq < 1 or self.learning_starts < 0:
            raise ValueError("SACConfig: n_step, buffer_capacity and train_freq must be >= 1, learning_starts >= 0")
        if self.priority is not None and not self.prioritized:
            raise ValueError("SACConfig: a priority config needs prioritized=True (the critic loss reads IS weights)")
        if not 0.0 <= self.tau <= 1.0:
            raise ValueError(f"SACConfig: tau must be in [0, 1], got {self.tau}")
        if self.step_mode not in ("eager", "graph"):
            raise ValueError(f"SACConfig: step_mode must be 'eager' or 'graph', got {self.step_mode!r}")

    def replay_priority(self) -> PriorityConfig | None:
        if not self.prioritized:
            return None
        return self.priority if self.priority is not None else PriorityConfig()


# --------------------------------------------------------------- twin Q ---

class TwinQ:
    """Both critics of a critic list as grouped launches.

    Each critic must be concat(s, a) -> [Linear -> ReLU]* -> Linear(1) with
    its parameters at a fixed stride from the first critic's in one arena,
    which is how `build_sac_nets` lays them out.
    """

    def __init__(self, critics):
        crit = list(critics)
        if len(crit) != 2:
            raise ValueError(f"TwinQ: expected two critics, got {len(crit)}")
        self.layers = []
        for c in crit:
            seq = list(c.head.layers)
            lins = []
            for i, layer in enumerate(seq):
                if isinstance(layer, Linear):
                    lins.append(layer)
                elif isinstance(layer, ReLU):
                    continue
                elif hasattr(layer, "value") and isinstance(layer.value, Linear):
                    lins.append(layer.value)
                else:
                    raise ValueError(f"TwinQ: unsupported critic layer {type(layer).__name__}")
            if len(c.encoder.tower) != 0:
                raise ValueError("TwinQ: the critic's observation tower must be the identity encoder")
            self.layers.append(lins)
        a, b = self.layers
        if len(a) != len(b):
            raise ValueError("TwinQ: the two critics differ in depth")
        info0 = a[0].weight._arena
        if info0 is None:
            raise ValueError("TwinQ: critics must be built inside one ParamArena")
        stride = b[0].weight._arena[1] - info0[1]
        for la, lb in zip(a, b):
            for pa, pb in ((la.weight, lb.weight), (la.bias, lb.bias)):
                if pa._arena is None or pb._arena is None or pa._arena[0] is not pb._arena[0]:
                    raise ValueError("TwinQ: critics must share one ParamArena")
                if pb._arena[1] - pa._arena[1] != stride or tuple(pa.shape) != tuple(pb.shape):
                    raise ValueError("TwinQ: critic parameters are not at a fixed stride")
        self.stride = stride
        self.obs_dim = a[0].in_features - crit[0].encoder.action_width
        self.act_dim = crit[0].encoder.action_width

    def params(self):
        out = []
        for lins in self.layers:
            for lin in lins:
                out += [lin.weight, lin.bias]
        return out

    def _run_layers(self, dev, B: int, sets, first: dict) -> list:
        """Every layer of len(sets) critics (sets[g]: critic g's Linear
        layers, all of one shape) in one launch per layer; the first layer
        reads concat(first["x"][g], first["x2"][g]).  -> each layer's output,
        (G, B, N)."""
        G = len(sets)
        acts = []
        h = None
        nl = len(sets[0])
        for j in range(nl):
            lin = sets[0][j]
            N = lin.out_features
            y = DeviceArray(dev, (G, B, N))
            d = _lib.LinearDesc()
            d.M, d.K, d.N, d.groups = B, lin.in_features, N, G
            if j == 0:
                d.x, d.ldx = first["x"][0], first["ldx"]
                x2 = first.get("x2")
                if x2 is not None:
                    d.x2, d.ldx2, d.k1 = x2[0], first["ldx2"], first["k1"]
                for g in range(G):
                    d.xg[g] = first["x"][g]
                    if x2 is not None:
                        d.x2g[g] = x2[g]
            else:
                prev = sets[0][j - 1].out_features
                d.x, d.ldx, d.gx = h.ptr, prev, B * prev
            d.W, d.b = lin.weight.data.ptr, lin.bias.data.ptr
            for g in range(G):
                d.Wg[g], d.bg[g] = sets[g][j].weight.data.ptr, sets[g][j].bias.data.ptr
            d.y, d.gy = y.ptr, B * N
            d.relu = int(j < nl - 1)
            dev.call("ttrl_linear_forward", C.byref(d))
            if d.relu and layers_mod.RECORD is not None:
                layers_mod.RECORD.append(y)
            acts.append(y)
            h = y
        return acts

    def forward(self, obs: Tensor | None = None, action: Tensor | None = None, *, obs_action: Tensor | None = None,
                train_params: bool = True) -> Tensor:
        """Q of both critics, (2, B, 1).  Pass a dense concat(s, a) as
        `obs_action` (required when training the critics) or `obs` and
        `action` separately."""
        if obs_action is not None:
            x, x2 = obs_action, None
        else:
            x, x2 = obs, action
        B = int(x.shape[0])
        first = {"x": [x.data.ptr] * 2, "ldx": int(x.shape[1])}
        if x2 is not None:
            first.update(x2=[x2.data.ptr] * 2, ldx2=int(x2.shape[1]), k1=int(x.shape[1]))
        acts = self._run_layers(x.device, B, self.layers, first)
        return self._tape(x, x2, acts, train_params)

    def forward_with_targets(self, targets: "TwinQ", next_obs: Tensor, next_action: DeviceArray, obs: Tensor,
                             action: Tensor, obs_action: Tensor):
        """The target critics on (s', a') and these critics on (s, a), four
        groups of one launch per layer.  -> (q (2, B, 1) on the tape, its
        first-layer weight gradient read from the dense `obs_action`;
        q_next (2, B, 1) off the tape)."""
        B = int(obs.shape[0])
        if tuple(int(d) for d in next_action.shape) != (B, self.act_dim):
            raise ValueError(f"TwinQ: next_action must be ({B}, {self.act_dim})")
        first = {"x": [next_obs.data.ptr] * 2 + [obs.data.ptr] * 2, "ldx": self.obs_dim,
                 "x2": [next_action.ptr] * 2 + [action.data.ptr] * 2, "ldx2": self.act_dim, "k1": self.obs_dim}
        acts = self._run_layers(obs.device, B, list(targets.layers) + list(self.layers), first)
        online = [a.view(2 * B * int(a.shape[2]), (2, B, int(a.shape[2]))) for a in acts]
        q_next = Tensor(acts[-1].view(0, (2, B, 1)))
        return self._tape(obs_action, None, online, True), q_next

    def _tape(self, x: Tensor, x2: Tensor | None, acts: list, train_params: bool) -> Tensor:
        """The tape node of both critics' outputs acts[-1] (acts: each
        layer's (2, B, N) output), from input x (and x2 after it)."""
        lins = self.layers[0]
        B = int(x.shape[0])
        dev = x.device
        S = self.stride
        nl = len(lins)
        h = acts[-1]
        params = self.params() if train_params else []
        inputs = [t for t in (x, x2) if t is not None]
        if not _needs(*inputs, *params):
            return Tensor(h)
        out = Tensor(h, True, tuple(inputs) + tuple(params), "twin_q")
        want_action = x2 is not None and x2.requires_grad
        first_in = x.data

        def _backward(grad):
            g = grad
            for j in range(nl - 1, -1, -1):
                lin = lins[j]
                N, Kin = lin.out_features, lin.in_features
                d = _lib.LinearDesc()
                d.M, d.K, d.N, d.groups = B, Kin, N, 2
                d.W, d.gW = lin.weight.data.ptr, S
                d.dy, d.gy = g.ptr, B * N  # hidden-layer dy arrives gated by the layer above
                if params:
                    c0, c1 = self.layers[0][j], self.layers[1][j]
                    (dw0, db0, dw1, db1), beta = grad_targets(c0.weight, c0.bias, c1.weight, c1.bias)
                    if dw1.ptr - dw0.ptr != 4 * S or db1.ptr - db0.ptr != 4 * S:
                        raise RuntimeError("TwinQ: critic gradients are not in the arena's gradient slots")
                    if j == 0 and x2 is not None:
                        raise ValueError("TwinQ: training the critics needs a dense obs_action input")
                    xin = first_in if j == 0 else acts[j - 1]
                    d.x, d.ldx = xin.ptr, Kin
                    d.gx = 0 if j == 0 else B * Kin
                    d.dW, d.db, d.gb = dw0.ptr, db0.ptr, S
                    d.beta_w = beta
                if j > 0:
                    dx = DeviceArray(dev, (2, B, Kin))
                    d.dx, d.lddx, d.gdx = dx.ptr, Kin, B * Kin
                    d.dxmask = acts[j - 1].ptr  # relu_bw of layer j-1, applied as dx is written
                elif want_action:
                    dx = DeviceArray(dev, (2, B, self.act_dim))
                    d.dx, d.lddx, d.gdx = dx.ptr, self.act_dim, B * self.act_dim
                    d.dx_col0, d.dx_cols = self.obs_dim, self.act_dim
                else:
                    dx = None
                if d.dW or d.dx:
                    dev.call("ttrl_linear_backward", C.byref(d))
                g = dx
            if want_action and g is not None:
                g0 = g.view(0, (B, self.act_dim))
                g1 = g.view(B * self.act_dim, (B, self.act_dim))
                if hasattr(x2, "_accept_pair"):
                    x2._accept_pair(g0, g1)
                else:
                    x2._accumulate(K.binary("add", g0, g1))

        out._backward = _backward
        return out


# ---------------------------------------------------------------- losses ---

def _out_array(out: dict | None, name: str, dev, shape) -> DeviceArray:
    """out[name] reshaped to `shape` when the caller supplies it, else a new array."""
    a = (out or {}).get(name)
    if a is None:
        return DeviceArray(dev, shape)
    if a.numel != int(np.prod(shape)) or a.dtype != np.float32:
        raise ValueError(f"SAC loss: out[{name!r}] must hold {int(np.prod(shape))} float32 values")
    return a.reshape(shape)


def sac_critic_loss(q: Tensor, q_next_target: Tensor, logp_next: Tensor, log_alpha: Tensor, rewards: Tensor,
                    dones: Tensor, discounts: Tensor, is_weights: Tensor | None = None, out: dict | None = None):
    """critic_loss of ttrl/algos/sac/losses.py:46-76 as one kernel.

    -> (loss (1, 1) differentiable in q, metrics {q_target, td_abs, alpha}).
    `out` may supply the arrays loss, q_target, td_abs and alpha go to."""
    B = int(q.shape[1])
    dev = q.device
    loss = _out_array(out, "loss", dev, (1, 1))
    q_target = _out_array(out, "q_target", dev, (B, 1))
    dq = DeviceArray(dev, (2, B, 1))
    td_abs = _out_array(out, "td_abs", dev, (B, 1))
    alpha = _out_array(out, "alpha", dev, (1, 1))
    dev.call("ttrl_sac_critic_loss", B, q.data.vp, q_next_target.data.vp, logp_next.data.vp, log_alpha.data.vp,
             rewards.data.vp, dones.data.vp, discounts.data.vp, None if is_weights is None else is_weights.data.vp,
             loss.vp, q_target.vp, dq.vp, td_abs.vp, alpha.vp)
    metrics = {"q_target": Tensor(q_target), "td_abs": Tensor(td_abs), "alpha": Tensor(alpha)}
    if not _needs(q):
        return Tensor(loss), metrics
    out = Tensor(loss, True, (q,), "sac_critic_loss")

    def _backward(grad):
        q._accumulate(dq if grad.unit else K.binary("mul", dq, grad.reshape((1, 1, 1))))

    out._backward = _backward
    return out, metrics


def sac_actor_losses(q_pi: Tensor, logp: Tensor, log_alpha: Tensor, target_entropy: float,
                     learn_alpha: bool = True, out: dict | None = None):
    """actor_loss and alpha_loss (ttrl/algos/sac/losses.py:79-94) as one
    kernel.  -> (actor_loss, alpha_loss | None), each (1, 1).  `out` may
    supply the arrays actor_loss and alpha_loss go to."""
    B = int(q_pi.shape[1])
    dev = q_pi.device
    la = _out_array(out, "actor_loss", dev, (1, 1))
    lalpha = _out_array(out, "alpha_loss", dev, (1, 1))
    dq = DeviceArray(dev, (2, B, 1))
    g_logp = DeviceArray(dev, (B, 1))
    # d alpha_loss / d log_alpha straight into log_alpha's gradient slot when
    # nothing else holds a gradient there yet: the backward then only claims it
    ahead = (log_alpha._grad_slot if learn_alpha and log_alpha.requires_grad and log_alpha.grad is None
             else None)
    d_log_alpha = ahead.reshape((1, 1)) if ahead is not None else DeviceArray(dev, (1, 1))
    dev.call("ttrl_sac_actor_loss", B, q_pi.data.vp, logp.data.vp, log_alpha.data.vp, C.c_float(target_entropy),
             int(learn_alpha), la.vp, lalpha.vp, dq.vp, g_logp.vp, d_log_alpha.vp)
    actor = Tensor(la)
    if _needs(q_pi, logp):
        actor = Tensor(la, True, (q_pi, logp), "sac_actor_loss")

        def _backward(grad):
            scale = None if grad.unit else grad.reshape((1, 1, 1))
            if q_pi.requires_grad:
                q_pi._accumulate(dq if scale is None else K.binary("mul", dq, scale))
            if logp.requires_grad:
                logp._accumulate(g_logp if scale is None else K.binary("mul", g_logp, scale.reshape((1, 1))))

        actor._backward = _backward
    alpha_loss = None
    if learn_alpha:
        alpha_loss = Tensor(lalpha)
        if _needs(log_alpha):
            alpha_loss = Tensor(lalpha, True, (log_alpha,), "sac_alpha_loss")

            def _backward_alpha(grad):
                if ahead is not None:
                    if log_alpha.grad is not None:
                        raise RuntimeError("sac_actor_losses: log_alpha received a gradient between the loss, "
                                           "which wrote its own into the gradient slot, and this backward")
                    log_alpha.grad, log_alpha._grad_owned = ahead, True
                    if not grad.unit:
                        K.binary_into("mul", ahead, grad.reshape(tuple(ahead.shape)), ahead)
                    return
                log_alpha._accumulate(d_log_alpha if grad.unit else K.binary("mul", d_log_alpha, grad))

            alpha_loss._backward = _backward_alpha
    return actor, alpha_loss


# --------------------------------------------------------------- learner ---

def policy_packed(policy, obs: Tensor) -> Tensor:
    """Policy forward to packed [mean | clamp(log_std)] rows."""
    head = policy.head
    if not isinstance(head, GaussianHead):
        raise ValueError("SAC needs a GaussianHead policy")
    return head.forward_packed(policy.encoder(obs))


def _linear_relu_pairs(encoder):
    """The encoder's layers as (linear, ReLU) pairs, else None."""
    items = list(getattr(encoder, "layers", ()))
    if not items or len(items) % 2:
        return None
    pairs = list(zip(items[0::2], items[1::2]))
    for lin, act in pairs:
        if not (isinstance(lin, Linear) and isinstance(act, ReLU)):
            return None
    return [lin for lin, _ in pairs]


def _encoder_rows(policy, obs_all: DeviceArray, B: int):
    """The policy's encoder over every row of obs_all, one launch per layer,
    the tape over its first B rows.  -> (tape node, output of every row)."""
    lins = _linear_relu_pairs(policy.encoder)
    if not isinstance(policy.head, GaussianHead) or lins is None:
        raise ValueError("the SAC policy path needs an MLP encoder of Linear -> ReLU pairs and a GaussianHead")
    rows = int(obs_all.shape[0])
    dev = obs_all.dev
    x_all = obs_all
    x = Tensor(obs_all.view(0, (B, int(obs_all.shape[1]))))
    for lin in lins:
        w = lin.effective_weight()
        N = lin.out_features
        y_all = DeviceArray(dev, (rows, N))
        d = _lib.LinearDesc()
        d.M, d.K, d.N, d.groups = rows, lin.in_features, N, 1
        d.x, d.ldx = x_all.ptr, lin.in_features
        d.W, d.b = w.data.ptr, None if lin.bias is None else lin.bias.data.ptr
        d.y, d.relu = y_all.ptr, 1
        dev.call("ttrl_linear_forward", C.byref(d))
        if layers_mod.RECORD is not None:
            layers_mod.RECORD.append(y_all)
        x = linear_node(x, w, lin.bias, y_all.view(0, (B, N)), relu=True)
        x_all = y_all
    return x, x_all


HEAD_SAMPLE_MAX_D = 16  # action dimensions ttrl_sac_head_sample takes


def policy_sample_rows(policy, obs_all: DeviceArray, B: int, noise_all: DeviceArray, scale: ActionScale,
                       logp_all: DeviceArray):
    """The policy over every row of obs_all, one launch per encoder layer,
    then its Gaussian head and the squashed sample of every row in one launch
    (ttrl_sac_head_sample; a packed head launch and squashed_sample_rows for
    more than 16 action dimensions), the tape over the first B rows (the
    actor's observations; the rest are the soft target's next observations,
    constants of the update).
    -> (action, logp) tensors of the first B rows and (action, logp) arrays
    of the rest; `logp_all` receives every row's log-probability."""
    head = policy.head
    mean, log_std = head.heads["mean"], head.heads["log_std"]
    x, x_all = _encoder_rows(policy, obs_all, B)
    rows, K = (int(s) for s in x_all.shape)
    d = head.action_dim
    if d > HEAD_SAMPLE_MAX_D or mean.bias is None or log_std.bias is None:
        h, h_all = packed_linear_pair_rows(mean, log_std, x, x_all, clamp=(head.log_std_min, head.log_std_max),
                                           op="gaussian_head")
        return squashed_sample_rows(h, h_all, noise_all, scale, logp_all, head.log_std_min, head.log_std_max)
    if tuple(noise_all.shape) != (rows, d) or logp_all.numel != rows or rows <= B:
        raise ValueError(f"policy_sample_rows: noise {noise_all.shape} and logp ({logp_all.numel}) must hold "
                         f"{rows} rows of {d}, more than B = {B}")
    if scale._centre is None:
        raise ValueError("squashed_sample needs the device-resident bounds; construct ActionScale with a device")
    dev = x_all.dev
    head_all = DeviceArray(dev, (rows, 2 * d))
    action_all = DeviceArray(dev, (rows, d))
    u = DeviceArray(dev, (rows, d))
    desc = _lib.SacHeadDesc()
    desc.rows, desc.K, desc.d = rows, K, d
    desc.x = x_all.ptr
    desc.W1, desc.b1 = mean.weight.data.ptr, mean.bias.data.ptr
    desc.W2, desc.b2 = log_std.weight.data.ptr, log_std.bias.data.ptr
    desc.lo, desc.hi = head.log_std_min, head.log_std_max
    desc.noise, desc.centre, desc.half_width = noise_all.ptr, scale._centre.data.ptr, scale._scale.data.ptr
    desc.log_det = scale.log_det
    desc.head, desc.action, desc.logp, desc.u = head_all.ptr, action_all.ptr, logp_all.ptr, u.ptr
    dev.call("ttrl_sac_head_sample", C.byref(desc))
    h = packed_tape(mean, log_std, x, head_all.view(0, (B, 2 * d)), "gaussian_head")
    return sampled_rows_tape(h, action_all, logp_all, noise_all, u, scale, head.log_std_min, head.log_std_max)


class _FusedUpdate:
    """The update as the library's eight fused stages (ttrl_sac_fused_stage)
    and the three optimizer launches, for the standard networks: a policy of
    two Linear -> ReLU layers of width H with a Gaussian head, twin critics
    (and targets) concat(s, a) -> H -> H -> 1, H a multiple of 64 up to 256,
    a batch a multiple of 16.  The stages' activation buffers are allocated
    once here; the weight and bias gradients are written into the arenas'
    gradient slots, the temperature's into its slot, every metric into the
    learner's metric block."""

    def __init__(self, learner, H: int):
        self.learner = learner
        dev, B = learner.device, learner.cfg.batch_size
        O, A = learner.obs_spec.size, learner.action_spec.dim
        nq = H // 64
        self.B, self.O, self.A, self.H = B, O, A, H
        shapes = {"h1": (2 * B, H), "h2": (2 * B, H), "headp": (nq, 2 * B, 2 * A), "head": (2 * B, 2 * A),
                  "act": (2 * B, A), "u": (2 * B, A), "q1": (4, B, H), "q2": (4, B, H), "qp": (4, nq, B),
                  "q1pi": (2, B, H), "q2pi": (2, B, H), "qppi": (2, nq, B), "dQ": (2, B), "dq2": (2, B, H),
                  "dq1": (2, B, H), "dap": (2, nq, B, A), "dhead": (B, 2 * A), "dh2": (B, H), "dh1": (B, H),
                  "terms": (4, B), "adam_scalars": (6,)}
        self.buf = {k: DeviceArray(dev, v) for k, v in shapes.items()}
        self._nparts: dict = {}

    @staticmethod
    def width(learner):
        """H when the learner's networks and batch fit the fused stages, else None."""
        cfg = learner.cfg
        if not cfg.fused_update or not learner._stacked:
            return None
        pol = learner.nets.policy
        lins = _linear_relu_pairs(pol.encoder)
        if lins is None or len(lins) != 2:
            return None
        H = lins[0].out_features
        O, A, B = learner.obs_spec.size, learner.action_spec.dim, cfg.batch_size
        if lins[0].in_features != O or lins[1].in_features != H or lins[1].out_features != H:
            return None
        if H % 64 or H > 256 or B % 16 or B > 1024 or A > 8 or O + A > 64:
            return None
        head = pol.head
        for lin in (head.heads["mean"], head.heads["log_std"]):
            if lin.in_features != H or lin.out_features != A or lin.bias is None:
                return None
        for twin in (learner.twin, learner.twin_targets):
            for lins_c in twin.layers:
                if len(lins_c) != 3:
                    return None
                l1, l2, l3 = lins_c
                if (l1.in_features, l1.out_features, l2.in_features, l2.out_features, l3.in_features,
                        l3.out_features) != (O + A, H, H, H, H, 1):
                    return None
                if any(x.bias is None for x in lins_c):
                    return None
        wide = [lins[1].weight] + [c[1].weight for c in learner.twin.layers]
        if any(w.data.ptr % 16 for w in wide):
            return None
        # the Polyak blend runs element by element beside the critics' step
        ca, ta = getattr(learner.nets.critics, "arena", None), getattr(learner.nets.targets, "arena", None)
        if ca is None or ta is None or ca.numel != ta.numel or list(ca.offsets) != list(ta.offsets):
            return None
        return H

    def _desc(self) -> "_lib.SacFusedDesc":
        L = self.learner
        b, cfg, buf = L.batch, L.cfg, self.buf
        pol = L.nets.policy
        p1, p2 = _linear_relu_pairs(pol.encoder)
        head = pol.head
        mean, log_std = head.heads["mean"], head.heads["log_std"]
        d = _lib.SacFusedDesc()
        d.B, d.O, d.A, d.H = self.B, self.O, self.A, self.H
        d.P1, d.p1, d.P2, d.p2 = p1.weight.data.ptr, p1.bias.data.ptr, p2.weight.data.ptr, p2.bias.data.ptr
        d.Wm, d.bm, d.Wl, d.bl = mean.weight.data.ptr, mean.bias.data.ptr, log_std.weight.data.ptr, \
            log_std.bias.data.ptr
        d.log_std_min, d.log_std_max = head.log_std_min, head.log_std_max
        d.centre, d.half_width, d.log_det = L.scale._centre.data.ptr, L.scale._scale.data.ptr, L.scale.log_det
        for i, lins_c in enumerate(list(L.twin_targets.layers) + list(L.twin.layers)):
            l1, l2, l3 = lins_c
            d.critic[i] = _lib.SacCriticParams(l1.weight.data.ptr, l1.bias.data.ptr, l2.weight.data.ptr,
                                               l2.bias.data.ptr, l3.weight.data.ptr, l3.bias.data.ptr)
        d.obs_pair, d.actions, d.obs_actions = b.obs_pair.ptr, b["actions"].data.ptr, b["obs_actions"].data.ptr
        d.noise_pair = b.noise_pair.ptr
        d.rewards, d.dones, d.discounts = b["rewards"].data.ptr, b["dones"].data.ptr, b["discounts"].data.ptr
        d.is_weights = b["is_weights"].data.ptr if cfg.prioritized else None
        d.log_alpha, d.target_entropy, d.learn_alpha = L.log_alpha.data.ptr, L.target_entropy, int(cfg.learn_alpha)
        for name in _lib.SAC_FUSED_BUFFERS:
            setattr(d, name, buf[name].ptr)
        out = {"critic_loss": L._critic_out["loss"], "alpha": L._critic_out["alpha"],
               "actor_loss": L._actor_out["actor_loss"], "alpha_loss": L._actor_out["alpha_loss"],
               "q_target": L._critic_out["q_target"], "td_abs": L._critic_out["td_abs"], "logp": L._logp_all}
        for name in _lib.SAC_FUSED_METRICS:
            setattr(d, name, out[name].ptr)
        grads = []
        for lin in (p1, p2, mean, log_std):
            grads += [lin.weight._grad_slot, lin.bias._grad_slot]
        for name, g in zip(_lib.SAC_FUSED_POLICY_GRADS, grads):
            setattr(d, name, g.ptr)
        for j, lins_c in enumerate(L.twin.layers):
            slots = [t._grad_slot for lin in lins_c for t in (lin.weight, lin.bias)]
            for k, g in enumerate(slots):
                d.g_critic[j][k] = g.ptr
        d.g_log_alpha = L.log_alpha._grad_slot.ptr if cfg.learn_alpha else None
        # the three Adam steps and the Polyak blend run inside stages 3 and 7
        d.fuse_adam = 1
        d.critic_adam = L.critic_opt.fused_range(0)
        d.actor_adam = L.actor_opt.fused_range(1)
        if cfg.learn_alpha:
            d.alpha_adam = L.alpha_opt.fused_range(2)
        d.polyak_dst, d.tau = L.nets.targets.arena.data.ptr, cfg.tau
        d.adam_scalars = buf["adam_scalars"].ptr
        return d

    def _parts(self, d, stage: int) -> int:
        """The partial sums of g^2 stage 3 or 7 leaves for its optimizer's finish."""
        if stage not in self._nparts:
            n = C.c_int(0)
            _lib.check(_lib.lib().ttrl_sac_fused_adam_parts(C.byref(d), int(stage), C.byref(n)),
                       "ttrl_sac_fused_adam_parts")
            self._nparts[stage] = int(n.value)
        return self._nparts[stage]

    def _stage(self, d, k: int) -> None:
        self.learner.device.call("ttrl_sac_fused_stage", int(k), C.byref(d))

    @staticmethod
    def _written(params) -> None:
        """Every parameter's gradient is in its slot (a stage wrote it)."""
        for p in params:
            p.grad, p._grad_owned, p._grad_masked = p._grad_slot, True, False

    def body(self) -> dict:
        L = self.learner
        cfg, buf = L.cfg, self.buf
        for opt in (L.critic_opt, L.actor_opt, L.alpha_opt):
            opt.zero_grad()
        d = self._desc()
        B, H = self.B, self.H
        rec = layers_mod.RECORD
        self._stage(d, 0)
        self._stage(d, 1)
        if rec is not None:
            rec += [buf["h1"], buf["h2"], buf["q1"], buf["q2"]]
        self._stage(d, 2)
        self._stage(d, 3)  # the critics' gradients, their Adam step and the Polyak blend
        self._written(L.critic_opt.params)
        self._stage(d, 4)
        if rec is not None:
            rec += [buf["q1pi"], buf["q2pi"]]
        self._stage(d, 5)
        self._stage(d, 6)
        self._stage(d, 7)  # the policy's gradients and Adam step, and the temperature's
        self._written(L.actor_opt.params)
        stepped = [(L.critic_opt, 0, self._parts(d, 3)), (L.actor_opt, 1, self._parts(d, 7))]
        if cfg.learn_alpha:
            self._written([L.log_alpha])
            stepped.append((L.alpha_opt, 2, 1))
        finish_steps(L.device, stepped)
        metrics = {"critic_loss": Tensor(L._critic_out["loss"]), "alpha": Tensor(L._critic_out["alpha"]),
                   "q_target": Tensor(L._critic_out["q_target"]), "actor_loss": Tensor(L._actor_out["actor_loss"]),
                   "logp": Tensor(L._logp_out), "critic_grad_sq": Tensor(L.critic_opt.grad_sq),
                   "actor_grad_sq": Tensor(L.actor_opt.grad_sq)}
        if cfg.prioritized:
            metrics["td_abs"] = Tensor(L._critic_out["td_abs"])
        if cfg.learn_alpha:
            metrics["alpha_loss"] = Tensor(L._actor_out["alpha_loss"])
        return metrics


class _BatchBuffers:
    """Bound device buffers of one SAC batch, back to back in one block
    (`block`), allocated once and written in place."""

    def __init__(self, device, B, obs_dim, act_dim, prioritized):
        def z(*shape):
            return np.zeros(shape, np.float32)

        # obs and next_obs (and the two noises) back to back, so the policy
        # runs over both in one launch per layer
        specs = [("obs_pair", z(2 * B, obs_dim)), ("actions", z(B, act_dim)),
                 ("obs_actions", z(B, obs_dim + act_dim)), ("rewards", z(B, 1)), ("dones", z(B, 1)),
                 ("discounts", z(B, 1)), ("noise_pair", z(2 * B, act_dim))]
        if prioritized:
            specs.append(("is_weights", np.ones((B, 1), np.float32)))
        arrays, self.block = bound_block(device, specs)
        self.obs_pair, self.noise_pair = arrays["obs_pair"], arrays["noise_pair"]
        arrays["obs"] = self.obs_pair.view(0, (B, obs_dim))
        arrays["next_obs"] = self.obs_pair.view(B * obs_dim, (B, obs_dim))
        arrays["noise"] = self.noise_pair.view(0, (B, act_dim))
        arrays["next_noise"] = self.noise_pair.view(B * act_dim, (B, act_dim))
        self.tensors = {name: Tensor(arr) for name, arr in arrays.items()}
        self.B = B
        # staged in a pinned image of the block, sent as one copy per update
        self.binder = InputBinder(device, dict(self.tensors, _block=self.block))

    def __getitem__(self, key):
        return self.tensors[key]

    def load(self, name, array):
        self.binder.load(name, np.asarray(array, np.float32))

    def flush(self):
        """Send what was loaded since the last update (one copy for a batch)."""
        self.binder.flush()

    def close(self):
        self.binder.close()

    def load_batch(self, batch: dict):
        B = self.B
        for name in ("obs", "next_obs", "actions", "noise", "next_noise"):
            self.load(name, batch[name])
        for name in ("rewards", "dones", "discounts"):
            self.load(name, np.asarray(batch[name], np.float32).reshape(B, 1))
        self.load("obs_actions", np.concatenate([np.asarray(batch["obs"], np.float32).reshape(B, -1),
                                                 np.asarray(batch["actions"], np.float32).reshape(B, -1)], 1))
        if "is_weights" in self.tensors:
            w = batch.get("is_weights")
            self.load("is_weights", np.ones((B, 1), np.float32) if w is None else w)


class SACLearner:
    """Policy, twin critics, targets, log_alpha, three Adams, one update, and
    the acting step (ttrl/algos/sac/agent.py:95-125)."""

    def __init__(self, obs_spec, action_spec, device, *, cfg: SACConfig = SACConfig(), seed: int | None = None,
                 n_envs: int = 1):
        if action_spec.kind != "continuous":
            raise ValueError(f"SAC supports continuous actions only, got {action_spec.kind!r}")
        self.cfg = cfg
        self.device = device
        self.obs_spec, self.action_spec = obs_spec, action_spec
        if seed is not None:
            np.random.seed(seed)
        self.nets = build_sac_nets(obs_spec, action_spec, device, batch=cfg.batch_size,
                                   critic_hidden=cfg.critic_hidden, encoder_kwargs={"hidden": cfg.policy_hidden})
        with ParamArena(device, "log_alpha") as aa:
            self.log_alpha = Tensor.from_numpy(np.full((1, 1), cfg.init_log_alpha, np.float32), device,
                                               requires_grad=True)
        self.alpha_arena = aa
        self.target_entropy = (-float(action_spec.dim) if cfg.target_entropy is None else float(cfg.target_entropy))
        self.scale = ActionScale(action_spec, device)
        self.actor_opt = Adam(self.nets.policy_parameters(), lr=cfg.lr, eps=cfg.adam_eps)
        self.critic_opt = Adam(self.nets.critic_parameters(), lr=cfg.lr, eps=cfg.adam_eps)
        self.alpha_opt = Adam([self.log_alpha], lr=cfg.lr, eps=cfg.adam_eps)
        self.twin = TwinQ(self.nets.critics)
        self.twin_targets = TwinQ(self.nets.targets)
        self.batch = _BatchBuffers(device, cfg.batch_size, obs_spec.size, action_spec.dim, cfg.prioritized)
        # Every metric of an update in one device block, read back with one copy:
        # [critic_loss, alpha, actor_loss, alpha_loss, critic_grad_sq, actor_grad_sq, -, -,
        #  q_target[B], logp[B], td_abs[B]].
        B = cfg.batch_size
        # scalars, q_target, td_abs, then the sample's log-probabilities of
        # obs (the logp metric) and next_obs back to back
        blk = DeviceArray(device, (8 + 4 * B,))
        blk.fill(0.0)
        self._metric_block = blk
        self._critic_out = {"loss": blk.view(0, (1, 1)), "alpha": blk.view(1, (1, 1)),
                            "q_target": blk.view(8, (B, 1)), "td_abs": blk.view(8 + B, (B, 1))}
        self._actor_out = {"actor_loss": blk.view(2, (1, 1)), "alpha_loss": blk.view(3, (1, 1))}
        self._logp_all = blk.view(8 + 2 * B, (2 * B, 1))
        self._logp_out = blk.view(8 + 2 * B, (B, 1))
        self._stacked = isinstance(self.nets.policy.head, GaussianHead) and \
            _linear_relu_pairs(self.nets.policy.encoder) is not None
        self.critic_opt.grad_sq = blk.view(4, (1, 1))
        self.actor_opt.grad_sq = blk.view(5, (1, 1))
        self._reader = MetricReader(device)
        self._graph = None
        self._graph_metrics = None
        # input slots (enable_input_slots): slot k's graph reads _slot_batches[k]
        self._slots = None
        self._slot_batches: list = []
        self._pool = None
        self.update_count = 0
        self.n_envs = int(n_envs)
        self._acting = ActingNet(self.nets.policy, obs_spec, device, width=cfg.batch_size, lanes=self.n_envs,
                                 decision=SquashedDecision(self.scale), mode=cfg.act_mode)
        self.frame_count = 0
        self._rng = np.random.default_rng(seed)
        self._eval_rng = np.random.default_rng(seed).spawn(1)[0]
        H = _FusedUpdate.width(self)
        self._fused = None if H is None else _FusedUpdate(self, H)

    # -- state ---------------------------------------------------------------

    _WEIGHT_KEYS = ("nets", "log_alpha")
    _RUN_KEYS = ("actor_opt", "critic_opt", "alpha_opt", "frame_count", "update_count", "rng_state")

    def state_dict(self, *, weights_only: bool = False) -> dict:
        """The reference agent's state tree (ttrl/algos/sac/agent.py:249-264)
        for the parts a learner holds; the agent loop's autoreset phase and
        update clock are not part of it."""
        nets = to_reference_keys(self.nets.state_dict(), TOWERS_SAC, self.obs_spec.name)
        return assemble(self.cfg, {"nets": nets, "log_alpha": self.log_alpha.numpy()},
                        {"actor_opt": self.actor_opt.state_dict(), "critic_opt": self.critic_opt.state_dict(),
                         "alpha_opt": self.alpha_opt.state_dict(), "frame_count": self.frame_count,
                         "update_count": self.update_count, "rng_state": self._rng.bit_generator.state},
                        weights_only=weights_only)

    def load_state_dict(self, state: dict, *, weights_only: bool = False) -> None:
        """In place, so the captured update keeps its buffers
        (ttrl/algos/sac/agent.py:266-282)."""
        load_run = validate(state, algo="SAC", config=self.cfg, weight_keys=self._WEIGHT_KEYS,
                            run_keys=self._RUN_KEYS, weights_only=weights_only)
        log_alpha = np.asarray(state["log_alpha"], np.float32)
        if log_alpha.size != 1:
            raise ValueError(f"SAC.load_state_dict: log_alpha must hold one value, got shape {log_alpha.shape}")
        self.nets.load_state_dict(from_reference_keys(state["nets"], TOWERS_SAC, self.obs_spec.name))
        self.log_alpha.data.upload(log_alpha.reshape(tuple(self.log_alpha.shape)))
        if not load_run:
            return
        self.actor_opt.load_state_dict(state["actor_opt"])
        self.critic_opt.load_state_dict(state["critic_opt"])
        self.alpha_opt.load_state_dict(state["alpha_opt"])
        self.frame_count = int(state["frame_count"])
        self.update_count = int(state["update_count"])
        self._rng.bit_generator.state = state["rng_state"]

    # -- acting --------------------------------------------------------------

    def act(self, obs, *, deterministic: bool = False, episode_starts=None) -> np.ndarray:
        """One action per lane from the squashed-Gaussian policy; the noise
        is drawn on the host from the same stream and in the same shape as
        the reference's sample (ttrl/algos/sac/agent.py:111-125,
        ttrl/algos/sac/policy.py:42-59), the sample itself on the device.
        `deterministic` takes tanh of the mean."""
        lanes = int(np.asarray(obs).shape[0])
        noise = None
        if not deterministic:
            noise = self._rng.standard_normal((lanes, self.action_spec.dim))
        out = self._acting.decide(obs, noise=noise, deterministic=deterministic)
        if not deterministic:
            self.frame_count += lanes
        return out["action"]

    # -- one update ----------------------------------------------------------

    def _policy_both(self):
        """The policy and its sample over [obs; next_obs], one launch each
        layer and one sample launch, the tape over the obs rows: the critic
        step leaves the policy unchanged, so the actor's forward can run with
        the soft target's.  -> (action, logp) on the tape, (a_next, logp_next)."""
        b = self.batch
        action, logp, (a_next, logp_next) = policy_sample_rows(self.nets.policy, b.obs_pair, b.B, b.noise_pair,
                                                               self.scale, self._logp_all)
        return (action, logp), (a_next, Tensor(logp_next))

    def _critic_region(self, nxt=None) -> dict:
        b = self.batch
        if nxt is not None:
            # the target critics on (s', a') and the critics on (s, a): one launch per layer
            a_next, logp_next = nxt
            q, q_next = self.twin.forward_with_targets(self.twin_targets, b["next_obs"], a_next, b["obs"],
                                                       b["actions"], b["obs_actions"])
        else:
            with no_grad():
                head_n = policy_packed(self.nets.policy, b["next_obs"])
                a_next, logp_next = squashed_sample(head_n, b["next_noise"], self.scale)
                q_next = self.twin_targets.forward(b["next_obs"], a_next)
            q = self.twin.forward(obs_action=b["obs_actions"])
        loss, m = sac_critic_loss(q, q_next, logp_next, self.log_alpha, b["rewards"], b["dones"], b["discounts"],
                                  b["is_weights"] if self.cfg.prioritized else None, out=self._critic_out)
        loss.backward()
        out = {"critic_loss": loss, "alpha": m["alpha"], "q_target": m["q_target"]}
        if self.cfg.prioritized:
            out["td_abs"] = m["td_abs"]
        return out

    def _actor_region(self, sampled=None) -> dict:
        b = self.batch
        if sampled is not None:
            action, logp = sampled
        else:
            head = policy_packed(self.nets.policy, b["obs"])
            action, logp = squashed_sample(head, b["noise"], self.scale, logp_out=self._logp_out)
        q_pi = self.twin.forward(b["obs"], action, train_params=False)
        actor, dual = sac_actor_losses(q_pi, logp, self.log_alpha, self.target_entropy, self.cfg.learn_alpha,
                                       out=self._actor_out)
        actor.backward()
        out = {"actor_loss": actor, "logp": Tensor(logp.data)}
        if dual is not None:
            dual.backward()
            out["alpha_loss"] = dual
        return out

    def _body(self) -> dict:
        if self._fused is not None:
            return self._fused.body()
        self.critic_opt.zero_grad()
        self.actor_opt.zero_grad()
        self.alpha_opt.zero_grad()
        # The reference's order (ttrl/algos/sac/agent.py:229-236): critic step, actor
        # and temperature steps, Polyak blend.  The critic's finish waits for the
        # others so all three finish in one launch; actor, temperature and blend
        # share one launch (disjoint buffers, the blend reading the stepped critic).
        if self._stacked:
            sampled, nxt = self._policy_both()
            critic = self._critic_region(nxt)
        else:
            sampled = None
            critic = self._critic_region()
        self.critic_opt.step_deferred(0)
        actor = self._actor_region(sampled)
        stepped = [(self.actor_opt, 1)] + ([(self.alpha_opt, 2)] if self.cfg.learn_alpha else [])
        adam_multi(self.device, stepped,
                   polyak=(self.nets.targets.arena.data, self.nets.critics.arena.data, self.cfg.tau))
        finish_steps(self.device, [(self.critic_opt, 0)] + stepped)
        metrics = dict(critic)
        metrics.update(actor)
        metrics["critic_grad_sq"] = Tensor(self.critic_opt.grad_sq)
        metrics["actor_grad_sq"] = Tensor(self.actor_opt.grad_sq)
        return metrics

    def enable_input_slots(self, n: int) -> None:
        """n batch blocks of one layout (slot 0 is `batch.block`), one graph
        captured against each at the first graph update (engine.slots);
        `slot_block(k)` is slot k's block and `replay_slot(k)` runs the update
        on it.  Graph mode, before the first update."""
        if self.cfg.step_mode != "graph":
            raise ValueError("SACLearner.enable_input_slots: input slots need step_mode='graph'")
        if self._graph is not None or self._slots is not None:
            raise RuntimeError("SACLearner.enable_input_slots: call it once, before the first update")
        check_slot_count("SACLearner.enable_input_slots", n)
        b = self.batch
        self._slot_batches = [b] + [_BatchBuffers(self.device, b.B, self.obs_spec.size, self.action_spec.dim,
                                                  self.cfg.prioritized) for _ in range(n - 1)]
        self._slots = InputSlots(self.device, [x.block for x in self._slot_batches])

    def slot_block(self, k: int) -> DeviceArray:
        if self._slots is None:
            raise RuntimeError("SACLearner.slot_block: call enable_input_slots() first")
        return self._slot_batches[k].block

    def _capture_slots(self) -> None:
        """Slot k >= 1's graph: the same update over slot k's batch block."""
        want = metric_ptrs(self._graph_metrics)
        self._slots.graphs[0] = self._graph
        first = self.batch
        try:
            for k, b in enumerate(self._slot_batches[1:], start=1):
                self.batch = b
                graph, metrics = capture(self.device, self._body)
                self._slots.graphs[k] = graph
                if metric_ptrs(metrics) != want:
                    raise RuntimeError("SACLearner.enable_input_slots: a slot's graph writes its metrics elsewhere")
        finally:
            self.batch = first

    def replay_slot(self, k: int) -> None:
        """Launch the captured update on slot k's batch block without
        reading metrics; they are read as after `replay()`."""
        if self._slots is None:
            raise RuntimeError("SACLearner.replay_slot: call enable_input_slots() before the first update")
        if self._graph is None:
            raise RuntimeError("SACLearner.replay_slot: update once in graph mode first (it captures)")
        self._slots.launch(k)
        self._replayed()

    def run_slot(self, k: int) -> dict:
        """Slot k's update with its metrics read back: one ttrl_graph_step
        replaying slot k's graph on the batch already in its block, the packed
        metric block copied to the host, one wait; -> the metrics as
        `update` returns them."""
        if self._slots is None or self._graph is None:
            raise RuntimeError("SACLearner.run_slot: enable_input_slots() and one graph update first")
        if not 0 <= k < len(self._slot_batches):
            raise IndexError(f"input slot {k} outside [0, {len(self._slot_batches)})")
        span = self._reader.span
        if span is None:
            self.replay_slot(k)
            out = self._reader.read(self._graph_metrics)
        else:
            ptr, n, _ = span
            self.device.call("ttrl_graph_step", self._slots.graphs[k]._graph, None, None, C.c_size_t(0),
                             C.c_void_p(self._reader.image.ptr), C.c_void_p(ptr), C.c_size_t(n))
            self._replayed()
            out = self._reader._unpack(self._graph_metrics)
        self.update_count += 1
        return self.summarize(out)

    def _run(self) -> dict:
        """One update; -> its metrics, read from the device."""
        binder = self.batch.binder
        if self.cfg.step_mode == "eager":
            binder.flush()
            metrics = self._body()
            self._reader.bind(metrics)
            return self._reader.read(metrics)
        dev = self.device
        if self._graph is None:
            # First update runs eagerly (warming the pool), then the body is
            # captured; later updates replay it.
            binder.flush()
            self._pool = dev.create_pool()
            with dev.use_pool(self._pool):
                metrics = self._body()
                dev.synchronize()
                self._graph, self._graph_metrics = capture(dev, self._body)
                if self._slots is not None:
                    self._capture_slots()
            self._reader.bind(self._graph_metrics)
            return self._reader.read(metrics)
        span = self._reader.span
        sent = binder.take_single_range() if span is not None else None
        if sent is None:
            self.replay()
            return self._reader.read(self._graph_metrics)
        # One call: the batch in, the replay, the metric block out, one wait.
        b, e = sent
        ptr, n, _ = span
        dev.call("ttrl_graph_step", self._graph._graph, C.c_void_p(binder.block.ptr + b),
                 C.c_void_p(binder.image.ptr + b), C.c_size_t(e - b), C.c_void_p(self._reader.image.ptr),
                 C.c_void_p(ptr), C.c_size_t(n))
        self._replayed()
        return self._reader._unpack(self._graph_metrics)

    def replay(self) -> None:
        """Launch the captured update without reading metrics (benchmark loop)."""
        self.batch.flush()
        self._graph.replay()
        self._replayed()

    def _replayed(self) -> None:
        for opt in (self.critic_opt, self.actor_opt) + ((self.alpha_opt,) if self.cfg.learn_alpha else ()):
            opt._replayed()

    def update(self, batch: dict | None = None) -> dict:
        if batch is not None:
            self.batch.load_batch(batch)
        out = self._run()
        self.update_count += 1
        return self.summarize(out)

    def summarize(self, m: dict) -> dict:
        """The reference's metric keys (ttrl/algos/sac/step.py:115-130)."""
        def s(v):
            return float(np.asarray(v).reshape(-1)[0])

        out = {
            "critic_loss": s(m["critic_loss"]),
            "actor_loss": s(m["actor_loss"]),
            "alpha_loss": s(m["alpha_loss"]) if self.cfg.learn_alpha else 0.0,
            "alpha": s(m["alpha"]),
            "entropy": float(-np.mean(np.asarray(m["logp"], np.float64))),
            "mean_q_target": float(np.mean(np.asarray(m["q_target"], np.float64))),
            "critic_grad_norm": float(np.sqrt(max(s(m["critic_grad_sq"]), 0.0))),
            "actor_grad_norm": float(np.sqrt(max(s(m["actor_grad_sq"]), 0.0))),
        }
        out["q_target"] = np.asarray(m["q_target"]).reshape(-1)
        out["logp"] = np.asarray(m["logp"]).reshape(-1)
        if "td_abs" in m:
            out["td_abs"] = np.asarray(m["td_abs"]).reshape(-1)
        return out

    def close(self) -> None:
        self._acting.close()
        self.batch.close()
        self._reader.close()
        slots, self._slots = self._slots, None
        if slots is not None:
            slots.close_extra()
            for b in self._slot_batches[1:]:
                b.close()
            self._slot_batches = []
        if self._graph is not None:
            self._graph.close()
            self._graph = None
            self._graph_metrics = None
        if self._pool is not None and not self.device.closed:
            self.device.release_pool(self._pool)
            self._pool = None
