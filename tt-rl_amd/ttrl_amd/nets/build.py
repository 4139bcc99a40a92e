"""Network builders (ttrl/nets/build.py:82-215).

Every network is built inside its own `ParamArena`, so its parameters are
one flat device buffer (one Adam launch, one target copy, one Polyak blend).
The SAC critics share one arena and so do the targets: the twin critics then
sit at a fixed stride from each other, which lets both run in one grouped
launch per layer.  Construction order, and so the init draws from the global
numpy RNG, is the reference's: policy tower, policy head, critics, targets.
"""

from __future__ import annotations

from ttrl_amd.engine.layers import Linear, ReLU, Sequential
from ttrl_amd.engine.nn import ModuleList
from ttrl_amd.engine.tensor import ParamArena
from ttrl_amd.nets.encoders import identity_encoder, image_encoder, vector_encoder
from ttrl_amd.nets.heads import CategoricalHead, GaussianHead, QHead, ValueHead
from ttrl_amd.nets.models import ActorCritic, ConcatEncoder, ContinuousCritic, EncoderHead, SacNets

__all__ = ["build_actor_critic", "build_encoder", "build_q_net", "build_sac_nets"]


def build_encoder(obs_spec, device, *, batch: int, name: str = "auto", role: str = "actor", **kwargs):
    if name == "auto":
        if obs_spec.kind == "image":
            name = "nature_cnn"
        else:
            name = "identity" if role == "critic" else "mlp"
    if name == "nature_cnn":
        return image_encoder(obs_spec, device, batch=batch, **kwargs)
    if name == "mlp":
        return vector_encoder(obs_spec, device, batch=batch, **kwargs)
    if name == "identity":
        return identity_encoder(obs_spec, device, batch=batch, **kwargs)
    raise ValueError(f"unknown encoder {name!r}; choose 'auto', 'nature_cnn', 'mlp' or 'identity'")


def build_q_net(obs_spec, action_spec, device, *, batch: int, encoder: str = "auto", **encoder_kwargs):
    """Encoder + raw Q head, for DQN (discrete actions only)."""
    if action_spec.kind != "discrete":
        raise ValueError(f"build_q_net supports discrete actions only, got {action_spec.kind!r}")
    with ParamArena(device, "q_net") as arena:
        tower = build_encoder(obs_spec, device, batch=batch, name=encoder, **encoder_kwargs)
        net = EncoderHead(tower, QHead(tower.out_features, action_spec.width, device))
    net.arena = arena
    return net


def build_actor_critic(obs_spec, action_spec, device, *, batch: int, encoder: str = "auto",
                       **encoder_kwargs) -> ActorCritic:
    """Shared trunk + categorical policy head + value head, for PPO
    (ttrl/nets/build.py:95-117, discrete actions; every observation field
    belongs to the actor here, so one trunk fills both slots)."""
    if action_spec.kind != "discrete":
        raise ValueError(f"build_actor_critic supports discrete actions only, got {action_spec.kind!r}")
    with ParamArena(device, "actor_critic") as arena:
        trunk = build_encoder(obs_spec, device, batch=batch, name=encoder, **encoder_kwargs)
        policy = CategoricalHead(trunk.out_features, action_spec.width, device)
        value = ValueHead(trunk.out_features, device)
        net = ActorCritic(trunk, trunk, policy, value)
    net.arena = arena
    return net


def build_sac_nets(obs_spec, action_spec, device, *, batch: int, encoder: str = "auto",
                   critic_encoder: str = "auto", n_critics: int = 2, critic_hidden=(256, 256), head_kwargs=None,
                   encoder_kwargs=None, critic_encoder_kwargs=None) -> SacNets:
    if action_spec.kind != "continuous":
        raise ValueError(f"build_sac_nets supports continuous actions only, got {action_spec.kind!r}")
    if n_critics < 2:
        raise ValueError(f"build_sac_nets: n_critics must be >= 2, got {n_critics}.")
    widths = tuple(int(w) for w in critic_hidden)
    if not widths or min(widths) < 1:
        raise ValueError(f"build_sac_nets: critic_hidden must hold at least one positive width, got {critic_hidden}.")

    def one_critic() -> ContinuousCritic:
        tower = build_encoder(obs_spec, device, batch=batch, name=critic_encoder, role="critic",
                              **(critic_encoder_kwargs or {}))
        joint = ConcatEncoder(tower, action_spec.width)
        layers = []
        in_features = joint.out_features
        for width in widths:
            layers += [Linear(in_features, width, device), ReLU()]
            in_features = width
        layers.append(ValueHead(in_features, device))
        return ContinuousCritic(joint, Sequential(*layers))

    with ParamArena(device, "policy") as pa:
        tower = build_encoder(obs_spec, device, batch=batch, name=encoder, **(encoder_kwargs or {}))
        policy = EncoderHead(tower, GaussianHead(tower.out_features, action_spec.width, device,
                                                 **(head_kwargs or {})))
    with ParamArena(device, "critics") as ca:
        critics = ModuleList([one_critic() for _ in range(n_critics)])
    with ParamArena(device, "targets") as ta:
        targets = ModuleList([one_critic() for _ in range(n_critics)])
    policy.arena, critics.arena, targets.arena = pa, ca, ta
    nets = SacNets(policy=policy, critics=critics, targets=targets)
    nets.sync_targets()
    return nets
