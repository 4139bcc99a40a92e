"""Spec-built networks (ttrl/nets): Nature-CNN and MLP towers, heads, and the
DQN / SAC / PPO network builders."""

from ttrl_amd.nets.build import build_actor_critic, build_q_net, build_sac_nets
from ttrl_amd.nets.encoders import Encoder, ScaledLinear, identity_encoder, image_encoder, vector_encoder
from ttrl_amd.nets.heads import CategoricalHead, GaussianHead, QHead, ValueHead
from ttrl_amd.nets.models import ActorCritic, ConcatEncoder, ContinuousCritic, EncoderHead, SacNets
from ttrl_amd.nets.towers import NATURE_CNN, ConvStage

__all__ = [
    "ActorCritic", "build_actor_critic", "build_q_net", "build_sac_nets", "Encoder", "ScaledLinear", "identity_encoder", "image_encoder",
    "vector_encoder", "CategoricalHead", "GaussianHead", "QHead", "ValueHead", "ConcatEncoder",
    "ContinuousCritic", "EncoderHead", "SacNets", "NATURE_CNN", "ConvStage",
]
