"""Network compositions (ttrl/nets/models.py:20-135, ttrl/nets/fusion.py:36-71)."""

from __future__ import annotations

from dataclasses import dataclass

from ttrl_amd.engine.nn import Module, ModuleDict, ModuleList
from ttrl_amd.engine.ops import concat


def _actor(obs):
    return getattr(obs, "actor", obs)


def _critic(obs):
    return getattr(obs, "critic", obs)


class EncoderHead(Module):
    """Encoder -> one head; forward returns whatever the head returns."""

    def __init__(self, encoder, head):
        self.encoder = encoder
        self.head = head

    def forward(self, obs):
        return self.head(self.encoder(_actor(obs)))


class ActorCritic(Module):
    """Actor trunk, critic trunk, policy head, value head
    (ttrl/nets/models.py:42-71).  Parameters are named `encoders.actor.*`
    and `heads.policy.*`; one trunk in both slots is the shared-trunk case,
    run once, whose gradient is the sum of the two heads'.
    `forward(obs) -> (policy_out, value)`."""

    def __init__(self, actor, critic, policy, value):
        self.encoders = ModuleDict({"actor": actor, "critic": critic})
        self.heads = ModuleDict({"policy": policy, "value": value})

    @property
    def shared_trunk(self) -> bool:
        return self.encoders["actor"] is self.encoders["critic"]

    def forward(self, obs):
        actor, critic = self.encoders["actor"], self.encoders["critic"]
        features = actor(_actor(obs))
        critic_features = features if critic is actor else critic(_critic(obs))
        return self.heads["policy"](features), self.heads["value"](critic_features)


class ConcatEncoder(Module):
    """A tower's features with the action appended: concat(tower(s), a)."""

    def __init__(self, tower, action_width: int):
        self.tower = tower
        self.action_width = int(action_width)
        self.out_features = tower.out_features + self.action_width

    def forward(self, obs, action):
        return concat([self.tower(obs), action], dim=-1)


class ContinuousCritic(Module):
    """Q(s, a): encode s, append a, then the MLP head."""

    def __init__(self, encoder: ConcatEncoder, head):
        self.encoder = encoder
        self.head = head

    def forward(self, obs, action):
        return self.head(self.encoder(_critic(obs), action))


@dataclass
class SacNets:
    """Policy, twin critics and their lagged targets."""

    policy: Module
    critics: ModuleList
    targets: ModuleList

    def sync_targets(self) -> None:
        for critic, target in zip(self.critics, self.targets):
            target.copy_from(critic)

    def policy_parameters(self):
        return list(self.policy.parameters())

    def critic_parameters(self):
        return list(self.critics.parameters())

    def state_dict(self) -> dict:
        out = {}
        for name, module in (("policy", self.policy), ("critics", self.critics), ("targets", self.targets)):
            for key, array in module.state_dict().items():
                out[f"{name}.{key}"] = array
        return out

    def load_state_dict(self, state: dict) -> None:
        for name, module in (("policy", self.policy), ("critics", self.critics), ("targets", self.targets)):
            prefix = f"{name}."
            module.load_state_dict({k[len(prefix):]: v for k, v in state.items() if k.startswith(prefix)})
