"""The recurrent actor-critic (ttrl/nets/recurrent.py:49-196): a trunk, a GRU
memory between the trunk and the heads, a policy head and a value head, the
heads sized from the memory's width.  Built here for a shared trunk (every
observation field belongs to the actor), so one trunk and one memory serve
both heads.

`forward(obs, h0, starts, seq_len)` is the training path over a minibatch of
whole sequences, rows time-major (row t * n_seq + sequence,
ttrl/buffers/sequences.py:141-155): the trunk over every row, the unroll over
(seq_len, n_seq, features) from h0 with the episode-start mask on the state
entering each step, and both heads in one launch as packed
[logits | value] rows.
"""

from __future__ import annotations

from ttrl_amd.engine.nn import Module, ModuleDict
from ttrl_amd.engine.recurrent import GRU, _reshape_node
from ttrl_amd.engine.tensor import ParamArena
from ttrl_amd.nets.heads import CategoricalHead, ValueHead, policy_value_packed

__all__ = ["ACTOR", "CRITIC", "RecurrentActorCritic", "build_recurrent_actor_critic"]

ACTOR = "actor"
CRITIC = "critic"


class RecurrentActorCritic(Module):
    def __init__(self, trunk, memory: GRU, policy, value, hidden_size: int):
        self.encoders = ModuleDict({ACTOR: trunk, CRITIC: trunk})
        self.memories = ModuleDict({ACTOR: memory, CRITIC: memory})
        self.heads = ModuleDict({"policy": policy, "value": value})
        self.hidden_size = int(hidden_size)

    @property
    def shared(self) -> bool:
        return True

    @property
    def hidden_sizes(self) -> dict:
        return {ACTOR: self.hidden_size}

    def forward_packed(self, obs, h0, starts, *, seq_len: int):
        """-> (rows, A + 1) packed [logits | value] over a sequence minibatch."""
        features = self.encoders[ACTOR](obs)
        rows, width = (int(d) for d in features.shape)
        if rows % seq_len:
            raise ValueError(f"RecurrentActorCritic: {rows} rows is not a whole number of sequences of "
                             f"seq_len={seq_len}. A recurrent minibatch is a set of whole sequences, so choose a "
                             f"minibatch_size that is a multiple of recurrent.seq_len.")
        n_seq = rows // seq_len
        sequence = _reshape_node(features, (seq_len, n_seq, width))
        outputs, _final = self.memories[ACTOR](sequence, h0, starts)
        state = _reshape_node(outputs, (rows, self.hidden_size))
        return policy_value_packed(self.heads["policy"], self.heads["value"], state)

    def forward(self, obs, h0, starts, *, seq_len: int):
        head = self.forward_packed(obs, h0, starts, seq_len=seq_len)
        A = int(head.shape[1]) - 1
        from ttrl_amd.engine.ops import split

        logits, value = split(head, (A, 1), dim=-1)
        return logits, value


def build_recurrent_actor_critic(obs_spec, action_spec, device, *, batch: int, hidden_size: int,
                                 encoder: str = "auto", **encoder_kwargs) -> RecurrentActorCritic:
    """Trunk, GRU(trunk width, hidden_size), categorical and value heads over
    the memory (ttrl/nets/recurrent.py:170-196), in one parameter arena."""
    from ttrl_amd.nets.build import build_encoder

    if hidden_size < 1:
        raise ValueError(f"build_recurrent_actor_critic: hidden_size must be >= 1, got {hidden_size}")
    if action_spec.kind != "discrete":
        raise ValueError("build_recurrent_actor_critic supports discrete actions only")
    with ParamArena(device, "recurrent_actor_critic") as arena:
        trunk = build_encoder(obs_spec, device, batch=batch, name=encoder, **encoder_kwargs)
        memory = GRU(trunk.out_features, hidden_size, device)
        policy = CategoricalHead(hidden_size, action_spec.width, device)
        value = ValueHead(hidden_size, device)
        net = RecurrentActorCritic(trunk, memory, policy, value, hidden_size)
    net.arena = arena
    return net
