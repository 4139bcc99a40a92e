"""Host side of the acting step, on the CPU: the oracle's acting rules pinned
by their closed forms and special cases, and the module-tree view that
`ActingNet` builds per lane count (ttrl/nets/acting.py:69-114; the sharing
case of the reference's tests/hardware/test_acting_width.py:135-148)."""

from __future__ import annotations

import numpy as np
import pytest


def test_epsilon_schedule_closed_forms():
    from oracle.act import epsilon

    assert epsilon(0, 1.0, 0.01, 1000) == 1.0
    assert epsilon(1000, 1.0, 0.01, 1000) == pytest.approx(0.01)
    assert epsilon(10 ** 9, 1.0, 0.01, 1000) == pytest.approx(0.01)
    assert epsilon(500, 1.0, 0.0, 1000) == pytest.approx(0.5)


def test_epsilon_greedy_special_cases():
    from oracle.act import epsilon_greedy

    greedy = np.array([3, 1, 4, 1, 5, 2])
    # eps = 0: the greedy actions, whatever the draws.
    assert np.array_equal(epsilon_greedy(greedy, 6, 0.0, np.random.default_rng(0)), greedy)
    # eps = 1: exactly the random actions, drawn after the uniform draws.
    rng = np.random.default_rng(1)
    rng.random(6)
    want = rng.integers(0, 6, size=6)
    assert np.array_equal(epsilon_greedy(greedy, 6, 1.0, np.random.default_rng(1)), want)
    # In between: each lane takes the random action iff its draw is below eps.
    rng = np.random.default_rng(2)
    draws = rng.random(6)
    rand = rng.integers(0, 6, size=6)
    got = epsilon_greedy(greedy, 6, 0.4, np.random.default_rng(2))
    assert np.array_equal(got, np.where(draws < 0.4, rand, greedy))


def test_sac_act_deterministic_is_tanh_of_mean_and_stochastic_is_the_sample():
    from oracle.act import sac_act
    from oracle.sac import SacParams

    rng = np.random.default_rng(3)
    trunk = [(rng.standard_normal((5, 8)) * 0.3, rng.standard_normal(8) * 0.1),
             (rng.standard_normal((8, 8)) * 0.3, rng.standard_normal(8) * 0.1)]
    mean = (rng.standard_normal((8, 2)) * 0.3, rng.standard_normal(2) * 0.1)
    log_std = (rng.standard_normal((8, 2)) * 0.1, rng.standard_normal(2) * 0.1)
    P = SacParams(trunk=trunk, mean=mean, log_std=log_std, critics=[], targets=[], log_alpha=0.0)
    obs = rng.standard_normal((4, 5))
    h = np.maximum(np.maximum(obs @ trunk[0][0] + trunk[0][1], 0) @ trunk[1][0] + trunk[1][1], 0)
    mu = h @ mean[0] + mean[1]
    a, lp, m, _ = sac_act(P, obs, deterministic=True, centre=np.array([0.5, -1.0]), half_width=np.array([2.0, 1.0]))
    assert np.allclose(m, mu)
    assert np.allclose(a, np.array([0.5, -1.0]) + np.array([2.0, 1.0]) * np.tanh(mu))
    assert np.all(lp == 0.0)
    # Stochastic with a zero log_std head: u = mean + noise, and the action
    # is tanh(u) on [-1, 1].
    P0 = SacParams(trunk=trunk, mean=mean, log_std=(np.zeros((8, 2)), np.zeros(2)), critics=[], targets=[],
                   log_alpha=0.0)
    a, lp, _m, ls = sac_act(P0, obs, rng=np.random.default_rng(4))
    noise = np.random.default_rng(4).standard_normal((4, 2))
    assert np.all(ls == 0.0)
    assert np.allclose(a, np.tanh(mu + noise))
    # N(0, 1) density of the noise times the tanh Jacobian.
    u = mu + noise
    want = np.sum(-0.5 * noise ** 2 - 0.5 * np.log(2 * np.pi) - np.log(1 - np.tanh(u) ** 2), axis=1)
    assert np.allclose(lp, want, rtol=1e-9, atol=1e-9)


def _toy_modules():
    from ttrl_amd.engine.nn import Module, ModuleDict, ModuleList

    class Leaf(Module):
        def __init__(self, tag):
            self.tag = tag

    class Net(Module):
        def __init__(self):
            trunk = Leaf("trunk")
            self.encoders = ModuleDict({"actor": trunk, "critic": trunk})
            self.heads = ModuleList([Leaf("a"), Leaf("b")])
            self.scale = 0.5

    return Net()


def test_net_at_batch_keeps_what_the_net_shared():
    from ttrl_amd.nets.acting import net_at_batch

    net = _toy_modules()
    assert net.encoders["actor"] is net.encoders["critic"]
    view = net_at_batch(net, 2)
    assert view is not net
    assert view.encoders["actor"] is view.encoders["critic"]
    assert view.encoders["actor"] is not net.encoders["actor"]
    assert [h.tag for h in view.heads] == ["a", "b"]
    assert view.scale == 0.5


def test_folded_convolutions_are_refused():
    from ttrl_amd.engine.nn import Module
    from ttrl_amd.nets.acting import check_encoder_layout

    class Geom:
        fold = 2

    class Folded(Module):
        def __init__(self):
            self.geom = Geom()

    class Net(Module):
        def __init__(self):
            self.conv = Folded()

    with pytest.raises(ValueError, match="fold=2"):
        check_encoder_layout(Net())


def test_a_shared_trunk_checkpoints_once():
    """One self-serialising module in two slots appears once in the state
    (ttrl/engine/nn/discovery.py:128-139), as a shared actor-critic trunk."""
    import numpy as np
    from ttrl_amd.engine.nn import Module, ModuleDict

    class Leaf(Module):
        def state_dict(self):
            return {"w": np.ones(2)}

    class Net(Module):
        def __init__(self):
            trunk = Leaf()
            self.encoders = ModuleDict({"actor": trunk, "critic": trunk})
            self.head = Leaf()

    assert list(Net().state_dict()) == ["encoders.actor.w", "head.w"]
