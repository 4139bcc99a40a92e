"""The committed golden fixtures (tests/golden/) on the CPU: the reference's
literal known answers against the oracle and the library's host-side
geometry check, and the oracle against every regression fixture it wrote
(a drift in the oracle, or in numpy's seeded streams, fails here)."""

from __future__ import annotations

import ctypes as C
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import adam, conv, ppo

GOLDEN = Path(__file__).resolve().parent / "golden"


def _known():
    return json.loads((GOLDEN / "known_answers.json").read_text())


def test_conv_out_size_known_answers_oracle_and_library():
    from ttrl_amd import _lib
    k = _known()
    for case in k["conv_out_size"]:
        assert conv.out_size(case["size"], case["kernel"], case["stride"], case["padding"]) == case["out"]
        out = C.c_int(0)
        assert _lib.lib().ttrl_conv_out_size(case["size"], case["kernel"], case["stride"], case["padding"],
                                             C.byref(out)) == _lib.TTRL_OK
        assert out.value == case["out"]
    for case in k["conv_out_size_ragged"]:
        with pytest.raises(ValueError, match="ragged"):
            conv.out_size(case["size"], case["kernel"], case["stride"], case["padding"])
        out = C.c_int(0)
        assert _lib.lib().ttrl_conv_out_size(case["size"], case["kernel"], case["stride"], case["padding"],
                                             C.byref(out)) == _lib.TTRL_EINVAL
    sizes = [k["nature_cnn_geometry"][0]]
    for kern, stride in ((8, 4), (4, 2), (3, 1)):
        sizes.append(conv.out_size(sizes[-1], kern, stride, 0))
    assert sizes == k["nature_cnn_geometry"]
    assert sizes[-1] * sizes[-1] * 64 == k["nature_cnn_flatten"]


def test_adam_fused_scalars_known_answers():
    for c in _known()["adam_fused_scalars"]:
        alpha_t, eps_t = adam.fused_scalars(c["lr"], c["b1"], c["b2"], c["eps"], c["t"])
        got = alpha_t * c["S"] / (math.sqrt(c["V"]) + eps_t)
        assert got == pytest.approx(c["update"], rel=1e-12)


def test_gae_padding_known_answer():
    g = _known()["gae_padding"]
    T = len(g["rewards"])
    adv, _ = ppo.gae(np.array(g["rewards"], np.float32).reshape(T, 1), np.zeros((T, 1), np.float32),
                     np.zeros((T, 1), np.float32), np.zeros(1, np.float32), g["gamma"], g["lam"],
                     np.array(g["valid"], np.float32).reshape(T, 1))
    assert adv.reshape(-1).tolist() == g["advantages"]


@pytest.mark.parametrize("name", ["conv_small.npz", "gae_128x8.npz", "ppo_b64.npz", "dqn_b4_36.npz"])
def test_oracle_reproduces_fixture(name):
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    fresh = mg.build_all()[name]
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        assert sorted(f.files) == sorted(fresh)
        for key in f.files:
            a, b = f[key], np.asarray(fresh[key])
            assert a.dtype == b.dtype and a.shape == b.shape, key
            assert np.array_equal(a, b), key
