"""The allocation-free Adam step (ttrl_adam_step_static) against
ttrl_adam_step, called through the C ABI: on identical copies of
parameters, gradients, moments and the device step counter, two calls in a
row -- the second over a smaller range -- must give bit-identical
parameters, moments, step counters and sums of squared gradients (the two
entry points run the same kernels; only where the per-workgroup partial
sums live differs)."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _arrays(device, n, seed):
    from ttrl_amd.engine.tensor import DeviceArray

    rng = np.random.default_rng(seed)
    host = {"p": rng.standard_normal(n).astype(np.float32), "g": rng.standard_normal(n).astype(np.float32),
            "S": (0.1 * rng.standard_normal(n)).astype(np.float32), "V": rng.random(n).astype(np.float32)}
    out = {}
    for k, v in host.items():
        a = DeviceArray(device, (n,))
        a.upload(v)
        out[k] = a
    step = DeviceArray(device, (1,), np.int32)
    step.upload(np.array([3], np.int32))
    gsq = DeviceArray(device, (1,))
    gsq.upload(np.array([0.5], np.float32))
    out["step"], out["gsq"] = step, gsq
    return out


def _read(arrs):
    return {k: a.numpy() for k, a in arrs.items()}


@pytest.mark.parametrize("accumulate", [0, 1])
def test_static_adam_matches_the_context_entry_point(device, accumulate):
    from ttrl_amd import _lib

    lib = _lib.lib()
    stream = C.c_void_p(lib.ttrl_stream(device.ctx))
    hyper = (C.c_float(3e-4), C.c_float(0.9), C.c_float(0.999), C.c_float(1e-8), C.c_float(0.0))
    for call, n in enumerate((1_687_206, 70_406 + 3)):  # the DQN arena, then a smaller range with a tail
        ref = _arrays(device, n, 10 + call)
        got = _arrays(device, n, 10 + call)
        device.call("ttrl_adam_step", ref["p"].vp, ref["g"].vp, ref["S"].vp, ref["V"].vp, C.c_long(n),
                    ref["step"].vp, *hyper, ref["gsq"].vp, accumulate)
        rc = lib.ttrl_adam_step_static(stream, got["p"].vp, got["g"].vp, got["S"].vp, got["V"].vp, C.c_long(n),
                                       got["step"].vp, *hyper, got["gsq"].vp, accumulate)
        assert rc == 0, lib.ttrl_last_error()
        device.synchronize()
        a, b = _read(ref), _read(got)
        for k in a:
            assert np.array_equal(a[k], b[k]), (call, k)
        assert int(b["step"][0]) == 4
        want = np.sum(np.square(a["g"].astype(np.float64)))
        assert abs(float(b["gsq"][0]) - (want + (0.5 if accumulate else 0.0))) <= 1e-5 * want


def test_static_adam_refuses_bad_arguments(device):
    from ttrl_amd import _lib

    lib = _lib.lib()
    arrs = _arrays(device, 64, 1)
    hyper = (C.c_float(3e-4), C.c_float(0.9), C.c_float(0.999), C.c_float(1e-8), C.c_float(0.0))
    stream = C.c_void_p(lib.ttrl_stream(device.ctx))
    rc = lib.ttrl_adam_step_static(stream, arrs["p"].vp, arrs["g"].vp, arrs["S"].vp, arrs["V"].vp, C.c_long(0),
                                   arrs["step"].vp, *hyper, None, 0)
    assert rc == _lib.TTRL_EINVAL and b"empty" in lib.ttrl_last_error()
    rc = lib.ttrl_adam_step_static(stream, C.c_void_p(arrs["p"].ptr + 4), arrs["g"].vp, arrs["S"].vp, arrs["V"].vp,
                                   C.c_long(60), arrs["step"].vp, *hyper, None, 0)
    assert rc == _lib.TTRL_EINVAL and b"aligned" in lib.ttrl_last_error()
