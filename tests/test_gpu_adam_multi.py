"""Deferred Adam steps (ttrl_adam_step_deferred, ttrl_adam_multi,
ttrl_adam_finish_slots) against one ttrl_adam_step per range and a
ttrl_polyak, called through the C ABI on identical copies of the inputs.
Every range keeps the block partition and the partial-sum order of its
single-range launch, so parameters, moments, the Polyak target, the step
counters and the sums of squared gradients must agree bit for bit, over two
updates in a row (the second reading the counters the first stored)."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (n, lr, beta1, beta2, eps, weight_decay): the SAC critic arena, the policy
# arena, the one-element temperature arena (a range that is all tail)
RANGES = [(140_802, 3e-4, 0.9, 0.999, 1e-8, 0.0), (70_406 + 2, 1e-3, 0.8, 0.99, 1e-6, 0.01),
          (1, 3e-4, 0.9, 0.999, 1e-8, 0.0)]
POLYAK_N, TAU = 140_802, 0.005


def _upload(device, host, dtype=np.float32):
    from ttrl_amd.engine.tensor import DeviceArray

    a = DeviceArray(device, host.shape, dtype)
    a.upload(host.astype(dtype))
    return a


def _state(device, seed):
    rng = np.random.default_rng(seed)
    ranges = []
    for i, (n, *_) in enumerate(RANGES):
        ranges.append({"p": _upload(device, rng.standard_normal(n)), "g": _upload(device, rng.standard_normal(n)),
                       "S": _upload(device, 0.1 * rng.standard_normal(n)), "V": _upload(device, rng.random(n)),
                       "step": _upload(device, np.array([5 + i]), np.int32),
                       "gsq": _upload(device, np.array([0.0]))})
    polyak = {"dst": _upload(device, rng.standard_normal(POLYAK_N)),
              "src": _upload(device, rng.standard_normal(POLYAK_N))}
    return ranges, polyak


def _hyper(r):
    return tuple(C.c_float(v) for v in r[1:])


def _reference(device, ranges, polyak):
    for r, a in zip(RANGES, ranges):
        device.call("ttrl_adam_step", a["p"].vp, a["g"].vp, a["S"].vp, a["V"].vp, C.c_long(r[0]), a["step"].vp,
                    *_hyper(r), a["gsq"].vp, 0)
    device.call("ttrl_polyak", polyak["dst"].vp, polyak["src"].vp, C.c_long(POLYAK_N), C.c_float(TAU))


def _deferred(device, ranges, polyak):
    from ttrl_amd import _lib

    first, rest = ranges[0], ranges[1:]
    device.call("ttrl_adam_step_deferred", first["p"].vp, first["g"].vp, first["S"].vp, first["V"].vp,
                C.c_long(RANGES[0][0]), first["step"].vp, *_hyper(RANGES[0]), 0)
    descs = [_lib.AdamRange(a["p"].ptr, a["g"].ptr, a["S"].ptr, a["V"].ptr, r[0], a["step"].ptr, *r[1:], slot)
             for slot, (r, a) in enumerate(zip(RANGES[1:], rest), start=1)]
    arr = (_lib.AdamRange * len(descs))(*descs)
    device.call("ttrl_adam_multi", len(descs), arr, polyak["dst"].vp, polyak["src"].vp, C.c_long(POLYAK_N),
                C.c_float(TAU))
    fins = [_lib.AdamFinish(slot, r[0], a["step"].ptr, a["gsq"].ptr, 0)
            for slot, (r, a) in enumerate(zip(RANGES, ranges))]
    device.call("ttrl_adam_finish_slots", len(fins), (_lib.AdamFinish * len(fins))(*fins))


def test_deferred_steps_match_single_steps(device):
    ref_r, ref_p = _state(device, 7)
    got_r, got_p = _state(device, 7)
    for update in range(2):
        _reference(device, ref_r, ref_p)
        _deferred(device, got_r, got_p)
        device.synchronize()
        for i, (a, b) in enumerate(zip(ref_r, got_r)):
            for k in a:
                assert np.array_equal(a[k].numpy(), b[k].numpy()), (update, i, k)
            assert int(b["step"].numpy()[0]) == 5 + i + update + 1
        for k in ref_p:
            assert np.array_equal(ref_p[k].numpy(), got_p[k].numpy()), (update, k)


def test_deferred_steps_refuse_bad_arguments(device):
    from ttrl_amd import _lib

    lib = _lib.lib()
    ranges, polyak = _state(device, 1)
    a = ranges[1]
    bad = _lib.AdamRange(a["p"].ptr, a["g"].ptr, a["S"].ptr, a["V"].ptr, RANGES[1][0], a["step"].ptr,
                         *RANGES[1][1:], 9)
    rc = lib.ttrl_adam_multi(device.ctx, 1, C.byref(bad), None, None, C.c_long(0), C.c_float(0.0))
    assert rc == _lib.TTRL_EINVAL and b"slot" in lib.ttrl_last_error()
    two = (_lib.AdamRange * 2)(*[_lib.AdamRange(a["p"].ptr, a["g"].ptr, a["S"].ptr, a["V"].ptr, RANGES[1][0],
                                                a["step"].ptr, *RANGES[1][1:], 3)] * 2)
    rc = lib.ttrl_adam_multi(device.ctx, 2, two, None, None, C.c_long(0), C.c_float(0.0))
    assert rc == _lib.TTRL_EINVAL and b"twice" in lib.ttrl_last_error()
    fin = _lib.AdamFinish(0, 0, a["step"].ptr, None, 0)
    rc = lib.ttrl_adam_finish_slots(device.ctx, 1, C.byref(fin))
    assert rc == _lib.TTRL_EINVAL and b"empty" in lib.ttrl_last_error()
