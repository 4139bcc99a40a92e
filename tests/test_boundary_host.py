"""The engine and learner boundary without a GPU: EngineConfig and DEFAULT
(ttrl/engine/config.py), `acquire` as a context manager over per-GPU locks
(ttrl/engine/device/acquire.py:55-140, liveness.py:262-299), the ALGOS
registry (ttrl/algos/registry.py, ttrl/nets/registry.py), check_agent, and
the input binder's range coalescing."""

from __future__ import annotations

import subprocess
import sys
import time

import pytest


# -- EngineConfig ---------------------------------------------------------------

def test_engine_exports_default_and_config():
    import ttrl_amd
    from ttrl_amd import engine
    from ttrl_amd.engine.config import DEFAULT, EngineConfig

    assert engine.DEFAULT is DEFAULT and engine.EngineConfig is EngineConfig
    assert ttrl_amd.DEFAULT is DEFAULT
    assert "DEFAULT" in engine.__all__ and "EngineConfig" in engine.__all__
    assert DEFAULT == EngineConfig(trace_blocking=False, l1_small_size=32768, trace_region_size=32 * 1024 * 1024)
    with pytest.raises(Exception):
        DEFAULT.trace_blocking = True  # frozen


def test_engine_config_refuses_fields_without_a_counterpart():
    from ttrl_amd.engine.config import DEFAULT, EngineConfig, check_engine_config

    assert check_engine_config(None, "x") is DEFAULT
    blocking = EngineConfig(trace_blocking=True)
    assert check_engine_config(blocking, "x") is blocking
    with pytest.raises(ValueError, match="l1_small_size"):
        check_engine_config(EngineConfig(l1_small_size=65536), "TrainStep")
    with pytest.raises(ValueError, match="trace_region_size"):
        check_engine_config(EngineConfig(trace_region_size=1 << 20), "acquire")
    with pytest.raises(ValueError, match="EngineConfig"):
        check_engine_config({"trace_blocking": True}, "TrainStep")


def test_train_step_takes_the_engine_config():
    from ttrl_amd.engine.config import DEFAULT, EngineConfig
    from ttrl_amd.engine.step import TrainStep

    step = TrainStep(lambda inputs: {}, {}, None)
    assert step.cfg is DEFAULT
    step = TrainStep(lambda inputs: {}, {}, None, cfg=EngineConfig(trace_blocking=True))
    assert step.cfg.trace_blocking
    with pytest.raises(ValueError, match="l1_small_size"):
        TrainStep(lambda inputs: {}, {}, None, cfg=EngineConfig(l1_small_size=1))


# -- acquire ------------------------------------------------------------------------

class _FakeDevice:
    opened: list = []

    def __init__(self, index, *, cfg=None):
        self.index, self.cfg, self.closed = index, cfg, False
        _FakeDevice.opened.append(self)

    def close(self):
        self.closed = True


@pytest.fixture
def fake_gpus(monkeypatch, tmp_path):
    """Three visible GPUs whose contexts are host stand-ins; locks in tmp_path."""
    from ttrl_amd.engine import device as D

    monkeypatch.setenv("TTRL_LOCK_DIR", str(tmp_path))
    for var in ("HIP_VISIBLE_DEVICES", "CUDA_VISIBLE_DEVICES", "ROCR_VISIBLE_DEVICES"):
        monkeypatch.delenv(var, raising=False)
    monkeypatch.setattr(D, "device_count", lambda: 3)
    monkeypatch.setattr(D, "Device", _FakeDevice)
    monkeypatch.setattr(D, "probe_profile", lambda dev, cfg: ("profile", dev.index, cfg.trace_blocking))
    purged = []
    monkeypatch.setattr(D, "purge_device_caches", lambda dev: purged.append(dev.index))
    _FakeDevice.opened = []
    return D, tmp_path, purged


def _hold(tmp_path, index):
    """A child process holding GPU `index`'s lock until killed."""
    code = ("import fcntl, os, sys, time\n"
            f"fh = open({str(tmp_path / f'gpu{index}.lock')!r}, 'a+')\n"
            "fcntl.flock(fh, fcntl.LOCK_EX)\n"
            "fh.seek(0); fh.truncate(); fh.write(str(os.getpid())); fh.flush()\n"
            "print('held', flush=True)\n"
            "time.sleep(60)\n")
    proc = subprocess.Popen([sys.executable, "-c", code], stdout=subprocess.PIPE, text=True)
    assert proc.stdout.readline().strip() == "held"
    return proc


def test_acquire_yields_device_and_profile_and_closes(fake_gpus):
    D, tmp, purged = fake_gpus
    with D.acquire(1) as (device, profile):
        assert device.index == 1 and not device.closed
        assert profile == ("profile", 1, False)
        assert D.survey() == {0: None, 1: D.os.getpid(), 2: None}
    assert device.closed and purged == [1]
    assert D.survey()[1] is None  # released


def test_acquire_skips_busy_gpus_and_refuses_when_all_are(fake_gpus):
    D, tmp, _ = fake_gpus
    holders = [_hold(tmp, 0)]
    try:
        with D.acquire() as (device, _):
            assert device.index == 1  # GPU 0 is held by another process
            with D.acquire() as (inner, _):
                assert inner.index == 2  # this process holds 1
        holders += [_hold(tmp, 1), _hold(tmp, 2)]
        with pytest.raises(D.NoDeviceAvailable, match="every candidate GPU is busy"):
            with D.acquire(wait=False):
                pass
        seen = []
        t0 = time.monotonic()
        with pytest.raises(D.NoDeviceAvailable, match="no GPU free after"):
            with D.acquire(0, timeout=0.3, poll=0.05, on_wait=seen.append):
                pass
        assert time.monotonic() - t0 < 5
        assert seen and seen[0] == {0: holders[0].pid}
    finally:
        for p in holders:
            p.kill()
            p.wait()


def test_acquire_waits_for_a_gpu_to_free(fake_gpus):
    D, tmp, _ = fake_gpus
    holder = _hold(tmp, 0)
    polls = []

    def on_wait(s):
        polls.append(s)
        if len(polls) == 2:
            holder.kill()
            holder.wait()

    with D.acquire(0, timeout=10, poll=0.05, on_wait=on_wait) as (device, _):
        assert device.index == 0
    assert len(polls) >= 2


def test_acquire_closes_the_device_when_the_body_raises(fake_gpus):
    D, tmp, purged = fake_gpus
    with pytest.raises(KeyError):
        with D.acquire(2) as (device, _):
            raise KeyError("body")
    assert device.closed and purged == [2] and D.survey()[2] is None


def test_acquire_refuses_an_invisible_gpu_and_bad_config(fake_gpus):
    D, _, _ = fake_gpus
    from ttrl_amd.engine.config import EngineConfig

    with pytest.raises(D.NoDeviceAvailable, match="not visible"):
        with D.acquire(7):
            pass
    with pytest.raises(ValueError, match="l1_small_size"):
        with D.acquire(0, cfg=EngineConfig(l1_small_size=1)):
            pass


def test_lock_names_follow_the_visibility_mapping(monkeypatch):
    from ttrl_amd.engine import device as D

    for var in ("HIP_VISIBLE_DEVICES", "CUDA_VISIBLE_DEVICES", "ROCR_VISIBLE_DEVICES"):
        monkeypatch.delenv(var, raising=False)
    assert D.physical_index(2) == "2"
    monkeypatch.setenv("HIP_VISIBLE_DEVICES", "5,3")
    assert D.physical_index(1) == "3"


def test_acquire_without_a_visible_gpu(monkeypatch, tmp_path):
    """This container has no GPU: acquire says so instead of opening one."""
    from ttrl_amd.engine import device as D

    monkeypatch.setenv("TTRL_LOCK_DIR", str(tmp_path))
    if D.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(D.NoDeviceAvailable, match="no GPU is visible"):
        with D.acquire():
            pass


# -- ALGOS -----------------------------------------------------------------------------

def test_algos_registry_names_without_importing():
    import importlib

    import ttrl_amd
    from ttrl_amd.algos import ALGOS, resolve_and_build
    from ttrl_amd.algos.registry import ALGOS as same

    assert ALGOS is same and ttrl_amd.ALGOS is ALGOS and ttrl_amd.resolve_and_build is resolve_and_build
    assert ALGOS.names() == ["dqn", "ppo", "sac"]
    assert "dqn" in ALGOS and "nope" not in ALGOS and len(ALGOS) == 3
    assert ALGOS.entry("sac") == "ttrl_amd.algos.agents:SACAgent"
    agents = importlib.import_module("ttrl_amd.algos.agents")
    assert ALGOS.resolve("dqn") is agents.DQNAgent
    assert ALGOS.resolve("ppo") is agents.PPOAgent


def test_algos_registry_refusals():
    from ttrl_amd.algos import ALGOS, resolve_and_build
    from ttrl_amd.algos.registry import Registry

    with pytest.raises(KeyError, match=r"unknown algo 'nope'; registered names are \['dqn', 'ppo', 'sac'\]"):
        resolve_and_build("nope", None, None, None)
    with pytest.raises(ValueError, match="already registered"):
        ALGOS.register("dqn", lambda *a, **k: None)
    reg = Registry("algos", module="m", allow_targets=True)
    with pytest.raises(KeyError, match="registry is empty"):
        reg.resolve("x")
    with pytest.raises(ValueError, match="module:attr"):
        reg.register("x", "no_colon")
    reg.register("bad_module", "ttrl_amd.no_such_module:X")
    with pytest.raises(ModuleNotFoundError, match="does not exist"):
        reg.resolve("bad_module")
    reg.register("bad_attr", "ttrl_amd.spaces:NoSuchThing")
    with pytest.raises(AttributeError, match="defines no such name"):
        reg.resolve("bad_attr")
    strict = Registry("things", module="m")
    with pytest.raises(TypeError, match="callables only"):
        strict.register("x", "a:b")

    @reg("mine")
    def build(obs_spec, action_spec, device, **kwargs):
        return ("built", obs_spec, action_spec, device, kwargs)

    assert reg.resolve("mine")(1, 2, 3, seed=4) == ("built", 1, 2, 3, {"seed": 4})
    reg.unregister("mine")
    assert "mine" not in reg
    with pytest.raises(KeyError):
        reg.unregister("mine")


def test_check_agent():
    from ttrl_amd.algos import check_agent
    from ttrl_amd.spaces import ActionSpec, ObsSpec

    class Partial:
        obs_spec = ObsSpec.vector(3)
        action_spec = ActionSpec.discrete(2)

        def act(self, obs):
            return obs

    with pytest.raises(TypeError, match="missing"):
        check_agent(Partial())
    with pytest.raises(TypeError, match="obs_spec"):
        check_agent(object())


# -- InputBinder ---------------------------------------------------------------------------

def _binder(ranges, dirty):
    from ttrl_amd.engine.step import InputBinder

    b = object.__new__(InputBinder)
    b._ranges, b._dirty = dict(ranges), set(dirty)
    return b


def test_pending_ranges_bridge_only_alignment_padding():
    # actions_onehot [32, 6] f32 (768 B), rewards [32, 1] (128 B), dones (128 B): each starts on 256 B
    ranges = {"actions_onehot": (0, 768), "rewards": (768, 896), "dones": (1024, 1152), "discounts": (1280, 1408)}
    assert _binder(ranges, {"actions_onehot", "dones"}).pending() == [(0, 768), (1024, 1152)]
    assert _binder(ranges, {"actions_onehot", "rewards", "dones"}).pending() == [(0, 1152)]
    assert _binder(ranges, {"rewards", "dones", "discounts"}).pending() == [(768, 1408)]
    assert _binder({"a": (0, 100), "b": (256, 300)}, {"a", "b"}).pending() == [(0, 300)]
    assert _binder({"a": (0, 256), "b": (256, 300), "c": (512, 600)}, {"a", "c"}).pending() == [(0, 256),
                                                                                                  (512, 600)]
    assert _binder(ranges, set()).pending() == []
