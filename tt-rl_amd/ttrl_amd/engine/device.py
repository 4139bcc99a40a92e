"""Device handle: one HIP context and stream per opened GPU, and `acquire`,
which opens a free GPU for the length of a `with` block
(ttrl/engine/device/acquire.py:55-140, ttrl/engine/device/liveness.py:262-299,
ttrl/engine/device/profile.py:18-97).

A `Device` owns a context from libttrl_hip; every kernel it launches runs on
that context's single stream, so ordering between ops, copies and graph
replays is stream order.  `acquire` takes an advisory lock per GPU (an
flock on a PID-tagged file, released with the process) so that processes
that share a machine through it never train on the same GPU, and yields the
device with its `DeviceProfile`.  `open_device` is the process-wide handle
this package's own tests and benchmarks share, outside any lock.
"""

from __future__ import annotations

import contextlib
import ctypes as C
import fcntl
import os
import threading
import time
import traceback
from contextlib import contextmanager
from dataclasses import dataclass
from pathlib import Path
from typing import Iterator

from ttrl_amd import _lib
from ttrl_amd.engine.config import DEFAULT, EngineConfig, check_engine_config

__all__ = ["Device", "DeviceProfile", "HostBlock", "NoDeviceAvailable", "acquire", "device_count", "lock_dir",
           "open_device", "probe_profile", "purge_device_caches", "register_device_cache", "survey"]

#: How long `acquire` waits for a busy GPU by default, and how often it looks
#: (ttrl/engine/device/liveness.py:23-28).
DEFAULT_WAIT_SECONDS = 120.0
POLL_SECONDS = 5.0

_LOCK_DIR_ENV = "TTRL_LOCK_DIR"


#: GEMM plans tuned on gfx950 for this package's learner workloads, loaded
#: into every context at open (TTRL_PLANS=<path> loads another file instead,
#: TTRL_PLANS=none none), so processes run the same plans and agree bit for bit.
PLAN_FILE = Path(__file__).resolve().parents[1] / "plans" / "gfx950.tsv"


class NoDeviceAvailable(RuntimeError):
    """No gfx950 device is visible to this process."""


def device_count() -> int:
    n = C.c_int(0)
    rc = _lib.lib().ttrl_device_count(C.byref(n))
    if rc != _lib.TTRL_OK:
        return 0
    return int(n.value)


class Device:
    """An open GPU: context, stream, allocation pools."""

    def __init__(self, index: int = 0, *, cfg: EngineConfig = DEFAULT):
        self.index = int(index)
        self.cfg = check_engine_config(cfg, "Device")
        handle = C.c_void_p()
        rc = _lib.lib().ttrl_init(self.index, C.byref(handle))
        if rc != _lib.TTRL_OK:
            msg = _lib.lib().ttrl_last_error().decode(errors="replace")
            raise NoDeviceAvailable(f"cannot open device {self.index}: {msg}")
        self.ctx = handle
        self._lock = threading.RLock()
        self.closed = False
        self._pool_stack = [0]
        # ordered sums queued for the next optimizer step (engine.pending)
        self.pending_sums: list = []
        plans = os.environ.get("TTRL_PLANS", "")
        if plans.lower() != "none":
            path = Path(plans) if plans else PLAN_FILE
            if path.is_file():
                self.load_plans(path)

    # -- plumbing ----------------------------------------------------------

    def call(self, name: str, *args) -> None:
        if self.closed:
            raise RuntimeError("device is closed")
        _lib.check(getattr(_lib.lib(), name)(self.ctx, *args), name)

    def synchronize(self) -> None:
        self.call("ttrl_sync")

    @property
    def capturing(self) -> bool:
        return getattr(self, "_capturing", False)

    # -- GEMM plans --------------------------------------------------------

    def export_plans(self) -> str:
        """The context's GEMM plan table as text (ttrl_plans_export)."""
        n = C.c_size_t(0)
        self.call("ttrl_plans_export", None, C.c_size_t(0), C.byref(n))
        buf = C.create_string_buffer(int(n.value) + 1)
        self.call("ttrl_plans_export", buf, C.c_size_t(len(buf)), C.byref(n))
        return buf.value.decode()

    def import_plans(self, text: str) -> int:
        """Add plans to the table; later calls of those signatures run them."""
        count = C.c_int(0)
        self.call("ttrl_plans_import", text.encode(), C.byref(count))
        return int(count.value)

    def save_plans(self, path) -> None:
        Path(path).write_text(self.export_plans())

    def load_plans(self, path) -> int:
        return self.import_plans(Path(path).read_text())

    # -- memory ------------------------------------------------------------

    def alloc(self, nbytes: int) -> int:
        ptr = C.c_void_p()
        self.call("ttrl_alloc", C.c_size_t(max(1, int(nbytes))), C.byref(ptr))
        return int(ptr.value)

    def free(self, ptr: int) -> None:
        if self.closed or not ptr:
            return
        _lib.lib().ttrl_free(self.ctx, C.c_void_p(ptr))

    def host_block(self, nbytes: int) -> "HostBlock":
        """Pinned host memory owned by this context (see `HostBlock`)."""
        return HostBlock(self, nbytes)

    def mapped_block(self, nbytes: int) -> "HostBlock":
        """Pinned host memory kernels read and write in place (`dptr` is its
        device address; see `HostBlock`)."""
        return HostBlock(self, nbytes, mapped=True)

    def create_pool(self) -> int:
        pid = C.c_int(0)
        self.call("ttrl_pool_create", C.byref(pid))
        return int(pid.value)

    def release_pool(self, pool: int) -> None:
        if self.closed:
            return
        self.call("ttrl_pool_release", int(pool))

    @contextmanager
    def use_pool(self, pool: int):
        """Allocations inside the block come from `pool`."""
        prev = C.c_int(0)
        self.call("ttrl_pool_use", int(pool), C.byref(prev))
        try:
            yield
        finally:
            if not self.closed:
                self.call("ttrl_pool_use", int(prev.value), None)

    def pool_stats(self, pool: int = 0) -> tuple[int, int]:
        reserved, live = C.c_size_t(0), C.c_size_t(0)
        self.call("ttrl_pool_stats", int(pool), C.byref(reserved), C.byref(live))
        return int(reserved.value), int(live.value)

    # -- lifecycle ---------------------------------------------------------

    def close(self) -> None:
        if self.closed:
            return
        _lib.lib().ttrl_shutdown(self.ctx)
        self.closed = True

    def __enter__(self) -> "Device":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __repr__(self) -> str:
        return f"Device({self.index}{', closed' if self.closed else ''})"


class HostBlock:
    """Pinned host memory from the device context (ttrl_host_alloc).

    `array` is a uint8 numpy view of it.  Copies between it and device memory
    read and write it in place (no staging pass), which makes it the host
    image of a bound input block or a metrics block.  A mapped block
    (`Device.mapped_block`) is also read and written by kernels in place at
    `dptr`.  The block owns the memory: views of `array` must not outlive it."""

    def __init__(self, dev: Device, nbytes: int, *, mapped: bool = False):
        import numpy as np

        self.dev = dev
        self.nbytes = max(1, int(nbytes))
        ptr = C.c_void_p()
        if mapped:
            dptr = C.c_void_p()
            dev.call("ttrl_host_alloc_mapped", C.c_size_t(self.nbytes), C.byref(ptr), C.byref(dptr))
            self.dptr = int(dptr.value)
        else:
            dev.call("ttrl_host_alloc", C.c_size_t(self.nbytes), C.byref(ptr))
            self.dptr = None
        self.ptr = int(ptr.value)
        self.array = np.frombuffer((C.c_uint8 * self.nbytes).from_address(self.ptr), dtype=np.uint8)

    def view(self, offset: int, shape, dtype):
        """A typed numpy view `offset` bytes into the block."""
        import numpy as np

        return np.ndarray(shape, dtype=dtype, buffer=self.array, offset=int(offset))

    def close(self) -> None:
        ptr, self.ptr = self.ptr, 0
        if ptr and not self.dev.closed:
            _lib.lib().ttrl_host_free(self.dev.ctx, C.c_void_p(ptr))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass(frozen=True)
class DeviceProfile:
    """Runtime-probed facts about an opened GPU, what the layers above may
    ask instead of knowing an architecture name
    (ttrl/engine/device/profile.py:18-29)."""

    arch: str
    name: str
    compute_units: int
    wavefront_size: int
    lds_per_cu: int
    lds_per_workgroup: int
    l2_bytes: int
    hbm_bytes: int
    clock_khz: int
    num_devices: int
    pci_bus_id: str
    trace_blocking: bool

    @property
    def gfx(self) -> str:
        """The ISA name without target features ("gfx950")."""
        return self.arch.split(":", 1)[0]


def _query(index: int) -> "_lib.DeviceInfo":
    info = _lib.DeviceInfo()
    _lib.check(_lib.lib().ttrl_device_query(int(index), C.byref(info)), "ttrl_device_query")
    return info


def probe_profile(device: "Device", cfg: EngineConfig = DEFAULT) -> DeviceProfile:
    info = _query(device.index)
    return DeviceProfile(
        arch=info.arch.decode(errors="replace"), name=info.name.decode(errors="replace"),
        compute_units=int(info.compute_units), wavefront_size=int(info.wavefront_size),
        lds_per_cu=int(info.lds_per_cu), lds_per_workgroup=int(info.lds_per_workgroup),
        l2_bytes=int(info.l2_bytes), hbm_bytes=int(info.hbm_bytes), clock_khz=int(info.clock_khz),
        num_devices=1,
        pci_bus_id=f"{info.pci_domain_id:04x}:{info.pci_bus_id:02x}:{info.pci_device_id:02x}",
        trace_blocking=bool(cfg.trace_blocking))


# -- device-keyed caches ------------------------------------------------------

_EXTRA_PURGERS: list = []


def register_device_cache(purge) -> None:
    """Register purge(device) for a cache keyed by id(device); it runs before
    the device closes (ttrl/engine/device/acquire.py:27-33)."""
    _EXTRA_PURGERS.append(purge)


def purge_device_caches(device) -> None:
    """Evict every process-global cache entry keyed by id(device), before
    the device closes: id() is reused once the object is freed
    (ttrl/engine/device/acquire.py:36-52)."""
    from ttrl_amd.engine.ops import purge_lane_caches, purge_matmul_caches

    purge_matmul_caches(device)
    purge_lane_caches(device)
    for purge in _EXTRA_PURGERS:
        purge(device)


# -- per-GPU advisory locks ----------------------------------------------------

def lock_dir() -> Path:
    """Directory of the per-GPU lock files, read per call ($TTRL_LOCK_DIR,
    else a per-user directory under the system temp dir)."""
    default = Path(os.environ.get("TMPDIR", "/tmp")) / f"ttrl-gpu-locks-{os.getuid()}"
    return Path(os.environ.get(_LOCK_DIR_ENV, str(default)))


def physical_index(index: int) -> str:
    """The GPU a visible index names, as the visibility variables map it,
    so that processes scoped to different GPU subsets lock the same file
    for the same GPU."""
    names = [str(int(index))]
    for var in ("HIP_VISIBLE_DEVICES", "CUDA_VISIBLE_DEVICES", "ROCR_VISIBLE_DEVICES"):
        value = os.environ.get(var, "").strip()
        if not value:
            continue
        entries = [e.strip() for e in value.split(",") if e.strip()]
        pos = int(names[-1])
        if 0 <= pos < len(entries) and entries[pos].isdigit():
            names.append(entries[pos])
    return names[-1]


def _lock_path(index: int) -> Path:
    return lock_dir() / f"gpu{physical_index(index)}.lock"


@contextmanager
def hold_lock(index: int) -> Iterator[bool]:
    """Try to take GPU `index`'s lock without blocking; yields whether it
    was taken (ttrl/engine/device/liveness.py:262-299).  The file holds the
    holder's PID while held; the lock dies with the process."""
    directory = lock_dir()
    directory.mkdir(parents=True, exist_ok=True)
    path = _lock_path(index)
    try:
        fh = open(path, "a+")
    except PermissionError as exc:
        raise PermissionError(f"cannot open the GPU lock {path}, which another user owns. "
                              f"Set {_LOCK_DIR_ENV} to a directory you own.") from exc
    try:
        try:
            fcntl.flock(fh, fcntl.LOCK_EX | fcntl.LOCK_NB)
        except BlockingIOError:
            yield False
            return
        fh.seek(0)
        fh.truncate()
        fh.write(str(os.getpid()))
        fh.flush()
        try:
            yield True
        finally:
            try:
                fh.seek(0)
                fh.truncate()
                fh.flush()
            finally:
                fcntl.flock(fh, fcntl.LOCK_UN)
    finally:
        fh.close()


def _holder(index: int) -> int | None:
    """PID recorded in GPU `index`'s lock file while it is held, else None."""
    path = _lock_path(index)
    try:
        with open(path, "a+") as fh:
            try:
                fcntl.flock(fh, fcntl.LOCK_EX | fcntl.LOCK_NB)
            except BlockingIOError:
                fh.seek(0)
                text = fh.read().strip()
                return int(text) if text.isdigit() else -1
            fcntl.flock(fh, fcntl.LOCK_UN)
            return None
    except FileNotFoundError:
        return None


def _visible() -> list[int]:
    return list(range(device_count()))


def survey(indices=None) -> dict[int, int | None]:
    """{visible GPU index: PID holding its lock, or None when free}."""
    return {i: _holder(i) for i in (_visible() if indices is None else indices)}


def describe_holders(held: dict) -> str:
    return "\n".join(f"  GPU {i}: " + ("free" if pid is None else f"held by pid {pid}" if pid > 0 else "held")
                     for i, pid in sorted(held.items()))


@contextlib.contextmanager
def acquire(chip_id: int | None = None, *, cfg: EngineConfig = DEFAULT, wait: bool = True,
            timeout: float | None = DEFAULT_WAIT_SECONDS, poll: float = POLL_SECONDS,
            on_wait=None) -> Iterator[tuple[Device, DeviceProfile]]:
    """Open a free GPU, waiting for one while all are held, and yield
    (device, profile) (ttrl/engine/device/acquire.py:55-140).

    `chip_id` is an index into the visible GPUs, or None for the first free
    one.  `on_wait(survey)` is called on each poll while blocked.  On the way
    out the device-keyed caches are purged, the device closes (its context,
    stream and every buffer it allocated) and the lock is released."""
    cfg = check_engine_config(cfg, "acquire")
    if chip_id is not None:
        index = int(chip_id)
        n = device_count()
        if not 0 <= index < max(n, 1) or n == 0:
            raise NoDeviceAvailable(f"GPU {chip_id} is not visible to this process ({n} visible GPUs); "
                                    f"check HIP_VISIBLE_DEVICES / ROCR_VISIBLE_DEVICES and that the amdgpu "
                                    f"driver is loaded (rocm-smi lists the GPUs it sees).")
        candidates = [index]
    else:
        candidates = _visible()
    if not candidates:
        raise NoDeviceAvailable("no GPU is visible to this process, so there is none to open; check "
                                "HIP_VISIBLE_DEVICES / ROCR_VISIBLE_DEVICES and that the amdgpu driver is loaded "
                                "(rocm-smi lists the GPUs it sees).")
    deadline = None if timeout is None else time.monotonic() + timeout
    while True:
        for index in candidates:
            with hold_lock(index) as got:
                if not got:
                    continue
                device = Device(index, cfg=cfg)
                body_exc: BaseException | None = None
                try:
                    try:
                        yield device, probe_profile(device, cfg)
                    except BaseException as exc:
                        body_exc = exc
                        raise
                finally:
                    try:
                        purge_device_caches(device)
                    except BaseException:
                        if body_exc is None:
                            raise
                        if hasattr(body_exc, "add_note"):
                            body_exc.add_note("device cache purge also failed:\n" + traceback.format_exc())
                    finally:
                        device.close()
                return
        if not wait:
            raise NoDeviceAvailable("every candidate GPU is busy:\n" + describe_holders(survey(candidates)))
        if deadline is not None and time.monotonic() >= deadline:
            raise NoDeviceAvailable(f"no GPU free after {timeout:.0f}s:\n" + describe_holders(survey(candidates)))
        if on_wait is not None:
            on_wait(survey(candidates))
        time.sleep(poll)


_DEFAULT: dict[int, Device] = {}


def open_device(index: int = 0) -> Device:
    """The process-wide Device for GPU `index`, opened on first use and kept
    until the process ends (no lock: callers that share a machine use
    `acquire`)."""
    dev = _DEFAULT.get(index)
    if dev is None or dev.closed:
        dev = Device(index)
        _DEFAULT[index] = dev
    return dev
