"""Device handle: one HIP context and stream per opened GPU.

Replaces `acquire` (ttrl/engine/device/acquire.py:56) and the chip scoping
around it.  A `Device` owns a context from libttrl_hip; every kernel it
launches runs on that context's single stream, so ordering between ops,
copies and graph replays is stream order.
"""

from __future__ import annotations

import ctypes as C
import os
import threading
from contextlib import contextmanager
from pathlib import Path

from ttrl_amd import _lib

__all__ = ["Device", "HostBlock", "acquire", "device_count", "NoDeviceAvailable"]


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

    def __init__(self, index: int = 0):
        self.index = int(index)
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
    image of a bound input block or a metrics block.  The block owns the
    memory: views of `array` must not outlive it."""

    def __init__(self, dev: Device, nbytes: int):
        import numpy as np

        self.dev = dev
        self.nbytes = max(1, int(nbytes))
        ptr = C.c_void_p()
        dev.call("ttrl_host_alloc", C.c_size_t(self.nbytes), C.byref(ptr))
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


_DEFAULT: dict[int, Device] = {}


def acquire(index: int = 0) -> Device:
    """The process-wide Device for GPU `index`, opened on first use."""
    dev = _DEFAULT.get(index)
    if dev is None or dev.closed:
        dev = Device(index)
        _DEFAULT[index] = dev
    return dev
