"""Device buffers and host<->device transfer.

`DeviceArray` is the storage behind every engine `Tensor`: a device pointer,
a shape and a dtype, freed back to its pool when the last view goes.
Address stability (ttrl/engine/tensor/__init__.py:1-8): a buffer bound into
a captured graph is only ever written in place, never rebound, so the helpers
that write into existing buffers (`restore_in_place`, `copy_in_place`) are the
ones a step may use.

`ParamArena` lays every parameter built inside its `with` block out in one
flat buffer, with gradients in a second buffer of the same layout, so one
kernel launch can step, blend or copy a whole network.
"""

from __future__ import annotations

import ctypes as C
import math

import numpy as np

from ttrl_amd.engine.device import Device

__all__ = [
    "DeviceArray", "MASTER_DTYPE", "ParamArena", "bound_block", "copy_in_place", "copy_tensor_in_place",
    "restore_in_place", "to_device", "to_host", "zeros",
]

MASTER_DTYPE = np.float32
_DTYPES = (np.dtype(np.float32), np.dtype(np.uint8), np.dtype(np.int32), np.dtype(np.float64))

#: Parameters start on 256-byte boundaries inside an arena, so weight rows,
#: vector loads and the Adam kernel's float4 accesses stay aligned.
ARENA_ALIGN_ELEMS = 64


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


class _Block:
    """One allocation; frees itself when no DeviceArray refers to it."""

    __slots__ = ("dev", "ptr", "nbytes", "__weakref__")

    def __init__(self, dev: Device, nbytes: int):
        self.dev = dev
        self.nbytes = int(nbytes)
        self.ptr = dev.alloc(self.nbytes)

    def __del__(self):
        try:
            if self.ptr and not self.dev.closed:
                self.dev.free(self.ptr)
        except Exception:
            pass
        self.ptr = 0


class _MappedBlock:
    """Pinned host memory that kernels read and write in place, as a block of
    DeviceArray views: kernels address it at `ptr` (its device address), the
    host through `host.array` (a uint8 numpy view).  Frees itself with its
    last view."""

    __slots__ = ("dev", "ptr", "nbytes", "host", "__weakref__")

    def __init__(self, dev: Device, nbytes: int):
        self.dev = dev
        self.host = dev.mapped_block(max(1, int(nbytes)))
        self.nbytes = self.host.nbytes
        self.ptr = self.host.dptr


class DeviceArray:
    """A dense, C-contiguous device array (a view into a `_Block`, or into a
    `_MappedBlock` of host memory)."""

    __slots__ = ("dev", "block", "offset", "shape", "dtype", "unit")

    def __init__(self, dev: Device, shape, dtype=np.float32, *, block: _Block | None = None, offset: int = 0):
        self.dev = dev
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        if self.dtype not in _DTYPES:
            raise ValueError(f"DeviceArray: unsupported dtype {self.dtype}")
        if block is None:
            block = _Block(dev, max(1, self.nbytes))
        self.block = block
        self.offset = int(offset)  # bytes
        self.unit = False  # set when every element is known to be exactly 1.0

    # -- geometry ------------------------------------------------------------

    @property
    def numel(self) -> int:
        return _numel(self.shape)

    @property
    def nbytes(self) -> int:
        return self.numel * self.dtype.itemsize

    @property
    def ptr(self) -> int:
        return self.block.ptr + self.offset

    @property
    def vp(self) -> C.c_void_p:
        return C.c_void_p(self.ptr)

    def reshape(self, shape) -> "DeviceArray":
        shape = tuple(int(d) for d in shape)
        if -1 in shape:
            known = _numel([d for d in shape if d != -1])
            shape = tuple(self.numel // known if d == -1 else d for d in shape)
        if _numel(shape) != self.numel:
            raise ValueError(f"cannot reshape {self.shape} to {shape}")
        out = DeviceArray(self.dev, shape, self.dtype, block=self.block, offset=self.offset)
        out.unit = self.unit
        return out

    def view(self, elem_offset: int, shape) -> "DeviceArray":
        """A contiguous sub-range starting `elem_offset` elements in."""
        n = _numel(shape)
        if elem_offset < 0 or elem_offset + n > self.numel:
            raise ValueError("DeviceArray.view out of range")
        return DeviceArray(self.dev, shape, self.dtype, block=self.block,
                           offset=self.offset + elem_offset * self.dtype.itemsize)

    def same_storage(self, other: "DeviceArray") -> bool:
        return self.block is other.block

    # -- transfer ------------------------------------------------------------

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes:
            self.dev.call("ttrl_d2h", out.ctypes.data_as(C.c_void_p), self.vp, C.c_size_t(out.nbytes))
        return out

    def upload(self, array) -> None:
        arr = np.ascontiguousarray(np.asarray(array, dtype=self.dtype))
        if arr.size != self.numel:
            raise ValueError(f"upload: {arr.shape} does not fit buffer {self.shape}")
        if arr.nbytes:
            self.dev.call("ttrl_h2d", self.vp, arr.ctypes.data_as(C.c_void_p), C.c_size_t(arr.nbytes))
        self.unit = False

    def fill(self, value: float) -> None:
        if self.dtype == np.float32:
            self.dev.call("ttrl_fill_f32", self.vp, C.c_float(value), C.c_long(self.numel))
        elif self.dtype == np.int32:
            self.dev.call("ttrl_fill_i32", self.vp, C.c_int(int(value)), C.c_long(self.numel))
        else:
            raise ValueError("fill: float32 or int32 buffers only")
        self.unit = self.dtype == np.float32 and float(value) == 1.0

    def copy_from(self, src: "DeviceArray") -> None:
        if src.nbytes != self.nbytes:
            raise ValueError(f"copy_from: {src.shape} -> {self.shape} size mismatch")
        if self.nbytes:
            self.dev.call("ttrl_d2d", self.vp, src.vp, C.c_size_t(self.nbytes))
        self.unit = src.unit

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype})"


def zeros(dev: Device, shape, dtype=np.float32) -> DeviceArray:
    out = DeviceArray(dev, shape, dtype)
    if dtype == np.uint8:
        out.upload(np.zeros(out.shape, np.uint8))
    else:
        out.fill(0)
    return out


def bound_block(device: Device, specs, *, mapped: bool = False):
    """Input buffers laid out back to back in one allocation.

    `specs` is a sequence of (name, host_array); each buffer starts on a
    256-byte boundary.  Returns ({name: DeviceArray}, whole block as uint8),
    so one device copy refreshes every input of a step.  With `mapped` the
    block is pinned host memory that kernels read and write in place
    (`_MappedBlock`; its host view is `whole.block.host.array`), so a step
    needs no copy at all.
    """
    layout, offset = [], 0
    for name, arr in specs:
        arr = np.ascontiguousarray(arr)
        layout.append((name, arr, offset))
        offset += int(math.ceil(max(arr.nbytes, 1) / 256.0)) * 256
    size = max(offset, 256)
    block = _MappedBlock(device, size) if mapped else _Block(device, size)
    whole = DeviceArray(device, (size,), np.uint8, block=block)
    out = {}
    for name, arr, off in layout:
        view = DeviceArray(device, arr.shape, arr.dtype, block=block, offset=off)
        if mapped:
            block.host.array[off:off + arr.nbytes] = arr.reshape(-1).view(np.uint8)
        else:
            view.upload(arr)
        out[name] = view
    return out, whole


def to_device(array, device: Device, dtype=np.float32, layout=None) -> DeviceArray:
    """Upload a host array (ttrl/engine/tensor/transfer.py:11-22)."""
    arr = np.asarray(array)
    dtype = np.dtype(dtype if dtype is not None else arr.dtype)
    out = DeviceArray(device, arr.shape, dtype)
    out.upload(arr)
    return out


def to_host(data: DeviceArray) -> np.ndarray:
    """Download a device array (ttrl/engine/tensor/transfer.py:42-51)."""
    return data.numpy()


def restore_in_place(data: DeviceArray, array) -> None:
    """Overwrite an existing buffer from host (ttrl/engine/tensor/transfer.py:23-39)."""
    data.upload(array)


def copy_in_place(dst: DeviceArray, src: DeviceArray) -> None:
    """Device copy into an existing buffer (ttrl/engine/tensor/arena.py:32)."""
    dst.copy_from(src)


def copy_tensor_in_place(dst, src) -> None:
    """`copy_in_place` over engine Tensors (target-network sync)."""
    dst.data.copy_from(src.data)


class ParamArena:
    """Collects parameters created inside `with arena:` into one flat buffer.

    On exit every collected Tensor's data is moved into the arena (in
    creation order, each start aligned to 64 elements) and given a gradient
    slot at the same offset of a zero-filled gradient arena.  The moved
    tensors keep their identity, so modules built inside the block see the
    arena buffers.  Two arenas built from the same construction sequence have
    identical layouts, which is what lets a Polyak blend or a hard target
    copy run as one launch over the whole buffer.
    """

    _active: "list[ParamArena]" = []

    def __init__(self, device: Device, name: str = ""):
        self.device = device
        self.name = name
        self.tensors: list = []
        self.offsets: list[int] = []
        self.data: DeviceArray | None = None
        self.grad: DeviceArray | None = None
        self.numel = 0

    @classmethod
    def current(cls):
        return cls._active[-1] if cls._active else None

    def register(self, tensor) -> None:
        if self.data is not None:
            raise RuntimeError("ParamArena: already sealed")
        self.tensors.append(tensor)

    def __enter__(self) -> "ParamArena":
        ParamArena._active.append(self)
        return self

    def __exit__(self, *exc) -> None:
        ParamArena._active.pop()
        if exc and exc[0] is not None:
            return
        self.seal()

    def seal(self) -> None:
        offset = 0
        for t in self.tensors:
            self.offsets.append(offset)
            n = t.data.numel
            offset += int(math.ceil(n / ARENA_ALIGN_ELEMS)) * ARENA_ALIGN_ELEMS
        self.numel = max(offset, ARENA_ALIGN_ELEMS)
        self.data = zeros(self.device, (self.numel,))
        self.grad = zeros(self.device, (self.numel,))
        for t, off in zip(self.tensors, self.offsets):
            view = self.data.view(off, t.data.shape)
            view.copy_from(t.data)
            t.data = view
            t._grad_slot = self.grad.view(off, t.data.shape)
            t._arena = (self, off)

    def covers(self, params) -> bool:
        """True when `params` are exactly this arena's tensors, in order."""
        params = list(params)
        return len(params) == len(self.tensors) and all(a is b for a, b in zip(params, self.tensors))


def arena_of(params):
    """The arena holding exactly `params` in order, else None."""
    params = list(params)
    if not params:
        return None
    info = getattr(params[0], "_arena", None)
    if info is None:
        return None
    arena = info[0]
    return arena if arena.covers(params) else None
