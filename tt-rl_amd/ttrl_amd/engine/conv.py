"""The Conv2d layer, its geometry, and the fused convolution op.

Same constructor and checkpoint surface as ttrl/engine/conv/module.py:28-263:
geometry fixed from `in_shape` and `batch`, PyTorch-default uniform init on
+-1/sqrt(C*k*k) drawn weight-then-bias, `input_scale` folded into the layer
(conv(s*x, W) = s*conv(x, W), dW = s*dW(x, dY), master weight unscaled,
ttrl/engine/conv/forward.py:160-205), `needs_input_grad=False` for a first
layer whose input is an observation, portable OIHW `state_dict`.

The master weight is kept in the GEMM layout the kernels read, Wt[k][O]:
k = (kh, kw, c) for fp32 NHWC inputs and k = (c, kh, kw) for uint8 NCHW
frames, the layout `input_layout="nchw_u8"` selects.  Activations are the
reference's flattened NHWC `[1, 1, N*H*W, C]`.
"""

from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from ttrl_amd import _lib
from ttrl_amd.engine.autograd import Tensor, is_grad_enabled, relu_mask
from ttrl_amd.engine.nn import Module
from ttrl_amd.engine.ops.fused import grad_targets
from ttrl_amd.engine.pending import PendingGrad
from ttrl_amd.engine.tensor import DeviceArray

__all__ = ["Conv2d", "ConvGeometry", "ConvDoesNotFit", "conv_out_size"]

LAYOUTS = {"nhwc": _lib.LAYOUT_NHWC_F32, "nchw_u8": _lib.LAYOUT_NCHW_U8}


class ConvDoesNotFit(ValueError):
    """A convolution geometry this device cannot run (kept for interface parity)."""


def conv_out_size(size: int, kernel: int, stride: int, padding: int = 0, *, axis: str = "h") -> int:
    """(size + 2p - k)/s + 1, refusing ragged geometry (ttrl/engine/conv/geometry.py:94-119)."""
    span = int(size) + 2 * int(padding) - int(kernel)
    if span < 0:
        raise ValueError(f"conv_out_size: kernel {kernel} is larger than the padded {axis} extent "
                         f"{size + 2 * padding}")
    if span % int(stride):
        raise ValueError(
            f"conv_out_size: ragged geometry on axis {axis}: size {size}, kernel {kernel}, "
            f"stride {stride}, padding {padding} leaves input rows that feed no output"
        )
    return span // int(stride) + 1


@dataclass(frozen=True)
class ConvGeometry:
    batch: int
    in_channels: int
    in_h: int
    in_w: int
    out_channels: int
    kernel: int
    stride: int = 1
    padding: int = 0
    fold: int = 1

    @property
    def out_h(self) -> int:
        return conv_out_size(self.in_h, self.kernel, self.stride, self.padding, axis="h")

    @property
    def out_w(self) -> int:
        return conv_out_size(self.in_w, self.kernel, self.stride, self.padding, axis="w")

    @property
    def out_shape(self) -> tuple[int, int, int]:
        return (self.out_channels, self.out_h, self.out_w)

    @property
    def in_numel(self) -> int:
        return self.batch * self.in_channels * self.in_h * self.in_w


def oihw_to_master(w: np.ndarray, layout: str) -> np.ndarray:
    """Logical (O, C, KH, KW) -> Wt[k][O] in the layer's k order."""
    o = w.shape[0]
    if layout == "nchw_u8":
        return np.ascontiguousarray(w.reshape(o, -1).T)  # k = (c, kh, kw)
    return np.ascontiguousarray(w.transpose(2, 3, 1, 0).reshape(-1, o))  # k = (kh, kw, c)


def master_to_oihw(wt: np.ndarray, shape, layout: str) -> np.ndarray:
    o, c, kh, kw = shape
    if layout == "nchw_u8":
        return np.ascontiguousarray(wt.T.reshape(o, c, kh, kw))
    return np.ascontiguousarray(wt.reshape(kh, kw, c, o).transpose(3, 2, 0, 1))


class Conv2d(Module):
    """A convolution holding its own master weight and optional bias."""

    def __init__(self, in_shape, out_channels: int, kernel: int, device, *, batch: int, stride: int = 1,
                 padding: int = 0, bias: bool = True, fold: int = 1, input_scale: float = 1.0, weight=None,
                 needs_input_grad: bool = True, profile=None, input_layout: str = "nhwc"):
        if len(tuple(in_shape)) != 3:
            raise ValueError(f"Conv2d: in_shape must be (channels, height, width), got {tuple(in_shape)}")
        if int(fold) != 1:
            raise ValueError(
                f"Conv2d: fold={fold} (space-to-depth) is not supported; the fold is a reindexing of the "
                "same convolution and this implementation runs the unfolded geometry directly"
            )
        if input_layout not in LAYOUTS:
            raise ValueError(f"Conv2d: input_layout must be one of {sorted(LAYOUTS)}, got {input_layout!r}")
        if input_layout == "nchw_u8" and needs_input_grad:
            raise ValueError("Conv2d: a uint8 frame input has no gradient; pass needs_input_grad=False")
        in_channels, in_h, in_w = (int(v) for v in in_shape)
        self.geom = ConvGeometry(batch=int(batch), in_channels=in_channels, in_h=in_h, in_w=in_w,
                                 out_channels=int(out_channels), kernel=int(kernel), stride=int(stride),
                                 padding=int(padding))
        _ = self.geom.out_shape  # validates the geometry
        self.device = device
        self.input_scale = float(input_scale)
        self.needs_input_grad = bool(needs_input_grad)
        self.input_layout = input_layout
        # Gradient bank (0-3) of the device context: when set, a backward
        # that writes the weight gradient fresh leaves its split-K sum to the
        # optimizer step (engine.pending).
        self.defer_bank = None
        if weight is None:
            bound = 1.0 / math.sqrt(in_channels * kernel * kernel)
            weight = np.random.uniform(-bound, bound, (out_channels, in_channels, kernel, kernel)).astype(np.float32)
        else:
            weight = np.asarray(weight, np.float32)
            want = (out_channels, in_channels, kernel, kernel)
            if weight.shape != want:
                raise ValueError(f"Conv2d: weight must have shape {want}, got {weight.shape}")
        self._oihw_shape = tuple(weight.shape)
        self.weight = Tensor.from_numpy(oihw_to_master(weight, input_layout), device, requires_grad=True)
        if bias:
            bound = 1.0 / math.sqrt(in_channels * kernel * kernel)
            b = np.random.uniform(-bound, bound, (1, 1, 1, out_channels)).astype(np.float32)
            self.bias = Tensor.from_numpy(b, device, requires_grad=True)
        else:
            self.bias = None

    # -- geometry ----------------------------------------------------------

    @property
    def out_shape(self) -> tuple[int, int, int]:
        return self.geom.out_shape

    @property
    def out_numel(self) -> int:
        return self.geom.batch * int(np.prod(self.geom.out_shape))

    def __repr__(self) -> str:
        g = self.geom
        return (f"Conv2d({g.in_channels}x{g.in_h}x{g.in_w} -> {self.out_shape}, k{g.kernel}, s{g.stride}, "
                f"p{g.padding}, {self.input_layout})")

    def _c_geom(self, batch: int) -> _lib.ConvGeom:
        g = self.geom
        return _lib.ConvGeom(batch, g.in_channels, g.in_h, g.in_w, g.out_channels, g.kernel, g.stride,
                             g.padding, LAYOUTS[self.input_layout])

    # -- parameters --------------------------------------------------------

    def weight_numpy(self) -> np.ndarray:
        """The logical (O, C, KH, KW) weight (host read)."""
        return master_to_oihw(self.weight.numpy(), self._oihw_shape, self.input_layout)

    def weight_grad_numpy(self) -> np.ndarray:
        if self.weight.grad is None:
            raise ValueError("Conv2d.weight_grad_numpy: no gradient has been accumulated")
        return master_to_oihw(self.weight.grad.numpy(), self._oihw_shape, self.input_layout)

    def load_weight_numpy(self, w_oihw) -> None:
        """Write a logical OIHW weight into the master, in place."""
        w = np.asarray(w_oihw, np.float32)
        if w.shape != self._oihw_shape:
            raise ValueError(f"Conv2d.load_weight_numpy: expected shape {self._oihw_shape}, got {w.shape}")
        self.weight.data.upload(oihw_to_master(w, self.input_layout))

    def state_dict(self) -> dict[str, np.ndarray]:
        state = {"weight": self.weight_numpy()}
        if self.bias is not None:
            state["bias"] = self.bias.numpy()
        return state

    def load_state_dict(self, state: dict, device=None) -> None:
        reference = self.state_dict()
        got, expected = set(state.keys()), set(reference)
        if got != expected:
            raise ValueError(
                "load_state_dict: checkpoint keys do not match module "
                f"parameters (missing={sorted(expected - got)}, extra={sorted(got - expected)})"
            )
        for name, want in reference.items():
            shape = tuple(int(d) for d in np.asarray(state[name]).shape)
            if shape != want.shape:
                raise ValueError(f"load_state_dict: shape mismatch for {name!r}: checkpoint has {shape}, "
                                 f"parameter expects {want.shape}")
        self.load_weight_numpy(state["weight"])
        if self.bias is not None:
            self.bias.data.upload(state["bias"])

    def at_batch(self, batch: int) -> "Conv2d":
        """This layer at another activation batch, sharing weight and bias."""
        view = object.__new__(Conv2d)
        view.__dict__.update(self.__dict__)
        g = self.geom
        view.geom = ConvGeometry(batch=int(batch), in_channels=g.in_channels, in_h=g.in_h, in_w=g.in_w,
                                 out_channels=g.out_channels, kernel=g.kernel, stride=g.stride, padding=g.padding)
        view.needs_input_grad = False
        return view

    # -- call --------------------------------------------------------------

    def forward(self, x: Tensor) -> Tensor:
        return self.forward_fused(x, relu=False)

    def _check_input(self, x: Tensor) -> int:
        """The activation batch, after validating dtype and geometry."""
        g = self.geom
        want_dtype = np.uint8 if self.input_layout == "nchw_u8" else np.float32
        if x.data.dtype != want_dtype:
            raise ValueError(f"conv2d: layer reads {np.dtype(want_dtype).name} {self.input_layout} input, "
                             f"got {x.data.dtype}")
        numel = x.data.numel
        if numel % (g.in_channels * g.in_h * g.in_w):
            raise ValueError(
                f"conv2d: activation has {numel} elements, not a whole number of "
                f"{g.in_channels}x{g.in_h}x{g.in_w} images; the layer was built for a different input."
            )
        batch = numel // (g.in_channels * g.in_h * g.in_w)
        if batch != g.batch:
            raise ValueError(
                f"conv2d: activation holds batch {batch} but this layer's geometry {g} requires "
                f"{g.batch}; build the layer for this batch or use at_batch()."
            )
        return batch

    def out_array(self, dev) -> DeviceArray:
        g = self.geom
        return DeviceArray(dev, (1, 1, g.batch * g.out_h * g.out_w, g.out_channels))

    def forward_fused(self, x: Tensor, relu: bool) -> Tensor:
        batch = self._check_input(x)
        cg = self._c_geom(batch)
        dev = x.device
        y = self.out_array(dev)
        bias = self.bias
        dev.call("ttrl_conv2d_forward", C.byref(cg), x.data.vp, self.weight.data.vp,
                 None if bias is None else bias.data.vp, y.vp, C.c_float(self.input_scale), int(relu))
        return self.node(x, y, relu)

    def node(self, x: Tensor, y: DeviceArray, relu: bool) -> Tensor:
        """The tape node of this layer's output `y` = conv(x) (+ReLU), computed elsewhere."""
        weight, bias = self.weight, self.bias
        needs = is_grad_enabled() and (x.requires_grad or weight.requires_grad or
                                       (bias is not None and bias.requires_grad))
        parents = (x, weight) + ((bias,) if bias is not None else ())
        out = Tensor(y, needs, parents if needs else (), "conv2d_relu" if relu else "conv2d")
        if not needs:
            return out
        cg = self._c_geom(self.geom.batch)
        dev = x.device
        x_data, w_data = x.data, weight.data
        scale = self.input_scale
        layer_has_dx = self.needs_input_grad
        bank = self.defer_bank

        def _backward(grad):
            if x.requires_grad and not layer_has_dx:
                raise RuntimeError(
                    "conv2d: this layer was built with needs_input_grad=False, "
                    "so it has no dX path, but its input requires a gradient. "
                    "Rebuild the layer with needs_input_grad=True, or detach "
                    "the activation it is given."
                )
            mask = y.vp if relu and not out._grad_masked else None
            (dw, db), beta_w = grad_targets(weight, bias)
            if dw is not None and bank is not None and beta_w == 0.0:
                src = _lib.GradSource()
                if x.requires_grad:
                    (dx,), beta_x = grad_targets(x)
                    xmask = relu_mask(x)
                    dev.call("ttrl_conv2d_backward_deferred", C.byref(cg), x_data.vp, C.c_float(scale), grad.vp, mask,
                             w_data.vp, dw.vp, None if db is None else db.vp, dx.vp,
                             None if xmask is None else xmask.vp, C.c_float(beta_x), int(bank), C.byref(src))
                    x._note_write(beta_x, xmask is not None)
                else:
                    dev.call("ttrl_conv2d_backward_weight_deferred", C.byref(cg), x_data.vp, C.c_float(scale),
                             grad.vp, mask, dw.vp, None if db is None else db.vp, int(bank), C.byref(src))
                if src.kind != _lib.GRAD_NONE:
                    PendingGrad(src, (weight, bias if db is not None else None))
                return
            if dw is not None and x.requires_grad:
                # both gradients in one call: the two GEMMs share a launch
                (dx,), beta_x = grad_targets(x)
                xmask = relu_mask(x)
                dev.call("ttrl_conv2d_backward", C.byref(cg), x_data.vp, C.c_float(scale), grad.vp, mask, w_data.vp,
                         dw.vp, None if db is None else db.vp, C.c_float(beta_w), dx.vp,
                         None if xmask is None else xmask.vp, C.c_float(beta_x))
                x._note_write(beta_x, xmask is not None)
                return
            if dw is not None:
                dev.call("ttrl_conv2d_backward_weight", C.byref(cg), x_data.vp, C.c_float(scale), grad.vp, mask,
                         dw.vp, None if db is None else db.vp, C.c_float(beta_w))
            elif db is not None:
                dw_tmp = DeviceArray(dev, w_data.shape)
                db_tmp = DeviceArray(dev, db.shape)
                dev.call("ttrl_conv2d_backward_weight", C.byref(cg), x_data.vp, C.c_float(scale), grad.vp, mask,
                         dw_tmp.vp, db_tmp.vp, C.c_float(0.0))
                from ttrl_amd.engine.ops import _kernels as Kk
                if beta_w:
                    Kk.binary_into("add", db, db_tmp, db)
                else:
                    db.copy_from(db_tmp)
            if x.requires_grad:
                (dx,), beta_x = grad_targets(x)
                xmask = relu_mask(x)
                dev.call("ttrl_conv2d_backward_input", C.byref(cg), grad.vp, mask, w_data.vp, dx.vp,
                         None if xmask is None else xmask.vp, C.c_float(scale), C.c_float(beta_x))
                x._note_write(beta_x, xmask is not None)

        out._backward = _backward
        return out
