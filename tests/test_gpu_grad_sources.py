"""Gradient sources: weight gradients left unreduced by one launch and
formed by a later one (ttrl_conv2d_backward_deferred,
ttrl_conv2d_backward_weight_deferred, ttrl_dqn_tail with loss_terms,
ttrl_grad_sources_materialize, ttrl_ordered_sums, ttrl_adam_step_sources),
called through the C ABI.

The bar is bit-exactness wherever the same floats are summed in the same
order: split partials summed in split order from zero and scaled as the
weight-gradient epilogue scales them (checked against the partials read back
and summed in float32 on the host), the tail's second-layer gradients and
batch means formed later against the tail's own, and the Adam step over an
arena with sources against forming the gradients first and stepping after.
Against the non-deferred launch, whose plan may split K differently, the
gradients agree to 1e-5 of their scale."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _up(device, host, dtype=np.float32):
    from ttrl_amd.engine.tensor import DeviceArray

    a = DeviceArray(device, np.shape(host), dtype)
    a.upload(np.asarray(host, dtype))
    return a


def _empty(device, shape):
    from ttrl_amd.engine.tensor import DeviceArray

    a = DeviceArray(device, shape)
    a.fill(0.0)
    return a


def _read(device, ptr, n):
    out = np.empty(n, np.float32)
    device.synchronize()
    device.call("ttrl_d2h", C.c_void_p(out.ctypes.data), C.c_void_p(ptr), C.c_size_t(out.nbytes))
    return out


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _split_sum(device, src, weight_rows, cols, has_bias):
    """The gradient the split partials describe, summed on the host in split
    order in float32 and scaled once (alpha * acc rounded, as an FMA with a
    zero addend rounds it)."""
    rows = weight_rows + int(has_bias)
    part = _read(device, src.part, src.splits * rows * cols).reshape(src.splits, rows, cols)
    acc = np.zeros((rows, cols), np.float32)
    for s in range(src.splits):
        acc = acc + part[s]
    w = (np.float64(np.float32(src.scale)) * acc[:weight_rows].astype(np.float64)).astype(np.float32)
    b = (np.float64(np.float32(src.bias_scale)) * acc[weight_rows].astype(np.float64)).astype(np.float32) \
        if has_bias else None
    return w, b


# conv2 and conv3 of the Nature CNN at batch 32 (NHWC fp32 inputs)
PAIR_GEOMS = [(32, 32, 20, 20, 64, 4, 2), (32, 64, 9, 9, 64, 3, 1)]


@pytest.mark.parametrize("geom", PAIR_GEOMS)
def test_deferred_conv_backward_forms_the_same_gradient(device, geom):
    from ttrl_amd import _lib

    B, Cin, H, W, O, k, s = geom
    g = _lib.ConvGeom(B, Cin, H, W, O, k, s, 0, 0)
    oh, ow = (H - k) // s + 1, (W - k) // s + 1
    Kp = Cin * k * k
    rng = np.random.default_rng(sum(geom))
    x = _up(device, rng.standard_normal((B, H, W, Cin)))
    dy = _up(device, rng.standard_normal((B * oh * ow, O)))
    wt = _up(device, 0.1 * rng.standard_normal((Kp, O)))
    ref = [_empty(device, sh) for sh in ((Kp, O), (O,), (B, H, W, Cin))]
    device.call("ttrl_conv2d_backward", C.byref(g), x.vp, C.c_float(1.0), dy.vp, None, wt.vp, ref[0].vp, ref[1].vp,
                C.c_float(0.0), ref[2].vp, None, C.c_float(0.0))
    got = [_empty(device, sh) for sh in ((Kp, O), (O,), (B, H, W, Cin))]
    src = _lib.GradSource()
    device.call("ttrl_conv2d_backward_deferred", C.byref(g), x.vp, C.c_float(1.0), dy.vp, None, wt.vp, got[0].vp,
                got[1].vp, got[2].vp, None, C.c_float(0.0), 1, C.byref(src))
    assert src.kind in (_lib.GRAD_NONE, _lib.GRAD_SPLITS)
    if src.kind == _lib.GRAD_SPLITS:
        assert (src.rows, src.cols, src.dw, src.db) == (Kp, O, got[0].ptr, got[1].ptr)
        want_w, want_b = _split_sum(device, src, Kp, O, True)
        device.call("ttrl_grad_sources_materialize", 1, C.byref(src))
        assert np.array_equal(got[0].numpy(), want_w)
        assert np.array_equal(got[1].numpy(), want_b)
    for a, b in zip(got, ref):
        assert _rel(a.numpy(), b.numpy()) < 1e-5


def test_deferred_conv_weight_gradient_of_frames(device):
    """conv1: uint8 NCHW frames scaled by 1/255, no input gradient."""
    from ttrl_amd import _lib

    B, Cin, H, O, k, s = 32, 4, 84, 32, 8, 4
    g = _lib.ConvGeom(B, Cin, H, H, O, k, s, 0, 1)
    oh = (H - k) // s + 1
    Kp = Cin * k * k
    rng = np.random.default_rng(5)
    x = _up(device, rng.integers(0, 256, (B, Cin, H, H)), np.uint8)
    dy = _up(device, rng.standard_normal((B * oh * oh, O)))
    scale = C.c_float(1.0 / 255.0)
    ref = [_empty(device, sh) for sh in ((Kp, O), (O,))]
    device.call("ttrl_conv2d_backward_weight", C.byref(g), x.vp, scale, dy.vp, None, ref[0].vp, ref[1].vp,
                C.c_float(0.0))
    got = [_empty(device, sh) for sh in ((Kp, O), (O,))]
    src = _lib.GradSource()
    device.call("ttrl_conv2d_backward_weight_deferred", C.byref(g), x.vp, scale, dy.vp, None, got[0].vp, got[1].vp, 2,
                C.byref(src))
    if src.kind == _lib.GRAD_SPLITS:
        assert src.scale == np.float32(1.0 / 255.0) and src.bias_scale == 1.0
        want_w, want_b = _split_sum(device, src, Kp, O, True)
        device.call("ttrl_grad_sources_materialize", 1, C.byref(src))
        assert np.array_equal(got[0].numpy(), want_w)
        assert np.array_equal(got[1].numpy(), want_b)
    for a, b in zip(got, ref):
        assert _rel(a.numpy(), b.numpy()) < 1e-5


def _tail_setup(device, rng, B=32, K=256, F=512, A=6, G=3):
    from ttrl_amd import _lib

    ins = {
        "x": [_up(device, rng.random((B, K))) for _ in range(G)],
        "W1": [_up(device, 0.05 * rng.standard_normal((K, F))) for _ in range(G)],
        "b1": [_up(device, 0.1 * rng.standard_normal(F)) for _ in range(G)],
        "W2": [_up(device, 0.1 * rng.standard_normal((F, A))) for _ in range(G)],
        "b2": [_up(device, 0.1 * rng.standard_normal(A)) for _ in range(G)],
        "onehot": _up(device, np.eye(A)[rng.integers(0, A, B)]),
        "r": _up(device, rng.standard_normal(B)), "d": _up(device, (rng.random(B) < 0.2).astype(np.float32)),
        "disc": _up(device, np.full(B, 0.99 ** 3)), "w": _up(device, 0.5 + rng.random(B)),
    }

    def desc(out):
        d = _lib.DqnTailDesc()
        d.B, d.K, d.F, d.A, d.groups = B, K, F, A, G
        for g in range(G):
            d.x[g], d.W1[g], d.b1[g] = ins["x"][g].ptr, ins["W1"][g].ptr, ins["b1"][g].ptr
            d.W2[g], d.b2[g] = ins["W2"][g].ptr, ins["b2"][g].ptr
            d.h[g], d.q[g] = out["h"][g].ptr, out["q"][g].ptr
        d.actions_onehot, d.rewards, d.dones = ins["onehot"].ptr, ins["r"].ptr, ins["d"].ptr
        d.discounts, d.is_weights, d.delta = ins["disc"].ptr, ins["w"].ptr, 1.0
        d.loss, d.mean_q, d.td_abs, d.dq, d.dh = (out[k].ptr for k in ("loss", "mean_q", "td_abs", "dq", "dh"))
        d.dW2, d.db2, d.beta_w = out["dW2"].ptr, out["db2"].ptr, 0.0
        return d

    def outputs():
        return {"h": [_empty(device, (B, F)) for _ in range(G)], "q": [_empty(device, (B, A)) for _ in range(G)],
                "loss": _empty(device, (1,)), "mean_q": _empty(device, (1,)), "td_abs": _empty(device, (B,)),
                "dq": _empty(device, (B, A)), "dh": _empty(device, (B, F)), "dW2": _empty(device, (F, A)),
                "db2": _empty(device, (A,)), "terms": _empty(device, (B, 2))}

    return desc, outputs


def test_tail_with_deferred_head_gradients_and_means(device):
    """ttrl_dqn_tail leaving dW2, db2, loss and mean Q to an outer-product
    source and ordered sums gives the bits of the tail forming them itself."""
    from ttrl_amd import _lib

    B, F, A = 32, 512, 6
    desc, outputs = _tail_setup(device, np.random.default_rng(11), B=B, F=F, A=A)
    ref = outputs()
    device.call("ttrl_dqn_tail", C.byref(desc(ref)))
    got = outputs()
    d = desc(got)
    d.dW2, d.db2, d.loss_terms = None, None, got["terms"].ptr
    device.call("ttrl_dqn_tail", C.byref(d))
    src = _lib.GradSource(kind=_lib.GRAD_OUTER, rows=F, cols=A, dw=got["dW2"].ptr, db=got["db2"].ptr,
                          u=got["h"][0].ptr, v=got["dq"].ptr, batch=B)
    device.call("ttrl_grad_sources_materialize", 1, C.byref(src))
    inv_b = float(np.float32(1.0) / np.float32(B))
    sums = (_lib.OrderedSum * 2)(_lib.OrderedSum(got["terms"].ptr, B, 2, inv_b, got["loss"].ptr),
                                 _lib.OrderedSum(got["terms"].ptr + 4, B, 2, inv_b, got["mean_q"].ptr))
    device.call("ttrl_ordered_sums", 2, sums)
    for k in ("loss", "mean_q", "td_abs", "dq", "dh", "dW2", "db2"):
        assert np.array_equal(got[k].numpy(), ref[k].numpy()), k
    for g in range(3):
        assert np.array_equal(got["h"][g].numpy(), ref["h"][g].numpy())
        assert np.array_equal(got["q"][g].numpy(), ref["q"][g].numpy())
    # the outer product itself, in float64
    h0, dq = got["h"][0].numpy().astype(np.float64), got["dq"].numpy().astype(np.float64)
    assert _rel(got["dW2"].numpy(), h0.T @ dq) < 1e-6
    assert _rel(got["db2"].numpy(), dq.sum(0)) < 1e-6
    # the tail refuses second-layer gradients alongside deferred means
    d.dW2 = got["dW2"].ptr
    lib = _lib.lib()
    assert lib.ttrl_dqn_tail(device.ctx, C.byref(d)) == _lib.TTRL_EINVAL


def test_tail_vector_and_scalar_paths_agree_bitwise(device, monkeypatch):
    """ttrl_dqn_tail reads the split partials, biases and W2 as float4s when
    its first layer's GEMM split K, every buffer is 16-byte aligned and
    F % 4 == 0, and element by element otherwise; both form the same sums in
    the same order.  The DQN update's shape (K = 3136, the GEMM held at 7
    splits), then the same inputs with the first-layer outputs one float off
    alignment, which take the element path: every output carries the same
    bits."""
    B, K, F, A, G = 32, 3136, 512, 6, 3
    monkeypatch.setenv("TTRL_GEMM_FORCE", "7:7")  # 32 x 32 tiles, two k-groups, 7 splits
    desc, outputs = _tail_setup(device, np.random.default_rng(12), B=B, K=K, F=F, A=A, G=G)
    vec = outputs()
    device.call("ttrl_dqn_tail", C.byref(desc(vec)))
    sca = outputs()
    hbuf = [_empty(device, (B * F + 4,)) for _ in range(G)]
    d = desc(sca)
    for g in range(G):
        d.h[g] = hbuf[g].ptr + 4  # 4 bytes past a 16-byte boundary
    device.call("ttrl_dqn_tail", C.byref(d))
    for k in ("loss", "mean_q", "td_abs", "dq", "dh", "dW2", "db2"):
        assert np.array_equal(sca[k].numpy(), vec[k].numpy()), k
    for g in range(G):
        assert np.array_equal(hbuf[g].numpy()[1:1 + B * F].reshape(B, F), vec["h"][g].numpy()), g
        assert np.array_equal(sca["q"][g].numpy(), vec["q"][g].numpy()), g
    assert float(vec["loss"].numpy()[0]) > 0.0 and np.count_nonzero(vec["dh"].numpy()) > 0


# An arena of N floats: a split-partials source (weight 40 x 32 + bias 32)
# and an outer-product source (weight 64 x 6 + bias 6, padded to 8) inside it.
N = 16_384
SPLIT_W, SPLIT_B, OUTER_W, OUTER_B = 1024, 2432, 4096, 4480


def _arena_sources(device, g_ptr, rng):
    from ttrl_amd import _lib

    splits, rows, cols = 5, 40, 32
    part = _up(device, rng.standard_normal((splits, rows + 1, cols)))
    u = _up(device, rng.standard_normal((32, 64)))
    v = _up(device, rng.standard_normal((32, 6)))
    srcs = (_lib.GradSource * 2)(
        _lib.GradSource(kind=_lib.GRAD_SPLITS, rows=rows, cols=cols, dw=g_ptr + 4 * SPLIT_W, db=g_ptr + 4 * SPLIT_B,
                        part=part.ptr, splits=splits, scale=0.25, bias_scale=1.0),
        _lib.GradSource(kind=_lib.GRAD_OUTER, rows=64, cols=6, dw=g_ptr + 4 * OUTER_W, db=g_ptr + 4 * OUTER_B,
                        u=u.ptr, v=v.ptr, batch=32))
    return srcs, (part, u, v)


@pytest.mark.parametrize("n", [N, N + 3])
def test_adam_step_with_sources_matches_forming_then_stepping(device, n):
    from ttrl_amd import _lib

    rng = np.random.default_rng(n)
    p0, g0 = rng.standard_normal(n), rng.standard_normal(n)
    g0[OUTER_B + 6:OUTER_B + 8] = 0.0  # an arena's padding holds no gradient
    s0, v0 = 0.1 * rng.standard_normal(n), rng.random(n)
    hyper = (1e-3, 0.9, 0.999, 1e-8, 0.01)
    arenas = []
    for _ in range(2):
        arenas.append({"p": _up(device, p0), "g": _up(device, g0), "S": _up(device, s0), "V": _up(device, v0),
                       "step": _up(device, np.array([3]), np.int32), "gsq": _empty(device, (1,))})
    terms = _up(device, rng.standard_normal((32, 2)))
    # reference: form the gradients into the arena, then the plain step
    ref = arenas[0]
    srcs, keep = _arena_sources(device, ref["g"].ptr, np.random.default_rng(1))
    device.call("ttrl_grad_sources_materialize", 2, srcs)
    device.call("ttrl_adam_step", ref["p"].vp, ref["g"].vp, ref["S"].vp, ref["V"].vp, C.c_long(n), ref["step"].vp,
                *(C.c_float(h) for h in hyper), ref["gsq"].vp, 0)
    ref_sum = _empty(device, (2,))
    ref_sums = (_lib.OrderedSum * 2)(_lib.OrderedSum(terms.ptr, 32, 2, 0.5, ref_sum.ptr),
                                     _lib.OrderedSum(terms.ptr + 4, 32, 2, 1.0, ref_sum.ptr + 4))
    device.call("ttrl_ordered_sums", 2, ref_sums)
    # one launch pair: the step forming the sources, its finish the sums
    got = arenas[1]
    srcs2, keep2 = _arena_sources(device, got["g"].ptr, np.random.default_rng(1))
    got_sum = _empty(device, (2,))
    sums = (_lib.OrderedSum * 2)(_lib.OrderedSum(terms.ptr, 32, 2, 0.5, got_sum.ptr),
                                 _lib.OrderedSum(terms.ptr + 4, 32, 2, 1.0, got_sum.ptr + 4))
    d = _lib.AdamSourcesDesc(got["p"].ptr, got["g"].ptr, got["S"].ptr, got["V"].ptr, n, got["step"].ptr, *hyper,
                             got["gsq"].ptr, 0, 2, srcs2, 2, sums, store_grads=1)
    device.call("ttrl_adam_step_sources", C.byref(d))
    for k in ("p", "g", "S", "V", "step"):
        assert np.array_equal(got[k].numpy(), ref[k].numpy()), k
    assert got["gsq"].numpy()[0] == pytest.approx(float(ref["gsq"].numpy()[0]), rel=1e-6)
    assert np.array_equal(got_sum.numpy(), ref_sum.numpy())
    t = terms.numpy()
    acc = np.float32(0.0)
    for i in range(32):
        acc = np.float32(acc + t[i, 0])
    assert got_sum.numpy()[0] == np.float32(acc * np.float32(0.5))


def test_adam_step_without_storing_the_formed_gradients(device):
    """store_grads 0: the parameters, moments, count, sum of g^2 and ordered
    sums are those of the storing step, bit for bit, the sources' gradient
    ranges of g are left as they were, and materializing the same sources
    afterwards writes the gradients the storing step would have, after two
    steps in a row."""
    from ttrl_amd import _lib

    n = N
    rng = np.random.default_rng(7)
    p0, g0 = rng.standard_normal(n), rng.standard_normal(n)
    g0[OUTER_B + 6:OUTER_B + 8] = 0.0
    s0, v0 = 0.1 * rng.standard_normal(n), rng.random(n)
    hyper = (1e-3, 0.9, 0.999, 1e-8, 0.0)
    terms = _up(device, rng.standard_normal((32, 2)))
    out = []
    for store in (1, 0):
        a = {"p": _up(device, p0), "g": _up(device, g0), "S": _up(device, s0), "V": _up(device, v0),
             "step": _up(device, np.array([5]), np.int32), "gsq": _empty(device, (1,)), "sum": _empty(device, (1,))}
        srcs, keep = _arena_sources(device, a["g"].ptr, np.random.default_rng(1))
        sums = (_lib.OrderedSum * 1)(_lib.OrderedSum(terms.ptr, 32, 2, 0.5, a["sum"].ptr))
        for _ in range(2):
            d = _lib.AdamSourcesDesc(a["p"].ptr, a["g"].ptr, a["S"].ptr, a["V"].ptr, n, a["step"].ptr, *hyper,
                                     a["gsq"].ptr, 0, 2, srcs, 1, sums, store_grads=store)
            device.call("ttrl_adam_step_sources", C.byref(d))
        host = {k: v.numpy() for k, v in a.items()}
        if not store:
            g = host["g"]
            untouched = np.asarray(g0, np.float32)
            for lo, hi in ((SPLIT_W, SPLIT_W + 40 * 32), (OUTER_W, OUTER_W + 64 * 6)):
                assert np.array_equal(g[lo:hi], untouched[lo:hi])
            device.call("ttrl_grad_sources_materialize", 2, srcs)
            host["g"] = a["g"].numpy()
        out.append((host, keep))
    (ref, _), (got, _) = out
    for k in ("p", "g", "S", "V", "step", "gsq", "sum"):
        assert np.array_equal(got[k], ref[k]), k
    assert int(got["step"][0]) == 7


def test_adam_step_with_sources_refuses_bad_sources(device):
    from ttrl_amd import _lib

    lib = _lib.lib()
    a = {k: _empty(device, (N,)) for k in ("p", "g", "S", "V")}
    step = _up(device, np.array([0]), np.int32)

    def run(srcs):
        arr = (_lib.GradSource * len(srcs))(*srcs)
        d = _lib.AdamSourcesDesc(a["p"].ptr, a["g"].ptr, a["S"].ptr, a["V"].ptr, N, step.ptr, 1e-3, 0.9, 0.999, 1e-8,
                                 0.0, None, 0, len(srcs), arr, 0, None)
        return lib.ttrl_adam_step_sources(device.ctx, C.byref(d)), lib.ttrl_last_error()

    part = _empty(device, (4 * 8 * 32,))
    good = dict(kind=_lib.GRAD_SPLITS, rows=8, cols=32, part=part.ptr, splits=4, scale=1.0, bias_scale=1.0)
    g = a["g"].ptr
    rc, msg = run([_lib.GradSource(dw=g + 4 * 64, **good), _lib.GradSource(dw=g + 4 * 128, **good)])
    assert rc == _lib.TTRL_EINVAL and b"same gradient" in msg
    rc, msg = run([_lib.GradSource(dw=g + 4 * (N - 64), **good)])
    assert rc == _lib.TTRL_EINVAL and b"outside the arena" in msg
    rc, msg = run([_lib.GradSource(kind=7, rows=8, cols=32, dw=g)])
    assert rc == _lib.TTRL_EINVAL and b"unknown kind" in msg
    rc, msg = run([_lib.GradSource(dw=g + 4 * 64 + 8, **good)])
    assert rc == _lib.TTRL_EINVAL and b"aligned" in msg
    t = _empty(device, (4,))
    dup = (_lib.OrderedSum * 2)(_lib.OrderedSum(t.ptr, 2, 1, 1.0, t.ptr + 8),
                                _lib.OrderedSum(t.ptr, 2, 1, 0.5, t.ptr + 8))
    assert lib.ttrl_ordered_sums(device.ctx, 2, dup) == _lib.TTRL_EINVAL
    assert b"same value" in lib.ttrl_last_error()


@pytest.mark.parametrize("rows,cols,batch", [(100, 128, 32), (48, 512, 5)])
def test_wide_outer_source_formed_by_tiles(device, rows, cols, batch):
    """An outer-product source too wide for one row band of v in LDS (a
    linear layer's dW = x^T dZ, db = column sums of dZ) is formed by 16 x 64
    tiles, the last row band ragged: the step forming it equals forming it
    first and stepping after, bit for bit, and the formed gradient is x^T dZ
    and the column sums to float32 accuracy."""
    from ttrl_amd import _lib

    rng = np.random.default_rng(rows + batch)
    wn = rows * cols
    n = wn + cols + 40
    u = rng.standard_normal((batch, rows))
    v = rng.standard_normal((batch, cols))
    ud, vd = _up(device, u), _up(device, v)
    p0, g0 = rng.standard_normal(n), rng.standard_normal(n)
    s0, v0 = 0.1 * rng.standard_normal(n), rng.random(n)
    hyper = (1e-3, 0.9, 0.999, 1e-8, 0.0)

    def arena():
        return {"p": _up(device, p0), "g": _up(device, g0), "S": _up(device, s0), "V": _up(device, v0),
                "step": _up(device, np.array([1]), np.int32), "gsq": _empty(device, (1,))}

    def source(a):
        return (_lib.GradSource * 1)(_lib.GradSource(kind=_lib.GRAD_OUTER, rows=rows, cols=cols, dw=a["g"].ptr,
                                                     db=a["g"].ptr + 4 * wn, u=ud.ptr, v=vd.ptr, batch=batch))

    ref = arena()
    device.call("ttrl_grad_sources_materialize", 1, source(ref))
    g = ref["g"].numpy()
    want_w = np.asarray(u, np.float32).astype(np.float64).T @ np.asarray(v, np.float32).astype(np.float64)
    assert _rel(g[:wn], want_w.ravel()) < 1e-5
    assert _rel(g[wn:wn + cols], np.asarray(v, np.float32).astype(np.float64).sum(0)) < 1e-5
    assert np.array_equal(g[wn + cols:], np.asarray(g0[wn + cols:], np.float32))  # past the block: untouched
    device.call("ttrl_adam_step", ref["p"].vp, ref["g"].vp, ref["S"].vp, ref["V"].vp, C.c_long(n), ref["step"].vp,
                *(C.c_float(h) for h in hyper), ref["gsq"].vp, 0)
    got = arena()
    d = _lib.AdamSourcesDesc(got["p"].ptr, got["g"].ptr, got["S"].ptr, got["V"].ptr, n, got["step"].ptr, *hyper,
                             got["gsq"].ptr, 0, 1, source(got), 0, None, store_grads=1)
    device.call("ttrl_adam_step_sources", C.byref(d))
    for k in ("p", "g", "S", "V", "step"):
        assert np.array_equal(got[k].numpy(), ref[k].numpy()), k
    assert got["gsq"].numpy()[0] == pytest.approx(float(ref["gsq"].numpy()[0]), rel=1e-5)
