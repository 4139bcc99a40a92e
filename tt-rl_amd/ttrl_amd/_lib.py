"""ctypes binding of libttrl_hip.so (the C ABI declared in include/ttrl_hip.h).

The library is the only compute path: importing this module does not load it,
`lib()` does, and it raises if the shared object is missing rather than
falling back to any host implementation.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libttrl_hip.so"

TTRL_OK = 0
TTRL_EINVAL = -1
TTRL_EHIP = -2
TTRL_ENOMEM = -3
TTRL_ESTATE = -4

LAYOUT_NHWC_F32 = 0
LAYOUT_NCHW_U8 = 1

# unary / binary / reduce op codes (enum order in ttrl_hip.h)
U_OPS = ["relu", "abs", "sign", "square", "exp", "log", "tanh", "sigmoid", "sqrt", "neg",
         "add_s", "mul_s", "rsub_s", "div_s", "eqz", "gtz", "isfinite"]
U = {name: i for i, name in enumerate(U_OPS)}
B_OPS = ["add", "sub", "mul", "div", "relu_bw", "max", "min", "eq"]
BOP = {name: i for i, name in enumerate(B_OPS)}
R = {"sum": 0, "max": 1, "argmax": 2}


class LinearDesc(C.Structure):
    """Mirror of ttrl_linear_desc."""

    _fields_ = [
        ("M", C.c_int), ("K", C.c_int), ("N", C.c_int), ("groups", C.c_int),
        ("x", C.c_void_p), ("ldx", C.c_long), ("gx", C.c_long),
        ("x2", C.c_void_p), ("ldx2", C.c_long), ("gx2", C.c_long), ("k1", C.c_int),
        ("W", C.c_void_p), ("gW", C.c_long),
        ("b", C.c_void_p), ("gb", C.c_long),
        ("W2", C.c_void_p), ("b2", C.c_void_p), ("n1", C.c_int),
        ("y", C.c_void_p), ("gy", C.c_long),
        ("relu", C.c_int), ("clamp_col", C.c_int), ("lo", C.c_float), ("hi", C.c_float),
        ("ymask", C.c_void_p), ("dy", C.c_void_p),
        ("dW", C.c_void_p), ("db", C.c_void_p), ("dW2", C.c_void_p), ("db2", C.c_void_p),
        ("dx", C.c_void_p), ("lddx", C.c_long), ("gdx", C.c_long),
        ("dx_col0", C.c_int), ("dx_cols", C.c_int),
        ("beta_w", C.c_float), ("beta_x", C.c_float),
        ("dxmask", C.c_void_p),
        ("xg", C.c_void_p * 4), ("x2g", C.c_void_p * 4), ("Wg", C.c_void_p * 4), ("bg", C.c_void_p * 4),
    ]


class DeviceInfo(C.Structure):
    """Mirror of ttrl_device_info."""

    _fields_ = [
        ("name", C.c_char * 256), ("arch", C.c_char * 64), ("compute_units", C.c_int), ("wavefront_size", C.c_int),
        ("lds_per_cu", C.c_long), ("lds_per_workgroup", C.c_long), ("l2_bytes", C.c_long), ("hbm_bytes", C.c_long),
        ("clock_khz", C.c_int), ("memory_clock_khz", C.c_int), ("memory_bus_bits", C.c_int),
        ("pci_bus_id", C.c_int), ("pci_device_id", C.c_int), ("pci_domain_id", C.c_int),
    ]


class AdamRange(C.Structure):
    """Mirror of ttrl_adam_range."""

    _fields_ = [
        ("p", C.c_void_p), ("g", C.c_void_p), ("m_s", C.c_void_p), ("v_s", C.c_void_p), ("n", C.c_long),
        ("step", C.c_void_p), ("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
        ("weight_decay", C.c_float), ("slot", C.c_int),
    ]


class AdamFinish(C.Structure):
    """Mirror of ttrl_adam_finish."""

    _fields_ = [("slot", C.c_int), ("n", C.c_long), ("step", C.c_void_p), ("grad_sq", C.c_void_p),
                ("accumulate", C.c_int), ("parts", C.c_int)]


class DqnTailDesc(C.Structure):
    """Mirror of ttrl_dqn_tail_desc."""

    _fields_ = [
        ("B", C.c_int), ("K", C.c_int), ("F", C.c_int), ("A", C.c_int), ("groups", C.c_int),
        ("x", C.c_void_p * 3), ("W1", C.c_void_p * 3), ("b1", C.c_void_p * 3), ("h", C.c_void_p * 3),
        ("W2", C.c_void_p * 3), ("b2", C.c_void_p * 3), ("q", C.c_void_p * 3),
        ("actions_onehot", C.c_void_p), ("rewards", C.c_void_p), ("dones", C.c_void_p),
        ("discounts", C.c_void_p), ("is_weights", C.c_void_p), ("delta", C.c_float),
        ("loss", C.c_void_p), ("mean_q", C.c_void_p), ("td_abs", C.c_void_p), ("dq", C.c_void_p),
        ("next_actions", C.c_void_p), ("td_target", C.c_void_p), ("dh", C.c_void_p), ("dW2", C.c_void_p),
        ("db2", C.c_void_p), ("beta_w", C.c_float), ("loss_terms", C.c_void_p),
    ]


class SacHeadDesc(C.Structure):
    """Mirror of ttrl_sac_head_desc."""

    _fields_ = [
        ("rows", C.c_int), ("K", C.c_int), ("d", C.c_int), ("x", C.c_void_p), ("W1", C.c_void_p),
        ("b1", C.c_void_p), ("W2", C.c_void_p), ("b2", C.c_void_p), ("lo", C.c_float), ("hi", C.c_float),
        ("noise", C.c_void_p), ("centre", C.c_void_p), ("half_width", C.c_void_p), ("log_det", C.c_float),
        ("head", C.c_void_p), ("action", C.c_void_p), ("logp", C.c_void_p), ("u", C.c_void_p),
    ]


GRAD_NONE, GRAD_SPLITS, GRAD_OUTER = 0, 1, 2


class GradSource(C.Structure):
    """Mirror of ttrl_grad_source."""

    _fields_ = [
        ("kind", C.c_int), ("rows", C.c_int), ("cols", C.c_int), ("dw", C.c_void_p), ("db", C.c_void_p),
        ("part", C.c_void_p), ("splits", C.c_int), ("scale", C.c_float), ("bias_scale", C.c_float),
        ("u", C.c_void_p), ("v", C.c_void_p), ("batch", C.c_int),
    ]


class OrderedSum(C.Structure):
    """Mirror of ttrl_ordered_sum."""

    _fields_ = [("src", C.c_void_p), ("n", C.c_int), ("stride", C.c_int), ("scale", C.c_float),
                ("dst", C.c_void_p)]


class AdamSourcesDesc(C.Structure):
    """Mirror of ttrl_adam_sources_desc."""

    _fields_ = [
        ("p", C.c_void_p), ("g", C.c_void_p), ("m_s", C.c_void_p), ("v_s", C.c_void_p), ("n", C.c_long),
        ("step", C.c_void_p), ("lr", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float), ("eps", C.c_float),
        ("weight_decay", C.c_float), ("grad_sq", C.c_void_p), ("accumulate_grad_sq", C.c_int),
        ("nsources", C.c_int), ("sources", C.POINTER(GradSource)), ("nsums", C.c_int),
        ("sums", C.POINTER(OrderedSum)), ("store_grads", C.c_int),
    ]


class ReplayRing(C.Structure):
    """Mirror of ttrl_replay_ring."""

    _fields_ = [
        ("lanes", C.c_int), ("cols", C.c_int), ("obs_bytes", C.c_long),
        ("obs", C.c_void_p), ("actions", C.c_void_p), ("rewards", C.c_void_p), ("dones", C.c_void_p),
        ("ends", C.c_void_p), ("final_slot", C.c_void_p), ("final_obs", C.c_void_p), ("final_rows", C.c_int),
        ("weight", C.c_void_p), ("max_priority", C.c_void_p), ("alpha", C.c_double), ("epsilon", C.c_double),
        ("action_vec", C.c_void_p), ("action_dim", C.c_int),
    ]


class ReplayDraw(C.Structure):
    """Mirror of ttrl_replay_draw."""

    _fields_ = [
        ("n", C.c_int), ("lane", C.c_void_p), ("lanes_out", C.c_void_p), ("u", C.c_void_p), ("start", C.c_void_p),
        ("count", C.c_void_p),
        ("chunk", C.c_int), ("max_chunks", C.c_int), ("chunk_sums", C.c_void_p), ("sums", C.c_void_p),
        ("total_count", C.c_long), ("beta", C.c_double), ("cols_out", C.c_void_p), ("picked_weight", C.c_void_p),
        ("weights_out", C.c_void_p), ("n_step", C.c_int), ("gamma", C.c_double), ("obs_out", C.c_void_p),
        ("next_obs_out", C.c_void_p), ("actions_onehot", C.c_void_p), ("num_actions", C.c_int),
        ("actions_out", C.c_void_p), ("action_vec_out", C.c_void_p), ("rewards_out", C.c_void_p),
        ("dones_out", C.c_void_p), ("discounts_out", C.c_void_p),
    ]


class SacCriticParams(C.Structure):
    """Mirror of ttrl_sac_critic_params."""

    _fields_ = [(n, C.c_void_p) for n in ("W1", "b1", "W2", "b2", "w3", "b3")]


SAC_FUSED_BUFFERS = ("h1", "h2", "headp", "head", "act", "u", "q1", "q2", "qp", "q1pi", "q2pi", "qppi", "dQ", "dq2",
                     "dq1", "dap", "dhead", "dh2", "dh1", "terms")
SAC_FUSED_METRICS = ("critic_loss", "alpha", "actor_loss", "alpha_loss", "q_target", "td_abs", "logp")
SAC_FUSED_POLICY_GRADS = ("gP1", "gp1", "gP2", "gp2", "gWm", "gbm", "gWl", "gbl")


class SacFusedDesc(C.Structure):
    """Mirror of ttrl_sac_fused_desc."""

    _fields_ = ([("B", C.c_int), ("O", C.c_int), ("A", C.c_int), ("H", C.c_int)]
                + [(n, C.c_void_p) for n in ("P1", "p1", "P2", "p2", "Wm", "bm", "Wl", "bl")]
                + [("log_std_min", C.c_float), ("log_std_max", C.c_float), ("centre", C.c_void_p),
                   ("half_width", C.c_void_p), ("log_det", C.c_float), ("critic", SacCriticParams * 4)]
                + [(n, C.c_void_p) for n in ("obs_pair", "actions", "obs_actions", "noise_pair", "rewards", "dones",
                                             "discounts", "is_weights", "log_alpha")]
                + [("target_entropy", C.c_float), ("learn_alpha", C.c_int)]
                + [(n, C.c_void_p) for n in SAC_FUSED_BUFFERS + SAC_FUSED_METRICS + SAC_FUSED_POLICY_GRADS]
                + [("g_critic", (C.c_void_p * 6) * 2), ("g_log_alpha", C.c_void_p)]
                + [("fuse_adam", C.c_int), ("critic_adam", AdamRange), ("actor_adam", AdamRange),
                   ("alpha_adam", AdamRange), ("polyak_dst", C.c_void_p), ("tau", C.c_float),
                   ("adam_scalars", C.c_void_p)])


class ConvGeom(C.Structure):
    """Mirror of ttrl_conv_geom."""

    _fields_ = [(name, C.c_int) for name in (
        "batch", "in_c", "in_h", "in_w", "out_c", "kernel", "stride", "padding", "in_layout")]


P = C.c_void_p
I = C.c_int
L = C.c_long
F = C.c_float
SZ = C.c_size_t

#: name -> (argtypes, restype); every entry point of ttrl_hip.h.
SIGNATURES = {
    "ttrl_last_error": ([], C.c_char_p),
    "ttrl_version": ([], I),
    "ttrl_device_count": ([C.POINTER(I)], I),
    "ttrl_device_query": ([I, C.POINTER(DeviceInfo)], I),
    "ttrl_init": ([I, C.POINTER(P)], I),
    "ttrl_shutdown": ([P], I),
    "ttrl_sync": ([P], I),
    "ttrl_stream": ([P], P),
    "ttrl_pool_create": ([P, C.POINTER(I)], I),
    "ttrl_pool_release": ([P, I], I),
    "ttrl_pool_use": ([P, I, C.POINTER(I)], I),
    "ttrl_pool_stats": ([P, I, C.POINTER(SZ), C.POINTER(SZ)], I),
    "ttrl_alloc": ([P, SZ, C.POINTER(P)], I),
    "ttrl_free": ([P, P], I),
    "ttrl_h2d": ([P, P, P, SZ], I),
    "ttrl_h2d_enqueue": ([P, P, P, SZ], I),
    "ttrl_d2h": ([P, P, P, SZ], I),
    "ttrl_d2d": ([P, P, P, SZ], I),
    "ttrl_fill_f32": ([P, P, F, L], I),
    "ttrl_fill_i32": ([P, P, I, L], I),
    "ttrl_capture_begin": ([P], I),
    "ttrl_capture_end": ([P, C.POINTER(P)], I),
    "ttrl_capture_abort": ([P], I),
    "ttrl_graph_launch": ([P, P], I),
    "ttrl_graph_set_direct": ([P, I], I),
    "ttrl_mfma_rate": ([P, I, I, P, C.POINTER(C.c_double)], I),
    "ttrl_graph_launch_n": ([P, P, I], I),
    "ttrl_graph_step": ([P, P, P, P, SZ, P, P, SZ], I),
    "ttrl_host_alloc": ([P, SZ, C.POINTER(P)], I),
    "ttrl_host_free": ([P, P], I),
    "ttrl_host_alloc_mapped": ([P, SZ, C.POINTER(P), C.POINTER(P)], I),
    "ttrl_graph_nodes": ([P, C.POINTER(SZ)], I),
    "ttrl_graph_destroy": ([P], I),
    "ttrl_plans_export": ([P, C.c_char_p, SZ, C.POINTER(SZ)], I),
    "ttrl_plans_import": ([P, C.c_char_p, C.POINTER(I)], I),
    "ttrl_timer_start": ([P], I),
    "ttrl_timer_stop": ([P, C.POINTER(F)], I),
    "ttrl_matmul": ([P, I, I, I, P, L, I, P, L, I, P, L, F, F], I),
    "ttrl_linear_forward": ([P, C.POINTER(LinearDesc)], I),
    "ttrl_linear_backward": ([P, C.POINTER(LinearDesc)], I),
    "ttrl_linear_forward_multi": ([P, I, I, I, I, C.POINTER(P), C.POINTER(P), C.POINTER(P), C.POINTER(P), I], I),
    "ttrl_conv_out_size": ([I, I, I, I, C.POINTER(I)], I),
    "ttrl_conv2d_forward": ([P, C.POINTER(ConvGeom), P, P, P, P, F, I], I),
    "ttrl_conv2d_forward_multi": ([P, C.POINTER(ConvGeom), I, C.POINTER(P), C.POINTER(P), C.POINTER(P),
                                   C.POINTER(P), F, I], I),
    "ttrl_conv2d_backward_weight": ([P, C.POINTER(ConvGeom), P, F, P, P, P, P, F], I),
    "ttrl_conv2d_backward_input": ([P, C.POINTER(ConvGeom), P, P, P, P, P, F, F], I),
    "ttrl_conv2d_backward": ([P, C.POINTER(ConvGeom), P, F, P, P, P, P, P, F, P, P, F], I),
    "ttrl_conv2d_backward_deferred": ([P, C.POINTER(ConvGeom), P, F, P, P, P, P, P, P, P, F, I,
                                       C.POINTER(GradSource)], I),
    "ttrl_conv2d_backward_weight_deferred": ([P, C.POINTER(ConvGeom), P, F, P, P, P, P, I, C.POINTER(GradSource)], I),
    "ttrl_grad_sources_materialize": ([P, I, C.POINTER(GradSource)], I),
    "ttrl_dqn_loss": ([P, I, I, P, P, P, P, P, P, P, P, F, P, P, P, P, P, P], I),
    "ttrl_dqn_head": ([P, I, I, I, I, P, P, P, P, P, P, P, P, P, F, P, P, P, P, P, P], I),
    "ttrl_dqn_tail": ([P, C.POINTER(DqnTailDesc)], I),
    "ttrl_sac_sample": ([P, I, I, P, P, P, P, F, P, P, P], I),
    "ttrl_sac_head_sample": ([P, C.POINTER(SacHeadDesc)], I),
    "ttrl_q_act": ([P, I, I, I, P, P, P, P, P], I),
    "ttrl_gru_step": ([P, I, I, P, P, P, P, P, P], I),
    "ttrl_gru_mask": ([P, I, I, P, P, P], I),
    "ttrl_gru_step_backward": ([P, I, I, P, P, P, P, P, P, P, P, P], I),
    "ttrl_gru_step_fused": ([P, I, I, P, P, P, P, P, P, P, P], I),
    "ttrl_gru_step_backward_fused": ([P, I, I, P, P, P, P, P, P, P, P, P, P, P, P], I),
    "ttrl_replay_write": ([P, C.POINTER(ReplayRing), I, P, P, P, P, P, P, P, P, P, P], I),
    "ttrl_replay_lane_sums": ([P, C.POINTER(ReplayRing), P, P, I, I, P, P], I),
    "ttrl_replay_priority_pick": ([P, C.POINTER(ReplayRing), I, P, P, P, P, I, I, P, P, P, P], I),
    "ttrl_replay_is_weights": ([P, I, P, P, I, C.c_long, C.c_double, P], I),
    "ttrl_replay_assemble": ([P, C.POINTER(ReplayRing), I, P, P, I, C.c_double, P, P, P, I, P, P, P, P, P], I),
    "ttrl_replay_draw_batch": ([P, C.POINTER(ReplayRing), C.POINTER(ReplayDraw)], I),
    "ttrl_sac_fused_stage": ([P, I, C.POINTER(SacFusedDesc)], I),
    "ttrl_sac_fused_adam_parts": ([C.POINTER(SacFusedDesc), I, C.POINTER(I)], I),
    "ttrl_replay_update_priorities": ([P, C.POINTER(ReplayRing), I, P, P, P], I),
    "ttrl_replay_update_priorities_f64": ([P, C.POINTER(ReplayRing), I, P, P, P], I),
    "ttrl_gaussian_act": ([P, I, I, I, P, P, P, P, P, F, F, P, P, P, F, I, P, P, P], I),
    "ttrl_sac_sample_backward": ([P, I, I, P, P, P, P, P, P, P, F, F, P, F], I),
    "ttrl_sac_critic_loss": ([P, I, P, P, P, P, P, P, P, P, P, P, P, P, P], I),
    "ttrl_sac_actor_loss": ([P, I, P, P, P, F, I, P, P, P, P, P], I),
    "ttrl_adam_step": ([P, P, P, P, P, L, P, F, F, F, F, F, P, I], I),
    "ttrl_adam_step_clipped": ([P, P, P, P, P, L, P, F, F, F, F, F, P, I, F, P, P], I),
    "ttrl_adam_step_clipped_end": ([P, P, P, P, P, L, P, F, F, F, F, F, P, I, F, P, P, P, P, I, P, I], I),
    "ttrl_adam_step_static": ([P, P, P, P, P, L, P, F, F, F, F, F, P, I], I),
    "ttrl_adam_step_deferred": ([P, P, P, P, P, L, P, F, F, F, F, F, I], I),
    "ttrl_adam_multi": ([P, I, C.POINTER(AdamRange), P, P, L, F], I),
    "ttrl_adam_finish_slots": ([P, I, C.POINTER(AdamFinish)], I),
    "ttrl_adam_step_sources": ([P, C.POINTER(AdamSourcesDesc)], I),
    "ttrl_ordered_sums": ([P, I, C.POINTER(OrderedSum)], I),
    "ttrl_sum_squares": ([P, P, L, P, I], I),
    "ttrl_polyak": ([P, P, P, L, F], I),
    "ttrl_gae": ([P, I, I, P, P, P, P, P, C.c_double, C.c_double, P, P], I),
    "ttrl_normalize_advantages": ([P, P, P, L, F, P, P], I),
    "ttrl_ppo_loss_packed": ([P, I, I, P, P, P, P, P, P, P, F, F, F, F, P, P, P], I),
    "ttrl_gather_rows": ([P, I, I, P, P, P, C.c_long, P, C.c_long, P, I], I),
    "ttrl_step_end": ([P, P, P, I, P, I], I),
    "ttrl_ppo_loss": ([P, I, I, P, P, P, P, P, P, P, P, F, F, F, F, P, P, P, P], I),
    "ttrl_clip_grad_norm": ([P, P, L, F, P, P], I),
    "ttrl_unary": ([P, I, P, P, L, F], I),
    "ttrl_binary": ([P, I, P, P, P, I, C.POINTER(L), C.POINTER(L), C.POINTER(L)], I),
    "ttrl_copy_strided": ([P, P, P, I, C.POINTER(L), C.POINTER(L), C.POINTER(L)], I),
    "ttrl_reduce": ([P, I, P, P, L, L, L], I),
    "ttrl_one_hot": ([P, P, P, L, I], I),
}

_LIB = None


class TTRLError(RuntimeError):
    """A libttrl_hip call failed; `code` is the TTRL_E* status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def load(path: Path | str | None = None) -> C.CDLL:
    """Open the shared library without touching any device."""
    target = Path(path) if path else LIB_PATH
    if not target.exists():
        raise RuntimeError(
            f"libttrl_hip.so is not built ({target} missing). Run __graft_entry__.build() or "
            f"`python -m ttrl_amd._build` with tt-rl_amd on sys.path; there is no host fallback."
        )
    # Kernel arguments in device memory: every launch's first argument reads
    # are then HBM reads rather than host-memory reads across the bus (about
    # 1 us per update of the learners' 11 to 25 launches).  The HIP runtime
    # reads this when it initialises, which happens at the library's first
    # call; a value the caller set is kept.
    os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")
    dll = C.CDLL(str(target), mode=os.RTLD_LOCAL if hasattr(os, "RTLD_LOCAL") else 0)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(dll, name)
        fn.argtypes = args
        fn.restype = res
    return dll


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def check(rc: int, what: str = "") -> None:
    """Raise the reference's exception type for a failed call."""
    if rc == TTRL_OK:
        return
    msg = lib().ttrl_last_error().decode(errors="replace")
    text = f"{what}: {msg}" if what else msg
    if rc == TTRL_EINVAL:
        raise ValueError(text)
    raise TTRLError(rc, text)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptrs(values) -> C.Array:
    """A C array of void pointers (None for NULL)."""
    values = [None if v is None else int(v) for v in values]
    return (P * len(values))(*values)


def longs(values) -> C.Array:
    values = [int(v) for v in values]
    return (L * len(values))(*values)
