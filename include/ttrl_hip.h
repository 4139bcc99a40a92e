/*
 * libttrl_hip: the C ABI of the MI355X (gfx950) learner-update path.
 *
 * A drop-in for the ttnn device calls that tt-rl's engine makes from Python.
 * Every function returns TTRL_OK (0) or a negative TTRL_E* code and leaves a
 * thread-local message for ttrl_last_error().  Pointers are device pointers
 * unless the name says host; all float data is IEEE fp32, row-major.  Every
 * kernel entry point only enqueues work on the context's stream, so a
 * sequence of them can be recorded into one graph between
 * ttrl_capture_begin and ttrl_capture_end.  Nothing here allocates device
 * memory except ttrl_alloc (and ttrl_init, which reserves the stream-ordered
 * split-K workspace).
 *
 * Each declaration names the reference interface it replaces (paths are
 * relative to the tt-rl repository).
 */
#ifndef TTRL_HIP_H
#define TTRL_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTRL_ABI_VERSION 1

#define TTRL_OK 0
#define TTRL_EINVAL (-1) /* bad argument or shape: the reference raises ValueError */
#define TTRL_EHIP (-2)   /* HIP runtime error */
#define TTRL_ENOMEM (-3)
#define TTRL_ESTATE (-4) /* call not allowed in the current state (e.g. host read during capture) */

typedef struct ttrl_ctx ttrl_ctx;
typedef struct ttrl_graph ttrl_graph;

/* ------------------------------------------------------------ context --- */

/* Message of the last failed call on this thread. */
const char* ttrl_last_error(void);
int ttrl_version(void);
int ttrl_device_count(int* out);

/* What acquire() yields beside the device: the facts about it that the
 * layers above may ask (replaces probe_profile, ttrl/engine/device/profile.py:79-97,
 * whose grid and tile facts describe a Tenstorrent chip).  Reads the
 * runtime's properties of visible device `device`; opens no context. */
typedef struct ttrl_device_info {
  char name[256];          /* marketing name, e.g. "AMD Instinct MI355X" */
  char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int compute_units;
  int wavefront_size;
  long lds_per_cu;         /* bytes of LDS per compute unit */
  long lds_per_workgroup;  /* bytes one workgroup may allocate */
  long l2_bytes;
  long hbm_bytes;
  int clock_khz;           /* peak engine clock */
  int memory_clock_khz;
  int memory_bus_bits;
  int pci_bus_id;
  int pci_device_id;
  int pci_domain_id;
} ttrl_device_info;
int ttrl_device_query(int device, ttrl_device_info* out);
/* Open a device and its stream; replaces acquire() (ttrl/engine/device/acquire.py:56). */
int ttrl_init(int device, ttrl_ctx** out);
/* Close; replaces the device close in ttrl/engine/device/acquire.py:56-140. */
int ttrl_shutdown(ttrl_ctx* ctx);
/* Wait for the stream; replaces ttnn.synchronize_device (ttrl/engine/step/core.py:135-141). */
int ttrl_sync(ttrl_ctx* ctx);
/* The context's hipStream_t, as an opaque handle. */
void* ttrl_stream(ttrl_ctx* ctx);

/* ------------------------------------------------------------- memory --- */
/* Fixed-address device buffers (ttrl/engine/tensor/arena.py:21-87): blocks
 * come from slab pools and are reused only by later allocations of the same
 * pool, in stream order, so buffers recorded into a graph keep their
 * addresses for the graph's lifetime.  Pool 0 is the default pool. */
int ttrl_pool_create(ttrl_ctx* ctx, int* pool);
int ttrl_pool_release(ttrl_ctx* ctx, int pool);
int ttrl_pool_use(ttrl_ctx* ctx, int pool, int* previous);
int ttrl_pool_stats(ttrl_ctx* ctx, int pool, size_t* reserved, size_t* live);
int ttrl_alloc(ttrl_ctx* ctx, size_t bytes, void** out);
int ttrl_free(ttrl_ctx* ctx, void* ptr);

/* Host<->device copies; replace to_device/to_host/restore_in_place
 * (ttrl/engine/tensor/transfer.py:11-51) and InputBinder.load
 * (ttrl/engine/step/inputs.py:28-85).  Both refuse to run during capture. */
int ttrl_h2d(ttrl_ctx* ctx, void* dst, const void* host_src, size_t bytes);
/* The same copy queued on the stream without waiting (InputBinder.load,
 * ttrl/engine/step/inputs.py:28-85, as one input's part of a batch upload):
 * host_src must lie inside one ttrl_host_alloc block and stay unchanged
 * until the stream is next waited for (ttrl_sync, ttrl_h2d, ttrl_graph_step). */
int ttrl_h2d_enqueue(ttrl_ctx* ctx, void* dst, const void* host_src, size_t bytes);
int ttrl_d2h(ttrl_ctx* ctx, void* host_dst, const void* src, size_t bytes);
/* Device copy on the stream; replaces copy_in_place (ttrl/engine/tensor/arena.py:32). */
int ttrl_d2d(ttrl_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Fill with a kernel (never a memset node); replaces ttnn.full_like / zeros. */
int ttrl_fill_f32(ttrl_ctx* ctx, float* dst, float value, long n);
int ttrl_fill_i32(ttrl_ctx* ctx, int* dst, int value, long n);

/* ------------------------------------------------------------- graphs --- */
/* Replace ttnn trace capture/replay (ttrl/engine/trace.py:56-126). */
int ttrl_capture_begin(ttrl_ctx* ctx);
int ttrl_capture_end(ttrl_ctx* ctx, ttrl_graph** out);
/* Leave capture after a failure (ttrl/engine/trace.py:39-53). */
int ttrl_capture_abort(ttrl_ctx* ctx);
int ttrl_graph_launch(ttrl_ctx* ctx, ttrl_graph* g);
/* No counterpart in the reference (its traces replay on the device's command
 * queue): with on nonzero, every later replay of g (ttrl_graph_launch,
 * ttrl_graph_launch_n, ttrl_graph_step) launches the graph's kernels one by
 * one in dependency order on the context's stream, with the arguments they
 * were captured with, instead of one graph launch.  Same kernels, same
 * results; for a small graph replayed once per host step (an acting step),
 * where a graph launch's fixed cost exceeds the launches.  TTRL_EINVAL for a
 * graph with nodes other than kernels. */
int ttrl_graph_set_direct(ttrl_graph* g, int on);
int ttrl_graph_launch_n(ttrl_ctx* ctx, ttrl_graph* g, int n);
/* One acting step as one host call: copy in_bytes of host memory into the
 * bound device block in_dev, replay g (skipped when NULL), copy out_bytes of
 * out_dev back to host memory, and wait.  Both copies go through one pinned
 * staging buffer the context owns and grows on demand.  Replaces the acting
 * round trip of ttrl/nets/acting.py:164-169 (ObsViews.load, the eager
 * forward) and the action read of ttrl/algos/dqn/agent.py:107-109 and
 * ttrl/algos/sac/agent.py:118-121. */
int ttrl_graph_step(ttrl_ctx* ctx, ttrl_graph* g, void* in_dev, const void* in_host, size_t in_bytes,
                    void* out_host, const void* out_dev, size_t out_bytes);
/* Pinned host memory owned by the context (freed by ttrl_host_free or at
 * shutdown).  When both host buffers of ttrl_graph_step lie in such blocks
 * the step copies from and to them directly: one H2D, the replay, one D2H
 * and one wait.  Replaces the wide-row staging buffer of InputBinder
 * (ttrl/engine/step/inputs.py:28-102) and the packed metric read of
 * read_metrics (ttrl/engine/step/metrics.py:22-30). */
int ttrl_host_alloc(ttrl_ctx* ctx, size_t bytes, void** out);
int ttrl_host_free(ttrl_ctx* ctx, void* ptr);
/* Pinned host memory that kernels read and write in place through *device
 * (mapped, coherent: no copy, no staging), freed by ttrl_host_free(host) or
 * at shutdown.  For the few words a host decision and a kernel exchange: a
 * replay draw's run extents, lane sums and generator draws
 * (ttrl/buffers/sampling.py:135-240 keeps them in host arrays). */
int ttrl_host_alloc_mapped(ttrl_ctx* ctx, size_t bytes, void** host, void** device);
int ttrl_graph_nodes(ttrl_graph* g, size_t* out);
int ttrl_graph_destroy(ttrl_graph* g);

/* The context's table of GEMM plans (tile shape and K split per call
 * signature), as text: one "cfg bm bn tbk splits kchunk<TAB>signature" line
 * per entry, sorted.  A plan is otherwise chosen by timing candidates at the
 * first call of a signature, which can differ between processes and with it
 * the split-K summation order; importing a saved table makes a second
 * process run the same plans and produce the same bits.  With buf NULL,
 * *len receives the size.  Imported plans are checked against each call's
 * extents before use (an invalid one is re-planned).  No reference
 * counterpart: ttnn's program cache (ttrl/engine/step/core.py:44-141) holds
 * compiled kernels, not tuning choices. */
int ttrl_plans_export(ttrl_ctx* ctx, char* buf, size_t cap, size_t* len);
int ttrl_plans_import(ttrl_ctx* ctx, const char* text, int* count);

/* Stream timer (events on the context's stream). */
int ttrl_timer_start(ttrl_ctx* ctx);
int ttrl_timer_stop(ttrl_ctx* ctx, float* ms);
/* No counterpart in the reference (measurement only): `workgroups` x 256
 * threads issuing `iters` rounds of eight independent
 * v_mfma_f32_16x16x4f32 each, no memory traffic in the loop; each thread's
 * sum goes to out[workgroups * 256]; *flops receives the launch's FP32
 * matrix FLOPs.  Timed with the stream timer, it gives the achievable FP32
 * MFMA rate beside the published peak. */
int ttrl_mfma_rate(ttrl_ctx* ctx, int workgroups, int iters, float* out, double* flops);

/* ------------------------------------------------------ dense layers --- */

/* C[M][N] = alpha * op(A) op(B) + beta * C, op(X) = X or X^T.  Replaces the
 * HiFi4 ttnn.matmul and its transposed backward products
 * (ttrl/engine/ops/matmul.py:42-86). */
int ttrl_matmul(ttrl_ctx* ctx, int M, int N, int K, const float* A, long lda, int trans_a, const float* B,
                long ldb, int trans_b, float* C, long ldc, float alpha, float beta);

/* A linear layer y = x @ W + b with W stored (in, out) (ttrl/engine/layers.py:22-61),
 * optionally fused with ReLU (ttrl/engine/ops/unary.py:25-37) or a column clamp
 * (ttrl/nets/heads.py:65-93).  Extensions used by the SAC nets:
 *   groups     independent problems with element strides g* (twin critics),
 *   x2/k1      input columns k >= k1 come from x2: concat(s, a) folded into the
 *              load (ttrl/engine/ops/shape.py:10-48, ttrl/nets/fusion.py:36-71),
 *   W2/b2/n1   output columns n >= n1 use a second weight (N - n1 wide): the
 *              mean and log_std heads in one launch (ttrl/nets/heads.py:65-93).
 * Backward: dZ = dy * [ymask > 0] when ymask is given (relu_bw), then
 * dW = x^T dZ with db = column sums of dZ folded in as an implicit ones row
 * (ttrl/engine/ops/broadcast.py:11-30), and dx = dZ W^T restricted to input
 * columns [dx_col0, dx_col0 + dx_cols) when dx_cols > 0.  dxmask, laid out
 * like dx, multiplies dx by [dxmask > 0] as it is written: the relu_bw of
 * the layer below applied in this epilogue, so that layer's backward needs
 * no ymask.  beta_* = 1 accumulates into existing gradients
 * (ttrl/engine/autograd.py:106-114). */
typedef struct ttrl_linear_desc {
  int M, K, N;
  int groups;
  const float* x;
  long ldx, gx;
  const float* x2;
  long ldx2, gx2;
  int k1;
  const float* W;
  long gW;
  const float* b;
  long gb;
  const float* W2;
  const float* b2;
  int n1;
  float* y;
  long gy;
  int relu;
  int clamp_col;
  float lo, hi;
  const float* ymask;
  const float* dy;
  float* dW;
  float* db;
  float* dW2;
  float* db2;
  float* dx;
  long lddx, gdx;
  int dx_col0, dx_cols;
  float beta_w, beta_x;
  const float* dxmask;
  /* Forward only: per-group pointers (g < groups) in place of base + g *
   * stride where non-NULL, for groups whose buffers sit at no common stride
   * (the online and the target critics of one SAC update live in two
   * parameter arenas). */
  const float* xg[4];
  const float* x2g[4];
  const float* Wg[4];
  const float* bg[4];
} ttrl_linear_desc;

int ttrl_linear_forward(ttrl_ctx* ctx, const ttrl_linear_desc* desc);
/* `groups` (<= 4) independent y[g] = x[g] @ W[g] + b[g] (+ReLU), each [M][K] @ [K][N],
 * from pointer tables (b may be NULL): several networks' same-shaped layers in
 * one launch, e.g. the online and target Q networks of one DQN update
 * (ttrl/algos/dqn/losses.py:96-103).  No reference counterpart as one call. */
int ttrl_linear_forward_multi(ttrl_ctx* ctx, int M, int K, int N, int groups, const float* const* x,
                              const float* const* W, const float* const* b, float* const* y, int relu);
int ttrl_linear_backward(ttrl_ctx* ctx, const ttrl_linear_desc* desc);

/* ------------------------------------------------------- convolution --- */

#define TTRL_LAYOUT_NHWC_F32 0 /* [B][H][W][C] fp32 activations */
#define TTRL_LAYOUT_NCHW_U8 1  /* [B][C][H][W] uint8 frames */

/* Geometry of ConvGeometry (ttrl/engine/conv/geometry.py:94-199), square kernel. */
typedef struct ttrl_conv_geom {
  int batch, in_c, in_h, in_w, out_c, kernel, stride, padding;
  int in_layout;
} ttrl_conv_geom;

/* (size + 2p - k)/s + 1, refusing ragged geometry (ttrl/engine/conv/geometry.py:107-119). */
int ttrl_conv_out_size(int size, int kernel, int stride, int padding, int* out);

/* y[B][OH][OW][O] = x_scale * conv(x, W) + b (+ReLU).  W is the master
 * Wt[k][O], k = (kh, kw, c) for NHWC inputs and (c, kh, kw) for NCHW uint8
 * inputs.  Replaces ttnn.conv2d + bias add with the input-scale fold
 * (ttrl/engine/conv/forward.py:160-205, ttrl/engine/conv/module.py:257-263). */
int ttrl_conv2d_forward(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, const float* wt,
                        const float* bias, float* y, float x_scale, int relu);
/* The same convolution geometry over `groups` (<= 4) input/weight/bias/output
 * pointer tables in one launch (the online and target towers of a DQN update). */
int ttrl_conv2d_forward_multi(ttrl_ctx* ctx, const ttrl_conv_geom* geom, int groups, const void* const* x,
                              const float* const* wt, const float* const* bias, float* const* y, float x_scale,
                              int relu);
/* dWt = x_scale * sum over pixels of patch^T dZ, db = column sums of dZ,
 * dZ = dy * [ymask > 0].  Replaces weight_grad + dw_to_prepared
 * (ttrl/engine/conv/backward.py:45-78, ttrl/engine/conv/transform.py:232-254)
 * and the conv bias-gradient sum (ttrl/engine/ops/broadcast.py:11-30). */
int ttrl_conv2d_backward_weight(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                const float* dy, const float* ymask, float* dwt, float* db, float beta);
/* dx = x_scale * conv_transpose(dZ, W) for fp32 NHWC inputs, times
 * [xmask > 0] when xmask (laid out like dx: the ReLU output that fed this
 * layer) is given, so the layer below needs no ymask.  Replaces
 * input_grad / transpose_weight / conv_transpose2d
 * (ttrl/engine/conv/backward.py:33-42, ttrl/engine/conv/transform.py:71-129). */
int ttrl_conv2d_backward_input(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const float* dy, const float* ymask,
                               const float* wt, float* dx, const float* xmask, float x_scale, float beta);
/* Both gradients of one conv2d node's backward (ttrl/engine/conv/backward.py:33-78):
 * ttrl_conv2d_backward_weight(x, x_scale, dy, ymask, dwt, db, beta_w) and
 * ttrl_conv2d_backward_input(dy, ymask, wt, dx, xmask, x_scale, beta_x), the
 * two GEMMs sharing one launch or as two launches with their own tile shapes,
 * whichever the context measured faster for the geometry on its first call
 * outside capture (kept with the context's GEMM plans).  fp32 NHWC inputs
 * only (a uint8 frame input has no gradient); db may be NULL. */
int ttrl_conv2d_backward(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale, const float* dy,
                         const float* ymask, const float* wt, float* dwt, float* db, float beta_w, float* dx,
                         const float* xmask, float beta_x);

/* Gradient sources: a parameter's gradient that an earlier launch left
 * unreduced, formed by the optimizer step that consumes it
 * (ttrl_adam_step_sources) or by ttrl_grad_sources_materialize.  The
 * gradient is a [rows][cols] row-major block at dw and, when db is not
 * NULL, cols bias entries at db.
 *   TTRL_GRAD_SPLITS: split-K partial sums part[splits][rows (+1)][cols]
 *     (the extra row is the bias's): dw[r][c] = scale * sum_s part[s][r][c],
 *     db[c] = bias_scale * sum_s part[s][rows][c], summed in split order from
 *     zero, as the weight-gradient launch itself would.
 *   TTRL_GRAD_OUTER: dw[r][c] = sum_b u[b][r] * v[b][c] and
 *     db[c] = sum_b v[b][c], b = 0 .. batch-1 in order from zero (a linear
 *     layer's gradients from its input rows u[batch][rows] and output
 *     gradient rows v[batch][cols]).
 *   TTRL_GRAD_NONE: nothing pending (the launch wrote dw and db itself). */
#define TTRL_GRAD_NONE 0
#define TTRL_GRAD_SPLITS 1
#define TTRL_GRAD_OUTER 2
typedef struct ttrl_grad_source {
  int kind;
  int rows, cols;
  float* dw;
  float* db;
  const float* part; /* TTRL_GRAD_SPLITS */
  int splits;
  float scale, bias_scale;
  const float* u; /* TTRL_GRAD_OUTER */
  const float* v;
  int batch;
} ttrl_grad_source;
/* ttrl_conv2d_backward with the weight gradient's split-K sum left to the
 * optimizer step (ttrl/engine/conv/backward.py:33-78): when the planned
 * launch splits the weight-gradient GEMM, its partials stay in gradient
 * bank `bank` (0 <= bank < 4, 4 MiB each, owned by the context) and *out
 * describes them (TTRL_GRAD_SPLITS); otherwise dwt and db are written and
 * out->kind is TTRL_GRAD_NONE.  The weight gradient is not accumulated
 * (beta_w = 0).  A bank's partials live until the next deferred call that
 * names the same bank. */
int ttrl_conv2d_backward_deferred(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                  const float* dy, const float* ymask, const float* wt, float* dwt, float* db,
                                  float* dx, const float* xmask, float beta_x, int bank, ttrl_grad_source* out);
/* ttrl_conv2d_backward_weight with the same deferral (beta = 0). */
int ttrl_conv2d_backward_weight_deferred(ttrl_ctx* ctx, const ttrl_conv_geom* geom, const void* x, float x_scale,
                                         const float* dy, const float* ymask, float* dwt, float* db, int bank,
                                         ttrl_grad_source* out);
/* Writes the gradients `n` sources describe (<= 8), with the bits the
 * optimizer step that consumes them would form. */
int ttrl_grad_sources_materialize(ttrl_ctx* ctx, int n, const ttrl_grad_source* sources);

/* ---------------------------------------------------------- loss heads --- */

/* The DQN update head of update_loss (ttrl/algos/dqn/losses.py:77-140):
 * pred = gather_onehot(q, actions_onehot); a* = argmax q_next_select (first
 * index wins); y = r + discounts*(1 - done)*q_next_value[a*]; loss =
 * mean(w * huber(pred - y, delta)); mean_q = mean(pred); td_abs = |pred - y|;
 * dq = dloss/dq.  is_weights, mean_q, td_abs, next_actions, td_target may be
 * NULL.  Pass q_next_select = q_next_value for vanilla DQN. */
int ttrl_dqn_loss(ttrl_ctx* ctx, int B, int A, const float* q, const float* q_next_select,
                  const float* q_next_value, const float* actions_onehot, const float* rewards, const float* dones,
                  const float* discounts, const float* is_weights, float delta, float* loss, float* mean_q,
                  float* td_abs, float* dq, float* next_actions, float* td_target);
/* The Q head's last linear layer (ttrl/nets/heads.py QHead: q = h @ W + b,
 * ttrl/engine/layers.py:22-61) for `groups` feature sets in one launch,
 * followed by ttrl_dqn_loss on the results: group 0 = online(s) gives q,
 * group 1 selects a*, group groups-1 values it (3 groups: double DQN with
 * online(s'), target(s'); 2 groups: vanilla, the target both selects and
 * values).  h[g] is [B][K], W[g] is [K][A] (in, out), bias[g] may be NULL or
 * bias itself NULL; q_out[g] receives [B][A].  A <= 32. */
int ttrl_dqn_head(ttrl_ctx* ctx, int B, int K, int A, int groups, const float* const* h, const float* const* W,
                  const float* const* bias, float* const* q_out, const float* actions_onehot, const float* rewards,
                  const float* dones, const float* discounts, const float* is_weights, float delta, float* loss,
                  float* mean_q, float* td_abs, float* dq, float* next_actions, float* td_target);

/* A DQN Q network's last two layers over 2 or 3 feature sets, the DQN loss
 * and the head's backward (ttrl/algos/dqn/losses.py:77-140 over the Nature
 * CNN's Linear(K, F) -> ReLU -> QHead Linear(F, A), ttrl/nets/encoders.py,
 * ttrl/nets/heads.py): h[g] = relu(x[g] W1[g] + b1[g]) ([B][F]); q[g] =
 * h[g] W2[g] + b2[g] ([B][A]); the loss and metrics of ttrl_dqn_loss with q[0]
 * = online(s), q[1] selecting a* and q[groups-1] valuing it; dq = dloss/dq[0];
 * dh = dq W2[0]^T * [h[0] > 0], the gradient entering the first layer's
 * backward; dW2 = h[0]^T dq and db2 = column sums of dq, the second layer's
 * gradients (added to their values when beta_w = 1).  b1, b2, is_weights,
 * mean_q, td_abs, next_actions, td_target and db2 may be NULL.  dW2 NULL
 * leaves the second layer's gradients to the caller (an outer-product
 * gradient source over h[0] and dq).  loss_terms not NULL defers the batch
 * sums as well: sample b's weighted Huber term and prediction go to
 * loss_terms[2b] and loss_terms[2b + 1], loss and mean_q are not written
 * (the caller sums the terms in sample order and scales by 1/B), and dW2
 * must be NULL; the launch then needs no cross-workgroup step.
 * B <= 1024, F <= 2048, A <= 32. */
typedef struct ttrl_dqn_tail_desc {
  int B, K, F, A, groups;
  const float* x[3];
  const float* W1[3];
  const float* b1[3];
  float* h[3];
  const float* W2[3];
  const float* b2[3];
  float* q[3];
  const float* actions_onehot;
  const float* rewards;
  const float* dones;
  const float* discounts;
  const float* is_weights;
  float delta;
  float* loss;
  float* mean_q;
  float* td_abs;
  float* dq;
  float* next_actions;
  float* td_target;
  float* dh;
  float* dW2;
  float* db2;
  float beta_w;
  float* loss_terms;
} ttrl_dqn_tail_desc;
int ttrl_dqn_tail(ttrl_ctx* ctx, const ttrl_dqn_tail_desc* desc);

/* SquashedGaussian.sample (ttrl/algos/sac/policy.py:30-40) over head rows
 * [mean | log_std] ([B][2d], log_std already clamped): action =
 * centre + half_width * tanh(mean + exp(log_std)*noise), logp with the stable
 * softplus correction (ttrl/algos/gaussian.py:55-117) minus log_det. */
int ttrl_sac_sample(ttrl_ctx* ctx, int B, int d, const float* head, const float* noise, const float* centre,
                    const float* half_width, float log_det, float* action, float* logp, float* u_out);
/* GaussianHead.forward (ttrl/nets/heads.py:65-93: mean and log_std Linear
 * layers, log_std clamped to [lo, hi]) and the squashed sample above in one
 * launch (the acting kernel of ttrl_gaussian_act), over rows of x
 * ([rows][K]); W1, W2 are [K][d] with d <= 16, b1/b2 may be NULL.  Writes
 * head [rows][2d] = [mean | log_std] and u, which the sample's backward
 * takes, with action and logp. */
typedef struct ttrl_sac_head_desc {
  int rows, K, d;
  const float* x;
  const float* W1;
  const float* b1;
  const float* W2;
  const float* b2;
  float lo, hi;
  const float* noise;
  const float* centre;
  const float* half_width;
  float log_det;
  float* head;
  float* action;
  float* logp;
  float* u;
} ttrl_sac_head_desc;
int ttrl_sac_head_sample(ttrl_ctx* ctx, const ttrl_sac_head_desc* desc);
/* Its backward to d_head ([B][2d]), given dL/daction (g_action0 + g_action1,
 * either may be NULL) and dL/dlogp per row; the log_std clamp passes
 * gradient strictly inside (log_std_min, log_std_max) (ttrl/engine/ops/select.py:26-29). */
int ttrl_sac_sample_backward(ttrl_ctx* ctx, int B, int d, const float* head, const float* noise, const float* u,
                             const float* half_width, const float* g_action0, const float* g_action1,
                             const float* g_logp, float log_std_min, float log_std_max, float* d_head, float beta);
/* critic_loss (ttrl/algos/sac/losses.py:46-76) for two critics: q and
 * q_next_target are [2][B]; writes loss, q_target[B], dq [2][B],
 * td_abs (priority_errors, losses.py:30-43; may be NULL) and alpha = exp(log_alpha). */
int ttrl_sac_critic_loss(ttrl_ctx* ctx, int B, const float* q, const float* q_next_target, const float* logp_next,
                         const float* log_alpha, const float* rewards, const float* dones, const float* discounts,
                         const float* is_weights, float* loss, float* q_target, float* dq, float* td_abs,
                         float* alpha_out);
/* actor_loss and alpha_loss (ttrl/algos/sac/losses.py:79-94): q is [2][B] at
 * the reparameterised action; writes both losses, dq [2][B], dL/dlogp per
 * row and dL_alpha/dlog_alpha. */
int ttrl_sac_actor_loss(ttrl_ctx* ctx, int B, const float* q, const float* logp, const float* log_alpha,
                        float target_entropy, int learn_alpha, float* actor_loss, float* alpha_loss, float* dq,
                        float* g_logp, float* d_log_alpha);

/* One deferred Adam step over a flat arena (the deferred steps under
 * "optimizer" below run it; a fused SAC update applies it in its stages). */
typedef struct ttrl_adam_range {
  float* p;
  const float* g;
  float* m_s;
  float* v_s;
  long n;
  const int* step;
  float lr, beta1, beta2, eps, weight_decay;
  int slot;
} ttrl_adam_range;
/* The SAC update (ttrl/algos/sac/agent.py:218-238 over ttrl/algos/sac/losses.py:25-94,
 * ttrl/algos/gaussian.py:55-117, ttrl/algos/sac/policy.py:30-40 and the twin
 * critics and policy of ttrl/nets/build.py) as eight stages, each one
 * launch over blocks of 16 rows with each workgroup owning 64 of the H
 * columns of the stage's H x H product (H a multiple of 64 up to 256, the
 * first layer's inputs at most 64, at most 8 action dimensions, the batch B
 * a multiple of 16 up to 1024):
 *   0 policy over [obs; next_obs] to its Gaussian head's quarter partials;
 *   1 the target critics on (next_obs, a' sampled) and the critics on (obs, actions);
 *   2 soft target, twin-critic loss gradient, backward of both critics to layer 1;
 *   3 the critics' weight and bias gradients (outer products over the batch)
 *     into g_critic;
 *   4 the (stepped) critics on (obs, a sampled);
 *   5 actor loss gradient into the smaller critic of each row, backward to d/da;
 *   6 the sample's backward, dh2, dh1; the actor, critic and temperature
 *     losses and d alpha_loss / d log_alpha into g_log_alpha (learn_alpha);
 *   7 the policy's weight and bias gradients into gP1 .. gbl.
 * The caller steps the critics between stages 3 and 4 and the policy and
 * temperature after stage 7.  critic[0..1] are the targets, critic[2..3] the
 * trained critics; every weight is [in][out].  The activation buffers hold
 * what later stages and the weight gradients read; logp receives the
 * sample's log-density of all 2B rows (obs rows first). */
typedef struct ttrl_sac_critic_params {
  const float *W1, *b1, *W2, *b2, *w3, *b3;
} ttrl_sac_critic_params;
typedef struct ttrl_sac_fused_desc {
  int B, O, A, H;
  const float *P1, *p1, *P2, *p2, *Wm, *bm, *Wl, *bl;
  float log_std_min, log_std_max;
  const float *centre, *half_width;
  float log_det;
  ttrl_sac_critic_params critic[4];
  const float *obs_pair;    /* [2B][O] obs rows, then next_obs rows */
  const float *actions;     /* [B][A] */
  const float *obs_actions; /* [B][O + A] */
  const float *noise_pair;  /* [2B][A] */
  const float *rewards, *dones, *discounts, *is_weights; /* [B]; is_weights may be NULL */
  const float *log_alpha;
  float target_entropy;
  int learn_alpha;
  float *h1, *h2;           /* [2B][H] */
  float *headp;             /* [H/64][2B][2A] */
  float *head, *act, *u;    /* [2B][2A], [2B][A], [2B][A] */
  float *q1, *q2;           /* [4][B][H] */
  float *qp;                /* [4][H/64][B] */
  float *q1pi, *q2pi;       /* [2][B][H] */
  float *qppi;              /* [2][H/64][B] */
  float *dQ;                /* [2][B] */
  float *dq2, *dq1;         /* [2][B][H] */
  float *dap;               /* [2][H/64][B][A] */
  float *dhead;             /* [B][2A] */
  float *dh2, *dh1;         /* [B][H] */
  float *terms;             /* [4][B] */
  float *critic_loss, *alpha, *actor_loss, *alpha_loss, *q_target, *td_abs, *logp;
  float *gP1, *gp1, *gP2, *gp2, *gWm, *gbm, *gWl, *gbl;
  float *g_critic[2][6];    /* the trained critics' W1, b1, W2, b2, w3, b3 gradients */
  float *g_log_alpha;
  /* fuse_adam nonzero: the stages step the optimizers as they form the
   * gradients, each element with ttrl_adam_step's arithmetic.  Stage 3 steps
   * the critics' arena (critic_adam; g_critic lie inside its g) and then
   * blends each stepped critic parameter into polyak_dst, the target
   * critics' arena laid out like the critics' (dst = (1 - tau) dst + tau p,
   * ttrl/algos/sac/targets.py:45-52); stage 7 steps the policy's arena
   * (actor_adam; gP1 .. gbl inside its g) and, with learn_alpha, the
   * temperature (alpha_adam; g_log_alpha inside its g).  Each range's
   * partial sums of g^2 wait in its slot for ttrl_adam_finish_slots, with
   * the counts ttrl_sac_fused_adam_parts gives.  Arena elements no stage
   * forms a gradient for (the zero padding between tensors) are not
   * stepped: with a zero gradient and zero moments a step leaves them as
   * they are.  With fuse_adam zero the caller steps the optimizers after
   * stages 3 and 7. */
  int fuse_adam;
  ttrl_adam_range critic_adam, actor_adam, alpha_adam;
  float *polyak_dst;
  float tau;
  float *adam_scalars;      /* [6] the three steps' fused scalars, formed by stage 0 for stages 3 and 7 */
} ttrl_sac_fused_desc;
int ttrl_sac_fused_stage(ttrl_ctx* ctx, int stage, const ttrl_sac_fused_desc* desc);
/* The number of partial sums of g^2 a fused stage leaves in its Adam
 * range's slot: stage 3 (critic_adam) or 7 (actor_adam); the temperature's
 * range leaves one.  No counterpart in the reference: the count a caller
 * passes to ttrl_adam_finish_slots for these ranges. */
int ttrl_sac_fused_adam_parts(const ttrl_sac_fused_desc* desc, int stage, int* parts);

/* ----------------------------------------------------------- optimizer --- */

/* One Adam update over a flat range (ttrl/engine/optim/adam.py:93-134 with
 * ttrl/engine/optim/scalars.py:13-27): m_s and v_s hold S = m/(1-b1) and
 * V = v/(1-b2); *step (device int) is the update count before the call and
 * is incremented by it; grad_sq (may be NULL) receives sum(g^2)
 * (ttrl/algos/grads.py:46-60), added to its value when accumulate_grad_sq. */
int ttrl_adam_step(ttrl_ctx* ctx, float* p, const float* g, float* m_s, float* v_s, long n, int* step, float lr,
                   float beta1, float beta2, float eps, float weight_decay, float* grad_sq, int accumulate_grad_sq);
/* ttrl_clip_grad_norm then ttrl_adam_step (ttrl/algos/grads.py:13-43, then
 * ttrl/engine/optim/adam.py:93-134) with one read of g: norm = sqrt(sum
 * g^2); when norm > max_norm the step reads g * max_norm / (norm + 1e-6)
 * and writes that clipped g back, as the clip leaves it, else it reads g.
 * Same parameters, moments and gradient as the two calls.  *sq_out and
 * *norm_out (nullable) receive sum g^2 and the norm before clipping;
 * grad_sq as in ttrl_adam_step, over the clipped gradient. */
int ttrl_adam_step_clipped(ttrl_ctx* ctx, float* p, float* g, float* m_s, float* v_s, long n, int* step,
                           float lr, float beta1, float beta2, float eps, float weight_decay, float* grad_sq,
                           int accumulate_grad_sq, float max_norm, float* sq_out, float* norm_out);
/* ttrl_adam_step_clipped followed by ttrl_step_end(ctx, counter, metrics,
 * n_metrics, ring, slots), the step end done by the step's finishing launch
 * (one launch fewer; the same results as the two calls): the end of a
 * replayed PPO minibatch step (ttrl/algos/ppo/learn.py:94-112).  metrics may
 * hold the step's own norm_out. */
int ttrl_adam_step_clipped_end(ttrl_ctx* ctx, float* p, float* g, float* m_s, float* v_s, long n, int* step,
                               float lr, float beta1, float beta2, float eps, float weight_decay, float* grad_sq,
                               int accumulate_grad_sq, float max_norm, float* sq_out, float* norm_out, int* counter,
                               const float* metrics, int n_metrics, float* ring, int slots);
/* ttrl_adam_step with the same kernels and results, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops): no context
 * and no allocation of any kind.  It enqueues on `stream` (a hipStream_t;
 * NULL is the default stream) and keeps its per-workgroup sums of squared
 * gradients in a static device array of 1024 floats (4 KiB, one per
 * workgroup of the launch, which never exceeds 1024) that each GPU holds
 * until the process ends; every n > 0 fits.  Calls on one GPU share that
 * array: calls that can overlap (different streams, no ordering between
 * them) race and must not be issued.  The first call on a device resolves
 * the array's address for that device.  No counterpart in the reference. */
int ttrl_adam_step_static(void* stream, float* p, const float* g, float* m_s, float* v_s, long n, int* step,
                          float lr, float beta1, float beta2, float eps, float weight_decay, float* grad_sq,
                          int accumulate_grad_sq);
/* Deferred Adam steps, for an update that steps several optimizers (the
 * SAC critic, then actor and temperature, then the Polyak blend,
 * ttrl/algos/sac/agent.py:229-236) in fewer launches.
 * ttrl_adam_step_deferred is ttrl_adam_step without its finish: *step is
 * read, not stored, and the per-workgroup partial sums of g^2 go to partial
 * slot `slot` (0 <= slot < 8) of the context, which keeps them until
 * ttrl_adam_finish_slots.  ttrl_adam_multi runs up to 4 deferred ranges and
 * a Polyak blend dst = (1 - tau) dst + tau src (ttrl/algos/sac/targets.py:45-52;
 * polyak_n may be 0) in one launch.  ttrl_adam_finish_slots finishes up to 8
 * deferred steps in one launch: the partials of each slot (a range of n
 * parameters) summed into *grad_sq (added when accumulate; grad_sq may be
 * NULL) and *step incremented.  Each range gives the same bits as
 * ttrl_adam_step (ttrl/engine/optim/adam.py:93-134), grad_sq included.  A
 * slot must not be reused between its step and its finish. */
typedef struct ttrl_adam_finish {
  int slot;
  long n;
  int* step;
  float* grad_sq;
  int accumulate;
  int parts;  /* partial sums in the slot; 0: those of a deferred range of n parameters */
} ttrl_adam_finish;
int ttrl_adam_step_deferred(ttrl_ctx* ctx, float* p, const float* g, float* m_s, float* v_s, long n,
                            const int* step, float lr, float beta1, float beta2, float eps, float weight_decay,
                            int slot);
int ttrl_adam_multi(ttrl_ctx* ctx, int nranges, const ttrl_adam_range* ranges, float* polyak_dst,
                    const float* polyak_src, long polyak_n, float tau);
int ttrl_adam_finish_slots(ttrl_ctx* ctx, int n, const ttrl_adam_finish* finishes);
/* ttrl_adam_step over an arena whose gradients include up to 8 gradient
 * sources (ranges of g that earlier launches left unreduced): the step forms
 * each source's gradient, writes it into g, and updates those parameters
 * with it, so an update needs no separate reduction launch per source
 * (ttrl/engine/optim/adam.py:93-134 over the gradients of
 * ttrl/engine/conv/backward.py:45-78 and ttrl/engine/layers.py:22-61).  The
 * finishing launch also forms up to 4 ordered sums dst = scale * sum over
 * i < n of src[i * stride], in order from zero (an update's batch means,
 * ttrl/algos/dqn/losses.py:120-140).  Each source's dw (and db) must lie in
 * [g, g + n), 16-byte aligned, rows * cols a multiple of 4; a splits
 * source needs cols % 4 == 0. */
typedef struct ttrl_ordered_sum {
  const float* src;
  int n, stride;
  float scale;
  float* dst;
} ttrl_ordered_sum;
typedef struct ttrl_adam_sources_desc {
  float* p;
  float* g;
  float* m_s;
  float* v_s;
  long n;
  int* step;
  float lr, beta1, beta2, eps, weight_decay;
  float* grad_sq;
  int accumulate_grad_sq;
  int nsources;
  const ttrl_grad_source* sources;
  int nsums;
  const ttrl_ordered_sum* sums;
  int store_grads; /* 0: the formed gradients update the parameters but are not
                      written into g (ttrl_grad_sources_materialize writes them
                      from the same operands while those are unchanged) */
} ttrl_adam_sources_desc;
int ttrl_adam_step_sources(ttrl_ctx* ctx, const ttrl_adam_sources_desc* desc);
/* The ordered sums of ttrl_adam_step_sources without a step (up to 4). */
int ttrl_ordered_sums(ttrl_ctx* ctx, int n, const ttrl_ordered_sum* sums);
/* sum(x^2) into *out (grad_sq_device, ttrl/algos/grads.py:46-60). */
int ttrl_sum_squares(ttrl_ctx* ctx, const float* x, long n, float* out, int accumulate);
/* dst = (1 - tau) * dst + tau * src (ttrl/algos/sac/targets.py:45-52). */
int ttrl_polyak(ttrl_ctx* ctx, float* dst, const float* src, long n, float tau);

/* ---------------------------------------------------------------- PPO --- */

/* GAE-lambda over a [T][N] rollout (time-major, one column per env lane),
 * recursing t = T-1 .. 0 with last_values [N] as the value after the last
 * step: delta = r + gamma*V'*(1-done) - V; A = delta + gamma*lam*(1-done)*A';
 * A *= valid (a padding slot cuts the chain; valid may be NULL for all ones);
 * returns = A + V.  Products round as the reference's float32 recursion does.
 * Replaces RolloutBuffer.compute_gae (ttrl/buffers/rollout.py:195-226). */
int ttrl_gae(ttrl_ctx* ctx, int T, int N, const float* rewards, const float* values, const float* dones,
             const float* valid, const float* last_values, double gamma, double lam, float* advantages,
             float* returns);
/* out = (a - mean) / (std + eps) over the n entries with valid > 0 (population
 * std; valid NULL = all), 0 elsewhere; stats (nullable) receives {mean, std}.
 * The minibatch advantage normalisation of ttrl/buffers/rollout.py:269-270. */
int ttrl_normalize_advantages(ttrl_ctx* ctx, const float* adv, const float* valid, long n, float eps, float* out,
                              float* stats);
/* The PPO objective of one minibatch (ttrl/algos/ppo/loss.py:42-83) with the
 * categorical head's log-prob and entropy (ttrl/algos/ppo/policy.py:64-76,
 * ttrl/engine/ops/functional.py:160-178): logits [B][A], actions [B] (int32),
 * per-row old_logp, advantages, returns, old_values, values [B]; valid [B]
 * (nullable) selects the masked mean (masked_mean, loss.py:27-39).
 * out4 = {loss, policy_loss, value_loss, entropy}; new_logp [B];
 * dlogits [B][A] and dvalues [B] = d loss / d logits, d loss / d values. */
int ttrl_ppo_loss(ttrl_ctx* ctx, int B, int A, const float* logits, const int* actions, const float* old_logp,
                  const float* advantages, const float* returns, const float* old_values, const float* values,
                  const float* valid, float clip_eps, float value_clip_eps, float value_coef, float entropy_coef,
                  float* out4, float* new_logp, float* dlogits, float* dvalues);
/* ttrl_ppo_loss over the packed rows of the fused policy-and-value head:
 * head [B][A+1] holds the logits in columns 0..A-1 and the value in column A,
 * dhead is laid out the same; out5 = {loss, policy_loss, value_loss, entropy,
 * approx_kl}, approx_kl = mean(expm1(r) - r) with r = new_logp - old_logp
 * (ttrl/algos/ppo/learn.py:101-112). */
int ttrl_ppo_loss_packed(ttrl_ctx* ctx, int B, int A, const float* head, const int* actions, const float* old_logp,
                         const float* advantages, const float* returns, const float* old_values, const float* valid,
                         float clip_eps, float value_clip_eps, float value_coef, float entropy_coef, float* out5,
                         float* new_logp, float* dhead);
/* Minibatch assembly by index from a resident flattened rollout
 * (RolloutBuffer.minibatches, ttrl/buffers/rollout.py:239-282): for each of
 * nsrc (<= 8) sources, dst[s] row i = src[s] row idx[c * stride + i], rows of
 * row_bytes[s] bytes (a multiple of 4; 16-byte rows move as 16-byte units),
 * i < n, c = *counter (counter NULL: c = 0).  Table slots past idx_len and
 * indices outside [0, rows) are skipped. */
int ttrl_gather_rows(ttrl_ctx* ctx, int n, int nsrc, const void* const* src, void* const* dst, const long* row_bytes,
                     long rows, const int* idx, long idx_len, const int* counter, int stride);
/* End of one replayed minibatch step: ring[c][0..n) = metrics when
 * 0 <= c < slots, then *counter = c + 1 (the per-minibatch metric reads of
 * ttrl/algos/ppo/learn.py:94-112, kept on the device for one read per
 * update). */
int ttrl_step_end(ttrl_ctx* ctx, int* counter, const float* metrics, int n, float* ring, int slots);
/* Global L2 clip of one flat gradient arena, on the device (no host read):
 * norm = sqrt(sum g^2); if norm > max_norm, g *= max_norm / (norm + 1e-6).
 * *norm_out (nullable) receives the norm before clipping; sq_scratch is one
 * float.  Replaces clip_grad_norm (ttrl/algos/grads.py:13-43). */
int ttrl_clip_grad_norm(ttrl_ctx* ctx, float* g, long n, float max_norm, float* sq_scratch, float* norm_out);

/* ------------------------------------------------------ elementwise ops --- */

enum {
  TTRL_U_RELU = 0, TTRL_U_ABS, TTRL_U_SIGN, TTRL_U_SQUARE, TTRL_U_EXP, TTRL_U_LOG, TTRL_U_TANH,
  TTRL_U_SIGMOID, TTRL_U_SQRT, TTRL_U_NEG, TTRL_U_ADD_S, TTRL_U_MUL_S, TTRL_U_RSUB_S, TTRL_U_DIV_S,
  TTRL_U_EQZ, TTRL_U_GTZ, TTRL_U_ISFINITE, TTRL_U_COUNT
};
enum { TTRL_B_ADD = 0, TTRL_B_SUB, TTRL_B_MUL, TTRL_B_DIV, TTRL_B_RELU_BW, TTRL_B_MAX, TTRL_B_MIN, TTRL_B_EQ,
       TTRL_B_COUNT };
enum { TTRL_R_SUM = 0, TTRL_R_MAX, TTRL_R_ARGMAX, TTRL_R_COUNT };

/* y = f(a) elementwise, with a scalar operand for the *_S ops; replaces the
 * unary ttnn ops and scalar spellings (ttrl/engine/ops/unary.py:21-150,
 * ttrl/engine/ops/elementwise.py:15-148). */
int ttrl_unary(ttrl_ctx* ctx, int op, const float* a, float* y, long n, float scalar);
/* y = a op b over a contiguous output of rank ndim <= 6; operands are read
 * through element strides (0 broadcasts).  Replaces the binary ttnn ops and
 * relu_bw (ttrl/engine/ops/elementwise.py:15-148, ttrl/engine/ops/unary.py:34). */
int ttrl_binary(ttrl_ctx* ctx, int op, const float* a, const float* b, float* y, int ndim, const long* shape,
                const long* stride_a, const long* stride_b);
/* y[strided] = a[strided]: concat, split, slice and repeat
 * (ttrl/engine/ops/shape.py:10-151, ttrl/engine/ops/broadcast.py:33-54). */
int ttrl_copy_strided(ttrl_ctx* ctx, const float* a, float* y, int ndim, const long* shape, const long* stride_a,
                      const long* stride_y);
/* Sum, max or argmax (first index, as fp32) of the middle axis of an
 * [outer][dim][inner] view (ttrl/engine/ops/reduce.py:12-99). */
int ttrl_reduce(ttrl_ctx* ctx, int op, const float* a, float* y, long outer, long dim, long inner);
/* y[b][c] = (c - indices[b] == 0) (ttrl/engine/ops/functional.py:112-123). */
int ttrl_one_hot(ttrl_ctx* ctx, const float* indices, float* y, long batch, int num_classes);

/* ---- acting step -------------------------------------------------------- */

/* Greedy action of a Q network's last linear layer, fused: q = h W + bias
 * ([B][K] x [K][A], W in the (in, out) layout of ttrl/engine/layers.py:43-47;
 * bias may be NULL, q_out may be NULL) and actions[b] = the first index of
 * the row maximum, as int32.  Replaces the acting forward's QHead matmul and
 * argmax_dim_detached (ttrl/algos/dqn/agent.py:107-109,
 * ttrl/engine/ops/reduce.py:82-99).  A <= 32. */
int ttrl_q_act(ttrl_ctx* ctx, int B, int K, int A, const float* h, const float* W, const float* bias, float* q_out,
               int* actions);
/* Squashed-Gaussian action of a GaussianHead, fused: mean = h W_mean +
 * b_mean, log_std = clamp(h W_log_std + b_log_std, min, max)
 * (ttrl/nets/heads.py:65-93); stochastic: u = mean + exp(log_std) * noise,
 * action = centre + half_width * tanh(u), logp = squashed_logp(u) - log_det;
 * deterministic: action = centre + half_width * tanh(mean), logp = 0
 * (ttrl/algos/sac/policy.py:42-59, ttrl/algos/gaussian.py:106-167).
 * head_out ([B][2d] = [mean | clamped log_std]) may be NULL.  d <= 16. */
int ttrl_gaussian_act(ttrl_ctx* ctx, int B, int K, int d, const float* h, const float* W_mean, const float* b_mean,
                      const float* W_log_std, const float* b_log_std, float log_std_min, float log_std_max,
                      const float* noise, const float* centre, const float* half_width, float log_det,
                      int deterministic, float* head_out, float* action, float* logp);

/* ---- GRU unroll ------------------------------------------------------------ */

/* One timestep of a GRU (GRUCell, ttrl/engine/recurrent.py:39-110; gate order
 * reset, update, candidate): gi and gh are the [B][3H] projections x W_ih +
 * b_ih and hin W_hh + b_hh; writes hout = (1 - z) * n + z * hin and, when
 * hin_next is given, hin_next = hout * (1 - done_next) (done_next [B] may be
 * NULL: no reset), the state entering the next step (GRU.forward's
 * apply_done_mask, ttrl/engine/recurrent.py:144-168). */
int ttrl_gru_step(ttrl_ctx* ctx, int B, int H, const float* gi, const float* gh, const float* hin, float* hout,
                  const float* done_next, float* hin_next);
/* out = h * (1 - done) per row (done NULL: a copy): the reset of the initial
 * state (apply_done_mask, ttrl/engine/ops/functional.py:40-46). */
int ttrl_gru_mask(ttrl_ctx* ctx, int B, int H, const float* h, const float* done, float* out);
/* Backward of ttrl_gru_step: with dh = dout + (1 - done_next) * dhin_next
 * (either term may be NULL), writes the gate gradients dgi, dgh ([B][3H])
 * and dhin = z * dh, the direct part of the gradient of hin (a GEMM adds
 * dgh W_hh^T). */
int ttrl_gru_step_backward(ttrl_ctx* ctx, int B, int H, const float* gi, const float* gh, const float* hin,
                           const float* dout, const float* dhin_next, const float* done_next, float* dgi, float* dgh,
                           float* dhin);
/* ttrl_gru_step with its recurrent product in the same launch: gh = hin W_hh
 * + b_hh (W_hh [H][3H], b_hh [3H]) is formed, written to gh and used for the
 * cell (GRUCell.forward, ttrl/engine/recurrent.py:86-94).  H a multiple of
 * 16 (<= 8192); hin and W_hh 16-byte aligned. */
int ttrl_gru_step_fused(ttrl_ctx* ctx, int B, int H, const float* gi, const float* hin, const float* W_hh,
                        const float* b_hh, float* gh, float* hout, const float* done_next, float* hin_next);
/* One step of the GRU's reverse walk in one launch (the backward of
 * ttrl/engine/recurrent.py:88-168 through step t): d hin_t = dhz + dgh
 * W_hh^T, where dhz = z_t * dh_t is the direct part ttrl_gru_step_backward
 * or the previous call left; written to dhin when given.  With gi_prev,
 * also the cell backward of step t - 1 for dh_{t-1} = dout_prev + (1 - done)
 * d hin_t (dout_prev, done [B] nullable; done is done_t): its gate gradients
 * dgi_prev, dgh_prev and its direct part dhz_prev, the input of the next
 * call.  gh_prev, hin_prev, dgi_prev, dgh_prev and dhz_prev come with
 * gi_prev or not at all.  H a multiple of 16 (<= 8192); dgh and W_hh
 * 16-byte aligned. */
int ttrl_gru_step_backward_fused(ttrl_ctx* ctx, int B, int H, const float* dgh, const float* W_hh, const float* dhz,
                                 float* dhin, const float* gi_prev, const float* gh_prev, const float* hin_prev,
                                 const float* dout_prev, const float* done, float* dgi_prev, float* dgh_prev,
                                 float* dhz_prev);

/* ---- GPU-resident replay -------------------------------------------------- */

/* One replay ring in device memory (ttrl/buffers/replay.py:62-129): per lane
 * `cols` columns; column i holds the state its action was taken from.  One
 * observation leaf of obs_bytes bytes (a multiple of 4).  final_slot[l][c]
 * names the row of final_obs holding the episode-final observation of an
 * ending column (the boundary table of ttrl/buffers/boundaries.py), or -1.
 * weight (NULL for a uniform ring) holds (p + epsilon) ** alpha per column
 * and *max_priority the largest raw priority seen, both float64
 * (ttrl/buffers/sampling.py:111-133). */
typedef struct ttrl_replay_ring {
  int lanes, cols;
  long obs_bytes;
  unsigned char* obs;        /* [lanes][cols][obs_bytes] */
  int* actions;              /* [lanes][cols] */
  float* rewards;            /* [lanes][cols] */
  unsigned char* dones;      /* [lanes][cols] terminated */
  unsigned char* ends;       /* [lanes][cols] terminated or truncated */
  int* final_slot;           /* [lanes][cols] */
  unsigned char* final_obs;  /* [final_rows][obs_bytes] */
  int final_rows;
  double* weight;            /* [lanes][cols] or NULL */
  double* max_priority;      /* device scalar or NULL */
  double alpha, epsilon;
  float* action_vec;         /* [lanes][cols][action_dim] continuous actions, or NULL (index actions) */
  int action_dim;            /* 1..64 when action_vec is set */
} ttrl_replay_ring;

/* Write n transitions, entry e into (lane[e], col[e]): obs row e of obs
 * ([n][obs_bytes]), the action (action[e], or row e of action_vec
 * ([n][action_dim]) for a ring with vector actions, the continuous actions
 * of SAC's replay), reward, terminated and ended flags, and for an
 * ending entry (final_row[e] >= 0) row e of final_obs into that boundary
 * row; a prioritized ring gives the column the weight (max priority + eps)
 * ** alpha.  Replaces ReplayBuffer._write_slot (ttrl/buffers/replay.py:178-199)
 * and PrioritySampler.on_write (ttrl/buffers/sampling.py:130-133).  All
 * arrays are device arrays. */
int ttrl_replay_write(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const int* col,
                      const int* action, const float* action_vec, const float* reward,
                      const unsigned char* terminated, const unsigned char* ended, const int* final_row,
                      const void* obs, const void* final_obs);
/* Per-lane sums of the priority weights over each lane's sampleable run
 * (start[l], count[l] in ring order), as chunk sums of `chunk` run positions
 * ([lanes][max_chunks]) and their ordered totals sums[lanes]
 * (PrioritySampler.draw's lane sums, ttrl/buffers/sampling.py:135-166). */
int ttrl_replay_lane_sums(ttrl_ctx* ctx, const ttrl_replay_ring* ring, const int* start, const int* count, int chunk,
                          int max_chunks, double* chunk_sums, double* sums);
/* For sample b in lane[b] with uniform u[b]: the run position where the
 * cumulative weight first exceeds u[b] * sums[lane] (searchsorted 'right',
 * capped at the run's end, ttrl/buffers/sampling.py:216-222); writes the
 * ring column and that column's weight. */
int ttrl_replay_priority_pick(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const double* u,
                              const int* start, const int* count, int chunk, int max_chunks,
                              const double* chunk_sums, const double* sums, int* cols_out, double* picked_weight);
/* Importance-sampling weights (N * P) ** -beta over the batch maximum, P =
 * picked weight / sum of the lane sums, N = total_count sampleable
 * transitions (ttrl/buffers/sampling.py:225-236), as float32. */
int ttrl_replay_is_weights(ttrl_ctx* ctx, int n, const double* picked_weight, const double* sums, int lanes,
                           long total_count, double beta, float* weights_out);
/* The batch rows of the transitions at (lane[b], col[b]): the n-step return
 * in float64 cast to float32, terminated flag and gamma ** steps
 * (ttrl/buffers/indexing.py:94-131), the observation and the successor (the
 * next column, or the boundary row of an ending column), the action as an
 * index and/or one-hot row, or as a [n][action_dim] row of a ring with
 * vector actions (ttrl/buffers/replaybatch.py:15-76).  Output pointers may
 * be a learner's bound input buffers. */
int ttrl_replay_assemble(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const int* col,
                         int n_step, double gamma, void* obs_out, void* next_obs_out, float* actions_onehot,
                         int num_actions, int* actions_out, float* action_vec_out, float* rewards_out,
                         float* dones_out, float* discounts_out);
/* One prioritized batch after the host's draws (ttrl/buffers/sampling.py:195-240,
 * ttrl/buffers/replay.py:254-282): ttrl_replay_priority_pick (also copying
 * the batch's lanes into lanes_out), then ttrl_replay_is_weights into
 * weights_out, then ttrl_replay_assemble of the picked (lanes_out, cols_out),
 * enqueued by one call.  lane, u, start, count and sums may be mapped host
 * memory (ttrl_host_alloc_mapped); lanes_out and cols_out are device arrays a
 * later priority update reads. */
typedef struct ttrl_replay_draw {
  int n;
  const int* lane;
  int* lanes_out;
  const double* u;
  const int* start;
  const int* count;
  int chunk, max_chunks;
  const double* chunk_sums;
  const double* sums;
  long total_count;
  double beta;
  int* cols_out;
  double* picked_weight;
  float* weights_out;
  int n_step;
  double gamma;
  void* obs_out;
  void* next_obs_out;
  float* actions_onehot;
  int num_actions;
  int* actions_out;
  float* action_vec_out;
  float* rewards_out;
  float* dones_out;
  float* discounts_out;
} ttrl_replay_draw;
int ttrl_replay_draw_batch(ttrl_ctx* ctx, const ttrl_replay_ring* ring, const ttrl_replay_draw* draw);
/* weight[lane[b]][col[b]] = (|priorities[b]| + eps) ** alpha, the last of
 * duplicate columns winning, and *max_priority = max(*max_priority,
 * max |priorities|) (PrioritySampler.update, ttrl/buffers/sampling.py:168-193).
 * priorities is a device array, e.g. the TD errors an update left on the
 * device. */
int ttrl_replay_update_priorities(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const int* col,
                                  const float* priorities);
/* The same update from float64 priorities (host values, whose
 * (|p| + eps) ** alpha the reference computes in float64,
 * ttrl/buffers/sampling.py:180-193). */
int ttrl_replay_update_priorities_f64(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane,
                                      const int* col, const double* priorities);

#ifdef __cplusplus
}
#endif

#endif /* TTRL_HIP_H */
