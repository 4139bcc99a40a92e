// GRU cell arithmetic of one timestep of an unrolled GRU, forward and
// backward, fused per element (ttrl/engine/recurrent.py:39-168, PyTorch's
// gate order and placement of the reset gate):
//
//   r = sigmoid(gi_r + gh_r)   z = sigmoid(gi_z + gh_z)
//   n = tanh(gi_n + r * gh_n)  h' = (1 - z) * n + z * h
//
// gi = x W_ih + b_ih and gh = h W_hh + b_hh are [B][3H] rows produced by the
// GEMMs around these kernels (all timesteps' gi by one GEMM before the
// unroll).  The state entering step t is hin_t = h_{t-1} * (1 - done_t)
// (apply_done_mask, ttrl/engine/ops/functional.py:40-46); the forward kernel
// of step t writes h_t and hin_{t+1}.  The backward recomputes r, z, n from
// gi, gh and hin (the same expressions, so the same values) and writes the
// gate gradients d gi, d gh for the batched weight-gradient GEMMs and the
// direct part z * dh of d hin_t, to which a GEMM adds d gh W_hh^T.
//
// Fused steps (H a multiple of 16): the recurrent product and the cell
// arithmetic of a timestep in one launch.  Forward, gh_t = hin_t W_hh + b_hh
// and the cell; backward, d hin_t = z_t dh_t + d gh_t W_hh^T and then the
// cell backward of step t - 1, whose dh_{t-1} = dout_{t-1} + (1 - done_t)
// d hin_t needs only this workgroup's units.  A workgroup owns 8 hidden
// units (the gate columns u, H + u, 2H + u of each) and 8 batch rows, and
// runs each 16 x 16 MFMA as two 8 x 8 products over different k: lanes of
// column half h (c / 8) carry row or unit c % 8 at k offset 16 h, so the
// diagonal blocks of the output hold the two k halves and every lane loads
// distinct operands (an 8 x 8 tile puts half the bytes and MFMAs of a 16 x
// 16 one on each CU, over twice the CUs).  Its kFw wavefronts split the
// reduction into pair groups of 32 k (a contiguous run each, so a wavefront
// reads whole cache lines of each operand row); in pair group p a lane
// (c, quarter g = lane / 16) feeds k = 32p + 16h + 4g + j to MFMA j, the
// operand that runs along k in memory as one float4.  The partial tiles are
// summed in wavefront order through LDS, so every output has one fixed
// summation order.
#include "common.hpp"
#include "tile_gemm.hpp"

#include <cmath>

namespace ttrl {
namespace {

constexpr int kGruThreads = 256;

__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

__device__ __forceinline__ float keep_f(const float* done, int b) { return done ? 1.f - done[b] : 1.f; }

// h' = (1 - z) * n + z * h from the two projections' gate pre-activations.
__device__ __forceinline__ float cell_forward(float xr, float xz, float xn, float hr, float hz, float hn, float h) {
  const float r = sigmoid_f(xr + hr);
  const float z = sigmoid_f(xz + hz);
  const float c = tanhf(xn + r * hn);
  return (1.f - z) * c + z * h;
}

// The cell's backward for dh = d h': the gate gradients (d gi = [r, z, n],
// d gh = [r, z, hn]) and the direct part z * dh of d h.
struct CellGrad {
  float r, z, n, hn, hz;
};
__device__ __forceinline__ CellGrad cell_backward(float xr, float xz, float xn, float hr, float hz, float hn, float h,
                                                  float dh) {
  const float r = sigmoid_f(xr + hr);
  const float z = sigmoid_f(xz + hz);
  const float c = tanhf(xn + r * hn);
  const float dc = dh * (1.f - z);
  const float dz = dh * (h - c);
  const float dcp = dc * (1.f - c * c);
  const float dr = dcp * hn;
  const float drp = dr * (r * (1.f - r));
  const float dzp = dz * (z * (1.f - z));
  return CellGrad{drp, dzp, dcp, dcp * r, dh * z};
}

__global__ __launch_bounds__(kGruThreads) void k_gru_mask(int B, int H, const float* __restrict__ h,
                                                          const float* __restrict__ done, float* __restrict__ out) {
  const long n = long(B) * H;
  for (long i = long(blockIdx.x) * kGruThreads + threadIdx.x; i < n; i += long(gridDim.x) * kGruThreads) {
    const int b = int(i / H);
    out[i] = h[i] * keep_f(done, b);
  }
}

__global__ __launch_bounds__(kGruThreads) void k_gru_step(int B, int H, const float* __restrict__ gi,
                                                          const float* __restrict__ gh,
                                                          const float* __restrict__ hin, float* __restrict__ hout,
                                                          const float* __restrict__ done_next,
                                                          float* __restrict__ hin_next) {
  const long n = long(B) * H;
  for (long i = long(blockIdx.x) * kGruThreads + threadIdx.x; i < n; i += long(gridDim.x) * kGruThreads) {
    const int b = int(i / H), j = int(i - long(b) * H);
    const float* gib = gi + long(b) * 3 * H;
    const float* ghb = gh + long(b) * 3 * H;
    const float out = cell_forward(gib[j], gib[H + j], gib[2 * H + j], ghb[j], ghb[H + j], ghb[2 * H + j], hin[i]);
    hout[i] = out;
    if (hin_next) hin_next[i] = out * keep_f(done_next, b);
  }
}

// dh_t = dout_t + (1 - done_{t+1}) * dhin_{t+1} (dout, dhin_next nullable).
__global__ __launch_bounds__(kGruThreads) void k_gru_step_bwd(int B, int H, const float* __restrict__ gi,
                                                              const float* __restrict__ gh,
                                                              const float* __restrict__ hin,
                                                              const float* __restrict__ dout,
                                                              const float* __restrict__ dhin_next,
                                                              const float* __restrict__ done_next,
                                                              float* __restrict__ dgi, float* __restrict__ dgh,
                                                              float* __restrict__ dhin) {
  const long n = long(B) * H;
  for (long i = long(blockIdx.x) * kGruThreads + threadIdx.x; i < n; i += long(gridDim.x) * kGruThreads) {
    const int b = int(i / H), j = int(i - long(b) * H);
    const float* gib = gi + long(b) * 3 * H;
    const float* ghb = gh + long(b) * 3 * H;
    float dh = dout ? dout[i] : 0.f;
    if (dhin_next) dh += keep_f(done_next, b) * dhin_next[i];
    const CellGrad d =
        cell_backward(gib[j], gib[H + j], gib[2 * H + j], ghb[j], ghb[H + j], ghb[2 * H + j], hin[i], dh);
    float* dgib = dgi + long(b) * 3 * H;
    float* dghb = dgh + long(b) * 3 * H;
    dgib[j] = d.r;
    dgib[H + j] = d.z;
    dgib[2 * H + j] = d.n;
    dghb[j] = d.r;
    dghb[H + j] = d.z;
    dghb[2 * H + j] = d.hn;
    dhin[i] = d.hz;
  }
}

constexpr int kFw = 8;  // wavefronts of a fused-step workgroup
constexpr int kFt = 64 * kFw;
constexpr int kTile = 8;       // batch rows and hidden units of a workgroup
constexpr int kFwdChunk = 2;   // forward: pair groups in flight per wavefront (13 loads each)
constexpr int kBwdChunk = 6;   // backward: pair groups in flight per wavefront (2 float4 loads each)

__device__ __forceinline__ float ldb1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ f32x4 ldb4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ f32x4 mfma4(f32x4 a, f32x4 b, f32x4 acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
}

// The lane's place in the block-diagonal product: half h = c / 8 of the
// 16 MFMA rows and columns, index cc = c % 8 in its 8 x 8 block; kh = the
// lane's k offset in a pair group (16 h + 4 g), kmax = the reduction length.
struct DiagLane {
  int cc, h, g;
  uint32_t kh;
};
__device__ __forceinline__ DiagLane diag_lane(int lane) {
  const int c = lane & 15, g = lane >> 4;
  return DiagLane{c & 7, c >> 3, g, uint32_t(16 * (c >> 3) + 4 * g)};
}

// The pair groups [lo, hi) of this wavefront: a contiguous run, so it reads
// whole cache lines of each operand row.
__device__ __forceinline__ void wave_range(int wave, int np, int& lo, int& hi) {
  const int per = (np + kFw - 1) / kFw;
  lo = wave * per;
  hi = min(np, lo + per);
}

struct GruFwdArgs {
  int B, H;
  const float* gi;         // [B][3H]  x_t W_ih + b_ih
  const float* hin;        // [B][H]   state entering the step
  const float* W;          // [H][3H]  W_hh
  const float* bias;       // [3H]     b_hh
  float* gh;               // [B][3H]  out: hin W_hh + b_hh
  float* hout;             // [B][H]   out: h_t
  const float* done_next;  // [B] or null
  float* hin_next;         // [B][H] or null: h_t * (1 - done_next)
};

__global__ __launch_bounds__(kFt) void k_gru_fwd_fused(GruFwdArgs a) {
  __shared__ float part[kFw * 3 * 256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int B = a.B, H = a.H, G = 3 * H;
  const int u0 = blockIdx.x * kTile, r0 = blockIdx.y * kTile;
  // The output element of threads 0..63 (row r0 + t / 8, unit u0 + t % 8);
  // the other threads load the same operands and store nothing.  The loads
  // are unconditional so that none of them waits before the product's.
  const int t = tid & 63;
  const bool ep = tid < 64;  // wavefront 0
  const int er = r0 + t / kTile, eu = u0 + t % kTile, erc = min(er, B - 1);
  const float* gib = a.gi + long(erc) * G;
  const float xr = gib[eu], xz = gib[H + eu], xn = gib[2 * H + eu];
  const float br = a.bias[eu], bz = a.bias[H + eu], bn = a.bias[2 * H + eu];
  const float h = a.hin[long(erc) * H + eu];
  const float dv = *(a.done_next ? a.done_next + erc : a.bias);
  const float keep = a.done_next ? 1.f - dv : 1.f;
  // A: hin[r0 + cc][k] (one float4), B: W[k][e H + u0 + cc], k = 32p + kh + j.
  const DiagLane L = diag_lane(lane);
  const __amdgpu_buffer_rsrc_t rA = make_res(a.hin, uint32_t(B) * uint32_t(H) * 4u);
  const __amdgpu_buffer_rsrc_t rB = make_res(a.W, uint32_t(H) * uint32_t(G) * 4u);
  const uint32_t va = uint32_t(min(r0 + L.cc, B - 1)) * uint32_t(H) * 4u;
  const uint32_t vb = uint32_t(u0 + L.cc) * 4u;
  const int np = (H + 31) >> 5;
  int lo, hi;
  wave_range(wave, np, lo, hi);
  f32x4 acc[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  for (int p0 = lo; p0 < hi; p0 += kFwdChunk) {
    f32x4 av[kFwdChunk], bv[kFwdChunk][3];
    bool in[kFwdChunk];
#pragma unroll
    for (int s = 0; s < kFwdChunk; ++s) {
      // past the end of the run (re-reads its last group) or of k (H % 32 ==
      // 16: re-reads the last 16 k): loaded, then zeroed below
      const uint32_t k = 32u * uint32_t(min(p0 + s, hi - 1)) + L.kh;
      in[s] = p0 + s < hi && k < uint32_t(H);
      const uint32_t kc = min(k, uint32_t(H - 16) + 4u * L.g);
      av[s] = ldb4(rA, va + kc * 4u, 0);
#pragma unroll
      for (int e = 0; e < 3; ++e) {
#pragma unroll
        for (int j = 0; j < 4; ++j) bv[s][e][j] = ldb1(rB, vb + ((kc + j) * uint32_t(G) + e * uint32_t(H)) * 4u, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the chunk issues before the first product
#pragma unroll
    for (int s = 0; s < kFwdChunk; ++s) {
      const f32x4 x = in[s] ? av[s] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 3; ++e) acc[e] = mfma4(x, bv[s][e], acc[e]);
    }
  }
  // lane (c, g) holds rows 4g + i of column c
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int e = 0; e < 3; ++e) {
#pragma unroll
    for (int i = 0; i < 4; ++i) part[(wave * 3 + e) * 256 + (4 * g + i) * 16 + c] = acc[e][i];
  }
  __syncthreads();
  if (!ep) return;
  // the element's two diagonal blocks (k halves), summed in wavefront order
  const int o0 = (t / kTile) * 16 + t % kTile, o1 = o0 + 8 * 16 + 8;
  float s3[3];
#pragma unroll
  for (int e = 0; e < 3; ++e) {
    float v = part[e * 256 + o0] + part[e * 256 + o1];
#pragma unroll
    for (int w = 1; w < kFw; ++w) v += part[(w * 3 + e) * 256 + o0] + part[(w * 3 + e) * 256 + o1];
    s3[e] = v;
  }
  const float hr = s3[0] + br, hz = s3[1] + bz, hn = s3[2] + bn;
  if (er >= B) return;
  const float out = cell_forward(xr, xz, xn, hr, hz, hn, h);
  float* ghb = a.gh + long(er) * G;
  ghb[eu] = hr;
  ghb[H + eu] = hz;
  ghb[2 * H + eu] = hn;
  a.hout[long(er) * H + eu] = out;
  if (a.hin_next) a.hin_next[long(er) * H + eu] = out * keep;
}

struct GruBwdArgs {
  int B, H;
  const float* dgh;  // [B][3H]  d gh_t
  const float* W;    // [H][3H]  W_hh
  const float* dhz;  // [B][H]   z_t * dh_t
  float* dhin;       // [B][H] or null: out d hin_t = dhz + d gh_t W_hh^T
  // the cell backward of step t - 1 (gi null: none)
  const float *gi, *gh, *hin;  // step t - 1's [B][3H], [B][3H], [B][H]
  const float* dout;           // [B][H] or null: d out_{t-1}
  const float* done;           // [B] or null: done_t, the reset between the steps
  float *dgi, *dgh_prev;       // [B][3H] out
  float* dhz_prev;             // [B][H]  out: z_{t-1} * dh_{t-1}
};

__global__ __launch_bounds__(kFt) void k_gru_bwd_fused(GruBwdArgs a) {
  __shared__ float part[kFw * 256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int B = a.B, H = a.H, G = 3 * H;
  const int u0 = blockIdx.x * kTile, r0 = blockIdx.y * kTile;
  const int t = tid & 63;
  const bool ep = tid < 64;
  const int er = r0 + t / kTile, eu = u0 + t % kTile, erc = min(er, B - 1);
  const bool cell = a.gi != nullptr;
  // Unconditional loads (see k_gru_fwd_fused); an absent operand reads a
  // buffer of the same shape and is not used.
  const long eh = long(erc) * H + eu;
  const float dz0 = a.dhz[eh];
  const float* gib = (cell ? a.gi : a.dgh) + long(erc) * G;
  const float* ghb = (cell ? a.gh : a.dgh) + long(erc) * G;
  const float xr = gib[eu], xz = gib[H + eu], xn = gib[2 * H + eu];
  const float hr = ghb[eu], hz = ghb[H + eu], hn = ghb[2 * H + eu];
  const float h = (cell ? a.hin : a.dhz)[eh];
  const float ov = (a.dout ? a.dout : a.dhz)[eh];
  const float dv = *(a.done ? a.done + erc : a.dhz);
  const float dout = a.dout ? ov : 0.f;
  const float keep = a.done ? 1.f - dv : 1.f;
  // A: d gh[r0 + cc][k], B: W[u0 + cc][k], k = 32p + kh + j; one float4 each.
  const DiagLane L = diag_lane(lane);
  const __amdgpu_buffer_rsrc_t rA = make_res(a.dgh, uint32_t(B) * uint32_t(G) * 4u);
  const __amdgpu_buffer_rsrc_t rB = make_res(a.W, uint32_t(H) * uint32_t(G) * 4u);
  const uint32_t va = uint32_t(min(r0 + L.cc, B - 1)) * uint32_t(G) * 4u;
  const uint32_t vb = uint32_t(u0 + L.cc) * uint32_t(G) * 4u;
  const int np = (G + 31) >> 5;
  int lo, hi;
  wave_range(wave, np, lo, hi);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int p0 = lo; p0 < hi; p0 += kBwdChunk) {
    f32x4 av[kBwdChunk], bv[kBwdChunk];
    bool in[kBwdChunk];
#pragma unroll
    for (int s = 0; s < kBwdChunk; ++s) {
      const uint32_t k = 32u * uint32_t(min(p0 + s, hi - 1)) + L.kh;
      in[s] = p0 + s < hi && k < uint32_t(G);
      const uint32_t kc = min(k, uint32_t(G - 16) + 4u * L.g);
      av[s] = ldb4(rA, va + kc * 4u, 0);
      bv[s] = ldb4(rB, vb + kc * 4u, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the chunk issues before the first product
#pragma unroll
    for (int s = 0; s < kBwdChunk; ++s) acc = mfma4(in[s] ? av[s] : f32x4{0.f, 0.f, 0.f, 0.f}, bv[s], acc);
  }
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) part[wave * 256 + (4 * g + i) * 16 + c] = acc[i];
  __syncthreads();
  if (!ep) return;
  const int o0 = (t / kTile) * 16 + t % kTile, o1 = o0 + 8 * 16 + 8;
  float v = part[o0] + part[o1];
#pragma unroll
  for (int w = 1; w < kFw; ++w) v += part[w * 256 + o0] + part[w * 256 + o1];
  const float dhin = v + dz0;
  if (er >= B) return;
  if (a.dhin) a.dhin[long(er) * H + eu] = dhin;
  if (!cell) return;
  const float dh = dout + keep * dhin;
  const CellGrad d = cell_backward(xr, xz, xn, hr, hz, hn, h, dh);
  float* dgib = a.dgi + long(er) * G;
  float* dghb = a.dgh_prev + long(er) * G;
  dgib[eu] = d.r;
  dgib[H + eu] = d.z;
  dgib[2 * H + eu] = d.n;
  dghb[eu] = d.r;
  dghb[H + eu] = d.z;
  dghb[2 * H + eu] = d.hn;
  a.dhz_prev[long(er) * H + eu] = d.hz;
}

unsigned grid_for(long n) {
  long g = (n + kGruThreads - 1) / kGruThreads;
  return unsigned(g < 1 ? 1 : (g > 4096 ? 4096 : g));
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_gru_mask(ttrl_ctx* ctx, int B, int H, const float* h, const float* done, float* out) {
  TTRL_REQUIRE(ctx && h && out, "ttrl_gru_mask: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0, "ttrl_gru_mask: bad extents");
  if (B == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_gru_mask, dim3(grid_for(long(B) * H)), dim3(kGruThreads), 0, stream_of(ctx), B, H, h, done,
                     out);
  return check_launch("ttrl_gru_mask");
}

int ttrl_gru_step(ttrl_ctx* ctx, int B, int H, const float* gi, const float* gh, const float* hin, float* hout,
                  const float* done_next, float* hin_next) {
  TTRL_REQUIRE(ctx && gi && gh && hin && hout, "ttrl_gru_step: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0, "ttrl_gru_step: bad extents");
  if (B == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_gru_step, dim3(grid_for(long(B) * H)), dim3(kGruThreads), 0, stream_of(ctx), B, H, gi, gh, hin,
                     hout, done_next, hin_next);
  return check_launch("ttrl_gru_step");
}

int ttrl_gru_step_backward(ttrl_ctx* ctx, int B, int H, const float* gi, const float* gh, const float* hin,
                           const float* dout, const float* dhin_next, const float* done_next, float* dgi, float* dgh,
                           float* dhin) {
  TTRL_REQUIRE(ctx && gi && gh && hin && dgi && dgh && dhin, "ttrl_gru_step_backward: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0, "ttrl_gru_step_backward: bad extents");
  if (B == 0) return TTRL_OK;
  hipLaunchKernelGGL(k_gru_step_bwd, dim3(grid_for(long(B) * H)), dim3(kGruThreads), 0, stream_of(ctx), B, H, gi, gh,
                     hin, dout, dhin_next, done_next, dgi, dgh, dhin);
  return check_launch("ttrl_gru_step_backward");
}

int ttrl_gru_step_fused(ttrl_ctx* ctx, int B, int H, const float* gi, const float* hin, const float* W_hh,
                        const float* b_hh, float* gh, float* hout, const float* done_next, float* hin_next) {
  TTRL_REQUIRE(ctx && gi && hin && W_hh && b_hh && gh && hout, "ttrl_gru_step_fused: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0 && H % 16 == 0 && H <= 8192,
               "ttrl_gru_step_fused: H must be a positive multiple of 16 up to 8192 (got B=%d, H=%d)", B, H);
  TTRL_REQUIRE((reinterpret_cast<uintptr_t>(hin) | reinterpret_cast<uintptr_t>(W_hh)) % 16 == 0,
               "ttrl_gru_step_fused: hin and W_hh must be 16-byte aligned");
  if (B == 0) return TTRL_OK;
  GruFwdArgs a{B, H, gi, hin, W_hh, b_hh, gh, hout, done_next, hin_next};
  hipLaunchKernelGGL(k_gru_fwd_fused, dim3(unsigned(H / kTile), ceil_div(B, kTile)), dim3(kFt), 0, stream_of(ctx), a);
  return check_launch("ttrl_gru_step_fused");
}

int ttrl_gru_step_backward_fused(ttrl_ctx* ctx, int B, int H, const float* dgh, const float* W_hh, const float* dhz,
                                 float* dhin, const float* gi_prev, const float* gh_prev, const float* hin_prev,
                                 const float* dout_prev, const float* done, float* dgi_prev, float* dgh_prev,
                                 float* dhz_prev) {
  TTRL_REQUIRE(ctx && dgh && W_hh && dhz, "ttrl_gru_step_backward_fused: null argument");
  TTRL_REQUIRE(B >= 0 && H > 0 && H % 16 == 0 && H <= 8192,
               "ttrl_gru_step_backward_fused: H must be a positive multiple of 16 up to 8192 (got B=%d, H=%d)", B,
               H);
  TTRL_REQUIRE((reinterpret_cast<uintptr_t>(dgh) | reinterpret_cast<uintptr_t>(W_hh)) % 16 == 0,
               "ttrl_gru_step_backward_fused: dgh and W_hh must be 16-byte aligned");
  const bool cell = gi_prev != nullptr;
  TTRL_REQUIRE(cell ? (gh_prev && hin_prev && dgi_prev && dgh_prev && dhz_prev)
                    : !(gh_prev || hin_prev || dout_prev || done || dgi_prev || dgh_prev || dhz_prev),
               "ttrl_gru_step_backward_fused: the previous step's gi, gh, hin, dgi, dgh and dhz are given together");
  TTRL_REQUIRE(cell || dhin, "ttrl_gru_step_backward_fused: nothing to write (dhin and gi_prev both NULL)");
  if (B == 0) return TTRL_OK;
  GruBwdArgs a{B, H, dgh, W_hh, dhz, dhin, gi_prev, gh_prev, hin_prev, dout_prev, done, dgi_prev, dgh_prev, dhz_prev};
  hipLaunchKernelGGL(k_gru_bwd_fused, dim3(unsigned(H / kTile), ceil_div(B, kTile)), dim3(kFt), 0, stream_of(ctx), a);
  return check_launch("ttrl_gru_step_backward_fused");
}

}  // extern "C"
