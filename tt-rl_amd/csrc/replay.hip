// GPU-resident replay: the ring of transitions lives in HBM and a sampled
// batch is assembled there, straight into the learner's bound inputs.
//
// write      one transition per entry into (lane, column): the observation,
//            action, reward, terminated / ended flags, the episode-final
//            observation of an ending column (a row of the boundary pool, or
//            none), and, for a prioritized ring, the fresh column's weight
//            (max priority + eps) ** alpha (ttrl/buffers/replay.py:178-199,
//            ttrl/buffers/sampling.py:126-133).
// lane sums  each lane's total weight over its sampleable run, summed as
//            chunk sums in run order (ttrl/buffers/sampling.py:135-166).
// pick       per sample, the position in its lane's run where the cumulative
//            weight first exceeds u * lane total -- numpy's
//            searchsorted(cumsum, x, 'right') capped at the run's end
//            (ttrl/buffers/sampling.py:216-222); one wavefront per sample
//            scans the lane's chunk sums, then the one chunk.
// weights    (N * P) ** -beta over the batch maximum (sampling.py:225-236).
// assemble   per sample the n-step walk in float64 (g += disc * r,
//            disc *= gamma, stop at the first ending column, only a
//            termination zeroes the bootstrap), the successor (the next
//            column, or the final observation of an ending column), and the
//            batch rows: observation, successor, action (index and one-hot),
//            float32 return, done, gamma ** steps
//            (ttrl/buffers/indexing.py:94-131, ttrl/buffers/replaybatch.py:15-76).
// priorities (|p| + eps) ** alpha into the sampled columns, the last of
//            duplicate columns winning as numpy's fancy assignment does, and
//            the running max priority (ttrl/buffers/sampling.py:168-193).
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>

namespace ttrl {
namespace {

constexpr int kReplayThreads = 256;

struct Ring {
  int lanes, cols;
  long obs_bytes;
  unsigned char* obs;
  int* actions;
  float* rewards;
  unsigned char* dones;
  unsigned char* ends;
  int* final_slot;
  unsigned char* final_obs;
  int final_rows;
  double* weight;
  double* max_priority;
  double alpha, epsilon;
  float* action_vec;
  int action_dim;
};

Ring ring_of(const ttrl_replay_ring* r) {
  return Ring{r->lanes,      r->cols,       r->obs_bytes,  r->obs,        r->actions,
              r->rewards,    r->dones,      r->ends,       r->final_slot, r->final_obs,
              r->final_rows, r->weight,     r->max_priority, r->alpha,    r->epsilon,
              r->action_vec, r->action_vec ? r->action_dim : 0};
}

// Copy one row of `bytes` bytes with the whole block, 16-byte units when the
// row size and both addresses allow, else 4-byte units.
__device__ __forceinline__ void copy_row(unsigned char* dst, const unsigned char* src, long bytes) {
  const bool vec = ((bytes | reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0;
  if (vec) {
    const long n = bytes >> 4;
    for (long i = threadIdx.x; i < n; i += blockDim.x)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else {
    const long n = bytes >> 2;
    for (long i = threadIdx.x; i < n; i += blockDim.x)
      reinterpret_cast<unsigned*>(dst)[i] = reinterpret_cast<const unsigned*>(src)[i];
  }
}

__global__ __launch_bounds__(kReplayThreads) void k_replay_write(Ring r, int n, const int* __restrict__ lane,
                                                                 const int* __restrict__ col,
                                                                 const int* __restrict__ action,
                                                                 const float* __restrict__ action_vec,
                                                                 const float* __restrict__ reward,
                                                                 const unsigned char* __restrict__ term,
                                                                 const unsigned char* __restrict__ end,
                                                                 const int* __restrict__ fslot,
                                                                 const unsigned char* __restrict__ obs,
                                                                 const unsigned char* __restrict__ fin) {
  const int e = blockIdx.x;
  if (e >= n) return;
  const int l = lane[e], c = col[e], f = fslot[e];
  if (l < 0 || l >= r.lanes || c < 0 || c >= r.cols) return;
  const long at = long(l) * r.cols + c;
  copy_row(r.obs + at * r.obs_bytes, obs + long(e) * r.obs_bytes, r.obs_bytes);
  const bool has_final = f >= 0 && f < r.final_rows;
  if (has_final) copy_row(r.final_obs + long(f) * r.obs_bytes, fin + long(e) * r.obs_bytes, r.obs_bytes);
  for (int i = threadIdx.x; i < r.action_dim; i += blockDim.x)
    r.action_vec[at * r.action_dim + i] = action_vec[long(e) * r.action_dim + i];
  if (threadIdx.x == 0) {
    r.actions[at] = action ? action[e] : 0;
    r.rewards[at] = reward[e];
    r.dones[at] = term[e];
    r.ends[at] = end[e];
    r.final_slot[at] = has_final ? f : -1;
    if (r.weight) r.weight[at] = pow(*r.max_priority + r.epsilon, r.alpha);
  }
}

// csum[l * max_chunks + k] = sum of the weights at run positions
// [k * chunk, min((k + 1) * chunk, count)) of lane l: one workgroup per
// (chunk, lane), coalesced loads, a tree sum.
__global__ __launch_bounds__(kReplayThreads) void k_replay_chunk_sums(Ring r, const int* __restrict__ start,
                                                                      const int* __restrict__ count, int chunk,
                                                                      int max_chunks, double* __restrict__ csum) {
  __shared__ double red[kReplayThreads];
  const int l = blockIdx.y, k = blockIdx.x;
  const int cnt = count[l], st = start[l];
  const int p0 = k * chunk, p1 = min(p0 + chunk, cnt);
  const double* w = r.weight + long(l) * r.cols;
  double s = 0.0;
  for (int p = p0 + threadIdx.x; p < p1; p += kReplayThreads) {
    int c = st + p;
    c = c >= r.cols ? c - r.cols : c;
    s += w[c];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int h = kReplayThreads / 2; h > 0; h >>= 1) {
    if (threadIdx.x < h) red[threadIdx.x] += red[threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0 && k < max_chunks) csum[long(l) * max_chunks + k] = red[0];
}

// sums[l] = the lane's chunk sums added in order, one wavefront per lane:
// the wavefront stages up to kLaneSumBatch chunk sums in LDS with all its
// loads in flight at once, then one thread adds them in chunk order (the
// same additions in the same order as a sequential loop over the chunks).
constexpr int kLaneSumBatch = 2048;
__global__ __launch_bounds__(64) void k_replay_lane_sums(int lanes, int max_chunks, const double* __restrict__ csum,
                                                         double* __restrict__ sums) {
  __shared__ double stage[kLaneSumBatch];
  const int l = blockIdx.x;
  if (l >= lanes) return;  // uniform over the workgroup
  const double* cs = csum + long(l) * max_chunks;
  double s = 0.0;
  for (int k0 = 0; k0 < max_chunks; k0 += kLaneSumBatch) {
    const int m = min(kLaneSumBatch, max_chunks - k0);
    for (int i = threadIdx.x; i < m; i += 64) stage[i] = cs[k0 + i];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < m; ++i) s += stage[i];
    __syncthreads();
  }
  if (threadIdx.x == 0) sums[l] = s;
}

// Wavefront inclusive prefix sum.
__device__ __forceinline__ double wave_incl_scan(double v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const double o = __shfl_up(v, off);
    if (lane >= off) v += o;
  }
  return v;
}

__device__ __forceinline__ int wave_min_int(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = min(v, __shfl_xor(v, off));
  return v;
}

// First index i in [0, m) of vals (read through `get`) whose running sum from
// `base` exceeds x, or m when none does; also the running sum before it.
template <class Get>
__device__ __forceinline__ int wave_first_above(int m, double base, double x, Get get, double* before) {
  const int lane = threadIdx.x & 63;
  const int per = (m + 63) / 64;
  const int i0 = lane * per, i1 = min(i0 + per, m);
  double mine = 0.0;
  for (int i = i0; i < i1; ++i) mine += get(i);
  const double incl = wave_incl_scan(mine);
  double excl = __shfl_up(incl, 1);
  excl = lane == 0 ? 0.0 : excl;
  double run = base + excl;  // running sum before this lane's items
  int hit = m;
  double hit_before = 0.0;
  for (int i = i0; i < i1; ++i) {
    const double nxt = run + get(i);
    if (nxt > x) {
      hit = i;
      hit_before = run;
      break;
    }
    run = nxt;
  }
  const int first = wave_min_int(hit);
  // The lane that owns `first` holds its running sum before it.
  const int owner = first < m ? first / max(per, 1) : 0;
  *before = __shfl(hit_before, owner);
  return first;
}

__global__ __launch_bounds__(kReplayThreads) void k_replay_pick(Ring r, int n, const int* __restrict__ lane,
                                                                const double* __restrict__ u,
                                                                const int* __restrict__ start,
                                                                const int* __restrict__ count, int chunk,
                                                                int max_chunks, const double* __restrict__ csum,
                                                                const double* __restrict__ sums,
                                                                int* __restrict__ cols_out,
                                                                double* __restrict__ w_out,
                                                                int* __restrict__ lanes_out) {
  const int b = blockIdx.x * (kReplayThreads / 64) + (threadIdx.x >> 6);
  if (b >= n) return;  // uniform per wavefront
  const int l = lane[b];
  if (lanes_out && (threadIdx.x & 63) == 0) lanes_out[b] = l;
  if (l < 0 || l >= r.lanes) return;
  const int cnt = count[l], st = start[l];
  if (cnt <= 0) return;
  const int nchunks = (cnt + chunk - 1) / chunk;
  const double x = u[b] * sums[l];
  const double* cs = csum + long(l) * max_chunks;
  double base = 0.0;
  int k = wave_first_above(nchunks, 0.0, x, [&](int i) { return cs[i]; }, &base);
  int pos;
  if (k >= nchunks) {
    pos = cnt - 1;  // u * total at or past the end: the last column, as the capped searchsorted
  } else {
    const int p0 = k * chunk, m = min(chunk, cnt - p0);
    const double* w = r.weight + long(l) * r.cols;
    double dummy;
    auto get = [&](int i) {
      int c = st + p0 + i;
      c = c >= r.cols ? c - r.cols : c;
      return w[c];
    };
    const int i = wave_first_above(m, base, x, get, &dummy);
    // No crossing inside the chunk the chunk sums chose can only come from
    // the two sums rounding differently: take the chunk's last column.
    pos = i >= m ? p0 + m - 1 : p0 + i;
  }
  if ((threadIdx.x & 63) == 0) {
    int c = st + pos;
    c = c >= r.cols ? c - r.cols : c;
    cols_out[b] = c;
    w_out[b] = r.weight[long(l) * r.cols + c];
  }
}

__global__ __launch_bounds__(kReplayThreads) void k_replay_is_weights(int n, const double* __restrict__ w,
                                                                      const double* __restrict__ sums, int lanes,
                                                                      double total_count, double beta,
                                                                      float* __restrict__ out) {
  __shared__ double red[kReplayThreads];
  __shared__ double grand;
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int l = 0; l < lanes; ++l) s += sums[l];
    grand = s;
  }
  __syncthreads();
  double mx = 0.0;
  for (int b = threadIdx.x; b < n; b += kReplayThreads) mx = fmax(mx, pow(total_count * (w[b] / grand), -beta));
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int s = kReplayThreads / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  const double top = red[0];
  for (int b = threadIdx.x; b < n; b += kReplayThreads)
    out[b] = float(pow(total_count * (w[b] / grand), -beta) / top);
}

__global__ __launch_bounds__(kReplayThreads) void k_replay_assemble(
    Ring r, int n, const int* __restrict__ lane, const int* __restrict__ col, int n_step, double gamma,
    unsigned char* __restrict__ obs_out, unsigned char* __restrict__ next_out, float* __restrict__ onehot, int A,
    int* __restrict__ actions_out, float* __restrict__ action_vec_out, float* __restrict__ rewards_out,
    float* __restrict__ dones_out, float* __restrict__ discounts_out) {
  __shared__ int s_end, s_ok;
  const int b = blockIdx.x;
  if (b >= n) return;
  const int l = lane[b], c = col[b];
  if (threadIdx.x == 0) {
    // Separate multiply and add, no fused multiply-add: the float64 walk
    // rounds as the reference's numpy expression g += disc * r does.
#pragma clang fp contract(off)
    const bool ok = l >= 0 && l < r.lanes && c >= 0 && c < r.cols;
    s_ok = ok;
    if (ok) {
      const long row = long(l) * r.cols;
      double g = 0.0, disc = 1.0;
      int end_col = c, steps = 0;
      bool term = false;
      for (int k = 0; k < n_step; ++k) {
        int j = c + k;
        j = j % r.cols;
        end_col = j;
        g += disc * double(r.rewards[row + j]);
        disc *= gamma;
        ++steps;
        if (r.ends[row + j]) {
          term = r.dones[row + j] != 0;
          break;
        }
      }
      s_end = end_col;
      const int a = r.actions[row + c];
      if (actions_out) actions_out[b] = a;
      rewards_out[b] = float(g);
      dones_out[b] = term ? 1.f : 0.f;
      discounts_out[b] = float(pow(gamma, double(steps)));
      if (onehot)
        for (int i = 0; i < A; ++i) onehot[long(b) * A + i] = i == a ? 1.f : 0.f;
    }
  }
  __syncthreads();
  if (!s_ok) return;
  const long row = long(l) * r.cols;
  if (action_vec_out)
    for (int i = threadIdx.x; i < r.action_dim; i += blockDim.x)
      action_vec_out[long(b) * r.action_dim + i] = r.action_vec[(row + c) * r.action_dim + i];
  copy_row(obs_out + long(b) * r.obs_bytes, r.obs + (row + c) * r.obs_bytes, r.obs_bytes);
  const int e = s_end;
  const unsigned char* succ;
  if (r.ends[row + e]) {
    const int f = r.final_slot[row + e];
    succ = (f >= 0 && f < r.final_rows) ? r.final_obs + long(f) * r.obs_bytes : nullptr;
  } else {
    const int nxt = e + 1 == r.cols ? 0 : e + 1;
    succ = r.obs + (row + nxt) * r.obs_bytes;
  }
  if (succ) copy_row(next_out + long(b) * r.obs_bytes, succ, r.obs_bytes);
}

// The priorities arrive as float32 (TD errors an update left on the device)
// or float64 (host priorities, kept in the reference's float64).
template <typename P>
__global__ __launch_bounds__(kReplayThreads) void k_replay_priorities(Ring r, int n, const int* __restrict__ lane,
                                                                      const int* __restrict__ col,
                                                                      const P* __restrict__ prio) {
  __shared__ double red[kReplayThreads];
  double mx = 0.0;
  for (int b = threadIdx.x; b < n; b += kReplayThreads) {
    const int l = lane[b], c = col[b];
    const double p = fabs(double(prio[b]));
    mx = fmax(mx, p);
    bool last = l >= 0 && l < r.lanes && c >= 0 && c < r.cols;
    for (int d = b + 1; d < n && last; ++d) last = !(lane[d] == l && col[d] == c);
    if (last) r.weight[long(l) * r.cols + c] = pow(p + r.epsilon, r.alpha);
  }
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int s = kReplayThreads / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) *r.max_priority = fmax(*r.max_priority, red[0]);
}

int check_ring(const ttrl_replay_ring* r, const char* name) {
  TTRL_REQUIRE(r && r->obs && r->actions && r->rewards && r->dones && r->ends && r->final_slot,
               "%s: incomplete ring", name);
  TTRL_REQUIRE(r->lanes > 0 && r->cols > 0 && r->obs_bytes > 0 && r->obs_bytes % 4 == 0,
               "%s: bad ring extents (lanes %d, cols %d, obs_bytes %ld)", name, r->lanes, r->cols, r->obs_bytes);
  TTRL_REQUIRE(r->final_rows >= 0 && (r->final_rows == 0 || r->final_obs), "%s: bad boundary pool", name);
  TTRL_REQUIRE(!r->action_vec || (r->action_dim > 0 && r->action_dim <= 64), "%s: action_dim %d outside [1, 64]",
               name, r->action_dim);
  return TTRL_OK;
}

}  // namespace
}  // namespace ttrl

using namespace ttrl;

extern "C" {

int ttrl_replay_write(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const int* col,
                      const int* action, const float* action_vec, const float* reward,
                      const unsigned char* terminated, const unsigned char* ended, const int* final_row,
                      const void* obs, const void* final_obs) {
  int rc = check_ring(ring, "ttrl_replay_write");
  if (rc) return rc;
  TTRL_REQUIRE(ctx && lane && col && reward && terminated && ended && final_row && obs,
               "ttrl_replay_write: null argument");
  TTRL_REQUIRE(ring->action_vec ? (action_vec != nullptr) : (action != nullptr),
               "ttrl_replay_write: a ring with %s actions needs the %s action array",
               ring->action_vec ? "vector" : "index", ring->action_vec ? "vector" : "index");
  TTRL_REQUIRE(!ring->weight || (ring->max_priority && ring->alpha >= 0.0), "ttrl_replay_write: bad priorities");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_replay_write, dim3(unsigned(n)), dim3(kReplayThreads), 0, stream_of(ctx), ring_of(ring), n,
                     lane, col, action, action_vec, reward, terminated, ended, final_row,
                     static_cast<const unsigned char*>(obs), static_cast<const unsigned char*>(final_obs));
  return check_launch("ttrl_replay_write");
}

int ttrl_replay_lane_sums(ttrl_ctx* ctx, const ttrl_replay_ring* ring, const int* start, const int* count, int chunk,
                          int max_chunks, double* chunk_sums, double* sums) {
  int rc = check_ring(ring, "ttrl_replay_lane_sums");
  if (rc) return rc;
  TTRL_REQUIRE(ctx && ring->weight && start && count && chunk_sums && sums, "ttrl_replay_lane_sums: null argument");
  TTRL_REQUIRE(chunk > 0 && max_chunks > 0 && long(chunk) * max_chunks >= ring->cols,
               "ttrl_replay_lane_sums: %d chunks of %d do not cover %d columns", max_chunks, chunk, ring->cols);
  hipLaunchKernelGGL(k_replay_chunk_sums, dim3(unsigned(max_chunks), unsigned(ring->lanes)), dim3(kReplayThreads), 0,
                     stream_of(ctx), ring_of(ring), start, count, chunk, max_chunks, chunk_sums);
  rc = check_launch("ttrl_replay_lane_sums");
  if (rc) return rc;
  hipLaunchKernelGGL(k_replay_lane_sums, dim3(unsigned(ring->lanes)), dim3(64), 0, stream_of(ctx), ring->lanes,
                     max_chunks, chunk_sums, sums);
  return check_launch("ttrl_replay_lane_sums");
}

int ttrl_replay_priority_pick(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const double* u,
                              const int* start, const int* count, int chunk, int max_chunks,
                              const double* chunk_sums, const double* sums, int* cols_out, double* picked_weight) {
  int rc = check_ring(ring, "ttrl_replay_priority_pick");
  if (rc) return rc;
  TTRL_REQUIRE(ctx && ring->weight && lane && u && start && count && chunk_sums && sums && cols_out && picked_weight,
               "ttrl_replay_priority_pick: null argument");
  TTRL_REQUIRE(chunk > 0 && max_chunks > 0, "ttrl_replay_priority_pick: bad chunking");
  if (n <= 0) return TTRL_OK;
  const int per_block = kReplayThreads / 64;
  hipLaunchKernelGGL(k_replay_pick, dim3(unsigned((n + per_block - 1) / per_block)), dim3(kReplayThreads), 0,
                     stream_of(ctx), ring_of(ring), n, lane, u, start, count, chunk, max_chunks, chunk_sums, sums,
                     cols_out, picked_weight, static_cast<int*>(nullptr));
  return check_launch("ttrl_replay_priority_pick");
}

int ttrl_replay_is_weights(ttrl_ctx* ctx, int n, const double* picked_weight, const double* sums, int lanes,
                           long total_count, double beta, float* weights_out) {
  TTRL_REQUIRE(ctx && picked_weight && sums && weights_out, "ttrl_replay_is_weights: null argument");
  TTRL_REQUIRE(lanes > 0 && total_count > 0 && beta >= 0.0, "ttrl_replay_is_weights: bad arguments");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_replay_is_weights, dim3(1), dim3(kReplayThreads), 0, stream_of(ctx), n, picked_weight, sums,
                     lanes, double(total_count), beta, weights_out);
  return check_launch("ttrl_replay_is_weights");
}

int ttrl_replay_assemble(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const int* col,
                         int n_step, double gamma, void* obs_out, void* next_obs_out, float* actions_onehot,
                         int num_actions, int* actions_out, float* action_vec_out, float* rewards_out,
                         float* dones_out, float* discounts_out) {
  int rc = check_ring(ring, "ttrl_replay_assemble");
  if (rc) return rc;
  TTRL_REQUIRE(ctx && lane && col && obs_out && next_obs_out && rewards_out && dones_out && discounts_out,
               "ttrl_replay_assemble: null argument");
  TTRL_REQUIRE(n_step >= 1 && gamma > 0.0 && gamma <= 1.0, "ttrl_replay_assemble: bad n_step or gamma");
  TTRL_REQUIRE(!actions_onehot || num_actions > 0, "ttrl_replay_assemble: one-hot actions need num_actions");
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_replay_assemble, dim3(unsigned(n)), dim3(kReplayThreads), 0, stream_of(ctx), ring_of(ring), n,
                     lane, col, n_step, gamma, static_cast<unsigned char*>(obs_out),
                     static_cast<unsigned char*>(next_obs_out), actions_onehot, num_actions, actions_out,
                     ring->action_vec ? action_vec_out : nullptr, rewards_out, dones_out, discounts_out);
  return check_launch("ttrl_replay_assemble");
}

int ttrl_replay_draw_batch(ttrl_ctx* ctx, const ttrl_replay_ring* ring, const ttrl_replay_draw* d) {
  TTRL_REQUIRE(ctx && ring && d, "ttrl_replay_draw_batch: null argument");
  int rc = check_ring(ring, "ttrl_replay_draw_batch");
  if (rc) return rc;
  TTRL_REQUIRE(ring->weight && d->lane && d->u && d->start && d->count && d->chunk_sums && d->sums && d->cols_out &&
                   d->picked_weight && d->lanes_out,
               "ttrl_replay_draw_batch: null argument");
  TTRL_REQUIRE(d->chunk > 0 && d->max_chunks > 0, "ttrl_replay_draw_batch: bad chunking");
  if (d->n <= 0) return TTRL_OK;
  const int per_block = kReplayThreads / 64;
  hipLaunchKernelGGL(k_replay_pick, dim3(unsigned((d->n + per_block - 1) / per_block)), dim3(kReplayThreads), 0,
                     stream_of(ctx), ring_of(ring), d->n, d->lane, d->u, d->start, d->count, d->chunk, d->max_chunks,
                     d->chunk_sums, d->sums, d->cols_out, d->picked_weight, d->lanes_out);
  rc = check_launch("ttrl_replay_draw_batch");
  if (rc) return rc;
  rc = ttrl_replay_is_weights(ctx, d->n, d->picked_weight, d->sums, ring->lanes, d->total_count, d->beta,
                              d->weights_out);
  if (rc) return rc;
  return ttrl_replay_assemble(ctx, ring, d->n, d->lanes_out, d->cols_out, d->n_step, d->gamma, d->obs_out,
                              d->next_obs_out, d->actions_onehot, d->num_actions, d->actions_out, d->action_vec_out,
                              d->rewards_out, d->dones_out, d->discounts_out);
}

}  // extern "C"

namespace {

template <typename P>
int update_priorities(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const int* col,
                      const P* priorities, const char* name) {
  int rc = check_ring(ring, name);
  if (rc) return rc;
  TTRL_REQUIRE(ctx && ring->weight && ring->max_priority && lane && col && priorities, "%s: null argument", name);
  if (n <= 0) return TTRL_OK;
  hipLaunchKernelGGL(k_replay_priorities<P>, dim3(1), dim3(kReplayThreads), 0, stream_of(ctx), ring_of(ring), n,
                     lane, col, priorities);
  return check_launch(name);
}

}  // namespace

extern "C" {

int ttrl_replay_update_priorities(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane, const int* col,
                                  const float* priorities) {
  return update_priorities(ctx, ring, n, lane, col, priorities, "ttrl_replay_update_priorities");
}

int ttrl_replay_update_priorities_f64(ttrl_ctx* ctx, const ttrl_replay_ring* ring, int n, const int* lane,
                                      const int* col, const double* priorities) {
  return update_priorities(ctx, ring, n, lane, col, priorities, "ttrl_replay_update_priorities_f64");
}

}  // extern "C"
