// FP32 MFMA tile GEMM core for gfx950: C[g](m, n) = sum_k A[g](m, k) * B[g](k, n).
//
// Work decomposition.  A workgroup of WGM x WGN wavefronts (64 lanes each),
// times WGK groups along k, owns a BM x BN output tile; each wavefront owns
// a (BM/WGM) x (BN/WGN) sub-tile built from 16x16 v_mfma_f32_16x16x4f32
// fragments.  The reduction is staged through LDS in slices of TBK (up to
// 256), the next slice's global loads in flight while the current one's
// MFMAs run.  At the batch sizes of a learner update most workgroups own
// one or two slices, so a kernel's time is one workgroup's latency chain;
// the code below is arranged to keep that chain short.
//
// MFMA operand order.  Lane l of step s supplies A(row l%16, k = 4*(l/16)+s)
// and B(k = 4*(l/16)+s, col l%16): a fixed permutation of each 16-wide
// k-block shared by both operands, so the block is summed exactly once.
//
// Operands come from loader objects, so one core serves dense matrices in
// either storage order, implicit-GEMM convolution patches and the implicit
// ones row that folds a bias gradient into a weight-gradient GEMM.  A
// KCONTIG loader returns four consecutive k of one row and is staged
// row-major ([rows][TBK+4], one 128-bit LDS read feeds four MFMAs); any
// other loader returns four consecutive rows at one k and is staged k-major
// ([TBK][rows+4], 128-bit LDS stores, 32-bit reads), so neither layout takes
// bank conflicts on its stores.  Loaders bounds-check and return zeros
// outside the operand, so ragged M, N and K need no padding.  Epilogues
// apply bias, ReLU, clamp, a ReLU gate of the consuming layer's input, a
// scale and beta-accumulation as the tile is stored.
//
// blockIdx.z = group * splits + split: groups are independent problems
// (per-group pointer tables: twin critics, online/target networks,
// convolution residue classes), splits partition K.  A split-K launch writes
// partial tiles to a workspace that a second kernel sums in split order, so
// results never depend on scheduling.
#pragma once

#include "common.hpp"

#include <algorithm>
#include <cstdio>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

namespace ttrl {

constexpr int kMaxGroups = 4;

// ------------------------------------------------------------- loaders ---
//
// Operands are read with buffer loads: a 32-bit byte offset into a buffer
// resource whose range covers the operand exactly, so an offset past the
// range reads zero.  Operands are under 2^30 bytes (the host refuses larger
// ones), and an out-of-operand element (ragged M, N, K; image borders) gets
// an offset of at least kBad = 2^30: the sum of any valid offset and kBad,
// or of two kBad, stays in [2^30, 2^32), out of range, so validity folds
// into one addition instead of per-element predicates.
//
// Loads are issued in two phases so that all of a stage's loads are in
// flight before any is waited on: issue() starts loads into a Fetch4 and
// never reads a loaded value; write_tile() converts and stores to LDS.
//
// A KCONTIG loader returns four consecutive k of one row.  The kernel
// arranges that every fetch of a thread has the same k offset within the
// stage, so the loader splits its address into a per-row part (Row,
// computed once per workgroup) and a per-k part (Kp, once per stage): one
// addition per fetch.  Any other loader returns four consecutive rows at one
// k; every fetch of a thread covers the same four rows (Row), its first k
// gives a per-stage base (Ks) and fetch j sits j*NT/CH k-rows further on,
// a uniform stride.

constexpr uint32_t kBad = 0x40000000u;

// Element paths whose source buffer differs from lane to lane read through
// plain pointers (a buffer resource chosen per lane would serialise the
// wavefront); an element outside the operand reads one of these instead.
__device__ const float g_zero_one[2] = {0.f, 1.f};
constexpr long kMaxOperandBytes = 1L << 30;

// Loads through a pointer known to address global memory.  A generic
// (flat) load counts against both the vector-memory and the LDS wait
// counters and may return out of order with LDS reads, so while one is in
// flight every LDS wait must drain everything, including the next stage's
// prefetch; a global load counts against the vector-memory counter only.
typedef __attribute__((address_space(1))) const float gfloat;
__device__ __forceinline__ float gload(const float* p) { return *(gfloat*)p; }

// Materialises a wave-uniform pointer in scalar registers at this point.
// Per-group pointers are read from the argument segment once, where they
// are bound, instead of being re-read inside every divergent branch that
// uses them (one dependent scalar-cache round trip per use).
// All operands of one asm statement, so their loads share one wait.
template <class T, class U>
__device__ __forceinline__ void pin(T*& a, U*& b) {
  asm volatile("" : "+s"(a), "+s"(b));
}

// A copy of a plain struct of wave-uniform words (at most 32), every word
// materialised in scalar registers by one asm statement: the values are
// read once, together, and the compiler cannot re-read them from memory.
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
template <class T>
__device__ __forceinline__ T pin_pod(const T& src) {
  static_assert(sizeof(T) % 4 == 0 && sizeof(T) <= 128, "pin_pod: at most 32 words");
  constexpr int N = int(sizeof(T) / 4);
  uint32_t w[32] = {};
  __builtin_memcpy(w, &src, sizeof(T));
  u32x8 c0, c1, c2, c3;
  // readfirstlane: words the compiler computed on the vector unit (uniform
  // by construction) move to scalar registers.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    c0[i] = __builtin_amdgcn_readfirstlane(w[i]);
    c1[i] = __builtin_amdgcn_readfirstlane(w[8 + i]);
    c2[i] = __builtin_amdgcn_readfirstlane(w[16 + i]);
    c3[i] = __builtin_amdgcn_readfirstlane(w[24 + i]);
  }
  if constexpr (N <= 8) asm volatile("" : "+s"(c0));
  else if constexpr (N <= 16) asm volatile("" : "+s"(c0), "+s"(c1));
  else if constexpr (N <= 24) asm volatile("" : "+s"(c0), "+s"(c1), "+s"(c2));
  else asm volatile("" : "+s"(c0), "+s"(c1), "+s"(c2), "+s"(c3));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    w[i] = c0[i];
    w[8 + i] = c1[i];
    w[16 + i] = c2[i];
    w[24 + i] = c3[i];
  }
  T out;
  __builtin_memcpy(&out, w, sizeof(T));
  return out;
}
constexpr int kBufFlags = 0x00020000;  // gfx9 buffer resource word 3: raw 32-bit dwords

// The base and size are wave-uniform by construction; reading them through
// readfirstlane keeps the resource in scalar registers even where the
// compiler computed them on the vector unit (a resource in vector registers
// makes every load that uses it a loop over the lanes' distinct values).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_res(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  void* base = reinterpret_cast<void*>((uint64_t(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(base, static_cast<short>(0),
                                           static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)), kBufFlags);
}
__device__ __forceinline__ f32x4 ld_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float ld_f1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t ld_u8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return uint32_t(__builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0));
}

// Element formats a loader leaves in Fetch4::v.
enum FetchFmt { kF32 = 0, kU8Word = 1, kU8Each = 2 };

struct Fetch4 {
  f32x4 v;  // kF32: four floats; kU8Word: four bytes packed in v.x; kU8Each: one byte per element (bits)
};

__device__ __forceinline__ f32x4 resolve4(const Fetch4& f, int fmt) {
  if (fmt == kU8Word) {
    const uint32_t w = __float_as_uint(f.v.x);
    return f32x4{float(w & 0xffu), float((w >> 8) & 0xffu), float((w >> 16) & 0xffu), float(w >> 24)};
  }
  if (fmt == kU8Each)
    return f32x4{float(__float_as_uint(f.v.x)), float(__float_as_uint(f.v.y)), float(__float_as_uint(f.v.z)),
                 float(__float_as_uint(f.v.w))};
  return f.v;
}

// Each loader is a host-side description (per-group pointer tables and
// extents, passed as a kernel argument) and a device-side Live view of one
// group: the parameters its device code reads, loaded together and pinned
// in scalar registers by live(g) before any load is issued.  Reading kernel
// arguments where they are used instead makes the compiler reload them in
// every branch, each reload a scalar-cache round trip the wavefront waits on.

// v(r, k) = p[g][r*ld + k]; k contiguous.
struct LdRowK {
  const float* p[kMaxGroups] = {};
  long ld = 0;
  int rows = 0, K = 0;
  bool vec = false;  // p[g] 16-byte aligned and ld, K multiples of 4 (set by vec_ok)

  __host__ void vec_ok(bool aligned) { vec = aligned && ld % 4 == 0 && K % 4 == 0; }
  __host__ __device__ long bytes() const { return rows > 0 ? ((long(rows) - 1) * ld + K) * 4 : 0; }

  struct Params {
    const float* p;
    uint32_t bytes;
    int ld, rows, K, vec;
  };
  struct Live {
    static constexpr bool KCONTIG = true;
    Params q;
    __amdgpu_buffer_rsrc_t rs;
    struct Row { uint32_t off; };
    struct Kp { uint32_t add; int k; };
    __device__ __forceinline__ int fmt() const { return kF32; }
    __device__ __forceinline__ Row row(int r) const { return Row{r < q.rows ? uint32_t(r * q.ld) * 4u : kBad}; }
    __device__ __forceinline__ Kp kpos(int k) const { return Kp{k < q.K ? uint32_t(k) * 4u : kBad, k}; }
    __device__ __forceinline__ void issue(const Row& r, const Kp& kp, Fetch4& f) const {
      if (q.vec) {  // K % 4 == 0: k < K covers all four
        f.v = ld_f4(rs, r.off + kp.add);
        return;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) f.v[j] = ld_f1(rs, r.off + (kp.k + j < q.K ? uint32_t(kp.k + j) * 4u : kBad));
    }
  };
  __device__ __forceinline__ Live live(int g) const {
    const Params q = pin_pod(Params{p[g], uint32_t(bytes()), int(ld), rows, K, vec ? 1 : 0});
    return Live{q, make_res(q.p, q.bytes)};
  }
};

// v(r, k) = p[g][k*ld + r]; r contiguous.  Row `real_rows` reads 1.0 when
// `ones` is set (the implicit ones row of a bias gradient); rows >= `split`
// read p2[g][k*ld2 + r - split] (a second weight matrix beside the first
// along the output axis).  With ld >= the real rows, every k >= K lies past
// the resource's range, so the vector path needs no k check.
struct LdColK {
  const float* p[kMaxGroups] = {};
  const float* p2[kMaxGroups] = {};
  long ld = 0, ld2 = 0;
  int rows = 0, K = 0;
  bool vec = false;
  int real_rows = 1 << 30;
  bool ones = false;
  int split = 1 << 30;

  // Vector loads need aligned bases and ld % 4 == 0; a 4-row chunk that
  // straddles `rows`, `real_rows` or `split` takes the element path.
  __host__ void vec_ok(bool aligned) { vec = aligned && ld % 4 == 0 && ld >= real_dense(); }
  __host__ __device__ int real_dense() const {
    int rr = rows < real_rows ? rows : real_rows;
    return rr < split ? rr : split;
  }
  __host__ __device__ long bytes() const {
    const int rr = real_dense();
    return (K > 0 && rr > 0) ? ((long(K) - 1) * ld + rr) * 4 : 0;
  }
  __host__ __device__ long bytes2() const {
    return (K > 0 && rows > split) ? ((long(K) - 1) * ld2 + (rows - split)) * 4 : 0;
  }

  struct Params {
    const float* base;
    const float* base2;
    uint32_t bytes;
    int ld, ld2, rows, K, vec, real_rows, ones, split;
  };
  struct Live {
    static constexpr bool KCONTIG = false;
    Params q;
    __amdgpu_buffer_rsrc_t rs;
    // mode 0: four real rows, one vector load; 1: no row inside, zeros; 2: element by element.
    struct Row { uint32_t off; int r; int mode; };
    struct Ks { uint32_t base; int k; };
    __device__ __forceinline__ int fmt() const { return kF32; }
    __device__ __forceinline__ Row row(int r) const {
      const bool whole = q.vec && r + 3 < q.real_rows && r + 3 < q.split && r + 3 < q.rows;
      return Row{uint32_t(r) * 4u, r, whole ? 0 : (r >= q.rows ? 1 : 2)};
    }
    __device__ __forceinline__ Ks kstage(const Row& r, int k) const { return Ks{uint32_t(k * q.ld) * 4u + r.off, k}; }
    __device__ __forceinline__ void issue(const Row& r, const Ks& ks, int dk, Fetch4& f) const {
      if (r.mode == 0) {
        f.v = ld_f4(rs, ks.base + uint32_t(dk * q.ld) * 4u);
        return;
      }
      if (r.mode == 1) {
        f.v = f32x4{0.f, 0.f, 0.f, 0.f};
        return;
      }
      const int k = ks.k + dk;
      const bool kv = k < q.K;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rr = r.r + j;
        const bool in = kv && rr < q.rows;
        const float* src = &g_zero_one[0];
        if (in && rr >= q.real_rows) src = &g_zero_one[(q.ones && rr == q.real_rows) ? 1 : 0];
        else if (in && rr >= q.split) src = q.base2 + (long(k) * q.ld2 + (rr - q.split));
        else if (in) src = q.base + (long(k) * q.ld + rr);
        f.v[j] = gload(src);
      }
    }
  };
  __device__ __forceinline__ Live live(int g) const {
    const Params q = pin_pod(Params{p[g], p2[g], uint32_t(bytes()), int(ld), int(ld2), rows, K, vec ? 1 : 0,
                                    real_rows, ones ? 1 : 0, split});
    return Live{q, make_res(q.base, q.bytes)};
  }
};

// Concatenation along k of two row-major operands: k < k1 reads p1[g][r*ld1+k],
// k >= k1 reads p2[g][r*ld2 + k-k1] (the SAC critic's concat(s, a) input;
// also the transposed view of two weight matrices side by side).
struct LdRowKCat {
  const float* p1[kMaxGroups] = {};
  const float* p2[kMaxGroups] = {};
  long ld1 = 0, ld2 = 0;
  int rows = 0, k1 = 0, K = 0;

  __host__ __device__ long bytes1() const { return rows > 0 ? ((long(rows) - 1) * ld1 + k1) * 4 : 0; }
  __host__ __device__ long bytes2() const {
    return rows > 0 && K > k1 ? ((long(rows) - 1) * ld2 + (K - k1)) * 4 : 0;
  }

  struct Params {
    const float* a;
    const float* b;
    int ld1, ld2, rows, k1, K;
  };
  struct Live {
    static constexpr bool KCONTIG = true;
    Params q;
    struct Row { int r; };
    struct Kp { int k; };
    __device__ __forceinline__ int fmt() const { return kF32; }
    __device__ __forceinline__ Row row(int r) const { return Row{r}; }
    __device__ __forceinline__ Kp kpos(int k) const { return Kp{k}; }
    __device__ __forceinline__ void issue(const Row& r, const Kp& kp, Fetch4& f) const {
      const bool rv = r.r < q.rows;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kk = kp.k + j;
        const float* src = &g_zero_one[0];
        if (rv && kk < q.K)
          src = kk < q.k1 ? q.a + (long(r.r) * q.ld1 + kk) : q.b + (long(r.r) * q.ld2 + (kk - q.k1));
        f.v[j] = gload(src);
      }
    }
  };
  __device__ __forceinline__ Live live(int g) const {
    return Live{pin_pod(Params{p1[g], p2[g], int(ld1), int(ld2), rows, k1, K})};
  }
};

// ----------------------------------------------------------- epilogues ---

// Element (m, n) of group g goes to one of four row-major blocks: rows
// >= rsplit and columns >= csplit address the tail blocks with their index
// rebased to 0.  v = alpha*acc (+ bias) (relu | clamp) (* [mask > 0])
// (+ beta*old); the mask (the ReLU output of the layer whose gradient this
// is) applies to the leading block and is indexed like it.
struct EpAux {
  float* dst;  // pointer path
  float add, keep, old;
  uint32_t off;  // buffer path: byte offset, kBad for an element outside the output
};

__device__ __forceinline__ void st_f1(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
}

struct EpStore {
  int M = 0, N = 0;
  float* C[kMaxGroups] = {};    long ldc = 0;
  float* Cr[kMaxGroups] = {};                     // rows >= rsplit, ld = ldc
  float* Cc[kMaxGroups] = {};   long ldcc = 0;    // cols >= csplit
  float* Crc[kMaxGroups] = {};                    // both tails, ld = ldcc
  int rsplit = 1 << 30, csplit = 1 << 30;
  float alpha = 1.f, beta = 0.f;
  float alpha_r = 1.f;                            // scale of rows >= rsplit
  const float* bias[kMaxGroups] = {};             // cols < csplit
  const float* bias2[kMaxGroups] = {};            // cols >= csplit
  int relu = 0;
  int clamp_col = 1 << 30;                        // cols >= clamp_col clamp to [lo, hi]
  float lo = 0.f, hi = 0.f;
  const float* mask[kMaxGroups] = {};

  __device__ __forceinline__ int rows(int) const { return M; }
  // A copy that writes every element into `sink` (at least tune_span()
  // floats) and reads nothing old: timing a candidate plan must not disturb
  // the real output.
  __host__ long tune_span() const {
    const long ld = ldc > ldcc ? ldc : ldcc;
    return long(M) * (ld > 0 ? ld : N) + N + 64;
  }
  __host__ EpStore tune_copy(float* sink) const {
    EpStore e = *this;
    for (int g = 0; g < kMaxGroups; ++g) e.C[g] = e.Cr[g] = e.Cc[g] = e.Crc[g] = sink;
    e.beta = 0.f;
    return e;
  }
  // One group's epilogue, its pointers bound in scalar registers.
  // Everything element (m, n) reads besides the accumulator (its address,
  // the bias, the mask and, when beta != 0, the old value) comes from aux();
  // the kernel issues these loads for a batch of elements before it stores
  // any of them.
  // One group's epilogue, its pointers bound in scalar registers, in one
  // of two forms chosen once per workgroup.  Everything element (m, n) reads
  // besides the accumulator (the bias, the mask and, when beta != 0, the old
  // value) comes from aux(); the kernel issues these loads for a batch of
  // elements before it stores any of them.
  //
  // Fast: one output block (no row or column tail) under 2^30 bytes, read
  // and written with buffer instructions.  An out-of-range offset reads zero
  // and drops the store, so an element needs no branch, and the loads of a
  // batch are all in flight before the first store waits on them.
  // The three reads are unconditional: an absent bias, mask or old value
  // (beta == 0) has an empty resource and reads zero without a memory access.
  struct Fast {
    int M, N;
    uint32_t ldc;
    float alpha, beta;
    int relu, clamp_col;
    float lo, hi;
    bool has_mask;
    __amdgpu_buffer_rsrc_t rc, rb, rm, ro;

    __device__ __forceinline__ EpAux aux(int m, int n) const {
      EpAux x{nullptr, 0.f, 1.f, 0.f, kBad};
      x.off = (m < M && n < N) ? (uint32_t(m) * ldc + uint32_t(n)) * 4u : kBad;
      x.add = ld_f1(rb, uint32_t(n) * 4u);
      x.keep = ld_f1(rm, x.off);
      x.old = ld_f1(ro, x.off);
      return x;
    }
    __device__ __forceinline__ void store(int, int n, float acc, const EpAux& x) const {
      float v = alpha * acc + x.add;
      if (relu) v = v > 0.f ? v : 0.f;
      if (n >= clamp_col) v = fminf(fmaxf(v, lo), hi);
      if (has_mask && !(x.keep > 0.f)) v = 0.f;
      v += beta * x.old;
      st_f1(rc, x.off, v);
    }
  };
  // General: row and column tails in separate blocks, through pointers.
  struct Split {
    int M, N;
    float* C;
    float* Cr;
    float* Cc;
    float* Crc;
    long ldc, ldcc;
    int rsplit, csplit;
    float alpha, beta, alpha_r;
    const float* bias;
    const float* bias2;
    int relu, clamp_col;
    float lo, hi;
    const float* mask;

    __device__ __forceinline__ EpAux aux(int m, int n) const {
      EpAux x{nullptr, 0.f, 1.f, 0.f, kBad};
      if (m >= M || n >= N) return x;
      const bool rt = m >= rsplit, ct = n >= csplit;
      const int mm = rt ? m - rsplit : m;
      const int nn = ct ? n - csplit : n;
      if (!ct && bias) x.add = gload(bias + nn);
      if (ct && bias2) x.add = gload(bias2 + nn);
      if (!rt && !ct && mask) x.keep = gload(mask + (long(mm) * ldc + nn));
      // Two two-way selects; the opaque step keeps the compiler from
      // turning a four-way choice into a table in scratch memory.
      float* lead = rt ? Cr : C;
      float* tail = rt ? Crc : Cc;
      asm("" : "+v"(lead), "+v"(tail));
      x.dst = (ct ? tail : lead) + (long(mm) * (ct ? ldcc : ldc) + nn);
      if (beta != 0.f) x.old = gload(x.dst);
      return x;
    }
    __device__ __forceinline__ void store(int m, int n, float acc, const EpAux& x) const {
      if (!x.dst) return;
      float v = (m >= rsplit ? alpha_r : alpha) * acc + x.add;
      if (relu) v = v > 0.f ? v : 0.f;
      if (n >= clamp_col) v = fminf(fmaxf(v, lo), hi);
      if (!(x.keep > 0.f)) v = 0.f;
      if (beta != 0.f) v += beta * x.old;
      *x.dst = v;
    }
  };
  // Calls f with group g's bound epilogue (its parameters pinned, as for
  // the loaders).
  struct Params {
    float* c0;
    float* c1;
    float* c2;
    float* c3;
    const float* b0;
    const float* b1;
    const float* mk;
    int M, N, ldc, ldcc, rsplit, csplit;
    float alpha, beta, alpha_r;
    int relu, clamp_col;
    float lo, hi;
  };
  template <class F>
  __device__ __forceinline__ void with_bound(int g, F&& f) const {
    const Params q = pin_pod(Params{C[g], Cr[g], Cc[g], Crc[g], bias[g], bias2[g], mask[g], M, N, int(ldc), int(ldcc),
                                    rsplit, csplit, alpha, beta, alpha_r, relu, clamp_col, lo, hi});
    const long cb = q.M > 0 ? (long(q.M - 1) * q.ldc + q.N) * 4 : 0;
    if (q.rsplit >= q.M && q.csplit >= q.N && cb < kMaxOperandBytes) {
      const uint32_t cbytes = uint32_t(cb);
      f(Fast{q.M, q.N, uint32_t(q.ldc), q.alpha, q.beta, q.relu, q.clamp_col, q.lo, q.hi, q.mk != nullptr,
             make_res(q.c0, cbytes), make_res(q.b0, q.b0 ? uint32_t(q.N) * 4u : 0u),
             make_res(q.mk, q.mk ? cbytes : 0u), make_res(q.c0, q.beta != 0.f ? cbytes : 0u)});
    } else {
      f(Split{q.M, q.N, q.c0, q.c1, q.c2, q.c3, q.ldc, q.ldcc, q.rsplit, q.csplit, q.alpha, q.beta, q.alpha_r, q.b0,
              q.b1, q.relu, q.clamp_col, q.lo, q.hi, q.mk});
    }
  }
};

// ----------------------------------------------------------- the core ----

// LDS footprint of one staged operand, in floats.
template <int ROWS, int TBK, bool KCONTIG>
struct TileLds {
  static constexpr int LD = KCONTIG ? TBK + 4 : ROWS + 4;  // padded leading dimension
  static constexpr int SIZE = KCONTIG ? ROWS * LD : TBK * LD;
};

// One operand stage: CH float4 chunks per LDS row, PER chunks per thread.
// Chunk i = tid + j*NT of a thread sits at LDS row i / CH, column i % CH;
// NT % CH == 0, so the column is tid % CH for every j.
template <int ROWS, int TBK, int NT, class L>
struct Stage {
  static constexpr int CH = L::KCONTIG ? TBK / 4 : ROWS / 4;
  static constexpr int TOTAL = (L::KCONTIG ? ROWS : TBK) * CH;
  static constexpr int PER = (TOTAL + NT - 1) / NT;
  static_assert(NT % CH == 0, "a thread's chunks must share one column");
  __device__ static constexpr bool live(int j, int tid) { return TOTAL % NT == 0 || tid + j * NT < TOTAL; }
};

// The per-workgroup part of a thread's fetch addresses: one Row per fetch
// for a KCONTIG loader (its rows differ), one shared Row otherwise.
template <class L, int PER, bool KC = L::KCONTIG>
struct Cursor;
template <class L, int PER>
struct Cursor<L, PER, true> {
  typename L::Row r[PER];
};
template <class L, int PER>
struct Cursor<L, PER, false> {
  typename L::Row r;
};

template <int ROWS, int TBK, int NT, class L, int PER>
__device__ __forceinline__ void make_cursor(Cursor<L, PER>& c, const L& ld, int r0, int tid) {
  using S = Stage<ROWS, TBK, NT, L>;
  if constexpr (L::KCONTIG) {
#pragma unroll
    for (int j = 0; j < PER; ++j) c.r[j] = ld.row(r0 + (tid + j * NT) / S::CH);
  } else {
    c.r = ld.row(r0 + (tid % S::CH) * 4);
  }
}

// Starts every load of one operand stage (no value is read here).
template <int ROWS, int TBK, int NT, class L, int PER>
__device__ __forceinline__ void issue_tile(Fetch4 (&f)[PER], const L& ld, const Cursor<L, PER>& c, int k0, int tid) {
  using S = Stage<ROWS, TBK, NT, L>;
  if constexpr (L::KCONTIG) {
    const auto kp = ld.kpos(k0 + (tid % S::CH) * 4);
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (S::live(j, tid)) ld.issue(c.r[j], kp, f[j]);
  } else {
    constexpr int KSTEP = NT / S::CH;  // k-rows between a thread's consecutive fetches
    const auto ks = ld.kstage(c.r, k0 + tid / S::CH);
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (S::live(j, tid)) ld.issue(c.r, ks, j * KSTEP, f[j]);
  }
}

// Converts the fetched values and writes them to the LDS tile.
template <int ROWS, int TBK, int NT, class L, int PER>
__device__ __forceinline__ void write_tile(float* T, const Fetch4 (&f)[PER], int fmt, int tid) {
  using S = Stage<ROWS, TBK, NT, L>;
  using Lds = TileLds<ROWS, TBK, L::KCONTIG>;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = tid + j * NT;
    if (S::live(j, tid)) {
      const int a = i / S::CH, b = (i - a * S::CH) * 4;
      *reinterpret_cast<f32x4*>(T + a * Lds::LD + b) = resolve4(f[j], fmt);
    }
  }
}

// Four consecutive-k operand values of tile row `row` at k-offset kk.
template <int ROWS, int TBK, bool KCONTIG>
__device__ __forceinline__ f32x4 lds_frag(const float* T, int row, int kk) {
  using Lds = TileLds<ROWS, TBK, KCONTIG>;
  if constexpr (KCONTIG) {
    return *reinterpret_cast<const f32x4*>(T + row * Lds::LD + kk);
  } else {
    return f32x4{T[(kk + 0) * Lds::LD + row], T[(kk + 1) * Lds::LD + row], T[(kk + 2) * Lds::LD + row],
                 T[(kk + 3) * Lds::LD + row]};
  }
}

// Fragments of one 16-wide k-block: rows ra + 16 i of A, rb + 16 j of B.
template <int BM, int BN, int TBK, bool KCA, bool KCB, int FM, int FN>
__device__ __forceinline__ void load_frags(f32x4 (&a)[FM], f32x4 (&b)[FN], const float* As, const float* Bs, int ra, int rb,
                                  int kk) {
#pragma unroll
  for (int i = 0; i < FM; ++i) a[i] = lds_frag<BM, TBK, KCA>(As, ra + i * 16, kk);
#pragma unroll
  for (int j = 0; j < FN; ++j) b[j] = lds_frag<BN, TBK, KCB>(Bs, rb + j * 16, kk);
}

template <int FM, int FN>
__device__ __forceinline__ void mma_block(f32x4 (&acc)[FM][FN], const f32x4 (&a)[FM], const f32x4 (&b)[FN]) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
    }
}

// The MFMAs of one full LDS stage.  The fragments of k-block q+1 are read
// while the MFMAs of block q run (two register sets, fully unrolled), so a
// wavefront waits on LDS latency once per stage rather than once per block;
// with one wavefront per SIMD nothing else would hide it.
template <int BM, int BN, int TBK, int WGK, bool KCA, bool KCB, int FM, int FN>
__device__ __forceinline__ void mma_stage_full(f32x4 (&acc)[FM][FN], const float* As, const float* Bs, int ra, int rb, int wk,
                                      int lk) {
  constexpr int NKB = TBK / (16 * WGK);
  static_assert(NKB >= 1 && TBK % (16 * WGK) == 0, "a stage must split evenly over the k-groups");
  f32x4 a0[FM], b0[FN], a1[FM], b1[FN];
  load_frags<BM, BN, TBK, KCA, KCB>(a0, b0, As, Bs, ra, rb, wk * 16 + lk);
#pragma unroll
  for (int q = 0; q < NKB; q += 2) {
    if (q + 1 < NKB) load_frags<BM, BN, TBK, KCA, KCB>(a1, b1, As, Bs, ra, rb, (wk + (q + 1) * WGK) * 16 + lk);
    __builtin_amdgcn_sched_barrier(0);  // keep the reads of block q+1 ahead of the MFMAs of block q
    mma_block(acc, a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    if (q + 1 < NKB) {
      if (q + 2 < NKB) load_frags<BM, BN, TBK, KCA, KCB>(a0, b0, As, Bs, ra, rb, (wk + (q + 2) * WGK) * 16 + lk);
      __builtin_amdgcn_sched_barrier(0);
      mma_block(acc, a1, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// The last, partial stage (kspan < TBK; the tile is zero past kspan): the
// same one-block-ahead reads in a loop.
template <int BM, int BN, int TBK, int WGK, bool KCA, bool KCB, int FM, int FN>
__device__ __forceinline__ void mma_stage_part(f32x4 (&acc)[FM][FN], const float* As, const float* Bs, int ra, int rb, int wk,
                                      int lk, int kspan) {
  int kb = wk * 16;
  if (kb >= kspan) return;
  f32x4 a0[FM], b0[FN], a1[FM], b1[FN];
  load_frags<BM, BN, TBK, KCA, KCB>(a0, b0, As, Bs, ra, rb, kb + lk);
  for (;;) {
    const int nk = kb + 16 * WGK;
    const bool more = nk < kspan;
    if (more) load_frags<BM, BN, TBK, KCA, KCB>(a1, b1, As, Bs, ra, rb, nk + lk);
    __builtin_amdgcn_sched_barrier(0);
    mma_block(acc, a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    if (!more) break;
#pragma unroll
    for (int i = 0; i < FM; ++i) a0[i] = a1[i];
#pragma unroll
    for (int j = 0; j < FN; ++j) b0[j] = b1[j];
    kb = nk;
  }
}

// Software pipeline over LDS stages: the loads of stage s+1 are issued into
// registers before the MFMAs of stage s run, so global-memory latency is
// paid once per workgroup rather than once per stage; both operands' loads
// of a stage are in flight together.
// WGK > 1 splits each LDS stage's k-blocks over WGK groups of wavefronts
// (interleaved, k-block b to group b % WGK); their partial accumulators are
// summed through LDS in group order before the epilogue, so a workgroup's
// MFMA chain, fetch count per thread and LDS traffic per wavefront shrink by
// WGK at the same tile size.
// LDS floats of one tile shape's A and B stages.
template <int BM, int BN, int TBK, class LA, class LB>
struct TileShared {
  static constexpr int A = TileLds<BM, TBK, LA::Live::KCONTIG>::SIZE;
  static constexpr int B = TileLds<BN, TBK, LB::Live::KCONTIG>::SIZE;
  static constexpr int SIZE = A + B;
};

// One workgroup's output tile (bx, by) of problem bz = group * splits +
// split, its stages in As and Bs.
template <int BM, int BN, int WGM, int WGN, int WGK, int TBK, class LA, class LB, class EP>
__device__ __forceinline__ void gemm_tile(const LA& la, const LB& lb, const EP& ep, float* ws, int M, int N, int K,
                                          int kchunk, int splits, int bx, int by, int bz, float* As, float* Bs) {
  constexpr int NT = 64 * WGM * WGN * WGK;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int FM = WTM / 16, FN = WTN / 16;
  static_assert(FM >= 1 && FN >= 1 && WTM % 16 == 0 && WTN % 16 == 0, "bad tile");
  static_assert(TBK % 16 == 0, "TBK must be a multiple of 16");
  using VA = typename LA::Live;
  using VB = typename LB::Live;
  using LdsA = TileLds<BM, TBK, VA::KCONTIG>;
  using LdsB = TileLds<BN, TBK, VB::KCONTIG>;
  constexpr int PA = Stage<BM, TBK, NT, VA>::PER;
  constexpr int PB = Stage<BN, TBK, NT, VB>::PER;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wk = wave / (WGM * WGN), wmn = wave - wk * (WGM * WGN);
  const int wm = wmn % WGM, wn = wmn / WGM;
  const int g = bz / splits, split = bz - g * splits;
  const int m0 = bx * BM, n0 = by * BN;
  if (m0 >= ep.rows(g)) return;  // uniform per block: ragged residue classes
  const int kbeg = split * kchunk;
  const int kend = min(K, kbeg + kchunk);

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const VA va = la.live(g);
  const VB vb = lb.live(g);
  Cursor<VA, PA> ca;
  Cursor<VB, PB> cb;
  make_cursor<BM, TBK, NT>(ca, va, m0, tid);
  make_cursor<BN, TBK, NT>(cb, vb, n0, tid);
  const int fa_fmt = va.fmt(), fb_fmt = vb.fmt();

  Fetch4 fa[PA], fb[PB];
  issue_tile<BM, TBK, NT>(fa, va, ca, kbeg, tid);
  issue_tile<BN, TBK, NT>(fb, vb, cb, kbeg, tid);

  const int lr = lane & 15, lk = (lane >> 4) * 4;
  for (int k0 = kbeg; k0 < kend; k0 += TBK) {
    if (k0 != kbeg) __syncthreads();  // the previous stage's LDS reads are done
    write_tile<BM, TBK, NT, VA>(As, fa, fa_fmt, tid);
    write_tile<BN, TBK, NT, VB>(Bs, fb, fb_fmt, tid);
    __syncthreads();
    if (k0 + TBK < kend) {
      issue_tile<BM, TBK, NT>(fa, va, ca, k0 + TBK, tid);
      issue_tile<BN, TBK, NT>(fb, vb, cb, k0 + TBK, tid);
    }
    const int kspan = min(TBK, kend - k0);  // zero padded past K
    if (kspan == TBK)
      mma_stage_full<BM, BN, TBK, WGK, VA::KCONTIG, VB::KCONTIG>(acc, As, Bs, wm * WTM + lr, wn * WTN + lr, wk, lk);
    else
      mma_stage_part<BM, BN, TBK, WGK, VA::KCONTIG, VB::KCONTIG>(acc, As, Bs, wm * WTM + lr, wn * WTN + lr, wk, lk,
                                                                  kspan);
  }

  // Fragment (i, j) register r holds C(row 4*(lane/16) + r, col lane%16).
  if constexpr (WGK > 1) {
    static_assert((WGK - 1) * BM * BN <= LdsA::SIZE, "k-group reduction must fit in the A tile");
    float* red = As;
    __syncthreads();  // every wavefront is done reading the tiles
    if (wk > 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = wm * WTM + i * 16 + (lane >> 4) * 4 + r, col = wn * WTN + j * 16 + lr;
            red[((wk - 1) * BM + row) * BN + col] = acc[i][j][r];
          }
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int q = 0; q < WGK - 1; ++q)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = wm * WTM + i * 16 + (lane >> 4) * 4 + r, col = wn * WTN + j * 16 + lr;
            acc[i][j][r] += red[(q * BM + row) * BN + col];
          }
  }
  // Each row of fragments first issues every load its elements need
  // (bias, mask, old value), then stores.
  if (splits > 1) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int mb = m0 + wm * WTM + i * 16 + (lane >> 4) * 4;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = mb + r, n = n0 + wn * WTN + j * 16 + lr;
          if (m < M && n < N) ws[((long(g) * splits + split) * M + m) * N + n] = acc[i][j][r];
        }
    }
    return;
  }
  ep.with_bound(g, [&](const auto& eb) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int mb = m0 + wm * WTM + i * 16 + (lane >> 4) * 4;
      EpAux x[FN][4];
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) x[j][r] = eb.aux(mb + r, n0 + wn * WTN + j * 16 + lr);
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) eb.store(mb + r, n0 + wn * WTN + j * 16 + lr, acc[i][j][r], x[j][r]);
    }
  });
}

template <int BM, int BN, int WGM, int WGN, int WGK, int TBK, class LA, class LB, class EP>
__global__ __launch_bounds__(64 * WGM * WGN * WGK) void k_gemm(LA la, LB lb, EP ep, float* ws, int M, int N, int K,
                                                               int kchunk, int splits) {
  using S = TileShared<BM, BN, TBK, LA, LB>;
  __shared__ __attribute__((aligned(16))) float lds[S::SIZE];
  warm_kernargs<int(sizeof(LA) + sizeof(LB) + sizeof(EP) + sizeof(float*) + 5 * sizeof(int))>();
  gemm_tile<BM, BN, WGM, WGN, WGK, TBK>(la, lb, ep, ws, M, N, K, kchunk, splits, blockIdx.x, blockIdx.y, blockIdx.z,
                                        lds, lds + S::A);
}

// Extents and grid of one problem of a paired launch.
struct PairDims {
  int M, N, K, kchunk, splits, gx, gy, blocks;
};

// Two independent GEMMs of one tile shape in one launch (a layer's weight
// and input gradients): workgroups [0, d1.blocks) run the first, the rest
// the second, so the two fill the device together instead of one after the
// other.  LDS is the larger of the two problems' stages.  Each problem's
// split-K partials go to its own buffer (ws1, ws2).  The two share the tile
// and the wavefront layout; their LDS stage depths (TBK1, TBK2) may differ,
// so a short reduction (a weight gradient over a batch of 32) and a long
// one (the input gradient through a wide layer) each get a stage to fit.
template <int BM, int BN, int WGM, int WGN, int WGK, int TBK1, int TBK2, class LA1, class LB1, class EP1, class LA2,
          class LB2, class EP2>
__global__ __launch_bounds__(64 * WGM * WGN * WGK) void k_gemm_pair(LA1 la1, LB1 lb1, EP1 ep1, LA2 la2, LB2 lb2,
                                                                    EP2 ep2, float* ws1, float* ws2, PairDims d1,
                                                                    PairDims d2) {
  using S1 = TileShared<BM, BN, TBK1, LA1, LB1>;
  using S2 = TileShared<BM, BN, TBK2, LA2, LB2>;
  constexpr int SIZE = S1::SIZE > S2::SIZE ? S1::SIZE : S2::SIZE;
  __shared__ __attribute__((aligned(16))) float lds[SIZE];
  warm_kernargs<int(sizeof(LA1) + sizeof(LB1) + sizeof(EP1) + sizeof(LA2) + sizeof(LB2) + sizeof(EP2) +
                    2 * sizeof(float*) + 2 * sizeof(PairDims))>();
  int b = blockIdx.x;
  if (b < d1.blocks) {
    const int bx = b % d1.gx, byz = b / d1.gx;
    gemm_tile<BM, BN, WGM, WGN, WGK, TBK1>(la1, lb1, ep1, ws1, d1.M, d1.N, d1.K, d1.kchunk, d1.splits, bx,
                                          byz % d1.gy, byz / d1.gy, lds, lds + S1::A);
  } else {
    b -= d1.blocks;
    const int bx = b % d2.gx, byz = b / d2.gx;
    gemm_tile<BM, BN, WGM, WGN, WGK, TBK2>(la2, lb2, ep2, ws2, d2.M, d2.N, d2.K, d2.kchunk, d2.splits, bx,
                                          byz % d2.gy, byz / d2.gy, lds, lds + S2::A);
  }
}

// Sums split-K partials in split order and applies the epilogue; group
// blockIdx.y.  Up to 32 partials are loaded before any is added (indices
// past the last split re-read it and are not added), so a split list of up
// to 32 costs one memory round trip.
template <class EP>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* ws, EP ep, int M, int N, int splits, FDiv dn) {
  constexpr int RB = 32;
  const int g = blockIdx.y;
  const int MN = M * N;
  const int rows = ep.rows(g);
  const float* wg = ws + long(g) * splits * MN;
  ep.with_bound(g, [&](const auto& eb) {
    for (int mn = blockIdx.x * 256 + threadIdx.x; mn < MN; mn += gridDim.x * 256) {
      const int m = dn.div(mn), n = mn - m * N;
      if (m >= rows) continue;
      const float* p = wg + mn;
      float s = 0.f;
      for (int sp = 0; sp < splits; sp += RB) {
        float v[RB];
#pragma unroll
        for (int j = 0; j < RB; ++j) v[j] = gload(p + long(min(sp + j, splits - 1)) * MN);
#pragma unroll
        for (int j = 0; j < RB; ++j)
          if (sp + j < splits) s += v[j];
      }
      eb.store(m, n, s, eb.aux(m, n));
    }
  });
}

// Tile shapes: BM x BN output tile, TBK reduction slice per LDS stage.
// K2 / K4: the same tile with 2 or 4 wavefront groups along k (8 or 16 wavefronts).
// S: a 32-deep stage for small K (the batch dimension of a weight gradient):
// a deeper stage would fetch and store zeros past K.
enum TileCfg {
  T32x32 = 0, T64x32 = 1, T32x64 = 2, T64x64 = 3, T128x32 = 4, T128x64 = 5, T64x128 = 6,
  T32x32K2 = 7, T32x32K4 = 8, T64x32K2 = 9, T32x64K2 = 10, T64x64K2 = 11,
  T32x32S = 12, T64x64S = 13, T128x64S = 14, kNumCfg = 15
};

struct TileDims {
  int bm, bn, tbk, wgm, wgn, wgk;
};

inline TileDims tile_dims(int cfg) {
  switch (cfg) {
    case T32x32: return {32, 32, 256, 2, 2, 1};
    case T64x32: return {64, 32, 128, 2, 2, 1};
    case T32x64: return {32, 64, 128, 2, 2, 1};
    case T64x64: return {64, 64, 128, 2, 2, 1};
    case T128x32: return {128, 32, 128, 4, 1, 1};
    case T128x64: return {128, 64, 64, 2, 2, 1};
    case T64x128: return {64, 128, 64, 2, 2, 1};
    case T32x32K2: return {32, 32, 256, 2, 2, 2};
    case T32x32K4: return {32, 32, 256, 2, 2, 4};
    case T64x32K2: return {64, 32, 128, 2, 2, 2};
    case T32x64K2: return {32, 64, 128, 2, 2, 2};
    case T32x32S: return {32, 32, 32, 2, 2, 1};
    case T64x64S: return {64, 64, 32, 2, 2, 1};
    case T128x64S: return {128, 64, 32, 2, 2, 1};
    default: return {64, 64, 128, 2, 2, 2};
  }
}

struct GemmPlan {
  int cfg, bm, bn, tbk, splits, kchunk;
};

// Chooses a tile among `allowed` (bit per TileCfg) and a split-K factor
// that minimise a cycle estimate, each split a whole number of LDS stages,
// within `ws_floats` of workspace.
GemmPlan plan_gemm(int M, int N, int K, int groups, long ws_floats, unsigned allowed);

// Workspace owned by the context (stream-ordered scratch for split-K).
float* ctx_workspace(ttrl_ctx* ctx, long* floats);

// dZ = src * [mask > 0] for `groups` blocks of n elements (element stride gs
// between blocks), written densely to the top of the context workspace
// (block g at offset g*n).  Adds the floats it occupies to *reserved, which
// the caller passes on to run_gemm; *rc receives the status.
const float* relu_mask_into_workspace(ttrl_ctx* ctx, const float* src, const float* mask, long n, long gs,
                                      int groups, long* reserved, int* rc);

template <int BM, int BN, int WGM, int WGN, int WGK, int TBK, class LA, class LB, class EP>
inline void launch_cfg(const LA& la, const LB& lb, const EP& ep, float* ws, int M, int N, int K, int groups,
                       const GemmPlan& p, hipStream_t st) {
  dim3 grid(ceil_div(M, BM), ceil_div(N, BN), unsigned(groups * p.splits));
  hipLaunchKernelGGL((k_gemm<BM, BN, WGM, WGN, WGK, TBK, LA, LB, EP>), grid, dim3(64 * WGM * WGN * WGK), 0, st, la,
                     lb, ep, ws, M, N, K, p.kchunk, p.splits);
  if (p.splits > 1) {
    unsigned blocks = unsigned(long(M) * N / 256 + 1);
    if (blocks > 2048) blocks = 2048;
    FDiv dn;
    dn.set(N);
    hipLaunchKernelGGL((k_splitk_reduce<EP>), dim3(blocks, unsigned(groups)), dim3(256), 0, st, ws, ep, M, N,
                       p.splits, dn);
  }
}

constexpr unsigned cfg_bit(int c) { return 1u << c; }
constexpr unsigned kCfgAll = (1u << kNumCfg) - 1;

// Plan cache and tuning resources of the context (runtime.hip).
bool ctx_capturing(ttrl_ctx* ctx);
const GemmPlan* ctx_plan_find(ttrl_ctx* ctx, const std::string& key);
void ctx_plan_store(ttrl_ctx* ctx, const std::string& key, const GemmPlan& p);
float* ctx_tune_sink(ttrl_ctx* ctx, size_t bytes);
bool ctx_tune_events(ttrl_ctx* ctx, hipEvent_t* a, hipEvent_t* b);
std::vector<GemmPlan> plan_candidates(int M, int N, int K, int groups, long ws_floats, unsigned allowed, int max_n);
// Tile shape `cfg` with K split `splits` ways (fewer if K has fewer LDS
// stages); false if the partials would not fit in `ws_floats`.
bool plan_with_splits(int cfg, int M, int N, int K, int groups, long ws_floats, int splits, GemmPlan* out);
// True when `p` is a plan of an allowed tile shape whose splits exactly cover
// K and whose partials fit `ws_floats`: checked on every plan taken from the
// context's table, which may have been imported from a file.
bool plan_valid(const GemmPlan& p, int M, int N, int K, int groups, long ws_floats, unsigned allowed);
bool gemm_tuning_enabled();
bool gemm_tuning_log();  // TTRL_GEMM_TUNE_LOG=1: print each tuned signature's candidates to stderr
// TTRL_GEMM_FORCE="cfg[:splits]" (read on every call, for tests): run that
// tile shape wherever a call site allows it, bypassing the plan cache.
bool gemm_forced(unsigned allowed, int M, int N, int K, int groups, long ws_floats, GemmPlan* out);

template <int ID_, int BM_, int BN_, int WGM_, int WGN_, int WGK_, int TBK_>
struct CfgTag {
  static constexpr int ID = ID_, BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, WGK = WGK_, TBK = TBK_;
};

// The tile shape with the same tile and wavefront layout and another LDS
// stage depth (a pair may run its two problems at different depths), or -1.
constexpr int twin_cfg(int c) {
  return c == T32x32 ? T32x32S : c == T32x32S ? T32x32 : c == T64x64 ? T64x64S : c == T64x64S ? T64x64
       : c == T128x64 ? T128x64S : c == T128x64S ? T128x64 : -1;
}
// True when a pair may run its problems with tile shapes c1 and c2.
constexpr bool pair_cfgs_ok(int c1, int c2) { return c1 == c2 || twin_cfg(c1) == c2; }

// Calls f(CfgTag<...>{}) for tile shape `cfg` if ALLOWED instantiates it.
template <unsigned ALLOWED, class F>
inline void dispatch_cfg(int cfg, F&& f) {
#define TTRL_CFG(C, BM, BN, WGM, WGN, WGK, TBK)                                            \
  case C:                                                                                 \
    if constexpr ((ALLOWED & cfg_bit(C)) != 0) f(CfgTag<C, BM, BN, WGM, WGN, WGK, TBK>{}); \
    break;
  switch (cfg) {
    TTRL_CFG(T32x32, 32, 32, 2, 2, 1, 256)
    TTRL_CFG(T64x32, 64, 32, 2, 2, 1, 128)
    TTRL_CFG(T32x64, 32, 64, 2, 2, 1, 128)
    TTRL_CFG(T64x64, 64, 64, 2, 2, 1, 128)
    TTRL_CFG(T128x32, 128, 32, 4, 1, 1, 128)
    TTRL_CFG(T128x64, 128, 64, 2, 2, 1, 64)
    TTRL_CFG(T64x128, 64, 128, 2, 2, 1, 64)
    TTRL_CFG(T32x32K2, 32, 32, 2, 2, 2, 256)
    TTRL_CFG(T32x32K4, 32, 32, 2, 2, 4, 256)
    TTRL_CFG(T64x32K2, 64, 32, 2, 2, 2, 128)
    TTRL_CFG(T32x64K2, 32, 64, 2, 2, 2, 128)
    TTRL_CFG(T64x64K2, 64, 64, 2, 2, 2, 128)
    TTRL_CFG(T32x32S, 32, 32, 2, 2, 1, 32)
    TTRL_CFG(T64x64S, 64, 64, 2, 2, 1, 32)
    TTRL_CFG(T128x64S, 128, 64, 2, 2, 1, 32)
    default: break;
  }
#undef TTRL_CFG
}

template <unsigned ALLOWED, class LA, class LB, class EP>
inline void launch_allowed(const LA& la, const LB& lb, const EP& ep, float* ws, int M, int N, int K, int groups,
                           const GemmPlan& p, hipStream_t st) {
  dispatch_cfg<ALLOWED>(p.cfg, [&](auto c) {
    using C = decltype(c);
    launch_cfg<C::BM, C::BN, C::WGM, C::WGN, C::WGK, C::TBK>(la, lb, ep, ws, M, N, K, groups, p, st);
  });
}

// A split-K plan's reduce is one more launch, which back-to-back timing
// outside a graph prices below what a node of a replayed graph costs; the
// tuners charge it this much per run, so a split must win by more.
constexpr float kReduceLaunchMs = 1.0e-3f;

// Best of three rounds of three back-to-back runs of `run` (milliseconds
// for three runs), -1 if an event call fails.  The minimum over rounds
// discards rounds slowed by clock ramps or other work on the device.
template <class F>
inline float time_best_of(hipEvent_t e0, hipEvent_t e1, hipStream_t st, F&& run) {
  float best = -1.f;
  for (int round = 0; round < 3; ++round) {
    if (hipEventRecord(e0, st) != hipSuccess) return -1.f;
    for (int r = 0; r < 3; ++r) run();
    float ms = 0.f;
    if (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
      return -1.f;
    if (best < 0.f || ms < best) best = ms;
  }
  return best;
}

// k_gemm alone: with a split plan the partial tiles stay in the workspace.
template <unsigned ALLOWED, class LA, class LB, class EP>
inline void launch_gemm_only(const LA& la, const LB& lb, const EP& ep, float* ws, int M, int N, int K, int groups,
                             const GemmPlan& p, hipStream_t st) {
  dispatch_cfg<ALLOWED>(p.cfg, [&](auto c) {
    using C = decltype(c);
    dim3 grid(ceil_div(M, C::BM), ceil_div(N, C::BN), unsigned(groups * p.splits));
    hipLaunchKernelGGL((k_gemm<C::BM, C::BN, C::WGM, C::WGN, C::WGK, C::TBK, LA, LB, EP>), grid,
                       dim3(64 * C::WGM * C::WGN * C::WGK), 0, st, la, lb, ep, ws, M, N, K, p.kchunk, p.splits);
  });
}

// Times the model's leading candidates on the real operands, writing into a
// sink instead of the output; returns the fastest (the model's first choice
// if timing is unavailable).  `reduce` false times k_gemm alone, for a
// consumer that sums the split partials itself.
template <unsigned ALLOWED, class LA, class LB, class EP>
inline GemmPlan tune_gemm(ttrl_ctx* ctx, const LA& la, const LB& lb, const EP& ep, float* ws, long ws_limit, int M,
                          int N, int K, int groups, hipStream_t st, bool reduce = true) {
  const std::vector<GemmPlan> cands = plan_candidates(M, N, K, groups, ws_limit, ALLOWED, 10);
  hipEvent_t e0, e1;
  float* sink = ctx_tune_sink(ctx, size_t(ep.tune_span()) * sizeof(float));
  if (cands.empty() || !sink || !ctx_tune_events(ctx, &e0, &e1)) return plan_gemm(M, N, K, groups, ws_limit, ALLOWED);
  const EP tep = ep.tune_copy(sink);
  GemmPlan best = cands.front();
  float best_ms = 1e30f;
  for (const GemmPlan& c : cands) {
    auto run = [&] {
      if (reduce)
        launch_allowed<ALLOWED>(la, lb, tep, ws, M, N, K, groups, c, st);
      else
        launch_gemm_only<ALLOWED>(la, lb, tep, ws, M, N, K, groups, c, st);
    };
    run();  // warm
    const float ms = time_best_of(e0, e1, st, run);
    if (ms < 0.f) break;
    if (gemm_tuning_log())
      fprintf(stderr, "[ttrl gemm tune] M=%d N=%d K=%d G=%d  %dx%d tbk%d splits=%d  %.2f us\n", M, N, K, groups, c.bm,
              c.bn, c.tbk, c.splits, ms * 1e3f / 3.f);
    const float cost = ms + (reduce && c.splits > 1 ? 3.f * kReduceLaunchMs : 0.f);
    if (cost < best_ms) {
      best_ms = cost;
      best = c;
    }
  }
  (void)hipGetLastError();
  return best;
}

// Plans and launches one GEMM.  ALLOWED restricts the tile shapes a call
// site instantiates (each is a separate kernel); `ws_reserved` floats at the
// top of the context workspace are in use by the caller.  The first call of
// a signature (kernel types and extents) outside graph capture times the
// model's leading candidates and keeps the fastest for the context; a call
// during capture uses the kept plan, or the model's, and keeps that.  Every
// later call of the signature in the context runs the same plan, so eager
// runs and graph replays sum split-K partials in the same order.
template <unsigned ALLOWED, class LA, class LB, class EP>
inline int run_gemm(ttrl_ctx* ctx, const LA& la, const LB& lb, const EP& ep, int M, int N, int K, int groups,
                    const char* name, long ws_reserved = 0) {
  static_assert((ALLOWED & kCfgAll) != 0, "no tile shape allowed");
  if (M <= 0 || N <= 0 || groups <= 0) return TTRL_OK;
  if (groups > kMaxGroups) return set_error(TTRL_EINVAL, "%s: at most %d groups", name, kMaxGroups);
  if (long(groups) * M * N >= (1L << 31)) return set_error(TTRL_EINVAL, "%s: output too large", name);
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const long ws_limit = wsf - ws_reserved;
  hipStream_t st = stream_of(ctx);
  char keybuf[96];
  snprintf(keybuf, sizeof(keybuf), "|%d|%d|%d|%d|%ld", M, N, K, groups, ws_limit);
  const std::string key = std::string(__PRETTY_FUNCTION__) + keybuf;
  GemmPlan p;
  if (gemm_forced(ALLOWED, M, N, K, groups, ws_limit, &p)) {
    launch_allowed<ALLOWED>(la, lb, ep, ws, M, N, K, groups, p, st);
    return check_launch(name);
  }
  const GemmPlan* hit = ctx_plan_find(ctx, key);
  if (hit && plan_valid(*hit, M, N, K, groups, ws_limit, ALLOWED)) {
    p = *hit;
  } else {
    if (!ctx_capturing(ctx) && gemm_tuning_enabled())
      p = tune_gemm<ALLOWED>(ctx, la, lb, ep, ws, ws_limit, M, N, K, groups, st);
    else
      p = plan_gemm(M, N, K, groups, ws_limit, ALLOWED);
    ctx_plan_store(ctx, key, p);
  }
  launch_allowed<ALLOWED>(la, lb, ep, ws, M, N, K, groups, p, st);
  return check_launch(name);
}

// run_gemm without the split-K reduction, for a consumer kernel that sums
// the partials itself: when the plan splits K, k_gemm leaves partial tiles
// at the start of the workspace as [groups][splits][M][N] floats, to be
// summed in split order from 0.f (as k_splitk_reduce does) and passed
// through the epilogue by that consumer; with one split the epilogue runs in
// the GEMM.  *plan receives the plan that ran.  `part` (room for
// part_floats) replaces the workspace as the partials' home when given.
template <unsigned ALLOWED, class LA, class LB, class EP>
inline int run_gemm_deferred(ttrl_ctx* ctx, const LA& la, const LB& lb, const EP& ep, int M, int N, int K,
                             int groups, const char* name, GemmPlan* plan, float* part = nullptr,
                             long part_floats = 0) {
  static_assert((ALLOWED & kCfgAll) != 0, "no tile shape allowed");
  if (M <= 0 || N <= 0 || groups <= 0) return set_error(TTRL_EINVAL, "%s: empty GEMM", name);
  if (groups > kMaxGroups) return set_error(TTRL_EINVAL, "%s: at most %d groups", name, kMaxGroups);
  if (long(groups) * M * N >= (1L << 31)) return set_error(TTRL_EINVAL, "%s: output too large", name);
  long wsf = part_floats;
  float* ws = part ? part : ctx_workspace(ctx, &wsf);
  hipStream_t st = stream_of(ctx);
  char keybuf[96];
  snprintf(keybuf, sizeof(keybuf), "|%d|%d|%d|%d|%ld", M, N, K, groups, wsf);
  const std::string key = std::string(__PRETTY_FUNCTION__) + keybuf;
  GemmPlan p;
  const GemmPlan* hit = ctx_plan_find(ctx, key);
  if (gemm_forced(ALLOWED, M, N, K, groups, wsf, &p)) {
  } else if (hit && plan_valid(*hit, M, N, K, groups, wsf, ALLOWED)) {
    p = *hit;
  } else {
    if (!ctx_capturing(ctx) && gemm_tuning_enabled())
      p = tune_gemm<ALLOWED>(ctx, la, lb, ep, ws, wsf, M, N, K, groups, st, false);
    else
      p = plan_gemm(M, N, K, groups, wsf, ALLOWED);
    ctx_plan_store(ctx, key, p);
  }
  launch_gemm_only<ALLOWED>(la, lb, ep, ws, M, N, K, groups, p, st);
  *plan = p;
  return check_launch(name);
}

// ---------------------------------------------------------- pairs -------

struct GemmDims {
  int M, N, K, groups;
};

// defer1 not null: the first problem's split-K partials go there and are
// left unreduced (a later launch sums them); otherwise both problems'
// partials share `ws` and each is reduced after the pair.
template <int BM, int BN, int WGM, int WGN, int WGK, int TBK1, int TBK2, class LA1, class LB1, class EP1, class LA2,
          class LB2, class EP2>
inline void launch_pair_cfg(const LA1& la1, const LB1& lb1, const EP1& ep1, const GemmDims& q1, const GemmPlan& p1,
                            const LA2& la2, const LB2& lb2, const EP2& ep2, const GemmDims& q2, const GemmPlan& p2,
                            float* ws, hipStream_t st, float* defer1) {
  const int gx1 = int(ceil_div(q1.M, BM)), gy1 = int(ceil_div(q1.N, BN));
  const int gx2 = int(ceil_div(q2.M, BM)), gy2 = int(ceil_div(q2.N, BN));
  const long part1 = p1.splits > 1 && !defer1 ? (long(p1.splits) * q1.groups * q1.M * q1.N + 63) / 64 * 64 : 0;
  const PairDims d1{q1.M, q1.N, q1.K, p1.kchunk, p1.splits, gx1, gy1, gx1 * gy1 * q1.groups * p1.splits};
  const PairDims d2{q2.M, q2.N, q2.K, p2.kchunk, p2.splits, gx2, gy2, gx2 * gy2 * q2.groups * p2.splits};
  float* ws1 = defer1 ? defer1 : ws;
  hipLaunchKernelGGL((k_gemm_pair<BM, BN, WGM, WGN, WGK, TBK1, TBK2, LA1, LB1, EP1, LA2, LB2, EP2>),
                     dim3(unsigned(d1.blocks + d2.blocks)), dim3(64 * WGM * WGN * WGK), 0, st, la1, lb1, ep1, la2, lb2,
                     ep2, ws1, ws + part1, d1, d2);
  auto reduce = [&](const auto& ep, const GemmDims& q, const GemmPlan& p, float* w) {
    if (p.splits <= 1) return;
    unsigned blocks = unsigned(long(q.M) * q.N / 256 + 1);
    if (blocks > 2048) blocks = 2048;
    FDiv dn;
    dn.set(q.N);
    using E = std::decay_t<decltype(ep)>;
    hipLaunchKernelGGL((k_splitk_reduce<E>), dim3(blocks, unsigned(q.groups)), dim3(256), 0, st, w, ep, q.M, q.N,
                       p.splits, dn);
  };
  if (!defer1) reduce(ep1, q1, p1, ws);
  reduce(ep2, q2, p2, ws + part1);
}

template <unsigned ALLOWED, class LA1, class LB1, class EP1, class LA2, class LB2, class EP2>
inline void launch_pair(const LA1& la1, const LB1& lb1, const EP1& ep1, const GemmDims& q1, const GemmPlan& p1,
                        const LA2& la2, const LB2& lb2, const EP2& ep2, const GemmDims& q2, const GemmPlan& p2,
                        float* ws, hipStream_t st, float* defer1 = nullptr) {
  dispatch_cfg<ALLOWED>(p1.cfg, [&](auto c1) {
    using C1 = decltype(c1);
    if (p2.cfg == C1::ID) {
      launch_pair_cfg<C1::BM, C1::BN, C1::WGM, C1::WGN, C1::WGK, C1::TBK, C1::TBK>(la1, lb1, ep1, q1, p1, la2, lb2,
                                                                                    ep2, q2, p2, ws, st, defer1);
      return;
    }
    constexpr int tw = twin_cfg(C1::ID);
    if constexpr (tw >= 0 && (ALLOWED & cfg_bit(tw)) != 0) {
      dispatch_cfg<cfg_bit(tw)>(p2.cfg, [&](auto c2) {
        using C2 = decltype(c2);
        static_assert(C2::BM == C1::BM && C2::BN == C1::BN && C2::WGM == C1::WGM && C2::WGN == C1::WGN &&
                          C2::WGK == C1::WGK,
                      "twin tile shapes share the tile and the wavefront layout");
        launch_pair_cfg<C1::BM, C1::BN, C1::WGM, C1::WGN, C1::WGK, C1::TBK, C2::TBK>(la1, lb1, ep1, q1, p1, la2, lb2,
                                                                                      ep2, q2, p2, ws, st, defer1);
      });
    }
  });
}

// Two independent GEMMs in one launch of one tile shape (k_gemm_pair),
// planned together: the first eager call of a signature times, for each
// allowed tile shape, the cost model's split of each problem, and keeps the
// fastest pair for the context (as run_gemm does for one GEMM).  The two
// problems' split-K partials share the workspace below `ws_reserved`.
// With `defer1` (room for defer1_floats), the first problem's partials go
// there instead and are not reduced: a later consumer sums them, and
// *plan1 receives the first problem's plan.
template <unsigned ALLOWED, class LA1, class LB1, class EP1, class LA2, class LB2, class EP2>
inline int run_gemm_pair(ttrl_ctx* ctx, const LA1& la1, const LB1& lb1, const EP1& ep1, const GemmDims& q1,
                         const LA2& la2, const LB2& lb2, const EP2& ep2, const GemmDims& q2, const char* name,
                         long ws_reserved = 0, float* defer1 = nullptr, long defer1_floats = 0,
                         GemmPlan* plan1 = nullptr) {
  static_assert((ALLOWED & kCfgAll) != 0, "no tile shape allowed");
  for (const GemmDims* q : {&q1, &q2}) {
    if (q->M <= 0 || q->N <= 0 || q->groups <= 0 || q->groups > kMaxGroups || long(q->groups) * q->M * q->N >= (1L << 31))
      return set_error(TTRL_EINVAL, "%s: bad extents", name);
  }
  long wsf = 0;
  float* ws = ctx_workspace(ctx, &wsf);
  const long half = (wsf - ws_reserved) / 2 / 64 * 64;
  // each problem's room for partials: the workspace is shared unless the
  // first problem's go to their own buffer
  const long room1 = defer1 ? defer1_floats : half;
  const long room2 = defer1 ? (wsf - ws_reserved) / 64 * 64 : half;
  hipStream_t st = stream_of(ctx);
  char keybuf[192];
  if (defer1)
    snprintf(keybuf, sizeof(keybuf), "|%d|%d|%d|%d|%d|%d|%d|%d|%ld|D%ld", q1.M, q1.N, q1.K, q1.groups, q2.M, q2.N,
             q2.K, q2.groups, room2, room1);
  else
    snprintf(keybuf, sizeof(keybuf), "|%d|%d|%d|%d|%d|%d|%d|%d|%ld", q1.M, q1.N, q1.K, q1.groups, q2.M, q2.N, q2.K,
             q2.groups, half);
  const std::string key = std::string(__PRETTY_FUNCTION__) + keybuf;
  GemmPlan p1, p2;
  if (gemm_forced(ALLOWED, q1.M, q1.N, q1.K, q1.groups, room1, &p1) &&
      gemm_forced(ALLOWED, q2.M, q2.N, q2.K, q2.groups, room2, &p2)) {
    launch_pair<ALLOWED>(la1, lb1, ep1, q1, p1, la2, lb2, ep2, q2, p2, ws, st, defer1);
    if (plan1) *plan1 = p1;
    return check_launch(name);
  }
  const std::string key2 = key + "#2";
  const GemmPlan* h1 = ctx_plan_find(ctx, key);
  const GemmPlan* h2 = ctx_plan_find(ctx, key2);
  if (h1 && h2 && pair_cfgs_ok(h1->cfg, h2->cfg) && plan_valid(*h1, q1.M, q1.N, q1.K, q1.groups, room1, ALLOWED) &&
      plan_valid(*h2, q2.M, q2.N, q2.K, q2.groups, room2, ALLOWED)) {
    p1 = *h1;
    p2 = *h2;
  } else {
    // Per tile shape: the cost model's split of each problem, then each
    // problem split 2 to 16 ways with the other at the model's split (the
    // model prices a long K loop of a small problem below its latency);
    // then the second problem at the twin stage depth, if allowed.
    std::vector<std::pair<GemmPlan, GemmPlan>> cands;
    auto add = [&](const GemmPlan& a, const GemmPlan& b) {
      for (const auto& e : cands)
        if (e.first.cfg == a.cfg && e.second.cfg == b.cfg && e.first.splits == a.splits &&
            e.second.splits == b.splits)
          return;
      cands.emplace_back(a, b);
    };
    for (int c = 0; c < kNumCfg; ++c) {
      if (!(ALLOWED & cfg_bit(c))) continue;
      const GemmPlan b1 = plan_gemm(q1.M, q1.N, q1.K, q1.groups, room1, cfg_bit(c));
      const GemmPlan b2 = plan_gemm(q2.M, q2.N, q2.K, q2.groups, room2, cfg_bit(c));
      add(b1, b2);
      for (int sp : {2, 4, 8, 16}) {
        GemmPlan v;
        if (plan_with_splits(c, q1.M, q1.N, q1.K, q1.groups, room1, sp, &v)) add(v, b2);
        if (plan_with_splits(c, q2.M, q2.N, q2.K, q2.groups, room2, sp, &v)) add(b1, v);
      }
      const int t = twin_cfg(c);
      if (t >= 0 && (ALLOWED & cfg_bit(t))) {
        add(b1, plan_gemm(q2.M, q2.N, q2.K, q2.groups, room2, cfg_bit(t)));
        for (int sp : {2, 4}) {
          GemmPlan v;
          if (plan_with_splits(t, q2.M, q2.N, q2.K, q2.groups, room2, sp, &v)) add(b1, v);
        }
      }
    }
    p1 = cands.front().first;
    p2 = cands.front().second;
    hipEvent_t e0, e1;
    const long span1 = ep1.tune_span();
    float* sink = nullptr;
    if (!ctx_capturing(ctx) && gemm_tuning_enabled() && cands.size() > 1 &&
        (sink = ctx_tune_sink(ctx, size_t(span1 + ep2.tune_span()) * sizeof(float))) != nullptr &&
        ctx_tune_events(ctx, &e0, &e1)) {
      const EP1 t1 = ep1.tune_copy(sink);
      const EP2 t2 = ep2.tune_copy(sink + span1);
      float best_ms = 1e30f;
      for (const auto& c : cands) {
        launch_pair<ALLOWED>(la1, lb1, t1, q1, c.first, la2, lb2, t2, q2, c.second, ws, st, defer1);  // warm
        const float ms = time_best_of(e0, e1, st, [&] {
          launch_pair<ALLOWED>(la1, lb1, t1, q1, c.first, la2, lb2, t2, q2, c.second, ws, st, defer1);
        });
        if (ms < 0.f) break;
        if (gemm_tuning_log())
          fprintf(stderr,
                  "[ttrl gemm tune pair] %dx%dx%d(G%d) + %dx%dx%d(G%d)  %dx%d tbk%d,%d splits=%d,%d  %.2f us\n",
                  q1.M, q1.N, q1.K, q1.groups, q2.M, q2.N, q2.K, q2.groups, c.first.bm, c.first.bn, c.first.tbk,
                  c.second.tbk, c.first.splits, c.second.splits, ms * 1e3f / 3.f);
        // a deferred first problem has no reduce launch to charge
        const float cost =
            ms + 3.f * kReduceLaunchMs * float(int(c.first.splits > 1 && !defer1) + int(c.second.splits > 1));
        if (cost < best_ms) {
          best_ms = cost;
          p1 = c.first;
          p2 = c.second;
        }
      }
      (void)hipGetLastError();
    }
    ctx_plan_store(ctx, key, p1);
    ctx_plan_store(ctx, key2, p2);
  }
  launch_pair<ALLOWED>(la1, lb1, ep1, q1, p1, la2, lb2, ep2, q2, p2, ws, st, defer1);
  if (plan1) *plan1 = p1;
  return check_launch(name);
}

// Per-group pointer table from a base pointer and an element stride.
template <class T>
inline void fill_groups(T* (&dst)[kMaxGroups], T* base, long stride, int groups) {
  for (int g = 0; g < kMaxGroups; ++g) dst[g] = (base && g < groups) ? base + g * stride : nullptr;
}

}  // namespace ttrl
