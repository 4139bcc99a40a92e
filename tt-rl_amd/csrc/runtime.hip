// Host runtime of libttrl_hip: device context, stream, slab-pool device
// allocator, host<->device transfers, fill, hipGraph capture and replay,
// stream timers.  Every entry point returns 0 or a negative TTRL_E* code and
// leaves a thread-local message for ttrl_last_error().
//
// Replaces the ttnn device plumbing the reference drives from Python:
//   device open/close            ttrl/engine/device/acquire.py:56-140
//   fixed-address buffers        ttrl/engine/tensor/arena.py:21-87
//   host<->device copies         ttrl/engine/tensor/transfer.py:11-51
//   trace capture / replay       ttrl/engine/trace.py:56-126
#include "common.hpp"
#include "tile_gemm.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_last_error;

constexpr size_t kAlign = 256;
constexpr size_t kSlabBytes = size_t(64) << 20;
constexpr size_t kWorkspaceBytes = size_t(64) << 20;

struct Pool {
  std::vector<std::pair<char*, size_t>> slabs;
  char* cursor = nullptr;
  size_t left = 0;
  std::unordered_map<size_t, std::vector<char*>> free_lists;
  size_t reserved = 0;
  size_t live = 0;
  bool retired = false;
  bool in_use = false;
};

struct Block {
  size_t size;
  int pool;
};

}  // namespace

struct ttrl_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  std::vector<Pool> pools;
  int current_pool = 0;
  std::unordered_map<void*, Block> blocks;
  bool capturing = false;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  float* ws = nullptr;  // stream-ordered scratch of split-K GEMMs and reductions
  long ws_floats = 0;
  unsigned* sync = nullptr;  // zeroed counters and partials (ctx_sync_words)
  float* adam_parts = nullptr;  // ctx_adam_partials
  float* grad_banks = nullptr;  // ctx_grad_bank
  // GEMM plans chosen by timing candidates on this device, by call signature.
  std::unordered_map<std::string, ttrl::GemmPlan> plans;
  float* tune_out = nullptr;  // output sink of candidate runs
  size_t tune_bytes = 0;
  hipEvent_t tune0 = nullptr, tune1 = nullptr;
  // Pinned host staging of ttrl_graph_step: inputs first, outputs after.
  unsigned char* pinned = nullptr;
  size_t pinned_bytes = 0;
  // Pinned host blocks handed out by ttrl_host_alloc (base -> bytes).
  std::unordered_map<void*, size_t> host_blocks;
  // Host blocks freed while the stream was capturing: releasing one waits for
  // the stream, which a capturing stream cannot do, so they go back once the
  // capture has ended (release_after_capture).
  std::vector<void*> host_frees_after_capture;
};

// One kernel node of a captured graph, as a direct launch.
struct DirectLaunch {
  const void* func;
  dim3 grid, block;
  unsigned shmem;
  void** args;  // owned by the graph's node, valid while the graph lives
};

struct ttrl_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  size_t nodes = 0;
  // The graph's kernels in dependency order, when every node is a kernel
  // (ttrl_graph_set_direct replays them as individual launches).
  std::vector<DirectLaunch> kernels;
  bool direct_ok = false;
  bool direct = false;
};

namespace ttrl {

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_error(hipError_t e, const char* what) {
  return set_error(TTRL_EHIP, "%s: %s (%d)", what, hipGetErrorString(e), int(e));
}

hipStream_t stream_of(ttrl_ctx* ctx) { return ctx->stream; }

unsigned* ctx_sync_words(ttrl_ctx* ctx) { return ctx->sync; }

float* ctx_adam_partials(ttrl_ctx* ctx) { return ctx->adam_parts; }
float* ctx_grad_bank(ttrl_ctx* ctx, int bank) { return ctx->grad_banks + long(bank) * kGradBankFloats; }

float* ctx_workspace(ttrl_ctx* ctx, long* floats) {
  if (floats) *floats = ctx->ws_floats;
  return ctx->ws;
}

bool ctx_capturing(ttrl_ctx* ctx) { return ctx->capturing; }

const GemmPlan* ctx_plan_find(ttrl_ctx* ctx, const std::string& key) {
  auto it = ctx->plans.find(key);
  return it == ctx->plans.end() ? nullptr : &it->second;
}

void ctx_plan_store(ttrl_ctx* ctx, const std::string& key, const GemmPlan& p) { ctx->plans[key] = p; }

float* ctx_tune_sink(ttrl_ctx* ctx, size_t bytes) {
  if (bytes > ctx->tune_bytes) {
    if (ctx->tune_out) (void)hipFree(ctx->tune_out);
    ctx->tune_out = nullptr;
    ctx->tune_bytes = 0;
    if (hipMalloc(&ctx->tune_out, bytes) != hipSuccess) return nullptr;
    ctx->tune_bytes = bytes;
  }
  return ctx->tune_out;
}

bool ctx_tune_events(ttrl_ctx* ctx, hipEvent_t* a, hipEvent_t* b) {
  if (!ctx->tune0 && hipEventCreate(&ctx->tune0) != hipSuccess) return false;
  if (!ctx->tune1 && hipEventCreate(&ctx->tune1) != hipSuccess) return false;
  *a = ctx->tune0;
  *b = ctx->tune1;
  return true;
}

int check_launch(const char* name) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_error(e, name);
  return TTRL_OK;
}

}  // namespace ttrl

using namespace ttrl;

namespace {

int pool_grow(Pool& p, size_t need) {
  size_t bytes = need > kSlabBytes ? need : kSlabBytes;
  void* ptr = nullptr;
  hipError_t e = hipMalloc(&ptr, bytes);
  if (e != hipSuccess) return hip_error(e, "hipMalloc (pool slab)");
  p.slabs.emplace_back(static_cast<char*>(ptr), bytes);
  p.cursor = static_cast<char*>(ptr);
  p.left = bytes;
  p.reserved += bytes;
  return TTRL_OK;
}

void pool_free_slabs(Pool& p) {
  for (auto& s : p.slabs) (void)hipFree(s.first);
  p.slabs.clear();
  p.free_lists.clear();
  p.cursor = nullptr;
  p.left = 0;
  p.reserved = 0;
}

// Releases held back while the stream captured a graph: host blocks freed in
// the meantime and retired pools whose last block went back.  A free can
// arrive during a capture from anywhere in the host program (a garbage
// collector finalising an unrelated object), and the stream wait a release
// needs would invalidate the capture.
void release_after_capture(ttrl_ctx* ctx) {
  std::lock_guard<std::mutex> g(ctx->mu);
  bool pools_due = false;
  for (auto& p : ctx->pools) pools_due |= p.retired && p.live == 0;
  if (!pools_due && ctx->host_frees_after_capture.empty()) return;
  (void)hipStreamSynchronize(ctx->stream);
  for (auto& p : ctx->pools) {
    if (p.retired && p.live == 0) {
      pool_free_slabs(p);
      p.retired = false;
      p.in_use = false;
    }
  }
  for (void* h : ctx->host_frees_after_capture) (void)hipHostFree(h);
  ctx->host_frees_after_capture.clear();
}

}  // namespace

extern "C" {

const char* ttrl_last_error(void) { return g_last_error.c_str(); }

int ttrl_version(void) { return TTRL_ABI_VERSION; }

int ttrl_device_count(int* out) {
  if (!out) return set_error(TTRL_EINVAL, "ttrl_device_count: null out");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    *out = 0;
    return hip_error(e, "hipGetDeviceCount");
  }
  *out = n;
  return TTRL_OK;
}

int ttrl_device_query(int device, ttrl_device_info* out) {
  if (!out) return set_error(TTRL_EINVAL, "ttrl_device_query: null out");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
  if (device < 0 || device >= n)
    return set_error(TTRL_EINVAL, "ttrl_device_query: device %d out of range (%d visible)", device, n);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_error(e, "hipGetDeviceProperties");
  std::memset(out, 0, sizeof(*out));
  std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
  std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
  out->compute_units = prop.multiProcessorCount;
  out->wavefront_size = prop.warpSize;
  out->lds_per_cu = long(prop.maxSharedMemoryPerMultiProcessor);
  out->lds_per_workgroup = long(prop.sharedMemPerBlock);
  out->l2_bytes = long(prop.l2CacheSize);
  out->hbm_bytes = long(prop.totalGlobalMem);
  out->clock_khz = prop.clockRate;
  out->memory_clock_khz = prop.memoryClockRate;
  out->memory_bus_bits = prop.memoryBusWidth;
  out->pci_bus_id = prop.pciBusID;
  out->pci_device_id = prop.pciDeviceID;
  out->pci_domain_id = prop.pciDomainID;
  return TTRL_OK;
}

int ttrl_init(int device, ttrl_ctx** out) {
  if (!out) return set_error(TTRL_EINVAL, "ttrl_init: null out");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
  if (device < 0 || device >= n)
    return set_error(TTRL_EINVAL, "ttrl_init: device %d out of range (%d visible)", device, n);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_error(e, "hipSetDevice");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_error(e, "hipGetDeviceProperties");
  if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
    return set_error(TTRL_EINVAL, "ttrl_init: device %d is %s; this library is built for gfx950 only",
                     device, prop.gcnArchName);
  auto* ctx = new ttrl_ctx();
  ctx->device = device;
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return hip_error(e, "hipStreamCreate");
  }
  (void)hipEventCreate(&ctx->t0);
  (void)hipEventCreate(&ctx->t1);
  // Split-K partial tiles and reduction partials are written and consumed
  // by consecutive kernels on this one stream, so one fixed buffer serves
  // every launch and every captured graph of the context.
  void* ws = nullptr;
  e = hipMalloc(&ws, kWorkspaceBytes);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_error(e, "hipMalloc (workspace)");
  }
  ctx->ws = static_cast<float*>(ws);
  ctx->ws_floats = long(kWorkspaceBytes / sizeof(float));
  const size_t sync_bytes = sizeof(unsigned) * (kSyncCounters + kSyncPartials);
  void* sync = nullptr;
  e = hipMalloc(&sync, sync_bytes);
  if (e == hipSuccess) e = hipMemset(sync, 0, sync_bytes);
  if (e != hipSuccess) {
    if (sync) (void)hipFree(sync);
    (void)hipFree(ws);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_error(e, "hipMalloc (sync words)");
  }
  ctx->sync = static_cast<unsigned*>(sync);
  void* parts = nullptr;
  e = hipMalloc(&parts, sizeof(float) * kAdamSlots * kAdamSlotFloats);
  if (e != hipSuccess) {
    (void)hipFree(sync);
    (void)hipFree(ws);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_error(e, "hipMalloc (Adam partial slots)");
  }
  ctx->adam_parts = static_cast<float*>(parts);
  void* banks = nullptr;
  e = hipMalloc(&banks, sizeof(float) * kGradBanks * kGradBankFloats);
  if (e != hipSuccess) {
    (void)hipFree(parts);
    (void)hipFree(sync);
    (void)hipFree(ws);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_error(e, "hipMalloc (gradient banks)");
  }
  ctx->grad_banks = static_cast<float*>(banks);
  ctx->pools.emplace_back();  // pool 0: the default pool
  ctx->pools[0].in_use = true;
  *out = ctx;
  return TTRL_OK;
}

int ttrl_shutdown(ttrl_ctx* ctx) {
  if (!ctx) return TTRL_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  for (auto& p : ctx->pools) pool_free_slabs(p);
  if (ctx->ws) (void)hipFree(ctx->ws);
  if (ctx->sync) (void)hipFree(ctx->sync);
  if (ctx->adam_parts) (void)hipFree(ctx->adam_parts);
  if (ctx->grad_banks) (void)hipFree(ctx->grad_banks);
  if (ctx->tune_out) (void)hipFree(ctx->tune_out);
  if (ctx->tune0) (void)hipEventDestroy(ctx->tune0);
  if (ctx->tune1) (void)hipEventDestroy(ctx->tune1);
  if (ctx->t0) (void)hipEventDestroy(ctx->t0);
  if (ctx->t1) (void)hipEventDestroy(ctx->t1);
  if (ctx->pinned) (void)hipHostFree(ctx->pinned);
  for (auto& hb : ctx->host_blocks) (void)hipHostFree(hb.first);
  for (void* h : ctx->host_frees_after_capture) (void)hipHostFree(h);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return TTRL_OK;
}

int ttrl_sync(ttrl_ctx* ctx) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_sync: null ctx");
  if (ctx->capturing) return set_error(TTRL_ESTATE, "ttrl_sync: the stream is capturing a graph");
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize");
  return TTRL_OK;
}

void* ttrl_stream(ttrl_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

// ---------------------------------------------------------------- pools ---

int ttrl_pool_create(ttrl_ctx* ctx, int* pool) {
  if (!ctx || !pool) return set_error(TTRL_EINVAL, "ttrl_pool_create: null argument");
  std::lock_guard<std::mutex> g(ctx->mu);
  for (size_t i = 1; i < ctx->pools.size(); ++i) {
    if (!ctx->pools[i].in_use) {
      ctx->pools[i] = Pool();
      ctx->pools[i].in_use = true;
      *pool = int(i);
      return TTRL_OK;
    }
  }
  ctx->pools.emplace_back();
  ctx->pools.back().in_use = true;
  *pool = int(ctx->pools.size() - 1);
  return TTRL_OK;
}

int ttrl_pool_release(ttrl_ctx* ctx, int pool) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_pool_release: null ctx");
  std::lock_guard<std::mutex> g(ctx->mu);
  if (pool <= 0 || pool >= int(ctx->pools.size()) || !ctx->pools[pool].in_use)
    return set_error(TTRL_EINVAL, "ttrl_pool_release: bad pool %d", pool);
  if (ctx->current_pool == pool) ctx->current_pool = 0;
  Pool& p = ctx->pools[pool];
  if (p.live == 0 && !ctx->capturing) {
    (void)hipStreamSynchronize(ctx->stream);
    pool_free_slabs(p);
    p.in_use = false;
  } else {
    p.retired = true;  // slabs go back when the last live block is freed, or after the capture
  }
  return TTRL_OK;
}

int ttrl_pool_use(ttrl_ctx* ctx, int pool, int* previous) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_pool_use: null ctx");
  std::lock_guard<std::mutex> g(ctx->mu);
  if (pool < 0 || pool >= int(ctx->pools.size()) || !ctx->pools[pool].in_use || ctx->pools[pool].retired)
    return set_error(TTRL_EINVAL, "ttrl_pool_use: bad pool %d", pool);
  if (previous) *previous = ctx->current_pool;
  ctx->current_pool = pool;
  return TTRL_OK;
}

int ttrl_pool_stats(ttrl_ctx* ctx, int pool, size_t* reserved, size_t* live) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_pool_stats: null ctx");
  std::lock_guard<std::mutex> g(ctx->mu);
  if (pool < 0 || pool >= int(ctx->pools.size()))
    return set_error(TTRL_EINVAL, "ttrl_pool_stats: bad pool %d", pool);
  if (reserved) *reserved = ctx->pools[pool].reserved;
  if (live) *live = ctx->pools[pool].live;
  return TTRL_OK;
}

int ttrl_alloc(ttrl_ctx* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return set_error(TTRL_EINVAL, "ttrl_alloc: null argument");
  std::lock_guard<std::mutex> g(ctx->mu);
  size_t size = ((bytes ? bytes : 1) + kAlign - 1) / kAlign * kAlign;
  int pid = ctx->current_pool;
  Pool& p = ctx->pools[pid];
  char* ptr = nullptr;
  auto it = p.free_lists.find(size);
  if (it != p.free_lists.end() && !it->second.empty()) {
    ptr = it->second.back();
    it->second.pop_back();
  } else {
    if (p.left < size) {
      int rc = pool_grow(p, size);
      if (rc) return rc;
    }
    ptr = p.cursor;
    p.cursor += size;
    p.left -= size;
  }
  p.live += size;
  ctx->blocks[ptr] = Block{size, pid};
  *out = ptr;
  return TTRL_OK;
}

int ttrl_free(ttrl_ctx* ctx, void* ptr) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_free: null ctx");
  if (!ptr) return TTRL_OK;
  std::lock_guard<std::mutex> g(ctx->mu);
  auto it = ctx->blocks.find(ptr);
  if (it == ctx->blocks.end()) return set_error(TTRL_EINVAL, "ttrl_free: %p was not allocated here", ptr);
  Block b = it->second;
  ctx->blocks.erase(it);
  Pool& p = ctx->pools[b.pool];
  p.live -= b.size;
  p.free_lists[b.size].push_back(static_cast<char*>(ptr));
  if (p.retired && p.live == 0 && !ctx->capturing) {
    (void)hipStreamSynchronize(ctx->stream);
    pool_free_slabs(p);
    p.retired = false;
    p.in_use = false;
  }
  return TTRL_OK;
}

// ------------------------------------------------------------ transfers ---

int ttrl_h2d(ttrl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return set_error(TTRL_EINVAL, "ttrl_h2d: null argument");
  if (ctx->capturing)
    return set_error(TTRL_ESTATE,
                     "ttrl_h2d: host-to-device writes are not allowed while a graph is being captured; "
                     "load inputs before the capture or between replays");
  if (!bytes) return TTRL_OK;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync H2D");
  e = hipStreamSynchronize(ctx->stream);  // the host buffer may be reused as soon as we return
  if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize after H2D");
  return TTRL_OK;
}

int ttrl_d2h(ttrl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return set_error(TTRL_EINVAL, "ttrl_d2h: null argument");
  if (ctx->capturing)
    return set_error(TTRL_ESTATE,
                     "ttrl_d2h: reads to host are not supported during graph capture; "
                     "read metrics after the replay");
  if (!bytes) return TTRL_OK;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync D2H");
  e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize after D2H");
  return TTRL_OK;
}

int ttrl_d2d(ttrl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return set_error(TTRL_EINVAL, "ttrl_d2d: null argument");
  if (!bytes) return TTRL_OK;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync D2D");
  return TTRL_OK;
}

// --------------------------------------------------------------- graphs ---

}  // extern "C"

namespace {

// Records g's kernel nodes in dependency order (Kahn's order over the
// node dependencies); leaves g->direct_ok false when a node is not a kernel
// or a query fails.
void record_kernels(ttrl_graph* g) {
  size_t n = 0;
  if (hipGraphGetNodes(g->graph, nullptr, &n) != hipSuccess || n == 0) return;
  std::vector<hipGraphNode_t> nodes(n);
  if (hipGraphGetNodes(g->graph, nodes.data(), &n) != hipSuccess) return;
  std::unordered_map<hipGraphNode_t, size_t> index;
  for (size_t i = 0; i < n; ++i) index[nodes[i]] = i;
  std::vector<int> pending(n, 0);
  std::vector<std::vector<size_t>> next(n);
  for (size_t i = 0; i < n; ++i) {
    size_t nd = 0;
    if (hipGraphNodeGetDependencies(nodes[i], nullptr, &nd) != hipSuccess) return;
    std::vector<hipGraphNode_t> deps(nd);
    if (nd && hipGraphNodeGetDependencies(nodes[i], deps.data(), &nd) != hipSuccess) return;
    for (hipGraphNode_t d : deps) {
      auto it = index.find(d);
      if (it == index.end()) return;
      next[it->second].push_back(i);
      ++pending[i];
    }
  }
  std::vector<size_t> order;
  for (size_t i = 0; i < n; ++i)
    if (pending[i] == 0) order.push_back(i);
  for (size_t h = 0; h < order.size(); ++h)
    for (size_t j : next[order[h]])
      if (--pending[j] == 0) order.push_back(j);
  if (order.size() != n) return;
  std::vector<DirectLaunch> ks;
  for (size_t i : order) {
    hipGraphNodeType type;
    if (hipGraphNodeGetType(nodes[i], &type) != hipSuccess || type != hipGraphNodeTypeKernel) return;
    hipKernelNodeParams kp{};
    if (hipGraphKernelNodeGetParams(nodes[i], &kp) != hipSuccess || kp.extra || !kp.func) return;
    ks.push_back(DirectLaunch{kp.func, kp.gridDim, kp.blockDim, kp.sharedMemBytes, kp.kernelParams});
  }
  g->kernels = std::move(ks);
  g->direct_ok = true;
}

// One replay of g on `stream`: the graph launch, or its kernels one by one.
hipError_t replay(ttrl_graph* g, hipStream_t stream) {
  if (!g->direct) return hipGraphLaunch(g->exec, stream);
  for (const DirectLaunch& k : g->kernels) {
    const hipError_t e = hipLaunchKernel(k.func, k.grid, k.block, k.args, k.shmem, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

extern "C" {

int ttrl_capture_begin(ttrl_ctx* ctx) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_capture_begin: null ctx");
  if (ctx->capturing) return set_error(TTRL_ESTATE, "ttrl_capture_begin: already capturing");
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) return hip_error(e, "hipStreamBeginCapture");
  ctx->capturing = true;
  return TTRL_OK;
}

int ttrl_capture_end(ttrl_ctx* ctx, ttrl_graph** out) {
  if (!ctx || !out) return set_error(TTRL_EINVAL, "ttrl_capture_end: null argument");
  if (!ctx->capturing) return set_error(TTRL_ESTATE, "ttrl_capture_end: not capturing");
  ctx->capturing = false;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
  release_after_capture(ctx);
  if (e != hipSuccess) {
    if (graph) (void)hipGraphDestroy(graph);
    return hip_error(e, "hipStreamEndCapture");
  }
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return hip_error(e, "hipGraphInstantiate");
  }
  auto* g = new ttrl_graph();
  g->graph = graph;
  g->exec = exec;
  size_t n = 0;
  if (hipGraphGetNodes(graph, nullptr, &n) == hipSuccess) g->nodes = n;
  record_kernels(g);
  *out = g;
  return TTRL_OK;
}

int ttrl_capture_abort(ttrl_ctx* ctx) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_capture_abort: null ctx");
  if (!ctx->capturing) return TTRL_OK;
  ctx->capturing = false;
  hipGraph_t graph = nullptr;
  (void)hipStreamEndCapture(ctx->stream, &graph);
  if (graph) (void)hipGraphDestroy(graph);
  (void)hipGetLastError();
  release_after_capture(ctx);
  return TTRL_OK;
}

int ttrl_graph_launch(ttrl_ctx* ctx, ttrl_graph* g) {
  if (!ctx || !g || !g->exec) return set_error(TTRL_EINVAL, "ttrl_graph_launch: null argument");
  if (ctx->capturing) return set_error(TTRL_ESTATE, "ttrl_graph_launch: the stream is capturing");
  hipError_t e = replay(g, ctx->stream);
  if (e != hipSuccess) return hip_error(e, g->direct ? "hipLaunchKernel (direct replay)" : "hipGraphLaunch");
  return TTRL_OK;
}

int ttrl_graph_set_direct(ttrl_graph* g, int on) {
  if (!g || !g->exec) return set_error(TTRL_EINVAL, "ttrl_graph_set_direct: null or destroyed graph");
  if (on && !g->direct_ok)
    return set_error(TTRL_EINVAL, "ttrl_graph_set_direct: the graph has nodes other than kernels (or none); "
                                  "only a graph of kernels replays as direct launches");
  g->direct = on != 0;
  return TTRL_OK;
}

int ttrl_host_alloc(ttrl_ctx* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return set_error(TTRL_EINVAL, "ttrl_host_alloc: null argument");
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault);
  if (e != hipSuccess) return hip_error(e, "hipHostMalloc (ttrl_host_alloc)");
  std::lock_guard<std::mutex> g(ctx->mu);
  ctx->host_blocks[p] = bytes ? bytes : 1;
  *out = p;
  return TTRL_OK;
}

int ttrl_host_alloc_mapped(ttrl_ctx* ctx, size_t bytes, void** host, void** device) {
  if (!ctx || !host || !device) return set_error(TTRL_EINVAL, "ttrl_host_alloc_mapped: null argument");
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocMapped | hipHostMallocCoherent);
  if (e != hipSuccess) return hip_error(e, "hipHostMalloc (ttrl_host_alloc_mapped)");
  void* d = nullptr;
  e = hipHostGetDevicePointer(&d, p, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(p);
    return hip_error(e, "hipHostGetDevicePointer (ttrl_host_alloc_mapped)");
  }
  std::lock_guard<std::mutex> g(ctx->mu);
  ctx->host_blocks[p] = bytes ? bytes : 1;
  *host = p;
  *device = d;
  return TTRL_OK;
}

int ttrl_host_free(ttrl_ctx* ctx, void* ptr) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_host_free: null ctx");
  if (!ptr) return TTRL_OK;
  std::lock_guard<std::mutex> g(ctx->mu);
  auto it = ctx->host_blocks.find(ptr);
  if (it == ctx->host_blocks.end()) return set_error(TTRL_EINVAL, "ttrl_host_free: %p was not allocated here", ptr);
  if (ctx->capturing) {
    ctx->host_blocks.erase(it);
    ctx->host_frees_after_capture.push_back(ptr);
    return TTRL_OK;
  }
  // A copy from or to the block may still be queued on the stream.
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipHostFree(ptr);
  ctx->host_blocks.erase(it);
  return TTRL_OK;
}

}  // extern "C"

namespace {

// True when [p, p + bytes) lies inside one block of ttrl_host_alloc.
bool in_host_block(ttrl_ctx* ctx, const void* p, size_t bytes) {
  const char* c = static_cast<const char*>(p);
  std::lock_guard<std::mutex> g(ctx->mu);
  for (auto& hb : ctx->host_blocks) {
    const char* base = static_cast<const char*>(hb.first);
    if (c >= base && c + bytes <= base + hb.second) return true;
  }
  return false;
}

}  // namespace

extern "C" {

int ttrl_h2d_enqueue(ttrl_ctx* ctx, void* dst, const void* host_src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!host_src && bytes))
    return set_error(TTRL_EINVAL, "ttrl_h2d_enqueue: null argument");
  if (ctx->capturing)
    return set_error(TTRL_ESTATE, "ttrl_h2d_enqueue: host-to-device writes are not allowed while a graph is being "
                                  "captured; load inputs before the capture or between replays");
  if (!bytes) return TTRL_OK;
  // Only pinned blocks: the copy reads the host range after this returns.
  if (!in_host_block(ctx, host_src, bytes))
    return set_error(TTRL_EINVAL, "ttrl_h2d_enqueue: the source must lie inside one ttrl_host_alloc block");
  const hipError_t e = hipMemcpyAsync(dst, host_src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync H2D (enqueued)");
  return TTRL_OK;
}

int ttrl_graph_step(ttrl_ctx* ctx, ttrl_graph* g, void* in_dev, const void* in_host, size_t in_bytes,
                    void* out_host, const void* out_dev, size_t out_bytes) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_graph_step: null ctx");
  if ((in_bytes && (!in_dev || !in_host)) || (out_bytes && (!out_dev || !out_host)))
    return set_error(TTRL_EINVAL, "ttrl_graph_step: null buffer with a nonzero size");
  if (g && !g->exec) return set_error(TTRL_EINVAL, "ttrl_graph_step: destroyed graph");
  if (ctx->capturing) return set_error(TTRL_ESTATE, "ttrl_graph_step: the stream is capturing");
  // Host buffers from ttrl_host_alloc are pinned already: the copies read
  // and write them in place, with no staging pass (an empty side needs none).
  const bool in_pinned = in_bytes == 0 || in_host_block(ctx, in_host, in_bytes);
  const bool out_pinned = out_bytes == 0 || in_host_block(ctx, out_host, out_bytes);
  if (in_pinned && out_pinned) {
    hipError_t e;
    if (in_bytes) {
      e = hipMemcpyAsync(in_dev, in_host, in_bytes, hipMemcpyHostToDevice, ctx->stream);
      if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync H2D (graph step)");
    }
    if (g) {
      e = replay(g, ctx->stream);
      if (e != hipSuccess) return hip_error(e, "replay (graph step)");
    }
    if (out_bytes) {
      e = hipMemcpyAsync(out_host, out_dev, out_bytes, hipMemcpyDeviceToHost, ctx->stream);
      if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync D2H (graph step)");
    }
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize (graph step)");
    return TTRL_OK;
  }
  const size_t out_at = (in_bytes + 255) & ~size_t(255);
  const size_t need = out_at + out_bytes;
  if (need > ctx->pinned_bytes) {
    // Grow only: the previous step has been waited for, so nothing reads the old staging.
    size_t cap = std::max(need, ctx->pinned_bytes * 2);
    unsigned char* p = nullptr;
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&p), cap, hipHostMallocDefault);
    if (e != hipSuccess) return hip_error(e, "hipHostMalloc (graph step staging)");
    if (ctx->pinned) (void)hipHostFree(ctx->pinned);
    ctx->pinned = p;
    ctx->pinned_bytes = cap;
  }
  hipError_t e;
  if (in_bytes) {
    std::memcpy(ctx->pinned, in_host, in_bytes);
    e = hipMemcpyAsync(in_dev, ctx->pinned, in_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync H2D (graph step)");
  }
  if (g) {
    e = replay(g, ctx->stream);
    if (e != hipSuccess) return hip_error(e, "replay (graph step)");
  }
  if (out_bytes) {
    e = hipMemcpyAsync(ctx->pinned + out_at, out_dev, out_bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e != hipSuccess) return hip_error(e, "hipMemcpyAsync D2H (graph step)");
  }
  e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipStreamSynchronize (graph step)");
  if (out_bytes) std::memcpy(out_host, ctx->pinned + out_at, out_bytes);
  return TTRL_OK;
}

int ttrl_graph_launch_n(ttrl_ctx* ctx, ttrl_graph* g, int n) {
  if (!ctx || !g || !g->exec) return set_error(TTRL_EINVAL, "ttrl_graph_launch_n: null argument");
  if (ctx->capturing) return set_error(TTRL_ESTATE, "ttrl_graph_launch_n: the stream is capturing");
  for (int i = 0; i < n; ++i) {
    hipError_t e = replay(g, ctx->stream);
    if (e != hipSuccess) return hip_error(e, g->direct ? "hipLaunchKernel (direct replay)" : "hipGraphLaunch");
  }
  return TTRL_OK;
}

int ttrl_graph_nodes(ttrl_graph* g, size_t* out) {
  if (!g || !out) return set_error(TTRL_EINVAL, "ttrl_graph_nodes: null argument");
  *out = g->nodes;
  return TTRL_OK;
}

int ttrl_graph_destroy(ttrl_graph* g) {
  if (!g) return TTRL_OK;
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
  return TTRL_OK;
}

// ---------------------------------------------------------------- plans ---

int ttrl_plans_export(ttrl_ctx* ctx, char* buf, size_t cap, size_t* len) {
  if (!ctx || !len) return set_error(TTRL_EINVAL, "ttrl_plans_export: null argument");
  std::vector<std::pair<std::string, GemmPlan>> rows(ctx->plans.begin(), ctx->plans.end());
  std::sort(rows.begin(), rows.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
  std::string text;
  char head[96];
  for (const auto& r : rows) {
    const GemmPlan& p = r.second;
    snprintf(head, sizeof(head), "%d %d %d %d %d %d\t", p.cfg, p.bm, p.bn, p.tbk, p.splits, p.kchunk);
    text += head;
    text += r.first;
    text += '\n';
  }
  *len = text.size();
  if (buf) {
    if (cap < text.size() + 1) return set_error(TTRL_EINVAL, "ttrl_plans_export: %zu bytes needed", text.size() + 1);
    std::memcpy(buf, text.c_str(), text.size() + 1);
  }
  return TTRL_OK;
}

int ttrl_plans_import(ttrl_ctx* ctx, const char* text, int* count) {
  if (!ctx || !text) return set_error(TTRL_EINVAL, "ttrl_plans_import: null argument");
  int n = 0;
  const char* line = text;
  while (*line) {
    const char* end = std::strchr(line, '\n');
    const size_t size = end ? size_t(end - line) : std::strlen(line);
    const std::string row(line, size);
    const size_t tab = row.find('\t');
    GemmPlan p;
    if (tab != std::string::npos && tab + 1 < row.size() &&
        std::sscanf(row.c_str(), "%d %d %d %d %d %d", &p.cfg, &p.bm, &p.bn, &p.tbk, &p.splits, &p.kchunk) == 6) {
      // A plan is checked against its call's extents when it is used.
      ctx->plans[row.substr(tab + 1)] = p;
      ++n;
    }
    if (!end) break;
    line = end + 1;
  }
  if (count) *count = n;
  return TTRL_OK;
}

// --------------------------------------------------------------- timing ---

int ttrl_timer_start(ttrl_ctx* ctx) {
  if (!ctx) return set_error(TTRL_EINVAL, "ttrl_timer_start: null ctx");
  hipError_t e = hipEventRecord(ctx->t0, ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipEventRecord");
  return TTRL_OK;
}

int ttrl_timer_stop(ttrl_ctx* ctx, float* ms) {
  if (!ctx || !ms) return set_error(TTRL_EINVAL, "ttrl_timer_stop: null argument");
  hipError_t e = hipEventRecord(ctx->t1, ctx->stream);
  if (e != hipSuccess) return hip_error(e, "hipEventRecord");
  e = hipEventSynchronize(ctx->t1);
  if (e != hipSuccess) return hip_error(e, "hipEventSynchronize");
  e = hipEventElapsedTime(ms, ctx->t0, ctx->t1);
  if (e != hipSuccess) return hip_error(e, "hipEventElapsedTime");
  return TTRL_OK;
}

}  // extern "C"
