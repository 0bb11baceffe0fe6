// Host side of the provider behind include/ohip.h: context, memory, weight
// residency, the dispatch gate and the op entry points that choose and launch
// the device kernels in kernels.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cctype>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <unordered_map>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/ohip.h"
#include "internal.hpp"

using namespace ohip;

// ------------------------------------------------------------------ errors
static thread_local std::string g_last_error;

static int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
static int hip_fail(hipError_t e, const char* what) {
  return fail(OHIP_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}
#define HIP_TRY(expr, what)                 \
  do {                                      \
    hipError_t _e = (expr);                 \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

extern "C" const char* ohip_last_error(void) { return g_last_error.c_str(); }

// Records a HIP failure of the node-level dispatcher as the last error.
int ohip_hip_error_internal(hipError_t e, const char* what) { return hip_fail(e, what); }
extern "C" const char* ohip_version(void) { return "oxionnx-hip 0.1.0 (gfx950)"; }

// oxionnx-cuda/src/context.rs:165-193: unset -> false; "", 0, false, no, off
// (trimmed, case-insensitive) -> false; anything else -> true.
extern "C" int ohip_env_flag(const char* name) {
  const char* v = name ? std::getenv(name) : nullptr;
  if (!v) return 0;
  std::string s(v);
  size_t b = s.find_first_not_of(" \t\r\n"), e = s.find_last_not_of(" \t\r\n");
  s = b == std::string::npos ? std::string() : s.substr(b, e - b + 1);
  for (auto& ch : s) ch = (char)std::tolower((unsigned char)ch);
  return !(s.empty() || s == "0" || s == "false" || s == "no" || s == "off");
}

// ------------------------------------------------------------------ types
enum WeightKind { WK_GEMM = 1, WK_CONV = 2, WK_QGEMM = 3, WK_QCONV = 4, WK_CONVT = 5 };

struct ohip_weight {
  ohip_ctx* ctx = nullptr;
  bool cached = false;
  int kind = 0;
  int dtype = 0;           // F32/F16/BF16 for float, I8 for integer
  int64_t rows = 0;        // N (gemm) or Cout (conv)
  int64_t k = 0;           // logical K (gemm) or Cin (conv)
  int64_t kh = 1, kw = 1;  // conv only
  int cpc = 0;             // conv: 16-byte channel chunks per tap
  int kc = 0;              // 16-byte chunks per packed row
  int64_t ld_bytes = 0;
  void* data = nullptr;
  bool pooled = false;            // data is a pool buffer (a transient weight)
  int32_t* colsum = nullptr;      // integer only
  int8_t* flip = nullptr;         // integer only, null when no channel is negated
  int kwrap = 0;                  // integer only: > 0 when each row holds two int8 halves
                                  // (chunks per half, a multiple of 8)
  int kreal = 0;                  // integer only: chunks of one half that hold K
  std::vector<float> scale;       // integer only (1 or rows entries)
  float* comb = nullptr;          // device, rows entries (integer only)
  float comb_a = NAN, comb_y = NAN;
  size_t bytes = 0;
  // ConvTranspose only: the sub-pixel phase filters (packed like a Conv
  // filter, phase ry * ph_sw + rx) for strides (ph_sh, ph_sw) and pad
  // residues (ph_pt, ph_pl); empty when the gather kernel serves the node.
  std::vector<ohip_weight*> phases;
  int64_t ph_sh = 0, ph_sw = 0, ph_pt = 0, ph_pl = 0;
  // all phase filters in one allocation, phase z at z * ph_zstride bytes
  // (when every phase has the same tap count and there are at most four)
  ohip_weight* ph_all = nullptr;
  int64_t ph_zstride = 0;
};

// Stream-ordered caching pool for device buffers (activations, staging).
// Every user of a pooled buffer runs on the context's stream, so a buffer
// returned to the pool may be handed out again at once: the next user's work
// is queued behind the last reads of the previous one.  Nothing is freed to
// HIP before the context is destroyed.
struct DevPool {
  std::multimap<size_t, void*> free_blocks;  // capacity -> buffer
  std::unordered_map<void*, size_t> live;    // buffer -> capacity
  size_t held = 0;                           // bytes held from HIP
  bool parking = false;                      // freed buffers are parked, not reused
  std::vector<std::pair<void*, size_t>> parked;
};

struct ohip_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  ohip_tuning tuning{};
  int tile_override = 0;
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  uint8_t* padtab = nullptr;  // 256 entries of 16 bytes: entry b is sixteen copies of byte b
  std::map<std::string, ohip_weight*> weights;
  std::vector<ohip_weight*> transients;  // freed with the context if never released
  ohip_counters counters{};
  std::string last_decline;
  std::mutex mu;
  std::mutex pool_mu;
  DevPool pool;
  std::map<std::string, uint8_t*> tables;  // device copies of 256-byte output tables, by content
  std::map<std::string, void*> consts;     // device copies of small initializer operands
  std::atomic<uint64_t> device_allocs{0};  // hipMalloc calls made for this context
};

// Every device allocation of a context goes through here, so the counters
// can show that a steady-state forward allocates nothing.
static hipError_t dev_malloc(ohip_ctx* ctx, void** p, size_t bytes) {
  hipError_t e = hipMalloc(p, bytes);
  if (e == hipSuccess) ctx->device_allocs.fetch_add(1, std::memory_order_relaxed);
  return e;
}

// A device buffer shared by a tensor and its aliases (Reshape and friends);
// the last owner returns it to the pool.
struct DevBuf {
  ohip_ctx* ctx;
  void* ptr;
  ~DevBuf();
};

struct ohip_dtensor {
  ohip_ctx* ctx = nullptr;
  std::shared_ptr<DevBuf> buf;
  void* ptr = nullptr;
  int dtype = 0;
  int rank = 0;
  int64_t shape[8] = {0};
  int layout = OHIP_NCHW;
  size_t bytes = 0;
  int64_t pitch = 0;   // NHWC: element slots between consecutive pixels (>= shape[1])
};

static int activate(ohip_ctx* ctx) {
  if (!ctx) return fail(OHIP_E_INVALID, "null context");
  HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
  return OHIP_OK;
}

// One bump-allocated scratch region per call.  The region only grows; growth
// synchronises the stream first so no in-flight kernel still reads the old one.
struct ScratchPlan {
  std::vector<size_t> sizes;
  size_t add(size_t b) {
    sizes.push_back((b + 255) & ~size_t(255));
    return sizes.size() - 1;
  }
  size_t total() const {
    size_t t = 0;
    for (auto s : sizes) t += s;
    return t;
  }
};

static int scratch_reserve(ohip_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return OHIP_OK;
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (ctx->scratch) HIP_TRY(hipFree(ctx->scratch), "hipFree(scratch)");
  ctx->scratch = nullptr;
  ctx->scratch_bytes = 0;
  size_t want = std::max<size_t>(bytes, size_t(1) << 20);
  hipError_t e = dev_malloc(ctx, &ctx->scratch, want);
  if (e != hipSuccess) return fail(OHIP_E_NOMEM, std::string("scratch hipMalloc: ") + hipGetErrorString(e));
  ctx->scratch_bytes = want;
  return OHIP_OK;
}

static void* scratch_at(ohip_ctx* ctx, const ScratchPlan& p, size_t idx) {
  size_t off = 0;
  for (size_t i = 0; i < idx; ++i) off += p.sizes[i];
  return static_cast<char*>(ctx->scratch) + off;
}

static void* plan_at(char* base, const ScratchPlan& p, size_t idx) {
  size_t off = 0;
  for (size_t i = 0; i < idx; ++i) off += p.sizes[i];
  return base + off;
}

// ------------------------------------------------------------------ static scratch
// The scratch of the allocation-free entry points (ohip_conv2d_noalloc): one
// array per GPU, held from the library's load until the process ends.  In
// host code `scratch` names a host-side stand-in, never the device memory:
// its device address is looked up once per device (at context creation, with
// that device current) and only that address is handed to kernels.  Every
// call on a GPU shares its array and it keeps the last call's contents;
// calls that overlap on one GPU (two streams, two contexts) race.
static constexpr size_t kStaticScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

static constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];
static bool g_scratch_looked_up[kMaxScratchDevices];

// Called with `device` current.
static int static_scratch_init(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return fail(OHIP_E_INVALID, "static scratch: device index");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_looked_up[device]) return g_scratch_ptr[device] ? OHIP_OK : fail(OHIP_E_HIP, "static scratch unavailable");
  g_scratch_looked_up[device] = true;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) return hip_fail(e == hipSuccess ? hipErrorInvalidSymbol : e, "hipGetSymbolAddress(scratch)");
  g_scratch_ptr[device] = p;
  return OHIP_OK;
}

// The scratch of one call: the context's growable region, or (noalloc) this
// device's static array, which is never grown.
static int call_scratch(ohip_ctx* ctx, size_t bytes, bool noalloc, char** base) {
  if (!noalloc) {
    int rc = scratch_reserve(ctx, bytes);
    if (rc) return rc;
    *base = static_cast<char*>(ctx->scratch);
    return OHIP_OK;
  }
  if (bytes > kStaticScratchBytes)
    return fail(OHIP_E_NOMEM, "ohip_conv2d_noalloc: needs " + std::to_string(bytes) +
                                  " bytes of scratch, more than the static " + std::to_string(kStaticScratchBytes));
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (ctx->device >= 0 && ctx->device < kMaxScratchDevices) p = g_scratch_ptr[ctx->device];
  }
  if (!p) return fail(OHIP_E_HIP, "ohip_conv2d_noalloc: the static scratch of this device was not set up");
  *base = static_cast<char*>(p);
  return OHIP_OK;
}

// ------------------------------------------------------------------ context
extern "C" int ohip_device_count(int* count) {
  if (!count) return fail(OHIP_E_INVALID, "null count");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;
  *count = n;
  return OHIP_OK;
}

extern "C" int ohip_ctx_create(int device, ohip_ctx** out) {
  if (!out) return fail(OHIP_E_INVALID, "null out");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(OHIP_E_NODEVICE, "no HIP device");
  if (device < 0 || device >= n) return fail(OHIP_E_INVALID, "device index out of range");
  HIP_TRY(hipSetDevice(device), "hipSetDevice");
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(OHIP_E_NODEVICE, std::string("kernels are built for gfx950, device is ") + prop.gcnArchName);
  auto* ctx = new (std::nothrow) ohip_ctx();
  if (!ctx) return fail(OHIP_E_NOMEM, "context allocation");
  ctx->device = device;
  hipError_t e = hipStreamCreateWithFlags(&ctx->own, hipStreamDefault);
  if (e != hipSuccess) {
    delete ctx;
    return hip_fail(e, "hipStreamCreate");
  }
  ctx->stream = ctx->own;
  {
    std::vector<uint8_t> tab(256 * 16);
    for (int b = 0; b < 256; ++b) std::memset(tab.data() + b * 16, b, 16);
    e = dev_malloc(ctx, (void**)&ctx->padtab, tab.size());
    if (e == hipSuccess) e = hipMemcpy(ctx->padtab, tab.data(), tab.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      if (ctx->padtab) (void)hipFree(ctx->padtab);
      (void)hipStreamDestroy(ctx->own);
      delete ctx;
      return hip_fail(e, "pad table");
    }
  }
  ohip_tuning_for_class(OHIP_CLASS_MI355X, &ctx->tuning);
  // A failed lookup leaves only ohip_conv2d_noalloc unusable on this device.
  if (static_scratch_init(device) != OHIP_OK) (void)hipGetLastError();
  *out = ctx;
  return OHIP_OK;
}

static int pool_free(ohip_ctx* ctx, void* p);

static void weight_free(ohip_weight* w) {
  if (!w) return;
  for (auto* p : w->phases) weight_free(p);
  if (w->ph_all) weight_free(w->ph_all);
  if (w->data && w->pooled) (void)pool_free(w->ctx, w->data);
  else if (w->data) (void)hipFree(w->data);
  if (w->colsum) (void)hipFree(w->colsum);
  if (w->flip) (void)hipFree(w->flip);
  if (w->comb) (void)hipFree(w->comb);
  delete w;
}

extern "C" void ohip_ctx_destroy(ohip_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  for (auto& kv : ctx->weights) weight_free(kv.second);
  for (auto* w : ctx->transients) weight_free(w);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->padtab) (void)hipFree(ctx->padtab);
  for (auto& kv : ctx->tables) (void)hipFree(kv.second);
  for (auto& kv : ctx->consts) (void)hipFree(kv.second);
  for (auto& kv : ctx->pool.free_blocks) (void)hipFree(kv.second);
  for (auto& kv : ctx->pool.live) (void)hipFree(kv.first);
  if (ctx->own) (void)hipStreamDestroy(ctx->own);
  delete ctx;
}

extern "C" int ohip_ctx_set_stream(ohip_ctx* ctx, void* s) {
  if (!ctx) return fail(OHIP_E_INVALID, "null context");
  ctx->stream = s ? static_cast<hipStream_t>(s) : ctx->own;
  return OHIP_OK;
}
extern "C" void* ohip_ctx_stream(ohip_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

extern "C" int ohip_sync(ohip_ctx* ctx) {
  int rc = activate(ctx);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  ctx->counters.stream_syncs++;
  return OHIP_OK;
}

extern "C" int ohip_set_tile_override(ohip_ctx* ctx, int tile_id) {
  if (!ctx) return fail(OHIP_E_INVALID, "null context");
  if (tile_id < 0 || tile_id > 18) return fail(OHIP_E_INVALID, "tile id must be 0..18");
  ctx->tile_override = tile_id;
  return OHIP_OK;
}

// ------------------------------------------------------------------ memory
static size_t pool_class(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= (64u << 10)) return (bytes + 255) & ~(size_t)255;
  if (bytes <= (16u << 20)) return (bytes + 4095) & ~(size_t)4095;
  return (bytes + (2u << 20) - 1) & ~(((size_t)2 << 20) - 1);
}

static int pool_alloc(ohip_ctx* ctx, size_t bytes, void** p) {
  const size_t cap = pool_class(bytes);
  std::lock_guard<std::mutex> lock(ctx->pool_mu);
  auto it = ctx->pool.free_blocks.lower_bound(cap);
  if (it != ctx->pool.free_blocks.end() && it->first <= 2 * cap) {
    *p = it->second;
    ctx->pool.live[*p] = it->first;
    ctx->pool.free_blocks.erase(it);
    return OHIP_OK;
  }
  hipError_t e = dev_malloc(ctx, p, cap);
  if (e != hipSuccess) {
    // give the cached blocks back to HIP once and retry
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->pool.free_blocks) { (void)hipFree(kv.second); ctx->pool.held -= kv.first; }
    ctx->pool.free_blocks.clear();
    e = dev_malloc(ctx, p, cap);
    if (e != hipSuccess) return fail(OHIP_E_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
  }
  ctx->pool.live[*p] = cap;
  ctx->pool.held += cap;
  return OHIP_OK;
}

static int pool_free(ohip_ctx* ctx, void* p) {
  if (!p) return OHIP_OK;
  std::lock_guard<std::mutex> lock(ctx->pool_mu);
  auto it = ctx->pool.live.find(p);
  if (it == ctx->pool.live.end()) return fail(OHIP_E_INVALID, "ohip_free: not a buffer of this context");
  if (ctx->pool.parking) ctx->pool.parked.emplace_back(p, it->second);
  else ctx->pool.free_blocks.emplace(it->second, p);
  ctx->pool.live.erase(it);
  return OHIP_OK;
}

// ------------------------------------------------------------------ graphs
// A captured forward.  While a capture (or a parking dry run) is open, freed
// pool buffers are parked instead of reused, so every buffer the captured
// kernels touch stays reserved for the graph; the graph returns them to the
// pool when destroyed.
struct ohip_graph {
  ohip_ctx* ctx = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<std::pair<void*, size_t>> held;
};

static void unpark_all(ohip_ctx* ctx, std::vector<std::pair<void*, size_t>>& v) {
  for (auto& pb : v) ctx->pool.free_blocks.emplace(pb.second, pb.first);
  v.clear();
}

extern "C" int ohip_pool_parking(ohip_ctx* ctx, int on) {
  if (!ctx) return fail(OHIP_E_INVALID, "null context");
  std::lock_guard<std::mutex> lock(ctx->pool_mu);
  ctx->pool.parking = on != 0;
  if (!on) unpark_all(ctx, ctx->pool.parked);
  return OHIP_OK;
}

extern "C" int ohip_graph_begin(ohip_ctx* ctx) {
  int rc = activate(ctx);
  if (rc) return rc;
  {
    std::lock_guard<std::mutex> lock(ctx->pool_mu);
    unpark_all(ctx, ctx->pool.parked);
    ctx->pool.parking = true;
  }
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) {
    std::lock_guard<std::mutex> lock(ctx->pool_mu);
    ctx->pool.parking = false;
    return hip_fail(e, "hipStreamBeginCapture");
  }
  return OHIP_OK;
}

extern "C" int ohip_graph_end(ohip_ctx* ctx, ohip_graph** out) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!out) return fail(OHIP_E_INVALID, "null out");
  auto* g = new ohip_graph();
  g->ctx = ctx;
  hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
  {
    std::lock_guard<std::mutex> lock(ctx->pool_mu);
    ctx->pool.parking = false;
    g->held.swap(ctx->pool.parked);
  }
  if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    if (g->graph) (void)hipGraphDestroy(g->graph);
    std::lock_guard<std::mutex> lock(ctx->pool_mu);
    unpark_all(ctx, g->held);
    delete g;
    return hip_fail(e, "graph capture");
  }
  *out = g;
  return OHIP_OK;
}

extern "C" int ohip_graph_launch(ohip_graph* g) {
  if (!g) return fail(OHIP_E_INVALID, "null graph");
  int rc = activate(g->ctx);
  if (rc) return rc;
  HIP_TRY(hipGraphLaunch(g->exec, g->ctx->stream), "hipGraphLaunch");
  return OHIP_OK;
}

extern "C" void ohip_graph_destroy(ohip_graph* g) {
  if (!g) return;
  (void)hipSetDevice(g->ctx->device);
  (void)hipStreamSynchronize(g->ctx->stream);
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  {
    std::lock_guard<std::mutex> lock(g->ctx->pool_mu);
    unpark_all(g->ctx, g->held);
  }
  delete g;
}

DevBuf::~DevBuf() {
  if (ptr && ctx) (void)pool_free(ctx, ptr);
}

// Device buffers come from the context's stream-ordered pool: ohip_free
// returns a buffer for reuse by later work on the same stream without a
// device synchronisation.
extern "C" int ohip_malloc(ohip_ctx* ctx, size_t bytes, void** p) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!p) return fail(OHIP_E_INVALID, "null out");
  return pool_alloc(ctx, bytes, p);
}
extern "C" int ohip_free(ohip_ctx* ctx, void* p) {
  int rc = activate(ctx);
  if (rc) return rc;
  return pool_free(ctx, p);
}
extern "C" int ohip_memcpy_h2d(ohip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = activate(ctx);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync H2D");
  ctx->counters.h2d_bytes += bytes;
  return OHIP_OK;
}
extern "C" int ohip_memcpy_d2h(ohip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = activate(ctx);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync D2H");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  ctx->counters.d2h_bytes += bytes;
  ctx->counters.stream_syncs++;
  return OHIP_OK;
}
extern "C" int ohip_memcpy_d2d(ohip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = activate(ctx);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream), "hipMemcpyAsync D2D");
  return OHIP_OK;
}

// ------------------------------------------------------------------ gate
// Thresholds for MI355X.  The reference's discrete-class numbers
// (tuning.rs:487-545) were measured for an RTX A4000 behind PCIe with a
// 24-thread host.  An MI355X finishes even the per-dispatch-upload cases far
// sooner, so the floors are derived from its own cost model (PCIe Gen5 x16
// ~50 GB/s effective, ~20 us fixed round trip, the reference's single-thread
// 2-D sgemm at ~50 GFLOP/s): a per-dispatch GEMM wins once 2mkn / 50e9 exceeds
// 20 us + 4 (mk + kn + mn) / 50e9, i.e. mkn >= ~1e6 and intensity >= ~8; a
// cached B removes the k·n upload, leaving the fixed cost (mkn >= ~5e5).
// Conv's implied GEMM uses the same fixed-cost floor.  bench.py and
// tests/test_gate.py record the measured crossovers these are checked by.
extern "C" int ohip_tuning_for_class(int cls, ohip_tuning* t) {
  if (!t) return fail(OHIP_E_INVALID, "null tuning");
  switch (cls) {
    case OHIP_CLASS_MI355X:
      // Measured crossovers against the reference's CPU algorithms on an
      // MI355X box's host (bench.py --only gate): the smallest sizes at and
      // above which every measured shape ran faster on the device.  No
      // intensity gate: no shape above the size floor lost, down to intensity 2.
      *t = ohip_tuning{OHIP_CLASS_MI355X, 4000000ull, 1500000ull, 0ull, 600000ull};
      return OHIP_OK;
    case OHIP_CLASS_PARITY:  // GpuTuning::PARITY (tuning.rs:409-425)
      *t = ohip_tuning{OHIP_CLASS_PARITY, 0, 0, 0, 0};
      return OHIP_OK;
    case OHIP_CLASS_NEVER:  // GpuTuning::NEVER (tuning.rs:441-456)
      *t = ohip_tuning{OHIP_CLASS_NEVER, UINT64_MAX, UINT64_MAX, UINT64_MAX, UINT64_MAX};
      return OHIP_OK;
    case OHIP_CLASS_LEGACY:  // GpuTuning::for_class(Discrete) (tuning.rs:487-545)
      *t = ohip_tuning{OHIP_CLASS_LEGACY, 25000000ull, 5000000ull, 56ull, 10000000ull};
      return OHIP_OK;
    default: return fail(OHIP_E_INVALID, "unknown perf class");
  }
}
extern "C" int ohip_set_tuning(ohip_ctx* ctx, const ohip_tuning* t) {
  if (!ctx || !t) return fail(OHIP_E_INVALID, "null argument");
  ctx->tuning = *t;
  return OHIP_OK;
}
extern "C" int ohip_get_tuning(ohip_ctx* ctx, ohip_tuning* t) {
  if (!ctx || !t) return fail(OHIP_E_INVALID, "null argument");
  *t = ctx->tuning;
  return OHIP_OK;
}

static bool mul_ok(uint64_t a, uint64_t b, uint64_t* r) { return !__builtin_mul_overflow(a, b, r); }

// gemm_mac (tuning.rs:500-503); false on u64 overflow.
static bool gemm_mac_checked(int64_t m, int64_t k, int64_t n, uint64_t* mac) {
  if (m < 0 || k < 0 || n < 0) return false;
  uint64_t mk;
  return mul_ok((uint64_t)m, (uint64_t)k, &mk) && mul_ok(mk, (uint64_t)n, mac);
}
extern "C" uint64_t ohip_gemm_mac(int64_t m, int64_t k, int64_t n) {
  uint64_t mac = 0;
  return gemm_mac_checked(m, k, n, &mac) ? mac : UINT64_MAX;
}
// gemm_intensity (tuning.rs:516-529): floor(2mkn / (mk + kn + mn)); 0 if
// degenerate or overflowing (the reference's None).
extern "C" uint64_t ohip_gemm_intensity(int64_t m, int64_t k, int64_t n) {
  if (m < 0 || k < 0 || n < 0) return 0;
  uint64_t mk, kn, mn, mkn, f;
  if (!mul_ok(m, k, &mk) || !mul_ok(k, n, &kn) || !mul_ok(m, n, &mn)) return 0;
  uint64_t moved;
  if (__builtin_add_overflow(mk, kn, &moved) || __builtin_add_overflow(moved, mn, &moved) || moved == 0) return 0;
  if (!mul_ok(mk, n, &mkn) || !mul_ok(mkn, 2, &f)) return 0;
  return f / moved;
}
// gemm_admits (tuning.rs:575-594): zero extents and overflow decline.
extern "C" int ohip_gemm_admits(const ohip_tuning* t, int64_t m, int64_t k, int64_t n, int cached) {
  if (!t || m <= 0 || k <= 0 || n <= 0) return 0;
  uint64_t mac;
  if (!gemm_mac_checked(m, k, n, &mac)) return 0;
  if (cached) return mac >= t->gemm_min_mac_cached;
  if (mac < t->gemm_min_mac) return 0;
  if (t->gemm_min_intensity == 0) return 1;
  uint64_t i = ohip_gemm_intensity(m, k, n);
  return i != 0 && i >= t->gemm_min_intensity;
}
// conv_admits (tuning.rs:606-610): only overflow declines outright.
extern "C" int ohip_conv_admits(const ohip_tuning* t, int64_t m, int64_t k, int64_t n) {
  uint64_t mac;
  if (!t || !gemm_mac_checked(m, k, n, &mac)) return 0;
  return mac >= t->conv_min_mac;
}

// ------------------------------------------------------------------ host conversions
static inline uint16_t f32_to_f16_rne(float f) { return f32_to_f16_bits(f); }
static inline float f16_to_f32(uint16_t h) { return f16_bits_to_f32(h); }
static inline uint16_t f32_to_bf16_rne(float f) { return f32_to_bf16_bits(f); }
static inline float bf16_to_f32(uint16_t h) { return bf16_bits_to_f32(h); }

static int elem_bytes(int dt) {
  switch (dt) {
    case OHIP_F32: case OHIP_I32: return 4;
    case OHIP_F16: case OHIP_BF16: return 2;
    case OHIP_U8: case OHIP_I8: return 1;
    default: return 0;
  }
}
static bool is_float(int dt) { return dt == OHIP_F32 || dt == OHIP_F16 || dt == OHIP_BF16; }
static int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

static float read_float(int dt, const void* p, int64_t i) {
  switch (dt) {
    case OHIP_F32: return static_cast<const float*>(p)[i];
    case OHIP_F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case OHIP_BF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    default: return 0.0f;
  }
}
// Write v (given as the source element's value) into a dtype slot.  A
// same-dtype copy keeps the exact bits.
static void write_elem(int dst_dt, void* dst, int64_t i, int src_dt, const void* src, int64_t si) {
  if (dst_dt == src_dt) {
    int b = elem_bytes(dst_dt);
    std::memcpy(static_cast<char*>(dst) + i * b, static_cast<const char*>(src) + si * b, b);
    return;
  }
  float v = read_float(src_dt, src, si);
  switch (dst_dt) {
    case OHIP_F32: static_cast<float*>(dst)[i] = v; break;
    case OHIP_F16: static_cast<uint16_t*>(dst)[i] = f32_to_f16_rne(v); break;
    case OHIP_BF16: static_cast<uint16_t*>(dst)[i] = f32_to_bf16_rne(v); break;
    default: break;
  }
}

// ------------------------------------------------------------------ weights
static std::string cache_key(const ohip_weight_key* key, int kind, int dtype, size_t src_bytes,
                             const std::vector<int64_t>& shape) {
  std::string k(key->name);
  k += '\x1f';
  k += key->label ? key->label : "";
  k += '\x1f' + std::to_string(kind) + '\x1f' + std::to_string(dtype) + '\x1f' + std::to_string(src_bytes);
  for (auto s : shape) k += '\x1f' + std::to_string(s);
  return k;
}

// Returns the cached weight for key or null; sets *key_str for the insert.
static ohip_weight* cache_lookup(ohip_ctx* ctx, const ohip_weight_key* key, const std::string& ks) {
  if (!key || !key->name) return nullptr;
  auto it = ctx->weights.find(ks);
  if (it == ctx->weights.end()) return nullptr;
  ctx->counters.weight_hits++;
  return it->second;
}

static int weight_upload(ohip_ctx* ctx, ohip_weight* w, const void* packed, size_t bytes) {
  hipError_t e = dev_malloc(ctx, &w->data, bytes ? bytes : 16);
  if (e != hipSuccess) return fail(OHIP_E_NOMEM, std::string("weight hipMalloc: ") + hipGetErrorString(e));
  HIP_TRY(hipMemcpyAsync(w->data, packed, bytes, hipMemcpyHostToDevice, ctx->stream), "weight upload");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "weight upload sync");
  w->bytes = bytes;
  ctx->counters.weight_uploaded_bytes += bytes;
  ctx->counters.h2d_bytes += bytes;
  return OHIP_OK;
}

static int weight_finish(ohip_ctx* ctx, const ohip_weight_key* key, const std::string& ks, ohip_weight* w,
                         ohip_weight** out) {
  w->ctx = ctx;
  if (key && key->name) {
    w->cached = true;
    ctx->weights[ks] = w;
    ctx->counters.weight_misses++;
    ctx->counters.weight_resident_bytes += w->bytes;
  } else {
    ctx->counters.weight_transient++;
    ctx->transients.push_back(w);
  }
  *out = w;
  return OHIP_OK;
}

extern "C" void ohip_weight_release(ohip_weight* w) {
  if (!w || w->cached) return;
  ohip_ctx* ctx = w->ctx;
  std::lock_guard<std::mutex> lock(ctx->mu);
  auto it = std::find(ctx->transients.begin(), ctx->transients.end(), w);
  if (it == ctx->transients.end()) return;
  ctx->transients.erase(it);
  (void)hipSetDevice(ctx->device);
  // a pooled weight goes back to the stream-ordered pool: work queued after
  // this on the stream may reuse it, so no wait is needed
  bool pool_only = w->pooled && !w->colsum && !w->flip && !w->comb && w->phases.empty() && !w->ph_all;
  if (!pool_only) (void)hipStreamSynchronize(ctx->stream);
  weight_free(w);
}
extern "C" size_t ohip_weight_bytes(const ohip_weight* w) { return w ? w->bytes : 0; }

static int chunk_elems(int dt) { return 16 / elem_bytes(dt); }

// Packs a Gemm B operand on the device: the host matrix is copied as it is
// into a pool buffer, converted to the compute dtype (the rounding of
// f32_to_f16_bits / f32_to_bf16_bits) and brought into [N][Kp] K-contiguous
// rows (zero padded) by the transpose or row-gather kernel.  A cached weight
// gets a buffer of its own; a transient one (no key) lives in a pool buffer,
// so a per-dispatch B costs one host copy and two small kernels, and no
// device allocation once the pool holds its size.
static int gemm_weight_pack_device(ohip_ctx* ctx, ohip_weight* w, const void* host, int src_dt, int64_t k, int64_t n,
                                   int trans_b, int64_t kp, bool cached) {
  w->ctx = ctx;
  const int dt = w->dtype, eb = elem_bytes(dt);
  const size_t raw = (size_t)(k * n) * elem_bytes(src_dt), packed = (size_t)(n * kp) * eb;
  if (k * n > INT_MAX || n * kp > INT_MAX) return fail(OHIP_DECLINED, "ohip_weight_gemm: operand too large");
  void* stage = nullptr;
  void* conv = nullptr;
  int rc = pool_alloc(ctx, raw, &stage);
  if (rc) return rc;
  auto cleanup = [&]() {
    if (conv && conv != stage) (void)pool_free(ctx, conv);
    (void)pool_free(ctx, stage);
  };
  hipError_t e = hipMemcpyAsync(stage, host, raw, hipMemcpyHostToDevice, ctx->stream);
  // the caller's host buffer may go away when this returns
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) { cleanup(); return hip_fail(e, "weight upload"); }
  conv = stage;
  if (src_dt != dt) {
    rc = pool_alloc(ctx, (size_t)(k * n) * eb, &conv);
    if (rc) { conv = nullptr; cleanup(); return rc; }
    e = run_convert_float(src_dt, dt, stage, conv, k * n, ctx->stream);
    if (e != hipSuccess) { cleanup(); return hip_fail(e, "weight conversion"); }
  }
  if (cached) {
    e = dev_malloc(ctx, &w->data, packed ? packed : 16);
    if (e != hipSuccess) { cleanup(); return fail(OHIP_E_NOMEM, std::string("weight hipMalloc: ") + hipGetErrorString(e)); }
  } else {
    rc = pool_alloc(ctx, packed ? packed : 16, &w->data);
    if (rc) { cleanup(); return rc; }
    w->pooled = true;
  }
  e = trans_b ? run_gather2d(eb, conv, k, 1, w->data, (int)n, (int)k, (int)kp, ctx->stream)
              : run_transpose_batched(eb, conv, w->data, 1, (int)k, (int)n, (int)kp, ctx->stream);
  cleanup();
  if (e != hipSuccess) return hip_fail(e, "weight packing");
  if (cached) {
    // a cached weight is read by later calls on any stream the caller picks
    HIP_TRY(hipStreamSynchronize(ctx->stream), "weight packing sync");
  }
  w->bytes = packed;
  ctx->counters.weight_uploaded_bytes += raw;
  ctx->counters.h2d_bytes += raw;
  return OHIP_OK;
}

extern "C" int ohip_weight_gemm(ohip_ctx* ctx, const ohip_weight_key* key, int src_dt, const void* host,
                                int64_t k, int64_t n, int trans_b, int dt, ohip_weight** out) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!host || !out || !is_float(src_dt) || !is_float(dt) || k <= 0 || n <= 0 || k > INT_MAX || n > INT_MAX)
    return fail(OHIP_E_INVALID, "ohip_weight_gemm: bad arguments");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const size_t src_bytes = (size_t)(k * n) * elem_bytes(src_dt);
  std::string ks = key && key->name ? cache_key(key, WK_GEMM, dt, src_bytes, {k, n, trans_b}) : std::string();
  if (ohip_weight* hit = cache_lookup(ctx, key, ks)) {
    *out = hit;
    return OHIP_OK;
  }
  const int64_t ce = chunk_elems(dt), kp = round_up(k, ce);
  auto* w = new ohip_weight();
  w->kind = WK_GEMM; w->dtype = dt; w->rows = n; w->k = k;
  w->kc = (int)(kp / ce); w->ld_bytes = kp * elem_bytes(dt);
  rc = gemm_weight_pack_device(ctx, w, host, src_dt, k, n, trans_b, kp, key && key->name);
  if (rc) { weight_free(w); return rc; }
  return weight_finish(ctx, key, ks, w, out);
}

extern "C" int ohip_weight_conv(ohip_ctx* ctx, const ohip_weight_key* key, int src_dt, const void* host,
                                int64_t cout, int64_t cin, int64_t kh, int64_t kw, int dt, ohip_weight** out) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!host || !out || !is_float(src_dt) || !is_float(dt) || cout <= 0 || cin <= 0 || kh <= 0 || kw <= 0)
    return fail(OHIP_E_INVALID, "ohip_weight_conv: bad arguments");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const size_t src_bytes = (size_t)(cout * cin * kh * kw) * elem_bytes(src_dt);
  std::string ks = key && key->name ? cache_key(key, WK_CONV, dt, src_bytes, {cout, cin, kh, kw}) : std::string();
  if (ohip_weight* hit = cache_lookup(ctx, key, ks)) {
    *out = hit;
    return OHIP_OK;
  }
  const int64_t ce = chunk_elems(dt), cp = round_up(cin, ce), kp = kh * kw * cp;
  if (kp > INT_MAX / 2) return fail(OHIP_E_INVALID, "ohip_weight_conv: filter too large");
  // [Cout][Cin][KH][KW] -> [Cout][KH][KW][Cp], channels innermost.
  std::vector<char> packed((size_t)(cout * kp) * elem_bytes(dt), 0);
  for (int64_t o = 0; o < cout; ++o)
    for (int64_t c = 0; c < cin; ++c)
      for (int64_t y = 0; y < kh; ++y)
        for (int64_t x = 0; x < kw; ++x)
          write_elem(dt, packed.data(), o * kp + (y * kw + x) * cp + c, src_dt, host, ((o * cin + c) * kh + y) * kw + x);
  auto* w = new ohip_weight();
  w->kind = WK_CONV; w->dtype = dt; w->rows = cout; w->k = cin; w->kh = kh; w->kw = kw;
  w->cpc = (int)(cp / ce); w->kc = (int)(kp / ce); w->ld_bytes = kp * elem_bytes(dt);
  rc = weight_upload(ctx, w, packed.data(), packed.size());
  if (rc) { weight_free(w); return rc; }
  return weight_finish(ctx, key, ks, w, out);
}

// ConvTranspose filter: [Cin][Cout/group][KH][KW] kept as is (converted to
// the compute dtype) for the gather kernel, plus, for group 1, dilation 1 and
// a kernel at least as wide as the stride, the sub-pixel phase filters.
// Output phase (ry, rx) = (oy mod sh, ox mod sw) receives exactly the taps
// ky = ky0 + sh * m with ky0 = (ry + pt) mod sh (likewise kx), and reads input
// row iy = (oy + pt - ky) / sh, so over the phase's output grid it is a
// stride-1 convolution with Mky = ceil((KH - ky0) / sh) taps, taken in
// reverse: phase tap m' holds ky0 + sh * (Mky - 1 - m').  Each phase filter is
// packed like a Conv filter, [Cout][Mky][Mkx][Cp].
extern "C" int ohip_weight_conv_transpose(ohip_ctx* ctx, const ohip_weight_key* key, int src_dt, const void* host,
                                          int64_t cin, int64_t coutg, int64_t kh, int64_t kw, int64_t stride_h,
                                          int64_t stride_w, int64_t pad_t, int64_t pad_l, int64_t dil_h,
                                          int64_t dil_w, int64_t group, int dt, ohip_weight** out) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!host || !out || !is_float(src_dt) || !is_float(dt) || cin <= 0 || coutg <= 0 || kh <= 0 || kw <= 0 ||
      stride_h <= 0 || stride_w <= 0 || pad_t < 0 || pad_l < 0 || dil_h <= 0 || dil_w <= 0 || group <= 0)
    return fail(OHIP_E_INVALID, "ohip_weight_conv_transpose: bad arguments");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const int64_t count = cin * coutg * kh * kw;
  const size_t src_bytes = (size_t)count * elem_bytes(src_dt);
  const bool phased = group == 1 && dil_h == 1 && dil_w == 1 && kh >= stride_h && kw >= stride_w;
  std::string ks;
  if (key && key->name)
    ks = cache_key(key, WK_CONVT, dt, src_bytes,
                   {cin, coutg, kh, kw, group, phased ? stride_h : 0, phased ? stride_w : 0,
                    phased ? pad_t % stride_h : 0, phased ? pad_l % stride_w : 0});
  if (ohip_weight* hit = cache_lookup(ctx, key, ks)) {
    *out = hit;
    return OHIP_OK;
  }
  const int eb = elem_bytes(dt);
  std::vector<char> conv((size_t)count * eb);
  for (int64_t i = 0; i < count; ++i) write_elem(dt, conv.data(), i, src_dt, host, i);
  auto* w = new ohip_weight();
  w->kind = WK_CONVT; w->dtype = dt; w->rows = cin; w->k = coutg; w->kh = kh; w->kw = kw;
  w->ld_bytes = coutg * kh * kw * eb;
  rc = weight_upload(ctx, w, conv.data(), conv.size());
  if (rc) { weight_free(w); return rc; }
  if (phased) {
    w->ph_sh = stride_h; w->ph_sw = stride_w; w->ph_pt = pad_t % stride_h; w->ph_pl = pad_l % stride_w;
    const int64_t ce = chunk_elems(dt), cp = round_up(cin, ce);
    std::vector<char> all;   // every phase's packed filter, in phase order
    int64_t all_kp = 0;      // their common K extent (-1: they differ)
    for (int64_t ry = 0; ry < stride_h; ++ry)
      for (int64_t rx = 0; rx < stride_w; ++rx) {
        const int64_t ky0 = (ry + pad_t) % stride_h, kx0 = (rx + pad_l) % stride_w;
        const int64_t mky = (kh - ky0 + stride_h - 1) / stride_h, mkx = (kw - kx0 + stride_w - 1) / stride_w;
        const int64_t kp = mky * mkx * cp;
        std::vector<char> packed((size_t)(coutg * kp) * eb, 0);
        for (int64_t o = 0; o < coutg; ++o)
          for (int64_t my = 0; my < mky; ++my)
            for (int64_t mx = 0; mx < mkx; ++mx) {
              const int64_t ky = ky0 + stride_h * (mky - 1 - my), kx = kx0 + stride_w * (mkx - 1 - mx);
              for (int64_t c = 0; c < cin; ++c)
                write_elem(dt, packed.data(), o * kp + (my * mkx + mx) * cp + c, src_dt, host,
                           ((c * coutg + o) * kh + ky) * kw + kx);
            }
        auto* ph = new ohip_weight();
        ph->ctx = ctx; ph->kind = WK_CONV; ph->dtype = dt; ph->rows = coutg; ph->k = cin; ph->kh = mky; ph->kw = mkx;
        ph->cpc = (int)(cp / ce); ph->kc = (int)(kp / ce); ph->ld_bytes = kp * eb;
        rc = weight_upload(ctx, ph, packed.data(), packed.size());
        if (rc) { weight_free(ph); weight_free(w); return rc; }
        w->bytes += ph->bytes;
        w->phases.push_back(ph);
        all.insert(all.end(), packed.begin(), packed.end());
        if (all_kp == 0) all_kp = kp;
        if (kp != all_kp) all_kp = -1;
      }
    const int64_t nph = stride_h * stride_w;
    if (all_kp > 0 && nph <= 4) {
      auto* pa = new ohip_weight();
      pa->ctx = ctx; pa->kind = WK_CONV; pa->dtype = dt; pa->rows = coutg; pa->k = cin;
      pa->kh = w->phases[0]->kh; pa->kw = w->phases[0]->kw; pa->cpc = w->phases[0]->cpc; pa->kc = w->phases[0]->kc;
      pa->ld_bytes = all_kp * eb;
      rc = weight_upload(ctx, pa, all.data(), all.size());
      if (rc) { weight_free(pa); weight_free(w); return rc; }
      w->bytes += pa->bytes;
      w->ph_all = pa;
      w->ph_zstride = coutg * all_kp * eb;
    }
  }
  return weight_finish(ctx, key, ks, w, out);
}

// Integer packing.  Each weight channel becomes v = w - w_zp[channel] in
// K-contiguous int8 rows, plus sum(v) for the epilogue's zero-point
// correction.  v spans at most 255 consecutive values inside [-255, 255]:
//   * a channel whose maximum exceeds 254 is stored negated (its range then
//     lies in [-255, 0]) and flagged, and the epilogue negates it back;
//   * when any stored value leaves [-128, 127], every row holds two int8
//     halves v1 = clamp(v, -128, 127) and v2 = v - v1 (both in range), laid
//     out as [v1 row | v2 row], each half padded with zeros to a multiple of
//     128 bytes (one MFMA stage); the activation is re-read for the second
//     half (kwrap), which doubles K but keeps the int8 MFMA path exact.
struct QPacked {
  std::vector<int8_t> data;
  std::vector<int32_t> colsum;
  std::vector<int8_t> flip;
  bool any_flip = false;
  int64_t kp = 0;
  int64_t half = 0;  // bytes per half of a split row (kp rounded up to 128)
  bool split = false;
};

template <class ValueAt>
static void qpack_rows(int64_t rows, int64_t kp, int64_t klen, ValueAt value_at, QPacked& q) {
  // value_at(row, j) gives v for j < klen, where j indexes the packed K axis
  // (positions the caller never fills are zero)
  std::vector<int32_t> v((size_t)(rows * kp), 0);
  q.colsum.assign((size_t)rows, 0);
  q.flip.assign((size_t)rows, 0);
  int32_t lo = 0, hi = 0;
  for (int64_t r = 0; r < rows; ++r) {
    int32_t mx = INT32_MIN;
    for (int64_t j = 0; j < klen; ++j) {
      int32_t x;
      if (!value_at(r, j, &x)) continue;
      v[(size_t)(r * kp + j)] = x;
      mx = std::max(mx, x);
    }
    const bool flip = mx > 254;
    int32_t s = 0;
    for (int64_t j = 0; j < kp; ++j) {
      int32_t& x = v[(size_t)(r * kp + j)];
      if (flip) x = -x;
      s += x;
      lo = std::min(lo, x);
      hi = std::max(hi, x);
    }
    q.colsum[(size_t)r] = s;
    q.flip[(size_t)r] = flip ? 1 : 0;
    q.any_flip |= flip;
  }
  q.kp = kp;
  q.split = lo < -128 || hi > 127;
  q.half = q.split ? (kp + 127) / 128 * 128 : kp;
  const int64_t width = q.split ? 2 * q.half : kp;
  q.data.assign((size_t)(rows * width), 0);
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < kp; ++j) {
      const int32_t x = v[(size_t)(r * kp + j)];
      const int32_t a = std::min(127, std::max(-128, x));
      q.data[(size_t)(r * width + j)] = (int8_t)a;
      if (q.split) q.data[(size_t)(r * width + q.half + j)] = (int8_t)(x - a);
    }
}

static int qpack_upload(ohip_ctx* ctx, ohip_weight* w, const QPacked& q, const float* scale, int n_scale) {
  w->kwrap = q.split ? (int)(q.half / 16) : 0;
  w->kreal = (int)(q.kp / 16);
  w->kc = (int)((q.split ? 2 * q.half : q.kp) / 16);
  w->ld_bytes = q.split ? 2 * q.half : q.kp;
  int rc = weight_upload(ctx, w, q.data.data(), q.data.size());
  if (rc) return rc;
  hipError_t e = dev_malloc(ctx, (void**)&w->colsum, q.colsum.size() * 4);
  if (e != hipSuccess) return fail(OHIP_E_NOMEM, "colsum hipMalloc");
  HIP_TRY(hipMemcpy(w->colsum, q.colsum.data(), q.colsum.size() * 4, hipMemcpyHostToDevice), "colsum upload");
  if (q.any_flip) {
    e = dev_malloc(ctx, (void**)&w->flip, q.flip.size());
    if (e != hipSuccess) return fail(OHIP_E_NOMEM, "flip hipMalloc");
    HIP_TRY(hipMemcpy(w->flip, q.flip.data(), q.flip.size(), hipMemcpyHostToDevice), "flip upload");
    w->bytes += q.flip.size();
  }
  e = dev_malloc(ctx, (void**)&w->comb, (size_t)w->rows * 4);
  if (e != hipSuccess) return fail(OHIP_E_NOMEM, "comb hipMalloc");
  if (scale && n_scale > 0) w->scale.assign(scale, scale + n_scale);
  w->bytes += q.colsum.size() * 4 + (size_t)w->rows * 4;
  return OHIP_OK;
}

// The weight scales of a cached integer weight are re-read on every dispatch
// (they are separate initializers); the combined scales are only recomputed
// when they changed.
static bool same_scales(const std::vector<float>& have, const float* s, int n) {
  if ((int)have.size() != n) return false;
  for (int i = 0; i < n; ++i)
    if (!(have[(size_t)i] == s[i])) return false;
  return true;
}

static int32_t int_at(int dt, const void* p, int64_t i) {
  return dt == OHIP_U8 ? (int32_t) static_cast<const uint8_t*>(p)[i] : (int32_t) static_cast<const int8_t*>(p)[i];
}

extern "C" int ohip_weight_qgemm(ohip_ctx* ctx, const ohip_weight_key* key, int src_dt, const void* host,
                                 int64_t k, int64_t n, int trans_b, const int32_t* zp, int n_zp,
                                 const float* scale, int n_scale, ohip_weight** out) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!host || !out || (src_dt != OHIP_U8 && src_dt != OHIP_I8) || k <= 0 || n <= 0 || k > INT_MAX / 4 ||
      n > INT_MAX)
    return fail(OHIP_E_INVALID, "ohip_weight_qgemm: bad arguments");
  if (zp && n_zp != 1 && n_zp != n) return fail(OHIP_E_SHAPE, "b_zero_point has the wrong length");
  if (scale && n_scale != 1 && n_scale != n) return fail(OHIP_E_SHAPE, "b_scale has the wrong length");
  std::lock_guard<std::mutex> lock(ctx->mu);
  std::string ks;
  if (key && key->name) {
    std::vector<int64_t> shape{k, n, trans_b, n_zp};
    for (int i = 0; zp && i < n_zp; ++i) shape.push_back(zp[i]);
    ks = cache_key(key, WK_QGEMM, src_dt, (size_t)(k * n), shape);
    if (ohip_weight* hit = cache_lookup(ctx, key, ks)) {
      if (scale && n_scale > 0 && !same_scales(hit->scale, scale, n_scale))
        hit->scale.assign(scale, scale + n_scale), hit->comb_a = NAN;
      *out = hit;
      return OHIP_OK;
    }
  }
  QPacked q;
  qpack_rows(n, round_up(k, 16), k, [&](int64_t j, int64_t p, int32_t* v) {
    const int32_t z = zp ? (n_zp == 1 ? zp[0] : zp[j]) : 0;
    *v = int_at(src_dt, host, trans_b ? j * k + p : p * n + j) - z;
    return true;
  }, q);
  auto* w = new ohip_weight();
  w->kind = WK_QGEMM; w->dtype = OHIP_I8; w->rows = n; w->k = k;
  rc = qpack_upload(ctx, w, q, scale, n_scale);
  if (rc) { weight_free(w); return rc; }
  return weight_finish(ctx, key, ks, w, out);
}

extern "C" int ohip_weight_qconv(ohip_ctx* ctx, const ohip_weight_key* key, int src_dt, const void* host,
                                 int64_t cout, int64_t cin, int64_t kh, int64_t kw, const int32_t* zp, int n_zp,
                                 const float* scale, int n_scale, ohip_weight** out) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!host || !out || (src_dt != OHIP_U8 && src_dt != OHIP_I8) || cout <= 0 || cin <= 0 || kh <= 0 || kw <= 0)
    return fail(OHIP_E_INVALID, "ohip_weight_qconv: bad arguments");
  if (zp && n_zp != 1 && n_zp != cout) return fail(OHIP_E_SHAPE, "w_zero_point has the wrong length");
  if (scale && n_scale != 1 && n_scale != cout) return fail(OHIP_E_SHAPE, "w_scale has the wrong length");
  std::lock_guard<std::mutex> lock(ctx->mu);
  std::string ks;
  if (key && key->name) {
    std::vector<int64_t> shape{cout, cin, kh, kw, n_zp};
    for (int i = 0; zp && i < n_zp; ++i) shape.push_back(zp[i]);
    ks = cache_key(key, WK_QCONV, src_dt, (size_t)(cout * cin * kh * kw), shape);
    if (ohip_weight* hit = cache_lookup(ctx, key, ks)) {
      if (scale && n_scale > 0 && !same_scales(hit->scale, scale, n_scale))
        hit->scale.assign(scale, scale + n_scale), hit->comb_a = NAN;
      *out = hit;
      return OHIP_OK;
    }
  }
  const int64_t cp = round_up(cin, 16), kp = kh * kw * cp;
  if (kp > INT_MAX / 4) return fail(OHIP_E_INVALID, "ohip_weight_qconv: filter too large");
  // packed K axis is (ky, kx, channel padded to cp)
  QPacked q;
  qpack_rows(cout, kp, kp, [&](int64_t o, int64_t j, int32_t* v) {
    const int64_t tap = j / cp, c = j - tap * cp;
    if (c >= cin) return false;
    const int64_t y = tap / kw, x = tap - y * kw;
    const int32_t z = zp ? (n_zp == 1 ? zp[0] : zp[o]) : 0;
    *v = int_at(src_dt, host, ((o * cin + c) * kh + y) * kw + x) - z;
    return true;
  }, q);
  auto* w = new ohip_weight();
  w->kind = WK_QCONV; w->dtype = OHIP_I8; w->rows = cout; w->k = cin; w->kh = kh; w->kw = kw;
  w->cpc = (int)(cp / 16);
  rc = qpack_upload(ctx, w, q, scale, n_scale);
  if (rc) { weight_free(w); return rc; }
  return weight_finish(ctx, key, ks, w, out);
}

// combined = a_scale * w_scale / y_scale, formed in f32 in that order
// (qlinear_matmul.rs:248, qlinear_conv.rs:99), cached on the weight.
static int ensure_comb(ohip_ctx* ctx, ohip_weight* w, float a_s, float y_s, int* n_comb) {
  if (w->scale.empty()) return fail(OHIP_E_INVALID, "weight has no scale");
  *n_comb = (int)w->scale.size();
  if (w->comb_a == a_s && w->comb_y == y_s) return OHIP_OK;
  std::vector<float> c(w->scale.size());
  for (size_t i = 0; i < c.size(); ++i) {
    volatile float prod = a_s * w->scale[i];
    c[i] = prod / y_s;
  }
  HIP_TRY(hipMemcpyAsync(w->comb, c.data(), c.size() * 4, hipMemcpyHostToDevice, ctx->stream), "comb upload");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "comb upload sync");
  w->comb_a = a_s;
  w->comb_y = y_s;
  return OHIP_OK;
}

// ------------------------------------------------------------------ helpers
static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Dense MFMA operands are addressed through a buffer resource with 32-bit
// offsets: the whole operand must lie below 2^31 bytes.
static bool dense_fits(const DenseOperand& d) {
  return (int64_t)d.rows * d.ld_bytes <= (int64_t)INT32_MAX - 4096;
}
#define DENSE_FITS_OR_DECLINE(op, where)                                          \
  do {                                                                          \
    if (!dense_fits(op)) return fail(OHIP_DECLINED, where ": operand exceeds 2 GiB"); \
  } while (0)

// Device address of sixteen copies of byte b (the MFMA loaders' pad source).
static const void* pad16(ohip_ctx* ctx, uint8_t b) { return ctx->padtab + (size_t)b * 16; }

extern "C" int64_t ohip_conv_out_dim(int64_t in, int64_t pb, int64_t pe, int64_t k, int64_t d, int64_t s) {
  if (s <= 0 || k <= 0 || d <= 0 || in < 0 || pb < 0 || pe < 0) return -1;
  int64_t eff = (k - 1) * d + 1, padded = in + pb + pe;
  if (padded < eff) return -1;
  return (padded - eff) / s + 1;
}

extern "C" int64_t ohip_conv_transpose_out_dim(int64_t in, int64_t s, int64_t op, int64_t k, int64_t d,
                                               int64_t pb, int64_t pe) {
  if (s <= 0 || k <= 0 || d <= 0 || in <= 0 || op < 0 || pb < 0 || pe < 0) return -1;
  const int64_t natural = s * (in - 1) + op + (k - 1) * d + 1;
  return natural - pb - pe >= 0 ? natural - pb - pe : -1;
}

// Bring an activation matrix [R][K] (row stride ld elements, or transposed
// [K][R]) into K-contiguous rows of whole 16-byte chunks.  Returns either the
// original pointer or a scratch copy.
struct RowsView {
  const void* p;
  int64_t ld_bytes;
  int kc;
};

static bool rows_direct(const void* a, int64_t k, int64_t ld, int eb, int trans) {
  const int ce = 16 / eb;
  return !trans && k % ce == 0 && (ld * eb) % 16 == 0 && aligned(a, 16);
}

// ------------------------------------------------------------------ float GEMM
static const int kMaxGemvM = 8;

extern "C" int ohip_gemm(ohip_ctx* ctx, const ohip_gemm_desc* d, const void* a, const ohip_weight* b,
                         const void* c, void* y) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!d || !a || !b || !y) return fail(OHIP_E_INVALID, "ohip_gemm: null argument");
  if (!is_float(d->dtype) || b->kind != WK_GEMM || b->dtype != d->dtype)
    return fail(OHIP_E_INVALID, "ohip_gemm: weight kind / dtype mismatch");
  if (d->k != b->k || d->n != b->rows || d->m < 0)
    return fail(OHIP_E_SHAPE, "ohip_gemm: shape disagrees with the packed weight");
  if (d->m > INT_MAX / 2 || d->n > INT_MAX / 2) return fail(OHIP_DECLINED, "ohip_gemm: extent too large");
  if (d->m == 0) return OHIP_OK;
  if (d->c_kind != OHIP_C_NONE && !c) return fail(OHIP_E_INVALID, "ohip_gemm: c_kind set but C is null");
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->counters.dispatches++;
  const int eb = elem_bytes(d->dtype), ce = 16 / eb;
  const int64_t M = d->m, N = d->n, K = d->k;
  const int64_t lda = d->lda ? d->lda : (d->trans_a ? M : K);
  const int64_t ldy = d->ldy ? d->ldy : N;
  const int64_t kp = round_up(K, ce);
  const bool direct = rows_direct(a, K, lda, eb, d->trans_a);
  const bool gemv = M <= kMaxGemvM;

  ScratchPlan plan;
  size_t ia = direct ? SIZE_MAX : plan.add((size_t)(M * kp) * eb);
  const SplitChoice sc = gemv ? SplitChoice{1, ctx->tile_override}
                              : plan_split_tile((int)N, (int)M, b->kc, ctx->tile_override, d->dtype == OHIP_F32);
  const int splits = sc.splits;
  size_t iw = splits > 1 ? plan.add(split_ws_bytes((int)N, (int)M, splits)) : SIZE_MAX;
  rc = scratch_reserve(ctx, plan.total());
  if (rc) return rc;

  RowsView av{a, lda * eb, (int)(kp / ce)};
  if (!direct) {
    void* pa = scratch_at(ctx, plan, ia);
    int64_t rs = d->trans_a ? 1 : lda, cs = d->trans_a ? lda : 1;
    HIP_TRY(run_gather2d(eb, a, rs, cs, pa, (int)M, (int)K, (int)kp, ctx->stream), "pack A");
    av = RowsView{pa, kp * eb, (int)(kp / ce)};
  }

  FloatOut o{};
  o.y = y; o.si = 1; o.sj = ldy; o.bstride = 0; o.ohw = INT_MAX; o.P = (int)N; o.Q = (int)M;
  o.vec = (ldy % 4 == 0) && aligned(y, 4 * eb);
  o.alpha = d->alpha; o.beta = d->beta; o.bias = c;
  o.bias_mode = d->c_kind == OHIP_C_SCALAR ? BIAS_SCALAR
              : d->c_kind == OHIP_C_ROW    ? BIAS_I
              : d->c_kind == OHIP_C_FULL   ? BIAS_FULL_JI
                                           : BIAS_NONE;
  o.act = d->act; o.lo = d->act_lo; o.hi = d->act_hi;
  if (o.act == ACT_CLIP) {
    if (std::isnan(o.lo)) o.lo = -INFINITY;
    if (std::isnan(o.hi)) o.hi = INFINITY;
    if (!(o.lo <= o.hi)) o.act = ACT_NONE;
  }

  hipError_t e;
  if (gemv) {
    GemvArgs g{av.p, av.ld_bytes / eb, b->data, b->ld_bytes / eb, (int)M, (int)N, b->kc};
    ctx->counters.contraction_launches++;
    e = run_gemv(d->dtype, g, o, ctx->stream);
  } else {
    DenseOperand x{b->data, b->ld_bytes, (int)N, b->kc, 0, 0u, pad16(ctx, 0)};
    DenseOperand yv{av.p, av.ld_bytes, (int)M, av.kc, 0, 0u, pad16(ctx, 0)};
    DENSE_FITS_OR_DECLINE(x, "ohip_gemm");
    DENSE_FITS_OR_DECLINE(yv, "ohip_gemm");
    o.splits = splits;
    o.split_ws = splits > 1 ? scratch_at(ctx, plan, iw) : nullptr;
    ctx->counters.contraction_launches++;
    e = run_dense_float(d->dtype, x, yv, o, sc.tile, ctx->stream);
  }
  if (e != hipSuccess) return hip_fail(e, "ohip_gemm launch");
  return OHIP_OK;
}

// ------------------------------------------------------------------ float Conv
struct ConvGeo {
  int64_t oh, ow;
};

static int conv_geo(int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t dh, int64_t dw,
                    int64_t pt, int64_t pl, int64_t pb, int64_t pr, ConvGeo* g) {
  g->oh = ohip_conv_out_dim(h, pt, pb, kh, dh, sh);
  g->ow = ohip_conv_out_dim(w, pl, pr, kw, dw, sw);
  if (g->oh < 0 || g->ow < 0) return fail(OHIP_E_SHAPE, "conv: padded input smaller than the dilated kernel");
  return OHIP_OK;
}

// OHIP_FEWOUT=0 keeps few-output convolutions on the MFMA engine (a
// measurement switch)
// OHIP_F32NCHW=0 keeps f32 NCHW convolutions on the staged engine path (a
// measurement switch)
static bool nchw_f32_allowed() {
  static const bool v = [] {
    const char* e = std::getenv("OHIP_F32NCHW");
    return !(e && e[0] == '0');
  }();
  return v;
}

static bool few_out_allowed() {
  static const bool v = [] {
    const char* e = std::getenv("OHIP_FEWOUT");
    return !(e && e[0] == '0');
  }();
  return v;
}

// OHIP_CONVT_ONE=0 runs ConvTranspose phases as a launch each (a measurement switch)
static bool ph_one_launch() {
  static const bool v = [] {
    const char* e = std::getenv("OHIP_CONVT_ONE");
    return !(e && e[0] == '0');
  }();
  return v;
}

// OHIP_HALO=0 keeps 3x3 convolutions on the engine's im2col path;
// OHIP_HALO_SPLITS=n forces the halo path's split count (measurement switches)
static bool halo_allowed() {
  static const bool v = [] {
    const char* e = std::getenv("OHIP_HALO");
    return !(e && e[0] == '0');
  }();
  return v;
}

// Split-K slices for the halo-patch kernel, or 0 where it does not apply:
// one group, 3x3, stride and dilation 1, an output width of 16, 32 or 64
// (256-pixel tiles of whole rows whose padded patch fits the stage) and an
// output height those tiles divide; automatically from 3 GFLOP up (below
// that the engine's shorter launches win; f32 512 -> 512 at 32x32: 53 us
// against 59 on the engine), always under tile override 15.  Slices are added until the grid gives every CU a
// block, keeping at least eight channel slabs per slice: every slice's
// partial sums make a round trip through memory (written at the end of the
// contraction, read by the reduction), which costs more than the extra
// slices' parallelism returns below that.
static int halo_plan(ohip_ctx* ctx, const ohip_conv_desc* d, int64_t G, int64_t w_in, const ConvGeo& g, int cpc,
                     int64_t img_bytes) {
  const bool forced = ctx->tile_override == 15;
  if (!halo_allowed() || (ctx->tile_override != 0 && !forced) || G != 1) return 0;
  if (d->kh != 3 || d->kw != 3 || d->stride_h != 1 || d->stride_w != 1 || d->dil_h != 1 || d->dil_w != 1) return 0;
  if (g.ow != 16 && g.ow != 32 && g.ow != 64 && g.ow != 128) return 0;
  const int64_t th = kHaloBPix / g.ow;
  const int pixmax = g.ow == 128 ? kHaloPixMaxWide : kHaloPixMax;
  if (g.oh % th != 0 || (th + 2) * (g.ow + 2) > pixmax || w_in > 65535) return 0;
  if (img_bytes >= ((int64_t)1 << 31) - 65536) return 0;
  const int64_t rows = d->n * g.oh * g.ow;
  const double flops = 2.0 * (double)rows * (double)d->cout * (double)d->c * 9.0;
  if (!forced && flops < 3e9) return 0;
  const int64_t nb = ((rows + kHaloBPix - 1) / kHaloBPix) * ((d->cout + 63) / 64);
  const int nslab = (cpc + 1) / 2;
  static const int forced_splits = [] {
    const char* e = std::getenv("OHIP_HALO_SPLITS");
    return e ? std::atoi(e) : 0;
  }();
  if (forced_splits >= 1 && forced_splits <= 64) return std::min(forced_splits, nslab);
  int64_t s = nb >= 256 ? 1 : (256 + nb - 1) / nb;
  s = std::min<int64_t>(s, std::max(1, nslab / 8));
  s = std::min<int64_t>(s, 16);
  return (int)std::max<int64_t>(s, 1);
}

static bool wk_allowed() {
  static const bool v = [] {
    const char* e = std::getenv("OHIP_WK");
    return !(e && e[0] == '0');
  }();
  return v;
}

// Whether a 3x3 stride-1 convolution runs the whole-K halo kernel
// (wk_conv_kernel): f16 / bf16, output rows 16, 32 or 64 wide tiling its
// pixel blocks (64 pixels at 32-wide rows, 128 otherwise) and 32-channel
// blocks into at least one block per CU (256), and enough work (1.5 GFLOP)
// for the launch to amortise.  Those are the mid-size convolutions the
// halo kernel would split four or more ways: the whole-K blocks write their
// outputs once instead (config 4's 512 -> 512 conv at 32x32: 12 us against
// 18 us plus the reduction of 8 MB of partial sums).  Tile override 17
// forces it wherever the geometry allows.
static bool wk_plan(ohip_ctx* ctx, const ohip_conv_desc* d, int64_t G, int64_t w_in, const ConvGeo& g,
                    int64_t img_bytes) {
  const bool forced = ctx->tile_override == 17;
  if (!wk_allowed() || (ctx->tile_override != 0 && !forced) || G != 1) return false;
  if (d->dtype != OHIP_F16 && d->dtype != OHIP_BF16 && d->dtype != OHIP_F32) return false;
  if (d->kh != 3 || d->kw != 3 || d->stride_h != 1 || d->stride_w != 1 || d->dil_h != 1 || d->dil_w != 1) return false;
  if (g.ow != 16 && g.ow != 32 && g.ow != 64) return false;
  const int64_t tpx = g.ow == 32 ? 64 : 128;
  if ((g.oh * g.ow) % tpx != 0 || w_in > 65535 || img_bytes >= ((int64_t)1 << 31) - 65536) return false;
  if (forced) return true;
  const int64_t rows = d->n * g.oh * g.ow;
  const int64_t blocks = rows / tpx * ((d->cout + 31) / 32);
  const double flops = 2.0 * (double)rows * (double)d->cout * (double)d->c * 9.0;
  return blocks >= 256 && flops >= 1.5e9;
}

// A fused instance normalisation for conv2d_impl (ohip_conv2d_instnorm).
struct ConvNorm {
  float eps;
  NormAffine aff;
};
// conv2d_impl's answer when a ConvNorm cannot read the split-K partial sums
// (no split, a grouped or direct convolution, an NHWC output, a large
// plane): nothing has been launched, and the caller runs the two steps.
constexpr int kNormTwoStep = 1 << 20;

static int conv2d_impl(ohip_ctx* ctx, const ohip_conv_desc* d, const void* x, const ohip_weight* w, const void* bias,
                       void* y, bool noalloc, const ConvNorm* norm = nullptr) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!d || !x || !w || !y) return fail(OHIP_E_INVALID, "ohip_conv2d: null argument");
  if (d->group < 1 || d->c % d->group || d->cout % d->group) return fail(OHIP_E_SHAPE, "ohip_conv2d: bad group");
  if (!is_float(d->dtype) || w->kind != WK_CONV || w->dtype != d->dtype)
    return fail(OHIP_E_INVALID, "ohip_conv2d: weight kind / dtype mismatch");
  const int64_t G = d->group, cg = d->c / G, coutg = d->cout / G;
  if (w->rows != d->cout || w->k != cg || w->kh != d->kh || w->kw != d->kw)
    return fail(OHIP_E_SHAPE, "ohip_conv2d: shape disagrees with the packed filter");
  ConvGeo g;
  rc = conv_geo(d->h, d->w, d->kh, d->kw, d->stride_h, d->stride_w, d->dil_h, d->dil_w, d->pad_t, d->pad_l,
                d->pad_b, d->pad_r, &g);
  if (rc) return rc;
  const int eb = elem_bytes(d->dtype), ce = 16 / eb;
  const int64_t cp = round_up(cg, ce);   // channel slots per group and tap
  const int64_t cpt = G * cp;            // channel slots per staged pixel
  const int64_t rows = d->n * g.oh * g.ow;
  if (rows > INT_MAX / 2 || d->n * d->h * d->w * cpt > (int64_t)INT_MAX * 4)
    return fail(OHIP_DECLINED, "ohip_conv2d: extent too large");
  if (rows == 0) return OHIP_OK;

  // A fused reflect / edge Pad is applied by the staging transpose, which
  // then writes the padded image; the convolution itself runs unpadded.
  const bool fused_pad = d->pad_mode == OHIP_PAD_REFLECT || d->pad_mode == OHIP_PAD_EDGE;
  if (d->pad_mode != OHIP_PAD_ZEROS && !fused_pad) return fail(OHIP_E_INVALID, "ohip_conv2d: pad_mode");
  // a fused Pad on an NHWC input is applied by the halo-patch loader (checked below)
  const bool nhwc_pad = fused_pad && d->in_layout == OHIP_NHWC;
  if (d->pad_mode == OHIP_PAD_REFLECT &&
      ((d->h > 1 && (d->pad_t >= d->h || d->pad_b >= d->h)) || (d->w > 1 && (d->pad_l >= d->w || d->pad_r >= d->w))))
    return fail(OHIP_DECLINED, "ohip_conv2d: reflect pad wider than the image");
  int act = d->act;
  float lo = d->act_lo, hi = d->act_hi;
  if (act == ACT_CLIP) {
    if (std::isnan(lo)) lo = -INFINITY;
    if (std::isnan(hi)) hi = INFINITY;
    if (!(lo <= hi)) act = ACT_NONE;
  }
  const int64_t ohw = g.oh * g.ow;
  const int64_t ldo = round_up(d->cout, ce);

  // Groups whose output or input channel span is too narrow to fill an MFMA
  // tile (depthwise, and small groups) run the direct kernel on the NCHW
  // input; wider groups run on the MFMA engine (one launch with the group on
  // the grid z, or a launch per group under split-K).  So do ungrouped
  // convolutions of an NCHW input with under 32 taps x channels (an RGB stem,
  // whose 16-byte channel padding would multiply the staged bytes).  A long
  // reduction stays on the engine even for a few output channels: one
  // thread per output walking thousands of taps is latency-bound (an RGB
  // head, 128 channels x 7x7 taps, ran 20x slower direct).
  const bool narrow = G == 1 && d->in_layout == OHIP_NCHW && cg * d->kh * d->kw < 32;
  const bool direct = (G > 1 && (coutg < 16 || cg * d->kh * d->kw < 32 || G > 64)) || narrow;
  if (G > 1 && d->in_layout != OHIP_NCHW && (direct || cg % ce != 0))
    return fail(OHIP_DECLINED, "ohip_conv2d: this grouped convolution needs an NCHW input");
  // A few output channels over a long reduction (an RGB head) would fill a
  // sliver of an f32 MFMA tile (f32 MFMA runs at a sixteenth of the f16
  // rate): the few-output kernel stages input patches in LDS and reduces over
  // channel slices instead (128 -> 3 channels, 7x7, 128x128: 50 us against
  // 232).  f16 / bf16 stay on the engine, which is faster there (the same
  // head in f16: 42.7 us on the engine, 55.5 us few-output).
  const bool fewout = !direct && d->dtype == OHIP_F32 && G == 1 && d->in_layout == OHIP_NCHW &&
                      d->cout <= kFewOutMax && cg * d->kh * d->kw >= 32 && rows * d->cout >= 16384 && few_out_allowed();
  // with a norm, out_layout is the normalised output's; the contraction
  // itself runs in the NCHW orientation (channel planes contiguous in the
  // partial sums)
  const bool norm_nhwc = norm && d->out_layout == OHIP_NHWC;
  DirectConvArgs a{};
  a.N = (int)d->n; a.C = (int)d->c; a.H = (int)d->h; a.W = (int)d->w; a.cout = (int)d->cout;
  a.cg = (int)cg; a.coutg = (int)coutg; a.KH = (int)d->kh; a.KW = (int)d->kw;
  a.sh = (int)d->stride_h; a.sw = (int)d->stride_w; a.dh = (int)d->dil_h; a.dw = (int)d->dil_w;
  a.pt = (int)d->pad_t; a.pl = (int)d->pad_l; a.pad_mode = fused_pad ? d->pad_mode : 0;
  a.OH = (int)g.oh; a.OW = (int)g.ow; a.ldw = w->ld_bytes / eb; a.cpg = (int)cp;
  a.nhwc_out = d->out_layout != OHIP_NCHW; a.ldo = ldo; a.act = act; a.lo = lo; a.hi = hi;
  // An NHWC f16 / bf16 input with at most 4 output channels (an RGB head)
  // runs the few-output MFMA kernel: a row's input patch staged once per
  // channel slab instead of the engine's per-tap gather, whose 64-column
  // tiles would be 1-4 columns full (128 -> 3 channels, 7x7, 128x128 with a
  // reflect pad: 45.9 us staged on the engine).
  const bool fewco = !direct && G == 1 && d->in_layout == OHIP_NHWC && few_out_allowed() &&
                     fewco_supported(d->dtype, a, (int)cpt);
  if (norm && (direct || fewout || fewco || G != 1 || g.oh * g.ow > kNormPartialsMaxSpatial || d->dtype == OHIP_BF16))
    return kNormTwoStep;
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->counters.dispatches++;
  if (fewco) {
    const int64_t slices = d->c / fewco_slice(a);
    ScratchPlan plan;
    const size_t iw = plan.add((size_t)(slices * d->n * d->cout * ohw) * 4);
    char* sbase = nullptr;
    rc = call_scratch(ctx, plan.total(), noalloc, &sbase);
    if (rc) return rc;
    if (!aligned(x, 16)) return fail(OHIP_E_INVALID, "ohip_conv2d: NHWC input must be 16-byte aligned");
    hipError_t e = run_conv_fewco(d->dtype, x, (int)cpt, w->data, bias, y, static_cast<float*>(plan_at(sbase, plan, iw)),
                                  a, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "ohip_conv2d few-output MFMA launch");
    return OHIP_OK;
  }
  // f32 3x3 / 1x1 stride-1 convolutions of an NCHW input, NCHW out: the
  // patch-staged kernel reads the input as it is, a fused reflect / edge pad
  // included (no staging transpose;
  // config 1: 27.7 -> 20.9 us).  Long reductions over few pixels keep the
  // halo-patch path, whose split-K fills the chip, and so do the ones the
  // whole-K kernel takes (the sums a fused norm's conv makes, bit for bit).
  const int64_t staged_w = fused_pad ? d->w + d->pad_l + d->pad_r : d->w;
  const int64_t staged_bytes =
      (fused_pad ? (d->h + d->pad_t + d->pad_b) * (d->w + d->pad_l + d->pad_r) : d->h * d->w) * cpt * eb;
  if (!norm && !direct && !fewout && d->dtype == OHIP_F32 && G == 1 && d->in_layout == OHIP_NCHW &&
      nchw_f32_allowed() && conv_nchw_f32_supported(a) && !wk_plan(ctx, d, G, staged_w, g, staged_bytes) &&
      halo_plan(ctx, d, G, staged_w, g, (int)(cp / ce), staged_bytes) == 0) {
    ctx->counters.contraction_launches++;
    hipError_t e = run_conv_nchw_f32(static_cast<const float*>(x), static_cast<const float*>(w->data),
                                     static_cast<const float*>(bias), static_cast<float*>(y), a, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "ohip_conv2d f32 NCHW launch");
    return OHIP_OK;
  }
  if (direct || fewout) {
    if (fewout) {
      const int cslice = fewout_slice(a);
      const int64_t slices = (d->c + cslice - 1) / cslice;
      ScratchPlan plan;
      const size_t iw = plan.add((size_t)(slices * d->n * d->cout * ohw) * 4);
      char* sbase = nullptr;
      rc = call_scratch(ctx, plan.total(), noalloc, &sbase);
      if (rc) return rc;
      hipError_t e = run_conv_fewout(d->dtype, x, w->data, bias, y, static_cast<float*>(plan_at(sbase, plan, iw)), a,
                                     cslice, ctx->stream);
      if (e != hipSuccess) return hip_fail(e, "ohip_conv2d few-output launch");
      return OHIP_OK;
    }
    hipError_t e = run_conv_direct(d->dtype, x, w->data, bias, y, a, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "ohip_conv2d direct launch");
    return OHIP_OK;
  }

  // extents of the buffer the contraction reads: an NCHW input is staged
  // with a fused Pad applied, an NHWC input is read as it is
  const bool pad_staged = fused_pad && !nhwc_pad;
  const int64_t sh_ = pad_staged ? d->h + d->pad_t + d->pad_b : d->h;
  const int64_t sw_ = pad_staged ? d->w + d->pad_l + d->pad_r : d->w;
  ScratchPlan plan;
  const bool stage = d->in_layout == OHIP_NCHW;
  size_t ix = stage ? plan.add((size_t)(d->n * sh_ * sw_ * cpt) * eb) : SIZE_MAX;
  const bool nchw_out = norm || d->out_layout == OHIP_NCHW;
  const int sP = nchw_out ? (int)rows : (int)coutg, sQ = nchw_out ? (int)coutg : (int)rows;
  // 3x3 stride-1 convolutions whose output rows tile 256-pixel blocks run
  // the halo-patch kernel (the input patch staged once per channel slab for
  // all nine taps) instead of the engine's im2col gather.
  const bool wk = wk_plan(ctx, d, G, sw_, g, (int64_t)(sh_ * sw_ * cpt * eb));
  const int hsplits = wk ? 0 : halo_plan(ctx, d, G, sw_, g, (int)(cp / ce), (int64_t)(sh_ * sw_ * cpt * eb));
  if (nhwc_pad && !hsplits && !wk)
    return fail(OHIP_DECLINED, "ohip_conv2d: a reflect / edge Pad on an NHWC input needs the halo-patch path");
  const SplitChoice sc = wk ? SplitChoice{1, 0} : hsplits ? SplitChoice{hsplits, 0}
                                 : plan_split_tile(sP, sQ, (int)(d->kh * d->kw * (cp / ce)), ctx->tile_override,
                                                   d->dtype == OHIP_F32);
  const int splits = sc.splits;
  if (norm && splits == 1 && !wk) {   // counted again by the two-step path's plain call
    ctx->counters.dispatches--;
    return kNormTwoStep;
  }
  // the whole-K kernel under a norm leaves its sums as one slice of f32
  // partial sums for the norm kernel
  // An f16 / f32 norm over planes of whole 64-pixel segments takes its
  // statistics from the whole-K kernel instead: the kernel stores the conv
  // output (NCHW) and each 64-pixel segment's moments, and the norm kernel
  // merges those and rescales the stored output in one elementwise pass.
  const bool wk_mom = wk && norm && (d->dtype == OHIP_F16 || d->dtype == OHIP_F32) && ohw % 64 == 0 &&
                      ohw <= kNormMomMaxSpatial && (!norm_nhwc || d->cout % 8 == 0) &&
                      (!norm->aff.residual || norm->aff.res_nhwc == (int)norm_nhwc) && aligned(y, 8 * eb) &&
                      aligned(norm->aff.residual, 8 * eb);
  const bool partials = splits > 1 || (wk && norm && !wk_mom);
  size_t iw = partials ? plan.add(splits > 1 ? split_ws_bytes(sP, sQ, splits) : (size_t)sQ * ((sP + 3) / 4 * 4) * 4)
                       : SIZE_MAX;
  const size_t ity = wk_mom ? plan.add((size_t)(d->n * d->cout * ohw) * eb) : SIZE_MAX;
  const size_t imom = wk_mom ? plan.add((size_t)(d->n * d->cout * (ohw / 64)) * 2 * 4) : SIZE_MAX;
  char* sbase = nullptr;
  rc = call_scratch(ctx, plan.total(), noalloc, &sbase);
  if (rc) return rc;
  const void* xin = x;
  if (stage) {
    void* px = plan_at(sbase, plan, ix);
    if (G > 1)
      HIP_TRY(run_stage_nhwc(eb, x, px, (int)d->n, (int)d->c, (int)d->h, (int)d->w, fused_pad ? (int)d->pad_t : 0,
                             fused_pad ? (int)d->pad_l : 0, fused_pad ? (int)d->pad_b : 0,
                             fused_pad ? (int)d->pad_r : 0, fused_pad ? d->pad_mode : 0, (int)cg, (int)cp, (int)G,
                             ctx->stream),
              "NCHW -> grouped NHWC");
    else if (fused_pad)
      HIP_TRY(run_nchw_to_nhwc_pad(eb, x, px, (int)d->n, (int)d->c, (int)d->h, (int)d->w, (int)cp, (int)d->pad_t,
                                   (int)d->pad_l, (int)d->pad_b, (int)d->pad_r, (int)d->pad_mode, ctx->stream),
              "NCHW -> padded NHWC");
    else
      HIP_TRY(run_nchw_to_nhwc(eb, x, px, (int)d->n, (int)d->c, (int)(d->h * d->w), (int)cp, ctx->stream),
              "NCHW -> NHWC");
    xin = px;
  } else if (!aligned(x, 16)) {
    return fail(OHIP_E_INVALID, "ohip_conv2d: NHWC input must be 16-byte aligned");
  }

  if (hsplits || wk) {
    HaloGeo hg{};
    hg.x = static_cast<const char*>(xin);
    hg.img_bytes = sh_ * sw_ * cpt * eb;
    hg.H = (int)sh_; hg.W = (int)sw_; hg.OH = (int)g.oh; hg.OW = (int)g.ow;
    hg.pt = pad_staged ? 0 : (int)d->pad_t; hg.pl = pad_staged ? 0 : (int)d->pad_l;
    hg.pad_mode = nhwc_pad ? d->pad_mode : 0;
    hg.pstride = (int)(cpt / ce); hg.cpc = (int)(cp / ce);
    hg.th = kHaloBPix / (int)g.ow;
    hg.ow_shift = 0;
    while ((1 << hg.ow_shift) < g.ow) ++hg.ow_shift;
    hg.w = static_cast<const char*>(w->data); hg.ldw = w->ld_bytes; hg.cout = (int)coutg;
    FloatOut o{};
    o.alpha = 1.0f; o.beta = 1.0f;
    o.bias = bias;
    o.act = act; o.lo = lo; o.hi = hi;
    o.y = wk_mom ? plan_at(sbase, plan, ity) : y;
    if (nchw_out) {
      o.si = 1; o.sj = ohw; o.bstride = d->cout * ohw; o.ohw = (int)ohw; o.P = (int)rows; o.Q = (int)coutg;
      o.vec = ohw % 4 == 0 && aligned(o.y, 4 * eb);
      o.bias_mode = BIAS_J;
    } else {
      o.si = 1; o.sj = ldo; o.bstride = 0; o.ohw = INT_MAX; o.P = (int)coutg; o.Q = (int)rows;
      o.vec = ldo % 4 == 0 && aligned(o.y, 4 * eb);
      o.bias_mode = BIAS_I;
    }
    o.splits = splits;
    o.split_ws = partials ? plan_at(sbase, plan, iw) : nullptr;
    o.defer_reduce = norm && !wk_mom ? 1 : 0;
    float* mom = wk_mom ? static_cast<float*>(plan_at(sbase, plan, imom)) : nullptr;
    ctx->counters.contraction_launches++;
    hipError_t e = wk ? run_wk_float(d->dtype, hg, nchw_out, o, mom, ctx->stream)
                      : run_halo_float(d->dtype, hg, nchw_out, o, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, wk ? "ohip_conv2d whole-K halo launch" : "ohip_conv2d halo launch");
    if (wk_mom) {
      e = run_instnorm_mom(d->dtype, o.y, mom, y, d->n, (int)d->cout, ohw, norm->eps, norm->aff, norm_nhwc,
                           ctx->stream);
      if (e != hipSuccess) return hip_fail(e, "ohip_conv2d_instnorm launch");
    } else if (norm) {
      e = run_instnorm_partials(d->dtype, static_cast<const float*>(o.split_ws), splits, (rows + 3) / 4 * 4, bias,
                                y, d->n, ohw, (int)d->cout, norm->eps, norm->aff, norm_nhwc, ctx->stream);
      if (e != hipSuccess) return hip_fail(e, "ohip_conv2d_instnorm launch");
    }
    return OHIP_OK;
  }

  // Groups without split-K run as one launch, group = blockIdx.z: the input
  // channel chunks, the weight rows, the bias and the output channels of
  // group z sit at fixed strides from group 0's.  Split plans share one
  // workspace, so those run a launch per group.
  const bool one_launch = G > 1 && G <= 65535 && splits == 1;
  for (int64_t gi = 0; gi < (one_launch ? 1 : G); ++gi) {
    Im2colOperand col{};
    col.base = static_cast<const char*>(xin) + gi * cp * eb;
    col.H = (int)sh_; col.W = (int)sw_; col.OH = (int)g.oh; col.OW = (int)g.ow;
    col.KW = (int)d->kw; col.cpc = (int)(cp / ce); col.pstride = (int)(cpt / ce);
    col.sh = (int)d->stride_h; col.sw = (int)d->stride_w; col.dh = (int)d->dil_h; col.dw = (int)d->dil_w;
    col.pt = fused_pad ? 0 : (int)d->pad_t; col.pl = fused_pad ? 0 : (int)d->pad_l;
    col.rows = (int)rows; col.kc = w->kc;
    col.xor_mask = 0; col.pad16 = pad16(ctx, 0);
    DenseOperand wt{static_cast<const char*>(w->data) + gi * coutg * w->ld_bytes, w->ld_bytes, (int)coutg, w->kc,
                    0, 0u, pad16(ctx, 0)};

    FloatOut o{};
    o.alpha = 1.0f; o.beta = 1.0f;
    o.bias = bias ? static_cast<const char*>(bias) + gi * coutg * eb : nullptr;
    o.act = act; o.lo = lo; o.hi = hi;
    bool col_on_x;
    if (nchw_out) {
      col_on_x = true;
      o.y = static_cast<char*>(y) + gi * coutg * ohw * eb;
      o.si = 1; o.sj = ohw; o.bstride = d->cout * ohw; o.ohw = (int)ohw; o.P = (int)rows; o.Q = (int)coutg;
      o.vec = ohw % 4 == 0 && aligned(o.y, 4 * eb);
      o.bias_mode = BIAS_J;
    } else {
      col_on_x = false;
      o.y = static_cast<char*>(y) + gi * coutg * eb;
      o.si = 1; o.sj = ldo; o.bstride = 0; o.ohw = INT_MAX; o.P = (int)coutg; o.Q = (int)rows;
      o.vec = ldo % 4 == 0 && aligned(o.y, 4 * eb);
      o.bias_mode = BIAS_I;
    }
    DENSE_FITS_OR_DECLINE(wt, "ohip_conv2d");
    o.splits = splits;
    o.split_ws = splits > 1 ? plan_at(sbase, plan, iw) : nullptr;
    if (one_launch) {
      col.zstride = cp * eb;
      wt.zmod = (int)G; wt.zstride = coutg * w->ld_bytes;
      o.batch = (int)G; o.zstride = nchw_out ? coutg * ohw * eb : coutg * eb;
      o.bias_z = coutg;
      // vector stores need every group's first output aligned, not only group 0's
      o.vec = o.vec && o.zstride % (4 * eb) == 0;
    }
    o.defer_reduce = norm ? 1 : 0;
    ctx->counters.contraction_launches++;
    hipError_t e = run_conv_float(d->dtype, col, wt, col_on_x, o, sc.tile, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "ohip_conv2d launch");
    if (norm) {
      e = run_instnorm_partials(d->dtype, static_cast<const float*>(o.split_ws), splits, (rows + 3) / 4 * 4, bias,
                                y, d->n, ohw, (int)d->cout, norm->eps, norm->aff, norm_nhwc, ctx->stream);
      if (e != hipSuccess) return hip_fail(e, "ohip_conv2d_instnorm launch");
    }
  }
  return OHIP_OK;
}

extern "C" int ohip_conv2d(ohip_ctx* ctx, const ohip_conv_desc* d, const void* x, const ohip_weight* w,
                           const void* bias, void* y) {
  return conv2d_impl(ctx, d, x, w, bias, y, false);
}

// The halo-patch split count an ungrouped convolution of a resident NHWC
// input would run with (0: not on the halo path), for the dispatcher's
// layout choices.
int ohip_conv_halo_splits_internal(ohip_ctx* ctx, const ohip_conv_desc* d) {
  if (!ctx || !d || d->group != 1 || !is_float(d->dtype)) return 0;
  ConvGeo g;
  if (conv_geo(d->h, d->w, d->kh, d->kw, d->stride_h, d->stride_w, d->dil_h, d->dil_w, d->pad_t, d->pad_l, d->pad_b,
               d->pad_r, &g) != OHIP_OK)
    return 0;
  const int eb = elem_bytes(d->dtype), ce = 16 / eb;
  const int64_t cp = round_up(d->c, ce);
  if (wk_plan(ctx, d, 1, d->w, g, d->h * d->w * cp * eb)) return 1;
  return halo_plan(ctx, d, 1, d->w, g, (int)(cp / ce), d->h * d->w * cp * eb);
}

// Whether ohip_conv2d would run this convolution of a resident NHWC input
// (channel pitch = the channels padded to 16 bytes) on the few-output MFMA
// kernel, which applies a fused reflect / edge pad in its loader.
int ohip_conv_fewco_internal(const ohip_conv_desc* d) {
  if (!d || d->group != 1 || !is_float(d->dtype) || !few_out_allowed()) return 0;
  ConvGeo g;
  if (conv_geo(d->h, d->w, d->kh, d->kw, d->stride_h, d->stride_w, d->dil_h, d->dil_w, d->pad_t, d->pad_l, d->pad_b,
               d->pad_r, &g) != OHIP_OK)
    return 0;
  const int ce = 16 / elem_bytes(d->dtype);
  const int64_t cp = round_up(d->c, ce);
  DirectConvArgs a{};
  a.N = (int)d->n; a.C = (int)d->c; a.H = (int)d->h; a.W = (int)d->w; a.cout = (int)d->cout;
  a.KH = (int)d->kh; a.KW = (int)d->kw; a.sh = (int)d->stride_h; a.sw = (int)d->stride_w;
  a.dh = (int)d->dil_h; a.dw = (int)d->dil_w; a.OH = (int)g.oh; a.OW = (int)g.ow;
  a.cpg = (int)cp; a.ldw = d->kh * d->kw * cp;
  return fewco_supported(d->dtype, a, (int)cp) ? 1 : 0;
}

// Conv -> instance normalisation.  With a split-K plan the normalisation
// reads the partial sums (one launch fewer, no conv output round trip);
// otherwise the conv writes a pooled temporary that the normalisation reads.
extern "C" int ohip_conv2d_instnorm(ohip_ctx* ctx, const ohip_conv_desc* d, const void* x, const ohip_weight* w,
                                    const void* bias, const ohip_norm_desc* nd, void* y) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!d || !nd || !y) return fail(OHIP_E_INVALID, "ohip_conv2d_instnorm: null argument");
  if (d->act != OHIP_ACT_NONE) return fail(OHIP_E_INVALID, "ohip_conv2d_instnorm: the conv must have no activation");
  if (d->out_layout == OHIP_NHWC && d->cout % (16 / elem_bytes(d->dtype)))
    return fail(OHIP_E_INVALID, "ohip_conv2d_instnorm: an NHWC output needs whole 16-byte pixels");
  if (d->dtype != OHIP_F32 && d->dtype != OHIP_F16) return fail(OHIP_DECLINED, "ohip_conv2d_instnorm: f32 / f16 only");
  if (nd->act != OHIP_ACT_NONE && nd->act != OHIP_ACT_RELU && nd->act != OHIP_ACT_LEAKY_RELU)
    return fail(OHIP_E_INVALID, "ohip_conv2d_instnorm: activation");
  ConvNorm cn{};
  cn.eps = nd->epsilon;
  cn.aff.scale = nd->scale; cn.aff.bias = nd->bias; cn.aff.per_sample = nd->per_sample; cn.aff.stride = nd->stride;
  cn.aff.same_type = nd->same_type;
  cn.aff.act = nd->act == OHIP_ACT_RELU ? UN_RELU : nd->act == OHIP_ACT_LEAKY_RELU ? UN_LEAKY_RELU : UN_IDENTITY;
  cn.aff.alpha = nd->alpha;
  cn.aff.residual = nd->residual;
  cn.aff.res_nhwc = nd->residual && nd->residual_layout == OHIP_NHWC;
  if (cn.aff.res_nhwc && d->cout % (16 / elem_bytes(d->dtype)))
    return fail(OHIP_E_INVALID, "ohip_conv2d_instnorm: an NHWC residual needs whole 16-byte pixels");
  rc = conv2d_impl(ctx, d, x, w, bias, y, false, &cn);
  if (rc != kNormTwoStep) return rc;
  // two steps: the conv (NCHW) into a pooled temporary, the normalisation
  // from it (NCHW), and for an NHWC output a transpose of that
  ConvGeo g;
  rc = conv_geo(d->h, d->w, d->kh, d->kw, d->stride_h, d->stride_w, d->dil_h, d->dil_w, d->pad_t, d->pad_l, d->pad_b,
                d->pad_r, &g);
  if (rc) return rc;
  const int64_t spatial = g.oh * g.ow;
  const size_t bytes = (size_t)(d->n * d->cout * spatial) * elem_bytes(d->dtype);
  const bool to_nhwc = d->out_layout == OHIP_NHWC;
  void* tmp = nullptr;
  void* tmp2 = nullptr;
  rc = pool_alloc(ctx, bytes, &tmp);
  if (!rc && to_nhwc) rc = pool_alloc(ctx, bytes, &tmp2);
  if (!rc) {
    ohip_conv_desc dc = *d;
    dc.out_layout = OHIP_NCHW;
    rc = conv2d_impl(ctx, &dc, x, w, bias, tmp, false, nullptr);
  }
  if (!rc) {
    hipError_t e = run_instnorm(d->dtype, tmp, to_nhwc ? tmp2 : y, d->n * d->cout, spatial, (int)d->cout, cn.eps,
                                cn.aff, ctx->stream);
    if (e == hipSuccess && to_nhwc)
      e = run_nchw_to_nhwc(elem_bytes(d->dtype), tmp2, y, (int)d->n, (int)d->cout, (int)spatial, (int)d->cout,
                           ctx->stream);
    if (e != hipSuccess) rc = hip_fail(e, "ohip_conv2d_instnorm: normalisation launch");
  }
  const int rf = pool_free(ctx, tmp);
  const int rf2 = pool_free(ctx, tmp2);
  return rc ? rc : (rf ? rf : rf2);
}

// Same kernels as ohip_conv2d; the staging copy and the split-K partial sums
// live in this device's static scratch array instead of the context's
// growable scratch, so the call makes no device allocation.
extern "C" int ohip_conv2d_noalloc(ohip_ctx* ctx, const ohip_conv_desc* d, const void* x, const ohip_weight* w,
                                   const void* bias, void* y) {
  return conv2d_impl(ctx, d, x, w, bias, y, true);
}

// ------------------------------------------------------------------ batched MatMul
extern "C" int ohip_matmul(ohip_ctx* ctx, const ohip_matmul_desc* d, const void* a, const void* b, void* y) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!d || !a || !b || !y) return fail(OHIP_E_INVALID, "ohip_matmul: null argument");
  if (!is_float(d->dtype)) return fail(OHIP_E_INVALID, "ohip_matmul: dtype");
  if (d->m < 0 || d->k <= 0 || d->n < 0 || d->batch < 1 || d->a_batches < 1 || d->b_batches < 1)
    return fail(OHIP_E_SHAPE, "ohip_matmul: bad extents");
  if (d->batch > 65535) return fail(OHIP_DECLINED, "ohip_matmul: more than 65535 slices");
  if (d->m == 0 || d->n == 0) return OHIP_OK;
  const int eb = elem_bytes(d->dtype), ce = 16 / eb;
  const int64_t M = d->m, K = d->k, N = d->n, kp = round_up(K, ce);
  if (M * d->a_batches > INT_MAX / 2 || N > INT_MAX / 2 || kp * eb > INT_MAX / 4)
    return fail(OHIP_DECLINED, "ohip_matmul: extent too large");
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->counters.dispatches++;
  const bool a_direct = (K * eb) % 16 == 0 && aligned(a, 16);
  ScratchPlan plan;
  size_t ib = plan.add((size_t)(d->b_batches * N * kp) * eb);
  size_t ia = a_direct ? SIZE_MAX : plan.add((size_t)(d->a_batches * M * kp) * eb);
  rc = scratch_reserve(ctx, plan.total());
  if (rc) return rc;
  void* pb = scratch_at(ctx, plan, ib);
  HIP_TRY(run_transpose_batched(eb, b, pb, (int)d->b_batches, (int)K, (int)N, (int)kp, ctx->stream),
          "MatMul B -> K-contiguous rows");
  const void* pa = a;
  if (!a_direct) {
    void* t = scratch_at(ctx, plan, ia);
    HIP_TRY(run_gather2d(eb, a, K, 1, t, (int)(d->a_batches * M), (int)K, (int)kp, ctx->stream), "MatMul A pack");
    pa = t;
  }
  const int64_t lda = a_direct ? K * eb : kp * eb;
  DenseOperand xo{pb, kp * eb, (int)N, (int)(kp / ce), 0, 0u, pad16(ctx, 0), (int)d->b_batches, N * kp * eb};
  DenseOperand yo{pa, lda, (int)M, (int)(kp / ce), 0, 0u, pad16(ctx, 0), (int)d->a_batches, M * lda};
  FloatOut o{};
  o.y = y; o.si = 1; o.sj = N; o.bstride = 0; o.ohw = INT_MAX; o.P = (int)N; o.Q = (int)M;
  o.vec = N % 4 == 0 && aligned(y, 4 * eb);
  o.alpha = 1.0f; o.beta = 1.0f; o.bias = nullptr; o.bias_mode = BIAS_NONE; o.act = ACT_NONE;
  o.splits = 1; o.split_ws = nullptr; o.batch = (int)d->batch; o.zstride = M * N * eb;
  DENSE_FITS_OR_DECLINE(xo, "ohip_matmul");
  DENSE_FITS_OR_DECLINE(yo, "ohip_matmul");
  ctx->counters.contraction_launches++;
  hipError_t e = run_dense_float(d->dtype, xo, yo, o, plain_tile_id(ctx->tile_override)
                                                          ? ctx->tile_override : 0, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "ohip_matmul launch");
  return OHIP_OK;
}

// ------------------------------------------------------------------ ConvTranspose
extern "C" int ohip_conv_transpose2d(ohip_ctx* ctx, const ohip_convt_desc* d, const void* x, const ohip_weight* w,
                                     const void* bias, void* y) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!d || !x || !w || !y) return fail(OHIP_E_INVALID, "ohip_conv_transpose2d: null argument");
  if (!is_float(d->dtype) || w->kind != WK_CONVT || w->dtype != d->dtype)
    return fail(OHIP_E_INVALID, "ohip_conv_transpose2d: weight kind / dtype mismatch");
  if (d->group < 1 || d->c % d->group || d->cout % d->group)
    return fail(OHIP_E_SHAPE, "ohip_conv_transpose2d: bad group");
  if (w->rows != d->c || w->k * d->group != d->cout || w->kh != d->kh || w->kw != d->kw)
    return fail(OHIP_E_SHAPE, "ohip_conv_transpose2d: shape disagrees with the filter");
  const int64_t oh = ohip_conv_transpose_out_dim(d->h, d->stride_h, d->out_pad_h, d->kh, d->dil_h, d->pad_t, d->pad_b);
  const int64_t ow = ohip_conv_transpose_out_dim(d->w, d->stride_w, d->out_pad_w, d->kw, d->dil_w, d->pad_l, d->pad_r);
  if (oh < 0 || ow < 0) return fail(OHIP_E_SHAPE, "ohip_conv_transpose2d: pads exceed the un-cropped extent");
  if (d->n * d->cout * oh * ow > (int64_t)INT_MAX * 8 || d->h * d->w > INT_MAX / 2)
    return fail(OHIP_DECLINED, "ohip_conv_transpose2d: extent too large");
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->counters.dispatches++;
  if (!w->phases.empty() && d->group == 1 && d->dil_h == 1 && d->dil_w == 1 && w->ph_sh == d->stride_h &&
      w->ph_sw == d->stride_w && w->ph_pt == d->pad_t % d->stride_h && w->ph_pl == d->pad_l % d->stride_w) {
    // sub-pixel phases on the MFMA engine: every phase is a stride-1
    // implicit-im2col convolution of the staged input, written to the
    // phase's strided output positions
    const int eb = elem_bytes(d->dtype), ce = 16 / eb;
    const int64_t cp = round_up(d->c, ce), sh = d->stride_h, sw = d->stride_w;
    int64_t max_rows = 0;
    for (int64_t ry = 0; ry < sh; ++ry)
      for (int64_t rx = 0; rx < sw; ++rx)
        max_rows = std::max<int64_t>(max_rows, ((oh - ry + sh - 1) / sh) * ((ow - rx + sw - 1) / sw));
    // Every phase in one launch, phase z = ry * sw + rx on the grid's z, when
    // the phases share one filter allocation and one output grid and none
    // runs split-K: the phase's pads, filter and output offset follow z.  A
    // combined grid of 256+ blocks fills the chip without splitting; a
    // forced split (tile 10 / 11, OHIP_SPLITS) keeps the per-phase launches.
    const int64_t ohp0 = oh / sh, owp0 = ow / sw;
    const int64_t blocks64 = ((ohp0 * owp0 + 63) / 64) * ((d->cout + 63) / 64) * sh * sw;
    const bool split_forced = ctx->tile_override == 10 || ctx->tile_override == 11 || forced_splits() != 0;
    const bool one = w->ph_all && oh % sh == 0 && ow % sw == 0 && ohp0 > 0 && owp0 > 0 && ph_one_launch() &&
                     !split_forced &&
                     (blocks64 >= 256 ||
                      plan_splits((int)(ohp0 * owp0), (int)d->cout, w->ph_all->kc, ctx->tile_override) == 1);
    int max_splits = 1;
    if (!one)
      for (auto* ph : w->phases)
        max_splits = std::max(max_splits, plan_splits((int)max_rows, (int)d->cout, ph->kc, ctx->tile_override));
    ScratchPlan plan;
    size_t ix = plan.add((size_t)(d->n * d->h * d->w * cp) * eb);
    size_t iw = max_splits > 1 ? plan.add(split_ws_bytes((int)max_rows, (int)d->cout, max_splits)) : SIZE_MAX;
    rc = scratch_reserve(ctx, plan.total());
    if (rc) return rc;
    void* px = scratch_at(ctx, plan, ix);
    HIP_TRY(run_nchw_to_nhwc(eb, x, px, (int)d->n, (int)d->c, (int)(d->h * d->w), (int)cp, ctx->stream),
            "NCHW -> NHWC");
    if (one) {
      const ohip_weight* pa = w->ph_all;
      for (int64_t n = 0; n < d->n; ++n) {
        Im2colOperand col{};
        col.base = static_cast<const char*>(px) + n * d->h * d->w * cp * eb;
        col.H = (int)d->h; col.W = (int)d->w; col.OH = (int)ohp0; col.OW = (int)owp0;
        col.KW = (int)pa->kw; col.cpc = (int)(cp / ce);
        col.sh = 1; col.sw = 1; col.dh = 1; col.dw = 1;
        col.rows = (int)(ohp0 * owp0); col.kc = pa->kc;
        col.xor_mask = 0; col.pad16 = pad16(ctx, 0);
        col.zpads = (int)(sh * sw);
        for (int64_t ry = 0; ry < sh; ++ry)
          for (int64_t rx = 0; rx < sw; ++rx) {
            const int64_t ky0 = (ry + d->pad_t) % sh, kx0 = (rx + d->pad_l) % sw;
            const int64_t c0y = (ry + d->pad_t - ky0) / sh, c0x = (rx + d->pad_l - kx0) / sw;
            col.zpt[ry * sw + rx] = (int)(pa->kh - 1 - c0y);
            col.zpl[ry * sw + rx] = (int)(pa->kw - 1 - c0x);
          }
        col.pt = col.zpt[0]; col.pl = col.zpl[0];
        DenseOperand wt{pa->data, pa->ld_bytes, (int)d->cout, pa->kc, 0, 0u, pad16(ctx, 0), (int)(sh * sw),
                        w->ph_zstride};
        FloatOut o{};
        o.y = static_cast<char*>(y) + n * d->cout * oh * ow * eb;
        o.alpha = 1.0f; o.beta = 1.0f; o.bias = bias; o.bias_mode = BIAS_J; o.act = ACT_NONE;
        o.si = sw; o.sj = oh * ow; o.bstride = sh * ow; o.ohw = (int)owp0;
        o.P = (int)(ohp0 * owp0); o.Q = (int)d->cout; o.vec = 0;
        o.splits = 1; o.split_ws = nullptr;
        o.batch = (int)(sh * sw); o.zsw = (int)sw; o.zrow = ow * eb; o.zstride = eb;   // phase (ry, rx) at ry * ow + rx
        DENSE_FITS_OR_DECLINE(wt, "ohip_conv_transpose2d");
        ctx->counters.contraction_launches++;
        hipError_t e = run_conv_float(d->dtype, col, wt, true, o, ctx->tile_override, ctx->stream);
        if (e != hipSuccess) return hip_fail(e, "ohip_conv_transpose2d phase launch");
      }
      return OHIP_OK;
    }
    for (int64_t n = 0; n < d->n; ++n)
      for (int64_t ry = 0; ry < sh; ++ry)
        for (int64_t rx = 0; rx < sw; ++rx) {
          const ohip_weight* ph = w->phases[(size_t)(ry * sw + rx)];
          const int64_t ohp = (oh - ry + sh - 1) / sh, owp = (ow - rx + sw - 1) / sw;
          if (ohp <= 0 || owp <= 0) continue;
          const int64_t ky0 = (ry + d->pad_t) % sh, kx0 = (rx + d->pad_l) % sw;
          const int64_t c0y = (ry + d->pad_t - ky0) / sh, c0x = (rx + d->pad_l - kx0) / sw;
          Im2colOperand col{};
          col.base = static_cast<const char*>(px) + n * d->h * d->w * cp * eb;
          col.H = (int)d->h; col.W = (int)d->w; col.OH = (int)ohp; col.OW = (int)owp;
          col.KW = (int)ph->kw; col.cpc = (int)(cp / ce);
          col.sh = 1; col.sw = 1; col.dh = 1; col.dw = 1;
          col.pt = (int)(ph->kh - 1 - c0y); col.pl = (int)(ph->kw - 1 - c0x);
          col.rows = (int)(ohp * owp); col.kc = ph->kc;
          col.xor_mask = 0; col.pad16 = pad16(ctx, 0);
          DenseOperand wt{ph->data, ph->ld_bytes, (int)d->cout, ph->kc, 0, 0u, pad16(ctx, 0)};
          FloatOut o{};
          o.y = static_cast<char*>(y) + (n * d->cout * oh * ow + ry * ow + rx) * eb;
          o.alpha = 1.0f; o.beta = 1.0f; o.bias = bias; o.bias_mode = BIAS_J; o.act = ACT_NONE;
          o.si = sw; o.sj = oh * ow; o.bstride = sh * ow; o.ohw = (int)owp;
          o.P = (int)(ohp * owp); o.Q = (int)d->cout; o.vec = 0;
          const int splits = plan_splits(o.P, o.Q, ph->kc, ctx->tile_override);
          o.splits = splits;
          o.split_ws = splits > 1 ? scratch_at(ctx, plan, iw) : nullptr;
          DENSE_FITS_OR_DECLINE(wt, "ohip_conv_transpose2d");
          ctx->counters.contraction_launches++;
          hipError_t e = run_conv_float(d->dtype, col, wt, true, o, ctx->tile_override, ctx->stream);
          if (e != hipSuccess) return hip_fail(e, "ohip_conv_transpose2d phase launch");
        }
    return OHIP_OK;
  }
  ConvTArgs a{};
  a.N = (int)d->n; a.C = (int)d->c; a.H = (int)d->h; a.W = (int)d->w; a.cout = (int)d->cout;
  a.cg = (int)(d->c / d->group); a.coutg = (int)(d->cout / d->group); a.KH = (int)d->kh; a.KW = (int)d->kw;
  a.sh = (int)d->stride_h; a.sw = (int)d->stride_w; a.dh = (int)d->dil_h; a.dw = (int)d->dil_w;
  a.pt = (int)d->pad_t; a.pl = (int)d->pad_l; a.OH = (int)oh; a.OW = (int)ow;
  hipError_t e = run_conv_transpose(d->dtype, x, w->data, bias, y, a, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "ohip_conv_transpose2d launch");
  return OHIP_OK;
}

// ------------------------------------------------------------------ integer GEMM
// |sum (a - a_zp)(w - w_zp)| <= K * 255 * 255; below this K neither the
// int32 MFMA accumulator nor the epilogue can overflow.
static const int64_t kMaxExactK = ((int64_t)INT32_MAX) / (255 * 255);

extern "C" int ohip_qgemm(ohip_ctx* ctx, const ohip_qgemm_desc* d, const void* a, const ohip_weight* b, void* y) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!d || !a || !b || !y) return fail(OHIP_E_INVALID, "ohip_qgemm: null argument");
  if (b->kind != WK_QGEMM) return fail(OHIP_E_INVALID, "ohip_qgemm: weight kind mismatch");
  if (d->a_dtype != OHIP_U8 && d->a_dtype != OHIP_I8) return fail(OHIP_E_INVALID, "ohip_qgemm: A must be u8/i8");
  if (d->k != b->k || d->n != b->rows || d->m < 0) return fail(OHIP_E_SHAPE, "ohip_qgemm: shape mismatch");
  if (d->n_azp != 1 && d->n_azp != d->m) return fail(OHIP_E_SHAPE, "a_zero_point has the wrong length");
  if (d->k > kMaxExactK) return fail(OHIP_DECLINED, "ohip_qgemm: K too large for an exact int32 accumulator");
  if (d->m > INT_MAX / 2) return fail(OHIP_DECLINED, "ohip_qgemm: extent too large");
  if (d->m == 0) return OHIP_OK;
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->counters.dispatches++;
  const int64_t M = d->m, N = d->n, K = d->k, kp = round_up(K, 16);
  const int64_t lda = d->lda ? d->lda : K, ldy = d->ldy ? d->ldy : N;
  const bool direct = rows_direct(a, K, lda, 1, 0);
  const bool u8 = d->a_dtype == OHIP_U8;
  const int32_t shift = u8 ? 128 : 0;
  int n_comb = 1;
  if (d->out_kind != OHIP_QOUT_I32) {
    rc = ensure_comb(ctx, const_cast<ohip_weight*>(b), d->a_scale, d->y_scale, &n_comb);
    if (rc) return rc;
  }
  ScratchPlan plan;
  size_t ia = direct ? SIZE_MAX : plan.add((size_t)(M * kp));
  size_t ir = d->n_azp > 1 ? plan.add((size_t)M * 4) : SIZE_MAX;
  const int splits = plan_splits((int)N, (int)M, b->kc, ctx->tile_override);
  size_t iw = splits > 1 ? plan.add(split_ws_bytes((int)N, (int)M, splits)) : SIZE_MAX;
  rc = scratch_reserve(ctx, plan.total());
  if (rc) return rc;
  const void* pa = a;
  int64_t lda_b = lda;
  if (!direct) {
    void* s = scratch_at(ctx, plan, ia);
    HIP_TRY(run_gather2d(1, a, lda, 1, s, (int)M, (int)K, (int)kp, ctx->stream), "pack A");
    pa = s;
    lda_b = kp;
  }
  int32_t* ca_rows = nullptr;
  if (d->n_azp > 1) {
    std::vector<int32_t> rows((size_t)M);
    for (int64_t i = 0; i < M; ++i) rows[(size_t)i] = shift - d->a_zp[i];
    ca_rows = static_cast<int32_t*>(scratch_at(ctx, plan, ir));
    HIP_TRY(hipMemcpyAsync(ca_rows, rows.data(), rows.size() * 4, hipMemcpyHostToDevice, ctx->stream), "a_zp upload");
    HIP_TRY(hipStreamSynchronize(ctx->stream), "a_zp upload sync");
  }
  QuantOut o{};
  o.y = y; o.si = 1; o.sj = ldy; o.bstride = 0; o.ohw = INT_MAX; o.P = (int)N; o.Q = (int)M;
  const int ob = (d->out_kind == OHIP_QOUT_I32 || d->out_kind == OHIP_QOUT_F32) ? 4 : 1;
  o.vec = ldy % 4 == 0 && aligned(y, 4 * ob);
  o.w_on_i = 1; o.colsum = b->colsum; o.flip = b->flip; o.bias = nullptr;
  o.ca = shift - (d->a_zp ? d->a_zp[0] : 0); o.ca_rows = ca_rows;
  o.comb = b->comb; o.n_comb = n_comb; o.out_kind = d->out_kind; o.y_zp = d->y_zp; o.lo = d->lo; o.hi = d->hi;
  DenseOperand x{b->data, b->ld_bytes, (int)N, b->kc, 0, 0u, pad16(ctx, 0)};
  DenseOperand yv{pa, lda_b, (int)M, (int)(kp / 16), b->kwrap, u8 ? 0x80808080u : 0u, pad16(ctx, 0)};
  DENSE_FITS_OR_DECLINE(x, "ohip_qgemm");
  DENSE_FITS_OR_DECLINE(yv, "ohip_qgemm");
  o.splits = splits;
  o.split_ws = splits > 1 ? scratch_at(ctx, plan, iw) : nullptr;
  ctx->counters.contraction_launches++;
  hipError_t e = run_dense_quant(x, yv, o, ctx->tile_override, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "ohip_qgemm launch");
  return OHIP_OK;
}

// Device copy of a 256-byte output table, uploaded once per distinct content
// (called with ctx->mu held).
static int device_table(ohip_ctx* ctx, const uint8_t* host, const uint8_t** out) {
  std::string key(reinterpret_cast<const char*>(host), 256);
  auto it = ctx->tables.find(key);
  if (it != ctx->tables.end()) { *out = it->second; return OHIP_OK; }
  uint8_t* d = nullptr;
  hipError_t e = dev_malloc(ctx, (void**)&d, 256);
  if (e != hipSuccess) return fail(OHIP_E_NOMEM, "table hipMalloc");
  HIP_TRY(hipMemcpy(d, host, 256, hipMemcpyHostToDevice), "table upload");
  ctx->tables.emplace(key, d);
  *out = d;
  return OHIP_OK;
}

extern "C" int ohip_qconv2d(ohip_ctx* ctx, const ohip_qconv_desc* d, const void* x, const ohip_weight* w,
                            const int32_t* bias, void* y) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!d || !x || !w || !y) return fail(OHIP_E_INVALID, "ohip_qconv2d: null argument");
  if (d->group < 1 || d->c % d->group || d->cout % d->group) return fail(OHIP_E_SHAPE, "ohip_qconv2d: bad group");
  if (w->kind != WK_QCONV) return fail(OHIP_E_INVALID, "ohip_qconv2d: weight kind mismatch");
  if (d->x_dtype != OHIP_U8 && d->x_dtype != OHIP_I8) return fail(OHIP_E_INVALID, "ohip_qconv2d: X must be u8/i8");
  const int64_t G = d->group, cg = d->c / G, coutg = d->cout / G;
  if (w->rows != d->cout || w->k != cg || w->kh != d->kh || w->kw != d->kw)
    return fail(OHIP_E_SHAPE, "ohip_qconv2d: shape disagrees with the packed filter");
  if (cg * d->kh * d->kw > kMaxExactK) return fail(OHIP_DECLINED, "ohip_qconv2d: K too large for exact int32");
  ConvGeo g;
  rc = conv_geo(d->h, d->w, d->kh, d->kw, d->stride_h, d->stride_w, d->dil_h, d->dil_w, d->pad_t, d->pad_l,
                d->pad_b, d->pad_r, &g);
  if (rc) return rc;
  const int64_t cp = round_up(cg, 16);   // channel slots per group and tap
  const int64_t cpt = G * cp;            // channel slots per staged pixel
  // pixel stride of an NHWC input: its own pitch (a channel range of a wider
  // tensor read in place), else the padded channel count
  const int64_t in_pstride = d->in_layout == OHIP_NHWC && d->in_pitch > 0 ? d->in_pitch : cpt;
  if (d->in_layout == OHIP_NHWC && d->in_pitch > 0 && (G > 1 || d->in_pitch % 16 || d->in_pitch < cp))
    return fail(OHIP_E_INVALID, "ohip_qconv2d: in_pitch must be a multiple of 16 covering the channels, group 1");
  const int64_t rows = d->n * g.oh * g.ow;
  if (rows > INT_MAX / 2) return fail(OHIP_DECLINED, "ohip_qconv2d: extent too large");
  if (rows == 0) return OHIP_OK;
  // narrow groups (depthwise and the like) run the exact direct kernel on the
  // NCHW input; wider groups run one MFMA launch per group.  So do ungrouped
  // convolutions of an NCHW input with under 32 taps x channels (as
  // ohip_conv2d).
  static const int stem_mode = [] { const char* e = std::getenv("OHIP_QSTEM"); return e ? std::atoi(e) : 1; }();
  const bool narrow = G == 1 && d->in_layout == OHIP_NCHW && cg * d->kh * d->kw < 32 && stem_mode == 1;
  const bool direct = (G > 1 && (coutg < 16 || cg * d->kh * d->kw < 32 || G > 64)) || narrow;
  if (G > 1 && d->in_layout != OHIP_NCHW && (direct || cg % 16 != 0))
    return fail(OHIP_DECLINED, "ohip_qconv2d: this grouped convolution needs an NCHW input");
  if (d->out_table && d->out_kind != OHIP_QOUT_U8 && d->out_kind != OHIP_QOUT_I8)
    return fail(OHIP_E_INVALID, "ohip_qconv2d: an output table needs a byte output");
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->counters.dispatches++;
  const bool u8 = d->x_dtype == OHIP_U8;
  const int32_t shift = u8 ? 128 : 0;
  int n_comb = 1;
  if (d->out_kind != OHIP_QOUT_I32) {
    rc = ensure_comb(ctx, const_cast<ohip_weight*>(w), d->x_scale, d->y_scale, &n_comb);
    if (rc) return rc;
  }
  const uint8_t* table = nullptr;
  if (d->out_table) {
    rc = device_table(ctx, d->out_table, &table);
    if (rc) return rc;
  }
  const int ob = (d->out_kind == OHIP_QOUT_I32 || d->out_kind == OHIP_QOUT_F32) ? 4 : 1;
  const int64_t ohw = g.oh * g.ow;
  const int64_t ldo = ob == 1 ? round_up(d->cout, 16) : round_up(d->cout, 4);
  const bool nchw_out = d->out_layout == OHIP_NCHW;

  if (direct) {
    DirectQConvArgs a{};
    a.N = (int)d->n; a.C = (int)d->c; a.H = (int)d->h; a.W = (int)d->w; a.cout = (int)d->cout;
    a.cg = (int)cg; a.coutg = (int)coutg; a.KH = (int)d->kh; a.KW = (int)d->kw;
    a.sh = (int)d->stride_h; a.sw = (int)d->stride_w; a.dh = (int)d->dil_h; a.dw = (int)d->dil_w;
    a.pt = (int)d->pad_t; a.pl = (int)d->pad_l; a.OH = (int)g.oh; a.OW = (int)g.ow;
    a.ldw = w->ld_bytes; a.cpg = (int)cp; a.half = w->kwrap > 0 ? (int64_t)w->kwrap * 16 : 0;
    a.x_signed = !u8; a.x_zp = d->x_zp; a.flip = w->flip; a.bias = bias; a.comb = w->comb; a.n_comb = n_comb;
    a.out_kind = d->out_kind; a.y_zp = d->y_zp; a.lo = d->lo; a.hi = d->hi; a.table = table;
    a.nhwc_out = !nchw_out; a.ldo = ldo;
    hipError_t e = run_qconv_direct(x, w->data, y, a, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "ohip_qconv2d direct launch");
    return OHIP_OK;
  }

  ScratchPlan plan;
  const bool stage = d->in_layout == OHIP_NCHW;
  size_t ix = stage ? plan.add((size_t)(d->n * d->h * d->w * cpt)) : SIZE_MAX;
  const int sP = nchw_out ? (int)rows : (int)coutg, sQ = nchw_out ? (int)coutg : (int)rows;
  const int splits = plan_splits(sP, sQ, w->kc, ctx->tile_override);
  size_t iw = splits > 1 ? plan.add(split_ws_bytes(sP, sQ, splits)) : SIZE_MAX;
  rc = scratch_reserve(ctx, plan.total());
  if (rc) return rc;
  const void* xin = x;
  if (stage) {
    void* px = scratch_at(ctx, plan, ix);
    if (G > 1)
      HIP_TRY(run_stage_nhwc(1, x, px, (int)d->n, (int)d->c, (int)d->h, (int)d->w, 0, 0, 0, 0, 0, (int)cg, (int)cp,
                             (int)G, ctx->stream),
              "NCHW -> grouped NHWC");
    else
      HIP_TRY(run_nchw_to_nhwc(1, x, px, (int)d->n, (int)d->c, (int)(d->h * d->w), (int)cp, ctx->stream),
              "NCHW -> NHWC");
    xin = px;
  } else if (!aligned(x, 16)) {
    return fail(OHIP_E_INVALID, "ohip_qconv2d: NHWC input must be 16-byte aligned");
  }
  // A padding tap stands for x == x_zp, i.e. (x_zp - shift) in the shifted
  // int8 domain, so it contributes exactly zero after the ca correction.  The
  // pad source is read before the XOR, so it holds the raw byte x_zp.  The
  // channel-padding slots of the staged input meet zero filter entries.
  const uint8_t padb = (uint8_t)(d->x_zp & 0xff);
  for (int64_t gi = 0; gi < G; ++gi) {
    Im2colOperand col{};
    col.base = static_cast<const char*>(xin) + gi * cp;
    col.H = (int)d->h; col.W = (int)d->w; col.OH = (int)g.oh; col.OW = (int)g.ow;
    col.KW = (int)d->kw; col.cpc = (int)(cp / 16); col.pstride = (int)((stage ? cpt : in_pstride) / 16);
    col.sh = (int)d->stride_h; col.sw = (int)d->stride_w; col.dh = (int)d->dil_h; col.dw = (int)d->dil_w;
    col.pt = (int)d->pad_t; col.pl = (int)d->pad_l; col.rows = (int)rows;
    col.kc = w->kwrap > 0 ? w->kreal : w->kc; col.kwrap = w->kwrap;
    col.xor_mask = u8 ? 0x80808080u : 0u;
    col.pad16 = pad16(ctx, padb);
    DenseOperand wt{static_cast<const char*>(w->data) + gi * coutg * w->ld_bytes, w->ld_bytes, (int)coutg, w->kc,
                    0, 0u, pad16(ctx, 0)};
    QuantOut o{};
    o.colsum = w->colsum + gi * coutg;
    o.flip = w->flip ? w->flip + gi * coutg : nullptr;
    o.bias = bias ? bias + gi * coutg : nullptr;
    o.ca = shift - d->x_zp; o.ca_rows = nullptr;
    o.comb = (n_comb > 1 && w->comb) ? w->comb + gi * coutg : w->comb;
    o.n_comb = n_comb; o.out_kind = d->out_kind; o.y_zp = d->y_zp; o.lo = d->lo; o.hi = d->hi;
    o.table = table;
    bool col_on_x;
    if (nchw_out) {
      col_on_x = true;
      o.y = static_cast<char*>(y) + gi * coutg * ohw * ob;
      o.si = 1; o.sj = ohw; o.bstride = d->cout * ohw; o.ohw = (int)ohw; o.P = (int)rows; o.Q = (int)coutg;
      o.vec = ohw % 4 == 0 && aligned(o.y, 4 * ob);
      o.w_on_i = 0;
    } else {
      col_on_x = false;
      o.y = static_cast<char*>(y) + gi * coutg * ob;
      o.si = 1; o.sj = ldo; o.bstride = 0; o.ohw = INT_MAX; o.P = (int)coutg; o.Q = (int)rows;
      o.vec = ldo % 4 == 0 && aligned(o.y, 4 * ob);
      o.w_on_i = 1;
    }
    DENSE_FITS_OR_DECLINE(wt, "ohip_qconv2d");
    o.splits = splits;
    o.split_ws = splits > 1 ? scratch_at(ctx, plan, iw) : nullptr;
    ctx->counters.contraction_launches++;
    hipError_t e = run_conv_quant(col, wt, col_on_x, o, ctx->tile_override, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "ohip_qconv2d launch");
  }
  return OHIP_OK;
}

// ------------------------------------------------------------------ device tensors
static int dt_bytes(int dtype, int rank, const int64_t* shape, int layout, size_t* out) {
  const int eb = elem_bytes(dtype);
  if (!eb || rank < 0 || rank > 8) return fail(OHIP_E_INVALID, "dtensor: bad dtype / rank");
  int64_t e = 1;
  for (int i = 0; i < rank; ++i) {
    if (shape[i] < 0) return fail(OHIP_E_INVALID, "dtensor: negative extent");
    e *= (layout == OHIP_NHWC && i == 1) ? round_up(shape[i], 16 / eb) : shape[i];
  }
  *out = (size_t)e * eb;
  return OHIP_OK;
}

extern "C" int ohip_dtensor_alloc(ohip_ctx* ctx, int dtype, int rank, const int64_t* shape, int layout,
                                  ohip_dtensor** out) {
  int rc = activate(ctx);
  if (rc) return rc;
  if (!out || (rank && !shape)) return fail(OHIP_E_INVALID, "dtensor: null argument");
  if (layout == OHIP_NHWC && rank != 4) return fail(OHIP_E_INVALID, "dtensor: NHWC needs rank 4");
  size_t bytes;
  rc = dt_bytes(dtype, rank, shape, layout, &bytes);
  if (rc) return rc;
  auto* t = new ohip_dtensor();
  t->ctx = ctx; t->dtype = dtype; t->rank = rank; t->layout = layout; t->bytes = bytes;
  for (int i = 0; i < rank; ++i) t->shape[i] = shape[i];
  rc = pool_alloc(ctx, bytes ? bytes : 16, &t->ptr);
  if (rc) { delete t; return rc; }
  t->buf = std::shared_ptr<DevBuf>(new DevBuf{ctx, t->ptr});
  if (layout == OHIP_NHWC) {  // channel padding must read as zero (a fill kernel: capture-safe)
    hipError_t e = run_zero_fill(t->ptr, bytes, ctx->stream);
    if (e != hipSuccess) { delete t; return hip_fail(e, "dtensor zero fill"); }
  }
  *out = t;
  return OHIP_OK;
}

extern "C" int ohip_dtensor_wrap(ohip_ctx* ctx, void* p, int dtype, int rank, const int64_t* shape,
                                 ohip_dtensor** out) {
  if (!ctx || !p || !out) return fail(OHIP_E_INVALID, "dtensor_wrap: null argument");
  size_t bytes;
  int rc = dt_bytes(dtype, rank, shape, OHIP_NCHW, &bytes);
  if (rc) return rc;
  auto* t = new ohip_dtensor();
  t->ctx = ctx; t->ptr = p; t->dtype = dtype; t->rank = rank; t->layout = OHIP_NCHW; t->bytes = bytes;
  t->buf = std::shared_ptr<DevBuf>(new DevBuf{ctx, p});
  for (int i = 0; i < rank; ++i) t->shape[i] = shape[i];
  *out = t;
  return OHIP_OK;
}

// Session-lifetime device copy of a small initializer operand (a bias, a Gemm
// C, a normalisation scale, a broadcast constant), in the form the caller
// converted it to: initializers are invariant for the context's life, as
// for the weight cache (oxionnx-cuda/src/lib.rs:519-541), so each is
// uploaded once instead of on every dispatch.
int ohip_const_operand_internal(ohip_ctx* ctx, const char* name, const char* label, int dtype, const void* host,
                                size_t bytes, const void** dev) {
  if (!ctx || !name || !*name || !host || !dev) return fail(OHIP_E_INVALID, "const operand: bad argument");
  std::string k(name);
  k += '\x1f';
  k += label ? label : "";
  k += '\x1f' + std::to_string(dtype) + '\x1f' + std::to_string(bytes);
  std::lock_guard<std::mutex> lock(ctx->mu);
  auto it = ctx->consts.find(k);
  if (it != ctx->consts.end()) { *dev = it->second; return OHIP_OK; }
  void* d = nullptr;
  hipError_t e = dev_malloc(ctx, &d, bytes ? bytes : 16);
  if (e != hipSuccess) return fail(OHIP_E_NOMEM, "const operand hipMalloc");
  HIP_TRY(hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, ctx->stream), "const operand upload");
  HIP_TRY(hipStreamSynchronize(ctx->stream), "const operand upload sync");
  ctx->counters.h2d_bytes += bytes;
  ctx->consts.emplace(k, d);
  *dev = d;
  return OHIP_OK;
}

// A second tensor over the same buffer (a Reshape / Flatten / Squeeze /
// Unsqueeze result): same bytes, new shape, shared ownership.
int ohip_dtensor_alias_internal(const ohip_dtensor* src, int rank, const int64_t* shape, ohip_dtensor** out) {
  if (!src || !out || rank < 0 || rank > 8) return fail(OHIP_E_INVALID, "dtensor_alias: bad argument");
  size_t bytes;
  int rc = dt_bytes(src->dtype, rank, shape, OHIP_NCHW, &bytes);
  if (rc) return rc;
  if (bytes != src->bytes || src->layout != OHIP_NCHW) return fail(OHIP_E_INVALID, "dtensor_alias: size mismatch");
  auto* t = new ohip_dtensor();
  t->ctx = src->ctx; t->buf = src->buf; t->ptr = src->ptr; t->dtype = src->dtype; t->rank = rank;
  t->layout = OHIP_NCHW; t->bytes = bytes;
  for (int i = 0; i < rank; ++i) t->shape[i] = shape[i];
  *out = t;
  return OHIP_OK;
}

// A tensor over a contiguous sub-range of another's buffer (a Slice that
// keeps one run of elements), starting byte_offset bytes in; shared ownership.
int ohip_dtensor_view_internal(const ohip_dtensor* src, int rank, const int64_t* shape, size_t byte_offset,
                               ohip_dtensor** out) {
  if (!src || !out || rank < 0 || rank > 8) return fail(OHIP_E_INVALID, "dtensor_view: bad argument");
  size_t bytes;
  int rc = dt_bytes(src->dtype, rank, shape, OHIP_NCHW, &bytes);
  if (rc) return rc;
  if (src->layout != OHIP_NCHW || byte_offset > src->bytes || bytes > src->bytes - byte_offset)
    return fail(OHIP_E_INVALID, "dtensor_view: range outside the source");
  auto* t = new ohip_dtensor();
  t->ctx = src->ctx; t->buf = src->buf; t->ptr = static_cast<char*>(src->ptr) + byte_offset; t->dtype = src->dtype;
  t->rank = rank; t->layout = OHIP_NCHW; t->bytes = bytes;
  for (int i = 0; i < rank; ++i) t->shape[i] = shape[i];
  *out = t;
  return OHIP_OK;
}

// NHWC resident tensors: a produced one is marked with its pixel pitch; a
// channel range of one is a view with the same pitch; the pitch is read by
// the consumers that take NHWC in place, and the conversion to NCHW serves
// the rest.
int ohip_dtensor_set_nhwc_internal(ohip_dtensor* t, int64_t pitch) {
  if (!t || t->rank != 4 || pitch < t->shape[1]) return fail(OHIP_E_INVALID, "dtensor: NHWC pitch");
  t->layout = OHIP_NHWC;
  t->pitch = pitch;
  return OHIP_OK;
}
int64_t ohip_dtensor_pitch_internal(const ohip_dtensor* t) { return t && t->layout == OHIP_NHWC ? t->pitch : 0; }
int ohip_dtensor_view_nhwc_internal(const ohip_dtensor* src, int64_t c0, int64_t cn, ohip_dtensor** out) {
  if (!src || !out || src->layout != OHIP_NHWC || c0 < 0 || cn < 0 || c0 + cn > src->shape[1])
    return fail(OHIP_E_INVALID, "dtensor_view: NHWC channel range");
  auto* t = new ohip_dtensor(*src);
  t->ptr = static_cast<char*>(src->ptr) + c0 * elem_bytes(src->dtype);
  t->shape[1] = cn;
  size_t nb = 0;   // the view's own element bytes (its NCHW form's size)
  if (dt_bytes(t->dtype, t->rank, t->shape, OHIP_NCHW, &nb) == OHIP_OK) t->bytes = nb;
  *out = t;
  return OHIP_OK;
}
// Writes the NCHW form of an NHWC tensor into dst (shape-product elements).
int ohip_dtensor_to_nchw_internal(ohip_ctx* ctx, const ohip_dtensor* t, void* dst) {
  if (!t || t->layout != OHIP_NHWC || !dst) return fail(OHIP_E_INVALID, "dtensor_to_nchw: not NHWC");
  HIP_TRY(run_nhwc_to_nchw(elem_bytes(t->dtype), t->ptr, dst, (int)t->shape[0], (int)t->shape[1],
                           (int)(t->shape[2] * t->shape[3]), (int)t->pitch, ctx->stream),
          "NHWC -> NCHW");
  return OHIP_OK;
}

extern "C" int ohip_dtensor_to_nchw(ohip_ctx* ctx, const ohip_dtensor* t, ohip_dtensor** out) {
  if (!t || !out) return fail(OHIP_E_INVALID, "dtensor_to_nchw: null argument");
  if (t->layout == OHIP_NCHW) return ohip_dtensor_alias_internal(t, t->rank, t->shape, out);
  int rc = activate(ctx);
  if (rc) return rc;
  size_t nb = 0;
  rc = dt_bytes(t->dtype, t->rank, t->shape, OHIP_NCHW, &nb);
  if (rc) return rc;
  void* p = nullptr;
  rc = ohip_malloc(ctx, nb ? nb : 16, &p);
  if (rc) return rc;
  rc = ohip_dtensor_to_nchw_internal(ctx, t, p);
  if (!rc) rc = ohip_dtensor_wrap(ctx, p, t->dtype, t->rank, t->shape, out);
  if (rc) ohip_free(ctx, p);
  return rc;
}

extern "C" int ohip_dtensor_upload(ohip_ctx* ctx, ohip_dtensor* t, const void* host) {
  if (!t || !host) return fail(OHIP_E_INVALID, "dtensor_upload: null argument");
  if (t->layout != OHIP_NCHW) return fail(OHIP_E_INVALID, "dtensor_upload: NCHW tensors only");
  return ohip_memcpy_h2d(ctx, t->ptr, host, t->bytes);
}
extern "C" int ohip_dtensor_download(ohip_ctx* ctx, const ohip_dtensor* t, void* host) {
  if (!t || !host) return fail(OHIP_E_INVALID, "dtensor_download: null argument");
  if (t->layout == OHIP_NHWC) {
    // the NCHW form through a temporary buffer
    int rc = activate(ctx);
    if (rc) return rc;
    size_t nb = 0;
    rc = dt_bytes(t->dtype, t->rank, t->shape, OHIP_NCHW, &nb);
    if (rc) return rc;
    void* tmp = nullptr;
    rc = ohip_malloc(ctx, nb ? nb : 16, &tmp);
    if (rc) return rc;
    rc = ohip_dtensor_to_nchw_internal(ctx, t, tmp);
    if (!rc) rc = ohip_memcpy_d2h(ctx, host, tmp, nb);
    ohip_free(ctx, tmp);
    return rc;
  }
  if (t->layout != OHIP_NCHW) return fail(OHIP_E_INVALID, "dtensor_download: NCHW tensors only");
  return ohip_memcpy_d2h(ctx, host, t->ptr, t->bytes);
}
extern "C" void* ohip_dtensor_ptr(const ohip_dtensor* t) { return t ? t->ptr : nullptr; }
extern "C" int ohip_dtensor_layout(const ohip_dtensor* t) { return t ? t->layout : -1; }
extern "C" int ohip_dtensor_info(const ohip_dtensor* t, int* dtype, int* rank, int64_t* shape8, size_t* bytes) {
  if (!t) return fail(OHIP_E_INVALID, "null dtensor");
  if (dtype) *dtype = t->dtype;
  if (rank) *rank = t->rank;
  if (shape8) for (int i = 0; i < 8; ++i) shape8[i] = i < t->rank ? t->shape[i] : 0;
  if (bytes) *bytes = t->bytes;
  return OHIP_OK;
}
extern "C" void ohip_dtensor_free(ohip_dtensor* t) {
  if (!t) return;
  delete t;  // the last owner of the buffer returns it to the pool
}

// ------------------------------------------------------------------ gating / declines
extern "C" int ohip_ctx_try_new(ohip_ctx** out) {
  if (!out) return fail(OHIP_E_INVALID, "null out");
  *out = nullptr;
  if (!ohip_env_flag("OXIONNX_HIP")) return fail(OHIP_DECLINED, "OXIONNX_HIP is not set");
  int dev = 0;
  if (const char* d = std::getenv("OXIONNX_HIP_DEVICE")) dev = std::atoi(d);
  int rc = ohip_ctx_create(dev, out);
  return rc == OHIP_E_NODEVICE ? fail(OHIP_DECLINED, "no gfx950 device") : rc;
}
extern "C" void ohip_note_declined(ohip_ctx* ctx, const char* why) {
  if (!ctx) return;
  std::lock_guard<std::mutex> lock(ctx->mu);
  ctx->counters.declined++;
  ctx->last_decline = why ? why : "";
}
extern "C" const char* ohip_last_decline(ohip_ctx* ctx) { return ctx ? ctx->last_decline.c_str() : ""; }

// ------------------------------------------------------------------ counters
extern "C" int ohip_get_counters(ohip_ctx* ctx, ohip_counters* out) {
  if (!ctx || !out) return fail(OHIP_E_INVALID, "null argument");
  *out = ctx->counters;
  out->device_allocs = ctx->device_allocs.load(std::memory_order_relaxed);
  {
    std::lock_guard<std::mutex> lock(ctx->pool_mu);
    out->pool_live = ctx->pool.live.size();
  }
  return OHIP_OK;
}
extern "C" int ohip_reset_counters(ohip_ctx* ctx) {
  if (!ctx) return fail(OHIP_E_INVALID, "null context");
  uint64_t resident = ctx->counters.weight_resident_bytes;
  ctx->counters = ohip_counters{};
  ctx->counters.weight_resident_bytes = resident;
  ctx->device_allocs.store(0, std::memory_order_relaxed);
  return OHIP_OK;
}
