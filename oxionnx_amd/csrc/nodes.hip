// Device kernels for the memory-bound nodes that sit between the
// contractions of a conv network (activations, broadcast arithmetic,
// instance normalisation, nearest resize, pad, max pool, slice, quantise /
// dequantise, byte tables).  They keep activations resident between the
// contraction nodes; each is one pass over its tensor, bound by HBM.
//
// Float tensors are f32 or f16 storage with f32 arithmetic; quantised
// tensors are u8 / i8 bytes.
#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

#include "internal.hpp"
#include "norm_stats.hpp"

namespace ohip {

namespace {

template <class T> __device__ __forceinline__ float ldf(const T* p, int64_t i) { return (float)p[i]; }
template <class T> __device__ __forceinline__ void stf(T* p, int64_t i, float v) { p[i] = (T)v; }

constexpr int kThreads = 256;

inline unsigned grid_for(int64_t n, int per_thread = 1) {
  int64_t b = (n + (int64_t)kThreads * per_thread - 1) / ((int64_t)kThreads * per_thread);
  if (b < 1) b = 1;
  if (b > 65535 * 16) b = 65535 * 16;  // grid-stride loops cover the rest
  return (unsigned)b;
}

// ---------------------------------------------------------------- unary
__device__ __forceinline__ float unary_op(float v, int op, float alpha) {
  switch (op) {
    case UN_RELU: return v > 0.0f ? v : 0.0f;
    case UN_LEAKY_RELU: return v >= 0.0f ? v : v * alpha;
    case UN_TANH: return tanhf(v);
    case UN_SIGMOID: return 1.0f / (1.0f + expf(-v));
    case UN_SILU: return v / (1.0f + expf(-v));
    default: return v;
  }
}

template <class T>
__global__ void __launch_bounds__(kThreads) unary_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n, int op,
                                                         float alpha) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    stf(y, i, unary_op(ldf(x, i), op, alpha));
}

// ---------------------------------------------------------------- binary with broadcasting
__device__ __forceinline__ float binary_op(float a, float b, int op) {
  switch (op) {
    case BIN_ADD: return a + b;
    case BIN_SUB: return a - b;
    case BIN_MUL: return a * b;
    default: return a / b;
  }
}

template <class T>
__global__ void __launch_bounds__(kThreads) binary_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                          T* __restrict__ y, int64_t n, BcastPlan p, int op) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    int64_t ia = 0, ib = 0, r = i;
#pragma unroll
    for (int d = kMaxRank - 1; d >= 0; --d) {
      if (d < kMaxRank - p.rank) break;
      const int64_t e = p.shape[d];
      const int64_t c = r % e;
      r /= e;
      ia += c * p.sa[d];
      ib += c * p.sb[d];
    }
    stf(y, i, binary_op(ldf(a, ia), ldf(b, ib), op));
  }
}

// Same-shape operands: no index arithmetic.
template <class T>
__global__ void __launch_bounds__(kThreads) binary_same_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                               T* __restrict__ y, int64_t n, int op) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    stf(y, i, binary_op(ldf(a, i), ldf(b, i), op));
}

// ---------------------------------------------------------------- instance normalisation
// One block per (n, c) plane: the plane is staged in LDS as f32 (planes of
// up to kNormPlaneLds values; larger ones are read from global memory), its
// statistics follow norm_stats.hpp (each thread a run's moments, sixteen
// lanes a segment's, one wave a group's tree, thread 0 the groups), then
// every thread rescales its share with the optional per-channel (or
// per-(n, c)) affine term and activation.
constexpr int64_t kNormPlaneLds = 15360;

template <class T>
__global__ void __launch_bounds__(kThreads) instnorm_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t spatial,
                                                            int C, float eps, NormAffine aff) {
  extern __shared__ float xs[];
  __shared__ float2 segm[kNormGroup];
  __shared__ float st[2];
  const int64_t plane = blockIdx.x;
  const T* xp = x + plane * spatial;
  T* yp = y + plane * spatial;
  const bool staged = spatial <= kNormPlaneLds;
  if (staged) {
    for (int64_t i = threadIdx.x; i < spatial; i += kThreads) xs[i] = ldf(xp, i);
    __syncthreads();
  }
  auto ld = [&](int64_t i) { return staged ? xs[i] : ldf(xp, i); };
  static_assert(kThreads == kNormGroup, "a group's threads");
  const int S = norm_segments(spatial);
  Moments acc{0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < S; s0 += kNormGroup) {
    const int cnt = S - s0 < kNormGroup ? S - s0 : kNormGroup;
    group_segments(ld, spatial, s0, cnt, segm, threadIdx.x);
    __syncthreads();
    const int64_t gend = (int64_t)(s0 + cnt) * kNormSeg < spatial ? (int64_t)(s0 + cnt) * kNormSeg : spatial;
    const int n_last = (int)(gend - (int64_t)(s0 + cnt - 1) * kNormSeg);
    if (threadIdx.x < 64) {
      float2 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = 4 * (int)threadIdx.x + j < cnt ? segm[4 * threadIdx.x + j] : float2{0.0f, 0.0f};
      const Moments gm = wave_tree(v, cnt, n_last, threadIdx.x);
      if (threadIdx.x == 0) {
        if (s0 == 0) acc = gm;
        else chan_merge(acc, gm);
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    st[0] = acc.m;
    st[1] = 1.0f / sqrtf(acc.m2 / (float)spatial + eps);
  }
  __syncthreads();
  const float mean = st[0], inv = st[1];
  const int c = (int)(plane % C);
  const int64_t n = plane / C;
  float sc = 1.0f, bi = 0.0f;
  bool affine = false;
  const int64_t ai = aff.per_sample ? n * aff.stride + c : c;
  if (aff.scale) {
    sc = aff.same_type ? ldf(static_cast<const T*>(aff.scale), ai) : static_cast<const float*>(aff.scale)[ai];
    affine = true;
  }
  if (aff.bias) {
    bi = aff.same_type ? ldf(static_cast<const T*>(aff.bias), ai) : static_cast<const float*>(aff.bias)[ai];
    affine = true;
  }
  // A fused affine tail keeps the unfused chain's storage roundings: the
  // normalised value, the product and the sum are each rounded to T, as the
  // OxiInstanceNorm -> Mul -> Add nodes store them.
  for (int64_t i = threadIdx.x; i < spatial; i += kThreads) {
    float v = (ld(i) - mean) * inv;
    if (affine) {
      v = round_to<T>(v);
      if (aff.scale) v = round_to<T>(v * sc);
      if (aff.bias) v = round_to<T>(v + bi);
    }
    if (aff.act == UN_RELU) v = v > 0.0f ? v : 0.0f;
    else if (aff.act == UN_LEAKY_RELU) v = round_to<T>(v), v = v >= 0.0f ? v : v * aff.alpha;
    if (aff.residual) {
      const T* r = static_cast<const T*>(aff.residual);
      v = round_to<T>(v) + (aff.res_nhwc ? ldf(r, (n * spatial + i) * C + c) : ldf(r + plane * spatial, i));
    }
    stf(yp, i, opaque(v));
  }
}

// The same normalisation over a plane rebuilt from split-K partial sums in
// LDS: x_i = T(sum over slices in slice order + bias), the value the split
// reduction would have stored; the statistics (norm_stats.hpp) and the
// rescale then read LDS instead of global memory, so the result is the
// unfused pair's.  PPB planes (channels of one image) per block, 256 threads
// each; with PPB > 1 (an NHWC output) each pixel's PPB channels are written
// (and a residual read) as one run.
#ifdef OHIP_KTIMING
// Diagnostic build only (never in the shipped library): per-block stamps of
// the 100 MHz real-time counter at the norm kernel's phase boundaries.
__device__ uint64_t ohip_ktime_nodes[8 * 65536];
extern "C" int ohip_ktime_read_nodes(void* host) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(ohip_ktime_nodes), sizeof(ohip_ktime_nodes));
}
#define NSTAMP(i) do { if (threadIdx.x == 0 && blockIdx.x < 65536) \
    ohip_ktime_nodes[(i) * 65536 + blockIdx.x] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define NSTAMP(i) do {} while (0)
#endif

template <class T, int PPB>
__global__ void __launch_bounds__(kThreads * PPB) instnorm_partials_kernel(const float* __restrict__ ws, int splits,
                                                                           int64_t slice, int64_t Pp,
                                                                           const T* __restrict__ cbias,
                                                                           T* __restrict__ y, int spatial, int C,
                                                                           float eps, NormAffine aff, int out_nhwc) {
#pragma clang fp contract(off)
  static_assert(kThreads == 256, "256 threads a plane");
  extern __shared__ float xs_all[];        // PPB planes of `spatial` values
  __shared__ float red[2][4 * PPB];   // each plane's mean and 1 / sqrt(var + eps) (slot 4 g)
  __shared__ float2 segm[PPB][kNormGroup];   // each plane's segment moments
  NSTAMP(0);
  const int g = threadIdx.x >> 8, lt = threadIdx.x & 255;
  const int groups = C / PPB;
  const int64_t n = blockIdx.x / groups;
  const int c0 = (int)(blockIdx.x % groups) * PPB, c = c0 + g;
  const int64_t plane = n * C + c;
  float* xs = xs_all + g * spatial;
  const float* src = ws + (int64_t)c * Pp + n * spatial;
  const float b = cbias ? (float)cbias[c] : -0.0f;
  // Loads the epilogue needs are issued here, so their round trip overlaps
  // the partial-sum reads instead of following the statistics: the affine
  // terms and, for an NHWC output, this thread's first residual run.
  const int64_t ai = aff.per_sample ? n * aff.stride + c : c;
  float sc = 1.0f, bi = 0.0f;
  if (aff.scale)
    sc = aff.same_type ? (float)static_cast<const T*>(aff.scale)[ai] : static_cast<const float*>(aff.scale)[ai];
  if (aff.bias)
    bi = aff.same_type ? (float)static_cast<const T*>(aff.bias)[ai] : static_cast<const float*>(aff.bias)[ai];
  const T* res = static_cast<const T*>(aff.residual);
  constexpr int kRunBytes = PPB * (int)sizeof(T);
  using Run = typename std::conditional<kRunBytes % 16 == 0, uint4,
              typename std::conditional<kRunBytes % 8 == 0, uint2, uint32_t>::type>::type;
  constexpr int kRuns = kRunBytes / (int)sizeof(Run) > 0 ? kRunBytes / (int)sizeof(Run) : 1;
  Run r0[kRuns];
  const bool pre = PPB > 1 && res && aff.res_nhwc && (int)threadIdx.x < spatial;
  if constexpr (PPB > 1) {
    if (pre) {
      const Run* rp = reinterpret_cast<const Run*>(res + (n * spatial + threadIdx.x) * C + c0);
#pragma unroll
      for (int k = 0; k < kRuns; ++k) r0[k] = rp[k];
    }
  }
  if ((spatial & 3) == 0 && ((uintptr_t)src & 15) == 0 && (slice & 3) == 0) {
    // four pixels a thread, 16-byte loads, up to four slices in flight; the
    // adds stay in slice order
    typedef float f4 __attribute__((ext_vector_type(4)));
    for (int i = 4 * lt; i < spatial; i += 4 * kThreads) {
      // every slice of a group of four loaded before the first add (one
      // round trip per group, not per slice); slice 0 starts the sum
      f4 acc;
      for (int s0 = 0; s0 < splits; s0 += 4) {
        f4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (s0 + u < splits) v[u] = *reinterpret_cast<const f4*>(src + (s0 + u) * slice + i);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (s0 + u < splits) acc = s0 + u == 0 ? v[u] : acc + v[u];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = acc[e];
        xs[i + e] = (float)(T)(a + b);
      }
    }
  } else {
    for (int i = lt; i < spatial; i += kThreads) {
      float acc = src[i];
      for (int s = 1; s < splits; ++s) acc += src[s * slice + i];
      xs[i] = (float)(T)(acc + b);
    }
  }
  __syncthreads();
  NSTAMP(1);
  // the plane's statistics (norm_stats.hpp): each thread a run's moments,
  // sixteen lanes a segment's, the plane's first wave the segments' tree
  static_assert(kThreads == kNormGroup, "a group's threads");
  const int S = norm_segments(spatial);   // <= 256 (kNormPartialsMaxSpatial): one group
  group_segments([&](int64_t i) { return xs[i]; }, spatial, 0, S, segm[g], lt);
  __syncthreads();
  if (lt < 64) {   // the plane's first wave merges its segments
    float2 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = 4 * lt + j < S ? segm[g][4 * lt + j] : float2{0.0f, 0.0f};
    const Moments pm = wave_tree(v, S, spatial - (S - 1) * kNormSeg, lt);
    if (lt == 0) {
      red[0][4 * g] = pm.m;
      red[1][4 * g] = 1.0f / sqrtf(pm.m2 / (float)spatial + eps);
    }
  }
  __syncthreads();
  const float mean = red[0][4 * g], inv = red[1][4 * g];
  NSTAMP(2);
  NSTAMP(3);
  const bool affine = aff.scale || aff.bias;
  T* yp = y + plane * spatial;
  for (int i = lt; i < spatial; i += kThreads) {
    float v = (xs[i] - mean) * inv;
    if (affine) {
      v = round_to<T>(v);
      if (aff.scale) v = round_to<T>(v * sc);
      if (aff.bias) v = round_to<T>(v + bi);
    }
    if (aff.act == UN_RELU) v = v > 0.0f ? v : 0.0f;
    else if (aff.act == UN_LEAKY_RELU) v = round_to<T>(v), v = v >= 0.0f ? v : v * aff.alpha;
    if constexpr (PPB == 1) {
      if (res) v = round_to<T>(v) + (float)(aff.res_nhwc ? res[(n * spatial + i) * C + c] : res[plane * spatial + i]);
      v = opaque(v);
      if (out_nhwc) y[(n * spatial + i) * C + c] = (T)v;   // channel c of each pixel (C per pixel)
      else yp[i] = (T)v;
    } else {
      xs[i] = round_to<T>(v);   // the stored value; the residual is added below, per run
    }
  }
  NSTAMP(4);
  if constexpr (PPB > 1) {
    __syncthreads();
    // each pixel's PPB channels as one run (NHWC output, C per pixel)
    for (int i = threadIdx.x; i < spatial; i += kThreads * PPB) {
      const int64_t pix = n * spatial + i;
      T r[PPB];
      if (res) {
        if (aff.res_nhwc) {
          const Run* rp = reinterpret_cast<const Run*>(res + pix * C + c0);
          Run w[kRuns];
          if (i == (int)threadIdx.x) {   // the run loaded up front
#pragma unroll
            for (int k = 0; k < kRuns; ++k) w[k] = r0[k];
          } else {
#pragma unroll
            for (int k = 0; k < kRuns; ++k) w[k] = rp[k];
          }
          __builtin_memcpy(r, w, sizeof(w));
        } else {
#pragma unroll
          for (int k = 0; k < PPB; ++k) r[k] = res[(n * C + c0 + k) * (int64_t)spatial + i];
        }
      }
      T o[PPB];
#pragma unroll
      for (int k = 0; k < PPB; ++k) {
        float v = xs_all[k * spatial + i];
        if (res) v = v + (float)r[k];
        o[k] = (T)opaque(v);
      }
      Run* dp = reinterpret_cast<Run*>(y + pix * C + c0);
#pragma unroll
      for (int k = 0; k < kRuns; ++k) {
        Run w;
        __builtin_memcpy(&w, reinterpret_cast<const char*>(o) + sizeof(Run) * k, sizeof(Run));
        dp[k] = w;
      }
    }
  }
  NSTAMP(5);
}

// ---------------------------------------------------------------- nearest resize (rank 4, H and W)
// Source index of output position j on one axis: transform_coord plus the
// nearest rule and the clamp of the reference's build_axis
// (oxionnx-ops/src/resize.rs:578-620, 712-722), evaluated in f32.
__device__ __forceinline__ int nearest_src(int j, int in_len, int out_len, float scale, int coord, int rule) {
  const float x = (float)j;
  float src;
  switch (coord) {
    case RZ_ASYMMETRIC: src = x / scale; break;
    case RZ_ALIGN_CORNERS: src = out_len <= 1 ? 0.0f : x * ((float)in_len - 1.0f) / ((float)out_len - 1.0f); break;
    case RZ_PYTORCH_HALF_PIXEL: src = out_len > 1 ? (x + 0.5f) / scale - 0.5f : 0.0f; break;
    case RZ_TF_HALF_PIXEL_FOR_NN: src = (x + 0.5f) / scale; break;
    default: src = (x + 0.5f) / scale - 0.5f; break;
  }
  const float guard = 6.0f;  // 2 * taps + 4 with one tap
  const float hi = (float)(in_len - 1);
  src = src < -guard ? -guard : (src > hi + guard ? hi + guard : src);
  float picked;
  switch (rule) {
    case RZ_ROUND_PREFER_CEIL: picked = floorf(src + 0.5f); break;
    case RZ_FLOOR: picked = floorf(src); break;
    case RZ_CEIL: picked = ceilf(src); break;
    default: picked = ceilf(src - 0.5f); break;
  }
  int64_t k = (int64_t)picked;
  k = k < 0 ? 0 : (k > in_len - 1 ? in_len - 1 : k);
  return (int)k;
}

template <class T>
__global__ void __launch_bounds__(kThreads) resize_nearest_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                  int64_t planes, ResizePlan p) {
  const int64_t n = planes * p.oh * p.ow;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int ox = (int)(i % p.ow);
    const int64_t t = i / p.ow;
    const int oy = (int)(t % p.oh);
    const int64_t pl = t / p.oh;
    const int iy = nearest_src(oy, p.ih, p.oh, p.sh, p.coord, p.rule);
    const int ix = nearest_src(ox, p.iw, p.ow, p.sw, p.coord, p.rule);
    y[i] = x[(pl * p.ih + iy) * p.iw + ix];
  }
}

// Row form: the source row is found once per output row and the source
// column of every output column once per block (an LDS table).  A thread
// writes one 16-byte run of a row (or one element when the row is not whole
// runs); the runs of one row share the block with the next rows.  32-bit
// row indices (the launcher checks the count).
constexpr int kResizeMaxCols = 4096;
template <class T>
__global__ void __launch_bounds__(kThreads) resize_nearest_rows_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                       int rows, ResizePlan p) {
  constexpr int V = 16 / (int)sizeof(T);
  __shared__ int ixmap[kResizeMaxCols];
  for (int ox = threadIdx.x; ox < p.ow; ox += kThreads) ixmap[ox] = nearest_src(ox, p.iw, p.ow, p.sw, p.coord, p.rule);
  __syncthreads();
  const bool vec = p.ow % V == 0;
  const int units = vec ? p.ow / V : p.ow;          // per row
  const int span = units < kThreads ? units : kThreads;
  const int rpi = kThreads / span;                  // rows per block iteration
  const int lr = threadIdx.x / span, u0 = threadIdx.x - lr * span;
  if (lr >= rpi) return;
  for (int r = blockIdx.x * rpi + lr; r < rows; r += gridDim.x * rpi) {
    const int oy = r % p.oh, pl = r / p.oh;
    const int iy = nearest_src(oy, p.ih, p.oh, p.sh, p.coord, p.rule);
    const T* xr = x + ((int64_t)pl * p.ih + iy) * p.iw;
    T* yr = y + (int64_t)r * p.ow;
    if (vec) {
      for (int u = u0; u < units; u += span) {
        T e[V];
#pragma unroll
        for (int k = 0; k < V; ++k) e[k] = xr[ixmap[u * V + k]];
        uint4 w;
        __builtin_memcpy(&w, e, 16);
        *reinterpret_cast<uint4*>(yr + u * V) = w;
      }
    } else {
      for (int ox = u0; ox < p.ow; ox += span) yr[ox] = xr[ixmap[ox]];
    }
  }
}

// ---------------------------------------------------------------- pad (rank <= 6)
__device__ __forceinline__ int64_t pad_src(int64_t o, int64_t begin, int64_t len, int mode, bool* inside) {
  int64_t s = o - begin;
  if (s >= 0 && s < len) return s;
  if (mode == PAD_CONSTANT) { *inside = false; return 0; }
  if (mode == PAD_EDGE) return s < 0 ? 0 : len - 1;
  if (mode == PAD_WRAP) { s %= len; return s < 0 ? s + len : s; }
  // reflect (len >= 2 is checked on the host, len == 1 maps everything to 0)
  if (len == 1) return 0;
  const int64_t period = 2 * (len - 1);
  s %= period;
  if (s < 0) s += period;
  return s < len ? s : period - s;
}

template <class T>
__global__ void __launch_bounds__(kThreads) pad_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n, PadPlan p) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    int64_t r = i, src = 0, mul = 1;
    bool inside = true;
    for (int d = p.rank - 1; d >= 0; --d) {
      const int64_t o = r % p.out[d];
      r /= p.out[d];
      src += pad_src(o, p.begin[d], p.in[d], p.mode, &inside) * mul;
      mul *= p.in[d];
    }
    y[i] = inside ? x[src] : (T)p.value_bits;
  }
}

// ---------------------------------------------------------------- max pool (2-D)
template <class T>
__global__ void __launch_bounds__(kThreads) maxpool_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t planes,
                                                           PoolPlan p) {
  const int64_t n = planes * p.oh * p.ow;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int ox = (int)(i % p.ow);
    const int64_t t = i / p.ow;
    const int oy = (int)(t % p.oh);
    const int64_t pl = t / p.oh;
    const T* xp = x + pl * p.ih * p.iw;
    // max_pool_into (conv/pooling.rs:166-240): strictly-greater update from
    // -inf, so a NaN sample never wins
    float best = -INFINITY;
    for (int ky = 0; ky < p.kh; ++ky) {
      const int iy = oy * p.sh - p.pt + ky * p.dh;
      if (iy < 0 || iy >= p.ih) continue;
      for (int kx = 0; kx < p.kw; ++kx) {
        const int ix = ox * p.sw - p.pl + kx * p.dw;
        if (ix < 0 || ix >= p.iw) continue;
        const float v = (float)xp[iy * p.iw + ix];
        if (v > best) best = v;
      }
    }
    y[i] = (T)best;
  }
}

// The same pool over an NHWC input with a pixel pitch: output element
// (n, oy, ox, c), compact NHWC, with the NCHW kernel's comparisons.
template <class T>
__global__ void __launch_bounds__(kThreads) maxpool_nhwc_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                int64_t images, PoolPlan p) {
  const int C = p.nhwc_c;
  const int64_t n = images * p.oh * p.ow * C;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int c = (int)(i % C);
    int64_t t = i / C;
    const int ox = (int)(t % p.ow);
    t /= p.ow;
    const int oy = (int)(t % p.oh);
    const int64_t img = t / p.oh;
    const T* xp = x + img * p.ih * p.iw * p.pitch + c;
    float best = -INFINITY;
    for (int ky = 0; ky < p.kh; ++ky) {
      const int iy = oy * p.sh - p.pt + ky * p.dh;
      if (iy < 0 || iy >= p.ih) continue;
      for (int kx = 0; kx < p.kw; ++kx) {
        const int ix = ox * p.sw - p.pl + kx * p.dw;
        if (ix < 0 || ix >= p.iw) continue;
        const float v = (float)xp[((int64_t)iy * p.iw + ix) * p.pitch];
        if (v > best) best = v;
      }
    }
    y[i] = (T)best;
  }
}

// Byte pools over an NHWC input whose channels come in 4-byte groups (C, the
// pitch and both pointers multiples of 4): a thread takes four channels of
// one output pixel, one 32-bit load per tap, and keeps a byte maximum per
// lane (the float kernel's comparison on the same integers).  With the
// window size a template argument (K x K, dilation 1) every tap's load is
// issued before the maxima, from a clamped address, and a tap outside the
// image is masked; K = 0 walks a general window.
template <bool SIGNED, int K>
__global__ void __launch_bounds__(kThreads) maxpool_nhwc_b4_kernel(const uint32_t* __restrict__ x,
                                                                   uint32_t* __restrict__ y, int64_t images,
                                                                   PoolPlan p) {
  const int G = p.nhwc_c / 4;
  const int64_t pitch = p.pitch / 4;
  const int64_t n = images * p.oh * p.ow * G;
  auto merge = [](int (&best)[4], uint32_t w) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int v = SIGNED ? (int)(int8_t)(w >> (8 * b)) : (int)((w >> (8 * b)) & 0xff);
      best[b] = v > best[b] ? v : best[b];
    }
  };
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int g = (int)(i % G);
    int64_t t = i / G;
    const int ox = (int)(t % p.ow);
    t /= p.ow;
    const int oy = (int)(t % p.oh);
    const int64_t img = t / p.oh;
    const uint32_t* xp = x + img * p.ih * p.iw * pitch + g;
    int best[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) best[b] = SIGNED ? -128 : 0;
    const int iy0 = oy * p.sh - p.pt, ix0 = ox * p.sw - p.pl;
    if constexpr (K > 0) {
      uint32_t w[K][K];
#pragma unroll
      for (int ky = 0; ky < K; ++ky) {
        const int iy = min(max(iy0 + ky, 0), p.ih - 1);
#pragma unroll
        for (int kx = 0; kx < K; ++kx) {
          const int ix = min(max(ix0 + kx, 0), p.iw - 1);
          w[ky][kx] = xp[((int64_t)iy * p.iw + ix) * pitch];
        }
      }
#pragma unroll
      for (int ky = 0; ky < K; ++ky)
#pragma unroll
        for (int kx = 0; kx < K; ++kx)
          if ((unsigned)(iy0 + ky) < (unsigned)p.ih && (unsigned)(ix0 + kx) < (unsigned)p.iw) merge(best, w[ky][kx]);
    } else {
      for (int ky = 0; ky < p.kh; ++ky) {
        const int iy = iy0 + ky * p.dh;
        if (iy < 0 || iy >= p.ih) continue;
        for (int kx = 0; kx < p.kw; ++kx) {
          const int ix = ix0 + kx * p.dw;
          if (ix < 0 || ix >= p.iw) continue;
          merge(best, xp[((int64_t)iy * p.iw + ix) * pitch]);
        }
      }
    }
    y[i] = (best[0] & 0xff) | ((best[1] & 0xff) << 8) | ((best[2] & 0xff) << 16) | ((uint32_t)(best[3] & 0xff) << 24);
  }
}

// ---------------------------------------------------------------- strided slice (rank <= 6)
template <class T>
__global__ void __launch_bounds__(kThreads) slice_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n, SlicePlan p) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    int64_t r = i, src = 0;
    for (int d = p.rank - 1; d >= 0; --d) {
      const int64_t o = r % p.out[d];
      r /= p.out[d];
      src += (p.start[d] + o * p.step[d]) * p.in_stride[d];
    }
    y[i] = x[src];
  }
}

// ---------------------------------------------------------------- quantise / dequantise / byte table
// QuantizeLinear (indexing/quantize.rs:96-150): round_ties_even(x / scale) + zp,
// clamped into [lo, hi]; the division is IEEE (correctly rounded), as on the host.
__global__ void __launch_bounds__(kThreads) quantize_kernel(const float* __restrict__ x, uint8_t* __restrict__ y, int64_t n,
                                                            float scale, float zp, float lo, float hi) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const float v = x[i] / scale;
    float r = __builtin_rintf(v);  // ties to even, the reference's round_ties_even
    if (!__builtin_isfinite(v)) r = v;
    float q = r + zp;
    q = q < lo ? lo : (q > hi ? hi : q);
    y[i] = (uint8_t)((int32_t)q & 0xff);
  }
}

// DequantizeLinear (indexing/quantize.rs:152-190): (x - zp) * scale in f32.
template <bool SIGNED>
__global__ void __launch_bounds__(kThreads) dequantize_kernel(const uint8_t* __restrict__ x, float* __restrict__ y,
                                                              int64_t n, float scale, float zp) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const float v = SIGNED ? (float)(int8_t)x[i] : (float)x[i];
    y[i] = (v - zp) * scale;
  }
}

// The dequantised residual sum in one pass: DequantizeLinear of both byte
// operands, their f32 Add and QuantizeLinear of the sum, each step the
// arithmetic of its own kernel above (no contraction across the steps).
__device__ __forceinline__ uint32_t qadd_one(uint32_t ra, uint32_t rb, const QAddArgs& q) {
#pragma clang fp contract(off)
  const float va = q.a_signed ? (float)(int8_t)ra : (float)(ra & 0xff);
  const float vb = q.b_signed ? (float)(int8_t)rb : (float)(rb & 0xff);
  const float da = (va - q.za) * q.sa;
  const float db = (vb - q.zb) * q.sb;
  const float sum = da + db;
  const float v = sum / q.sc;
  float r = __builtin_rintf(v);
  if (!__builtin_isfinite(v)) r = v;
  float o = r + q.zc;
  o = o < q.lo ? q.lo : (o > q.hi ? q.hi : o);
  return (uint32_t)((int32_t)o & 0xff);
}

// Two NHWC operands of one shape with their own pixel pitches (a resident
// channel slice is one), four channels a thread: 32-bit loads of both, the
// bytes through qadd_one, one 32-bit store into the compact output.
__global__ void __launch_bounds__(kThreads) qadd_pitched_b4_kernel(const uint32_t* __restrict__ a,
                                                                   const uint32_t* __restrict__ b,
                                                                   uint32_t* __restrict__ y, int64_t groups, int cg,
                                                                   int64_t pa, int64_t pb, QAddArgs q) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < groups; i += (int64_t)gridDim.x * kThreads) {
    const int64_t px = i / cg;
    const int c = (int)(i - px * cg);
    const uint32_t wa = a[px * pa + c], wb = b[px * pb + c];
    uint32_t o = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) o |= qadd_one(wa >> (8 * k), wb >> (8 * k), q) << (8 * k);
    y[i] = o;
  }
}

template <bool SAME>
__global__ void __launch_bounds__(kThreads) qadd_kernel(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b,
                                                        uint8_t* __restrict__ y, int64_t n, BcastPlan p, QAddArgs q) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    int64_t ia = i, ib = i;
    if (!SAME) {
      ia = ib = 0;
      int64_t r = i;
#pragma unroll
      for (int d = kMaxRank - 1; d >= 0; --d) {
        if (d < kMaxRank - p.rank) break;
        const int64_t e = p.shape[d];
        const int64_t c = r % e;
        r /= e;
        ia += c * p.sa[d];
        ib += c * p.sb[d];
      }
    }
    y[i] = (uint8_t)qadd_one(a[ia], b[ib], q);
  }
}

// ---------------------------------------------------------------- 2-D copy (Concat)
template <class T>
__global__ void __launch_bounds__(kThreads) copy2d_kernel(const T* __restrict__ src, int64_t sp, T* __restrict__ dst,
                                                          int64_t dp, int64_t width, int64_t rows) {
  const int64_t n = width * rows;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / width, c = i - r * width;
    dst[r * dp + c] = src[r * sp + c];
  }
}

// Concat of up to kConcatMax inputs in one launch: output row r is the
// inputs' rows r laid end to end; unit c of a row belongs to the input whose
// [off, off + w) range holds it.
template <class T>
__global__ void __launch_bounds__(kThreads) concat_rows_kernel(ConcatPlan p, int64_t row, int64_t rows) {
  const int64_t n = row * rows;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int64_t r = i / row, c = i - r * row;
    int k = 0;
#pragma unroll
    for (int j = 1; j < kConcatMax; ++j) k += (j < p.n && c >= p.off[j]) ? 1 : 0;
    reinterpret_cast<T*>(p.dst)[i] = reinterpret_cast<const T*>(p.src[k])[r * p.sp[k] + (c - p.off[k])];
  }
}

struct Table256 { uint8_t v[256]; };

__global__ void __launch_bounds__(kThreads) byte_table_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ y,
                                                              int64_t n, Table256 t) {
  __shared__ uint8_t tab[256];
  tab[threadIdx.x] = t.v[threadIdx.x];
  __syncthreads();
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
    y[i] = tab[x[i]];
}

}  // namespace

// ---------------------------------------------------------------- launchers
hipError_t run_unary(int dt, const void* x, void* y, int64_t n, int op, float alpha, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  if (dt == DT_F32)
    hipLaunchKernelGGL(unary_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const float*)x, (float*)y, n,
                       op, alpha);
  else if (dt == DT_F16)
    hipLaunchKernelGGL(unary_kernel<_Float16>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const _Float16*)x,
                       (_Float16*)y, n, op, alpha);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t run_binary(int dt, const void* a, const void* b, void* y, int64_t n, const BcastPlan& p, bool same, int op,
                      hipStream_t st) {
  if (n <= 0) return hipSuccess;
  if (dt == DT_F32) {
    if (same)
      hipLaunchKernelGGL(binary_same_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const float*)a,
                         (const float*)b, (float*)y, n, op);
    else
      hipLaunchKernelGGL(binary_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const float*)a,
                         (const float*)b, (float*)y, n, p, op);
  } else if (dt == DT_F16) {
    if (same)
      hipLaunchKernelGGL(binary_same_kernel<_Float16>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const _Float16*)a,
                         (const _Float16*)b, (_Float16*)y, n, op);
    else
      hipLaunchKernelGGL(binary_kernel<_Float16>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const _Float16*)a,
                         (const _Float16*)b, (_Float16*)y, n, p, op);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t run_instnorm(int dt, const void* x, void* y, int64_t planes, int64_t spatial, int C, float eps,
                        const NormAffine& aff, hipStream_t st) {
  if (planes <= 0 || spatial <= 0) return hipSuccess;
  if (planes > 0x7fffffff) return hipErrorInvalidValue;
  const size_t shm = spatial <= kNormPlaneLds ? (size_t)spatial * sizeof(float) : 0;
  if (dt == DT_F32)
    hipLaunchKernelGGL(instnorm_kernel<float>, dim3((unsigned)planes), dim3(kThreads), shm, st, (const float*)x,
                       (float*)y, spatial, C, eps, aff);
  else if (dt == DT_F16)
    hipLaunchKernelGGL(instnorm_kernel<_Float16>, dim3((unsigned)planes), dim3(kThreads), shm, st,
                       (const _Float16*)x, (_Float16*)y, spatial, C, eps, aff);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// Instance normalisation of f16 / f32 conv outputs whose statistics arrive
// as the moments of their 64-pixel segments (wk_conv_kernel with mom): a
// block takes 32 channels x 64 pixels of one image, merges each channel's
// segments as the plain kernel does (norm_stats.hpp's tree), and
// normalises its tile with the affine tail, activation and residual of the
// unfused chain, reading the conv output as NCHW rows and writing runs of
// eight elements (eight channels of a pixel for an NHWC output, eight
// pixels of a channel for NCHW).
template <class T>
__global__ void __launch_bounds__(256) instnorm_mom_kernel(const T* __restrict__ x, const float* __restrict__ mom,
                                                           T* __restrict__ y, int C, int spatial, float eps,
                                                           NormAffine aff, int out_nhwc) {
#pragma clang fp contract(off)
  typedef T h8 __attribute__((ext_vector_type(8)));   // eight elements: 16 bytes of f16, 32 of f32
  NSTAMP(0);
  __shared__ float st[2][32];
  __shared__ h8 tile[32][9];   // [channel][eight-pixel chunk] (one chunk of padding)
  __shared__ float afs[2][32];   // each channel's scale and bias
  const int S = spatial / kNormSeg;
  const int nct = (C + 31) / 32;
  const int pb = (int)(blockIdx.x % S), rest = (int)(blockIdx.x / S);
  const int c0 = (rest % nct) * 32, n = rest / nct, p0 = pb * kNormSeg;
  const int t = threadIdx.x;
  const int cw = C - c0 < 32 ? C - c0 : 32;
  // every global load of the block in flight before the first wait: this
  // thread's eight pixels (or, NHWC, eight channels) of the conv output and
  // of the residual, and its share of the first chunk of segment moments
  const T* res = static_cast<const T*>(aff.residual);
  h8 xv{}, r{};
  int64_t o;
  bool live;
  if (out_nhwc) {
    const int p = t >> 2, q = t & 3;
    live = 8 * q < cw;
    o = ((int64_t)n * spatial + p0 + p) * C + c0 + 8 * q;
  } else {
    const int cl = t >> 3, k = t & 7;
    live = cl < cw;
    o = ((int64_t)n * C + c0 + cl) * spatial + p0 + 8 * k;
  }
  {
    const int cl = t >> 3, k = t & 7;
    if (cl < cw) xv = *reinterpret_cast<const h8*>(x + ((int64_t)n * C + c0 + cl) * spatial + p0 + 8 * k);
  }
  if (res && live) r = *reinterpret_cast<const h8*>(res + o);
  if (t < cw) {
    const int64_t ai = aff.per_sample ? (int64_t)n * aff.stride + c0 + t : c0 + t;
    auto term = [&](const void* p) {
      return aff.same_type ? (float)static_cast<const T*>(p)[ai] : static_cast<const float*>(p)[ai];
    };
    afs[0][t] = aff.scale ? term(aff.scale) : 1.0f;
    afs[1][t] = aff.bias ? term(aff.bias) : 0.0f;
  }
  // each of the first cw threads merges its channel's segments in
  // registers (a whole plane of whole segments: S <= 64)
  if (t < cw) {
    const float2* mp = reinterpret_cast<const float2*>(mom) + ((int64_t)n * C + c0 + t) * S;
    auto plane = [&](auto nc) __attribute__((always_inline)) {
      constexpr int N = decltype(nc)::value;
      Moments r[N];
#pragma unroll
      for (int k = 0; k < N; ++k) {
        const float2 v = k < S ? mp[k] : float2{0.0f, 0.0f};
        r[k] = Moments{(float)kNormSeg, v.x, v.y};
      }
      tree_regs<N>(r, S);
      st[0][t] = r[0].m;
      st[1][t] = 1.0f / sqrtf(r[0].m2 / (float)spatial + eps);
    };
    if (S <= 16) plane(std::integral_constant<int, 16>{});
    else plane(std::integral_constant<int, 64>{});
  }
  tile[t >> 3][t & 7] = xv;
  __syncthreads();
  NSTAMP(1);
  if (!live) return;
  const bool affine = aff.scale || aff.bias;
  auto finish = [&](float v0, int cl, float r1) {
    const float sc = afs[0][cl], bi = afs[1][cl];
    float v = (v0 - st[0][cl]) * st[1][cl];
    if (affine) {
      v = round_to<T>(v);
      if (aff.scale) v = round_to<T>(v * sc);
      if (aff.bias) v = round_to<T>(v + bi);
    }
    if (aff.act == UN_RELU) v = v > 0.0f ? v : 0.0f;
    else if (aff.act == UN_LEAKY_RELU) v = round_to<T>(v), v = v >= 0.0f ? v : v * aff.alpha;
    if (res) v = round_to<T>(v) + r1;
    return (T)opaque(v);
  };
  h8 out;
  if (out_nhwc) {
    const int p = t >> 2, q = t & 3;
#pragma unroll
    for (int c = 0; c < 8; ++c) out[c] = finish((float)tile[8 * q + c][p >> 3][p & 7], 8 * q + c, (float)r[c]);
  } else {
    const int cl = t >> 3;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = finish((float)xv[e], cl, (float)r[e]);
  }
  *reinterpret_cast<h8*>(y + o) = out;
  NSTAMP(2);
}

hipError_t run_instnorm_mom(int dt, const void* x, const float* mom, void* y, int64_t N, int C, int64_t spatial,
                            float eps, const NormAffine& aff, bool out_nhwc, hipStream_t st) {
  if (N <= 0 || spatial <= 0) return hipSuccess;
  const uintptr_t run = dt == DT_F32 ? 32 : 16;   // eight elements
  if (spatial % kNormSeg != 0 || spatial > kNormMomMaxSpatial || (out_nhwc && C % 8 != 0) ||
      (aff.residual && aff.res_nhwc != (int)out_nhwc) || (uintptr_t)x % run || (uintptr_t)y % run ||
      (uintptr_t)aff.residual % run)
    return hipErrorInvalidValue;
  const int64_t blocks = N * ((C + 31) / 32) * (spatial / kNormSeg);
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  if (dt == DT_F16)
    hipLaunchKernelGGL(instnorm_mom_kernel<_Float16>, dim3((unsigned)blocks), dim3(256), 0, st, (const _Float16*)x,
                       mom, (_Float16*)y, C, (int)spatial, eps, aff, (int)out_nhwc);
  else if (dt == DT_F32)
    hipLaunchKernelGGL(instnorm_mom_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)x, mom,
                       (float*)y, C, (int)spatial, eps, aff, (int)out_nhwc);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t run_instnorm_partials(int dt, const float* ws, int splits, int64_t Pp, const void* conv_bias, void* y,
                                 int64_t N, int64_t spatial, int C, float eps, const NormAffine& aff, bool out_nhwc,
                                 hipStream_t st) {
  const int64_t planes = N * C;
  if (planes <= 0 || spatial <= 0) return hipSuccess;
  if (planes > 0x7fffffff || spatial > kNormPartialsMaxSpatial || splits < 1) return hipErrorInvalidValue;
  const int64_t slice = (int64_t)C * Pp;
  // an NHWC output takes PPB channels a block (runs of PPB elements per
  // pixel); OHIP_NORM_PPB (2 or 4) overrides the default of 4 (a
  // measurement switch)
  static const int ppb_env = [] { const char* e = std::getenv("OHIP_NORM_PPB"); return e ? std::atoi(e) : 4; }();
  const int eb = dt == DT_F32 ? 4 : 2;
  auto wide_ok = [&](int ppb) {
    return out_nhwc && C % ppb == 0 && (size_t)ppb * spatial * sizeof(float) <= 64 * 1024 &&
           (uintptr_t)y % (ppb * eb) == 0 &&
           (!aff.residual || !aff.res_nhwc || (uintptr_t)aff.residual % (ppb * eb) == 0);
  };
  auto launch_wide = [&](auto ppb_c) {
    constexpr int PPB = decltype(ppb_c)::value;
    const size_t shm = (size_t)PPB * spatial * sizeof(float);
    const unsigned blocks = (unsigned)(planes / PPB);
    if (dt == DT_F32)
      hipLaunchKernelGGL((instnorm_partials_kernel<float, PPB>), dim3(blocks), dim3(kThreads * PPB), shm, st, ws,
                         splits, slice, Pp, (const float*)conv_bias, (float*)y, (int)spatial, C, eps, aff, 1);
    else if (dt == DT_F16)
      hipLaunchKernelGGL((instnorm_partials_kernel<_Float16, PPB>), dim3(blocks), dim3(kThreads * PPB), shm, st, ws,
                         splits, slice, Pp, (const _Float16*)conv_bias, (_Float16*)y, (int)spatial, C, eps, aff, 1);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  };
  if (ppb_env == 2 && wide_ok(2)) return launch_wide(std::integral_constant<int, 2>{});
  if (ppb_env != 1 && wide_ok(4)) return launch_wide(std::integral_constant<int, 4>{});
  const size_t shm = (size_t)spatial * sizeof(float);
  if (dt == DT_F32)
    hipLaunchKernelGGL((instnorm_partials_kernel<float, 1>), dim3((unsigned)planes), dim3(kThreads), shm, st, ws,
                       splits, slice, Pp, (const float*)conv_bias, (float*)y, (int)spatial, C, eps, aff,
                       (int)out_nhwc);
  else if (dt == DT_F16)
    hipLaunchKernelGGL((instnorm_partials_kernel<_Float16, 1>), dim3((unsigned)planes), dim3(kThreads), shm, st, ws,
                       splits, slice, Pp, (const _Float16*)conv_bias, (_Float16*)y, (int)spatial, C, eps, aff,
                       (int)out_nhwc);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

#define OHIP_BY_ELEM_SIZE(eb, KERNEL, grid, ...)                                                                  \
  do {                                                                                                             \
    switch (eb) {                                                                                                  \
      case 1: hipLaunchKernelGGL(KERNEL<uint8_t>, grid, dim3(kThreads), 0, st, (const uint8_t*)x, (uint8_t*)y, __VA_ARGS__); break;     \
      case 2: hipLaunchKernelGGL(KERNEL<uint16_t>, grid, dim3(kThreads), 0, st, (const uint16_t*)x, (uint16_t*)y, __VA_ARGS__); break;  \
      case 4: hipLaunchKernelGGL(KERNEL<uint32_t>, grid, dim3(kThreads), 0, st, (const uint32_t*)x, (uint32_t*)y, __VA_ARGS__); break;  \
      default: return hipErrorInvalidValue;                                                                        \
    }                                                                                                              \
    return hipGetLastError();                                                                                      \
  } while (0)

// Nearest resize of an NHWC tensor (C elements a pixel, whole 16-byte
// pixels): every 16-byte chunk of an output pixel is the same chunk of its
// source pixel, the source row and column from the NCHW kernel's rule.
__global__ void __launch_bounds__(kThreads) resize_nearest_nhwc_kernel(const uint4* __restrict__ x,
                                                                       uint4* __restrict__ y, int64_t n, int cpp,
                                                                       ResizePlan p) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) {
    const int c = (int)(i % cpp);
    int64_t t = i / cpp;
    const int ox = (int)(t % p.ow);
    t /= p.ow;
    const int oy = (int)(t % p.oh);
    const int64_t img = t / p.oh;
    const int iy = nearest_src(oy, p.ih, p.oh, p.sh, p.coord, p.rule);
    const int ix = nearest_src(ox, p.iw, p.ow, p.sw, p.coord, p.rule);
    y[i] = x[((img * p.ih + iy) * p.iw + ix) * cpp + c];
  }
}

hipError_t run_resize_nearest_nhwc(int elem_bytes, const void* x, void* y, int64_t images, int64_t C,
                                   const ResizePlan& p, hipStream_t st) {
  if ((C * elem_bytes) % 16 != 0 || (uintptr_t)x % 16 != 0 || (uintptr_t)y % 16 != 0) return hipErrorInvalidValue;
  const int cpp = (int)(C * elem_bytes / 16);
  const int64_t n = images * p.oh * p.ow * cpp;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(resize_nearest_nhwc_kernel, dim3(grid_for(n)), dim3(kThreads), 0, st,
                     static_cast<const uint4*>(x), static_cast<uint4*>(y), n, cpp, p);
  return hipGetLastError();
}

hipError_t run_resize_nearest(int elem_bytes, const void* x, void* y, int64_t planes, const ResizePlan& p,
                              hipStream_t st) {
  const int64_t n = planes * p.oh * p.ow;
  if (n <= 0) return hipSuccess;
  const int64_t rows = planes * p.oh;
  if (p.ow <= kResizeMaxCols && rows < (int64_t)1 << 30 && (uintptr_t)y % 16 == 0) {
    const int v = 16 / elem_bytes;
    const int units = p.ow % v == 0 ? p.ow / v : p.ow;
    const int rpi = kThreads / (units < kThreads ? units : kThreads);
    const int64_t blocks = std::min<int64_t>((rows + rpi - 1) / rpi, 65536);
    OHIP_BY_ELEM_SIZE(elem_bytes, resize_nearest_rows_kernel, dim3((unsigned)blocks), (int)rows, p);
  }
  OHIP_BY_ELEM_SIZE(elem_bytes, resize_nearest_kernel, dim3(grid_for(n)), planes, p);
}

hipError_t run_pad(int elem_bytes, const void* x, void* y, int64_t n, const PadPlan& p, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  // the fill value travels as the element's bit pattern
  OHIP_BY_ELEM_SIZE(elem_bytes, pad_kernel, dim3(grid_for(n)), n, p);
}

hipError_t run_slice(int elem_bytes, const void* x, void* y, int64_t n, const SlicePlan& p, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  OHIP_BY_ELEM_SIZE(elem_bytes, slice_kernel, dim3(grid_for(n)), n, p);
}

hipError_t run_maxpool(int dt, const void* x, void* y, int64_t planes, const PoolPlan& p, hipStream_t st) {
  const int64_t n = planes * p.oh * p.ow;
  if (n <= 0) return hipSuccess;
  const dim3 g(grid_for(n));
  if (p.nhwc_c > 0) {
    const int64_t images = planes / p.nhwc_c;
    if ((dt == DT_U8 || dt == DT_I8) && p.nhwc_c % 4 == 0 && p.pitch % 4 == 0 && (uintptr_t)x % 4 == 0 &&
        (uintptr_t)y % 4 == 0) {
      const int k = p.kh == p.kw && p.dh == 1 && p.dw == 1 && (p.kh == 3 || p.kh == 5) ? p.kh : 0;
      const dim3 g4(grid_for(n / 4));
      const uint32_t* xs = static_cast<const uint32_t*>(x);
      uint32_t* ys = static_cast<uint32_t*>(y);
#define OHIP_POOL_B4(S)                                                                                  \
  switch (k) {                                                                                           \
    case 3: hipLaunchKernelGGL((maxpool_nhwc_b4_kernel<S, 3>), g4, dim3(kThreads), 0, st, xs, ys, images, p); break; \
    case 5: hipLaunchKernelGGL((maxpool_nhwc_b4_kernel<S, 5>), g4, dim3(kThreads), 0, st, xs, ys, images, p); break; \
    default: hipLaunchKernelGGL((maxpool_nhwc_b4_kernel<S, 0>), g4, dim3(kThreads), 0, st, xs, ys, images, p); break; \
  }
      if (dt == DT_I8) { OHIP_POOL_B4(true) } else { OHIP_POOL_B4(false) }
#undef OHIP_POOL_B4
      return hipGetLastError();
    }
    switch (dt) {
      case DT_U8: hipLaunchKernelGGL(maxpool_nhwc_kernel<uint8_t>, g, dim3(kThreads), 0, st, (const uint8_t*)x, (uint8_t*)y, images, p); break;
      case DT_I8: hipLaunchKernelGGL(maxpool_nhwc_kernel<int8_t>, g, dim3(kThreads), 0, st, (const int8_t*)x, (int8_t*)y, images, p); break;
      case DT_F16: hipLaunchKernelGGL(maxpool_nhwc_kernel<_Float16>, g, dim3(kThreads), 0, st, (const _Float16*)x, (_Float16*)y, images, p); break;
      case DT_F32: hipLaunchKernelGGL(maxpool_nhwc_kernel<float>, g, dim3(kThreads), 0, st, (const float*)x, (float*)y, images, p); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (dt) {
    case DT_F32: hipLaunchKernelGGL(maxpool_kernel<float>, g, dim3(kThreads), 0, st, (const float*)x, (float*)y, planes, p); break;
    case DT_F16: hipLaunchKernelGGL(maxpool_kernel<_Float16>, g, dim3(kThreads), 0, st, (const _Float16*)x, (_Float16*)y, planes, p); break;
    case DT_U8: hipLaunchKernelGGL(maxpool_kernel<uint8_t>, g, dim3(kThreads), 0, st, (const uint8_t*)x, (uint8_t*)y, planes, p); break;
    case DT_I8: hipLaunchKernelGGL(maxpool_kernel<int8_t>, g, dim3(kThreads), 0, st, (const int8_t*)x, (int8_t*)y, planes, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t run_quantize(const float* x, uint8_t* y, int64_t n, float scale, float zp, float lo, float hi,
                        hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(n)), dim3(kThreads), 0, st, x, y, n, scale, zp, lo, hi);
  return hipGetLastError();
}

hipError_t run_qadd(const uint8_t* a, const uint8_t* b, uint8_t* y, int64_t n, const BcastPlan& p, bool same,
                    const QAddArgs& q, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  // pixels x channels with each operand's pitch (or one contiguous run),
  // whole 4-byte channel groups: the vector kernel
  const int R = kMaxRank;
  const bool two_d = p.rank == 2 && p.sa[R - 1] == 1 && p.sb[R - 1] == 1;
  const int64_t C = two_d ? p.shape[R - 1] : n;
  const int64_t pa = two_d ? p.sa[R - 2] : n, pb = two_d ? p.sb[R - 2] : n;
  if ((two_d || same) && C % 4 == 0 && pa % 4 == 0 && pb % 4 == 0 && (uintptr_t)a % 4 == 0 &&
      (uintptr_t)b % 4 == 0 && (uintptr_t)y % 4 == 0 && C / 4 <= 0x7fffffff) {
    const int64_t groups = n / 4;
    hipLaunchKernelGGL(qadd_pitched_b4_kernel, dim3(grid_for(groups)), dim3(kThreads), 0, st,
                       reinterpret_cast<const uint32_t*>(a), reinterpret_cast<const uint32_t*>(b),
                       reinterpret_cast<uint32_t*>(y), groups, (int)(C / 4), pa / 4, pb / 4, q);
    return hipGetLastError();
  }
  if (same)
    hipLaunchKernelGGL(qadd_kernel<true>, dim3(grid_for(n)), dim3(kThreads), 0, st, a, b, y, n, p, q);
  else
    hipLaunchKernelGGL(qadd_kernel<false>, dim3(grid_for(n)), dim3(kThreads), 0, st, a, b, y, n, p, q);
  return hipGetLastError();
}

hipError_t run_dequantize(const uint8_t* x, bool is_signed, float* y, int64_t n, float scale, float zp,
                          hipStream_t st) {
  if (n <= 0) return hipSuccess;
  if (is_signed)
    hipLaunchKernelGGL(dequantize_kernel<true>, dim3(grid_for(n)), dim3(kThreads), 0, st, x, y, n, scale, zp);
  else
    hipLaunchKernelGGL(dequantize_kernel<false>, dim3(grid_for(n)), dim3(kThreads), 0, st, x, y, n, scale, zp);
  return hipGetLastError();
}

// Copies `rows` rows of `width` bytes (pitches in bytes), in 16-, 4- or
// 1-byte units as the alignment of every operand allows.
hipError_t run_copy2d(const void* src, int64_t src_pitch, void* dst, int64_t dst_pitch, int64_t width, int64_t rows,
                      hipStream_t st) {
  if (width <= 0 || rows <= 0) return hipSuccess;
  auto fits = [&](int u) {
    return (uintptr_t)src % u == 0 && (uintptr_t)dst % u == 0 && src_pitch % u == 0 && dst_pitch % u == 0 &&
           width % u == 0;
  };
  if (fits(16)) {
    const int64_t w = width / 16, n = w * rows;
    hipLaunchKernelGGL(copy2d_kernel<uint4>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const uint4*)src,
                       src_pitch / 16, (uint4*)dst, dst_pitch / 16, w, rows);
  } else if (fits(4)) {
    const int64_t w = width / 4, n = w * rows;
    hipLaunchKernelGGL(copy2d_kernel<uint32_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const uint32_t*)src,
                       src_pitch / 4, (uint32_t*)dst, dst_pitch / 4, w, rows);
  } else {
    const int64_t n = width * rows;
    hipLaunchKernelGGL(copy2d_kernel<uint8_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, (const uint8_t*)src,
                       src_pitch, (uint8_t*)dst, dst_pitch, width, rows);
  }
  return hipGetLastError();
}

// Zero fill (a kernel, not hipMemsetAsync, so it is safe inside a captured
// graph): 16-byte stores where the buffer allows, else bytes.
template <class T>
__global__ void __launch_bounds__(kThreads) zero_fill_kernel(T* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads) p[i] = T{};
}

hipError_t run_zero_fill(void* p, size_t bytes, hipStream_t st) {
  if (bytes == 0) return hipSuccess;
  if ((uintptr_t)p % 16 == 0 && bytes % 16 == 0) {
    const int64_t n = (int64_t)(bytes / 16);
    hipLaunchKernelGGL(zero_fill_kernel<uint4>, dim3(grid_for(n)), dim3(kThreads), 0, st, (uint4*)p, n);
  } else {
    hipLaunchKernelGGL(zero_fill_kernel<uint8_t>, dim3(grid_for((int64_t)bytes)), dim3(kThreads), 0, st,
                       (uint8_t*)p, (int64_t)bytes);
  }
  return hipGetLastError();
}

// widths and offsets in bytes on entry; converted to units of the widest
// element size that every pointer and width allows
hipError_t run_concat_rows(ConcatPlan p, int64_t row, int64_t rows, hipStream_t st) {
  if (row <= 0 || rows <= 0) return hipSuccess;
  if (p.n < 1 || p.n > kConcatMax) return hipErrorInvalidValue;
  auto fits = [&](int u) {
    if ((uintptr_t)p.dst % u || row % u) return false;
    for (int k = 0; k < p.n; ++k)
      if ((uintptr_t)p.src[k] % u || p.w[k] % u || p.sp[k] % u) return false;
    return true;
  };
  const int u = fits(16) ? 16 : fits(4) ? 4 : 1;
  for (int k = 0; k < p.n; ++k) { p.w[k] /= u; p.off[k] /= u; p.sp[k] /= u; }
  const int64_t ru = row / u, n = ru * rows;
  if (u == 16) hipLaunchKernelGGL(concat_rows_kernel<uint4>, dim3(grid_for(n)), dim3(kThreads), 0, st, p, ru, rows);
  else if (u == 4) hipLaunchKernelGGL(concat_rows_kernel<uint32_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, p, ru, rows);
  else hipLaunchKernelGGL(concat_rows_kernel<uint8_t>, dim3(grid_for(n)), dim3(kThreads), 0, st, p, ru, rows);
  return hipGetLastError();
}

hipError_t run_byte_table(const uint8_t* x, uint8_t* y, int64_t n, const uint8_t* table, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  Table256 t;
  for (int i = 0; i < 256; ++i) t.v[i] = table[i];
  hipLaunchKernelGGL(byte_table_kernel, dim3(grid_for(n)), dim3(kThreads), 0, st, x, y, n, t);
  return hipGetLastError();
}

}  // namespace ohip
