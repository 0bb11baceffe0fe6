// Device kernels and their launchers: MFMA GEMM / implicit-GEMM conv for
// f32, f16, bf16 and int8, the skinny-M GEMV path, and the layout kernels
// that feed them.  Host-side policy (what to launch) lives in ops.cpp.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "internal.hpp"
#include "mfma_core.hpp"

namespace ohip {

// ---------------------------------------------------------------- epilogues
template <class T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <class T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }

__device__ __forceinline__ float activate(float v, int act, float lo, float hi) {
  switch (act) {
    case ACT_RELU: return v > 0.0f ? v : 0.0f;  // f32::max(NaN, 0) == 0
    case ACT_CLIP: return v < lo ? lo : (v > hi ? hi : v);
    case ACT_LEAKY_RELU: return v >= 0.0f ? v : v * lo;
    default: return v;
  }
}

// Float output: v = acc; v *= alpha (when alpha != 1); v += beta * bias; act;
// round to OutT.  Output element (i, j) sits at
//   (i / ohw) * bstride + (i % ohw) * si + j * sj.
template <class OutT> struct FloatEpi {
  OutT* y;
  int64_t si, sj, bstride;
  int ohw, P, Q;
  int vec;            // si == 1 and every 4-run of i is contiguous and aligned
  int has_alpha;
  float alpha, beta;
  const OutT* bias;
  int bias_mode;      // BIAS_*
  int act;
  float lo, hi;

  __device__ __forceinline__ float bias_at(int i, int j) const {
    switch (bias_mode) {
      case BIAS_SCALAR: return to_f32(bias[0]);
      case BIAS_I: return to_f32(bias[i]);
      case BIAS_J: return to_f32(bias[j]);
      case BIAS_FULL_JI: return to_f32(bias[(int64_t)j * P + i]);
      default: return 0.0f;
    }
  }
  __device__ __forceinline__ float finish(float v, int i, int j) const {
    if (has_alpha) v = v * alpha;
    if (bias_mode != BIAS_NONE) v = v + beta * bias_at(i, j);
    return activate(v, act, lo, hi);
  }
  __device__ __forceinline__ int64_t index(int i, int j) const {
    const int n = i / ohw;
    return (int64_t)n * bstride + (int64_t)(i - n * ohw) * si + (int64_t)j * sj;
  }
  __device__ __forceinline__ void store(int i0, int j, f32x4 acc) const {
    if (j >= Q) return;
    if (vec && i0 + 3 < P) {
      OutT o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = from_f32<OutT>(finish(acc[r], i0 + r, j));
      OutT* dst = y + index(i0, j);
      if constexpr (sizeof(OutT) == 4) {
        *reinterpret_cast<f32x4*>(dst) = f32x4{__builtin_bit_cast(float, o[0]), __builtin_bit_cast(float, o[1]),
                                               __builtin_bit_cast(float, o[2]), __builtin_bit_cast(float, o[3])};
      } else {
        typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<u16x4*>(dst) =
            u16x4{__builtin_bit_cast(uint16_t, o[0]), __builtin_bit_cast(uint16_t, o[1]),
                  __builtin_bit_cast(uint16_t, o[2]), __builtin_bit_cast(uint16_t, o[3])};
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (i0 + r < P) y[index(i0 + r, j)] = from_f32<OutT>(finish(acc[r], i0 + r, j));
  }
};

// Integer output.  The MFMA sums A' * B'' where A' is the activation shifted
// into int8 (u8 ^ 0x80 == u8 - 128) and B'' = w - w_zp.  The true accumulator
// sum (a - a_zp)(w - w_zp) = sum A' B'' + ca * colsum(B'') with ca = shift -
// a_zp, plus the int32 bias.  Arithmetic is modulo 2^32, exact whenever the
// true value fits int32 (the host gate guarantees it).  Requantisation then
// follows SatRange::requantize: f64 product with the f32 combined scale, + zp,
// round half to even, clamp.
struct QuantEpi {
  void* y;
  int64_t si, sj, bstride;
  int ohw, P, Q;
  int vec;
  int w_on_i;               // weight channel index is i (else j)
  const int32_t* colsum;    // per weight channel
  const int8_t* flip;       // per weight channel: 1 = the packed channel holds -(w - w_zp)
  const int32_t* bias;      // per weight channel, may be null
  int32_t ca;               // per-tensor correction factor
  const int32_t* ca_rows;   // per activation row, may be null
  const float* comb;        // combined scale per channel (n_comb == 1 -> per tensor)
  int n_comb;
  int out_kind;             // QOUT_U8, QOUT_I8, QOUT_I32 (raw), QOUT_F32 (requantised, as f32)
  int32_t y_zp, lo, hi;

  __device__ __forceinline__ int64_t index(int i, int j) const {
    const int n = i / ohw;
    return (int64_t)n * bstride + (int64_t)(i - n * ohw) * si + (int64_t)j * sj;
  }
  __device__ __forceinline__ int32_t exact(int32_t acc, int i, int j) const {
    const int ch = w_on_i ? i : j;
    const int row = w_on_i ? j : i;
    const uint32_t c = (uint32_t)(ca_rows ? ca_rows[row] : ca);
    uint32_t v = (uint32_t)acc + c * (uint32_t)colsum[ch];
    if (flip && flip[ch]) v = 0u - v;
    if (bias) v += (uint32_t)bias[ch];
    return (int32_t)v;
  }
  __device__ __forceinline__ int32_t requant(int32_t v, int i, int j) const {
#pragma clang fp contract(off)
    const int ch = w_on_i ? i : j;
    const float cs = comb[n_comb > 1 ? ch : 0];
    double d = (double)v * (double)cs;
    d = d + (double)y_zp;
    d = __builtin_rint(d);
    d = d < (double)lo ? (double)lo : d;
    d = d > (double)hi ? (double)hi : d;
    return (int32_t)d;
  }
  __device__ __forceinline__ void store(int i0, int j, i32x4 acc) const {
    if (j >= Q) return;
    int32_t v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = exact(acc[r], i0 + r, j);
      if (out_kind != QOUT_I32) v[r] = requant(v[r], i0 + r, j);
    }
    if (out_kind == QOUT_F32) {
      // requantised lanes stored as f32, the reference Tensor's representation
      float* yy = reinterpret_cast<float*>(y);
      if (vec && i0 + 3 < P) {
        *reinterpret_cast<f32x4*>(yy + index(i0, j)) = f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (i0 + r < P) yy[index(i0 + r, j)] = (float)v[r];
      }
    } else if (out_kind == QOUT_I32) {
      int32_t* yy = reinterpret_cast<int32_t*>(y);
      if (vec && i0 + 3 < P) {
        *reinterpret_cast<i32x4*>(yy + index(i0, j)) = i32x4{v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (i0 + r < P) yy[index(i0 + r, j)] = v[r];
      }
    } else {
      uint8_t* yy = reinterpret_cast<uint8_t*>(y);
      if (vec && i0 + 3 < P) {
        uint32_t packed = (uint32_t)(v[0] & 0xff) | ((uint32_t)(v[1] & 0xff) << 8) |
                          ((uint32_t)(v[2] & 0xff) << 16) | ((uint32_t)(v[3] & 0xff) << 24);
        *reinterpret_cast<uint32_t*>(yy + index(i0, j)) = packed;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (i0 + r < P) yy[index(i0 + r, j)] = (uint8_t)(v[r] & 0xff);
      }
    }
  }
};

// ---------------------------------------------------------------- tiles
using T256 = Tile<256, 256, 2, 2>;
using T128 = Tile<128, 128, 2, 2>;
using T64 = Tile<64, 64, 2, 2>;

template <Op O, class Tl, class LX, class LY, class Epi>
static hipError_t launch_tile(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc,
                              hipStream_t st) {
  const int nP = (P + Tl::BP - 1) / Tl::BP, nQ = (Q + Tl::BQ - 1) / Tl::BQ;
  const int64_t nb = (int64_t)nP * nQ;
  if (nb <= 0) return hipSuccess;
  if (nb > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((mfma_gemm_kernel<O, Tl, LX, LY, Epi>), dim3((unsigned)nb), dim3(Tl::kThreads),
                     0, st, lx, ly, epi, nP, nQ, kc);
  return hipGetLastError();
}

static int pick_tile(int P, int Q, int forced) {
  if (forced == 256 || forced == 128 || forced == 64) return forced;
  auto blocks = [&](int b) { return (int64_t)((P + b - 1) / b) * ((Q + b - 1) / b); };
  if (blocks(256) >= 256) return 256;
  if (blocks(128) >= 200) return 128;
  return 64;
}

template <Op O, class LX, class LY, class Epi>
static hipError_t launch_any(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc, int tile,
                             hipStream_t st) {
  switch (pick_tile(P, Q, tile)) {
    case 256: return launch_tile<O, T256>(lx, ly, epi, P, Q, kc, st);
    case 128: return launch_tile<O, T128>(lx, ly, epi, P, Q, kc, st);
    default: return launch_tile<O, T64>(lx, ly, epi, P, Q, kc, st);
  }
}

template <class OutT>
static FloatEpi<OutT> make_float_epi(const FloatOut& o) {
  FloatEpi<OutT> e;
  e.y = reinterpret_cast<OutT*>(o.y);
  e.si = o.si; e.sj = o.sj; e.bstride = o.bstride; e.ohw = o.ohw; e.P = o.P; e.Q = o.Q;
  e.vec = o.vec; e.has_alpha = o.alpha != 1.0f; e.alpha = o.alpha; e.beta = o.beta;
  e.bias = reinterpret_cast<const OutT*>(o.bias); e.bias_mode = o.bias ? o.bias_mode : BIAS_NONE;
  e.act = o.act; e.lo = o.lo; e.hi = o.hi;
  return e;
}

static QuantEpi make_quant_epi(const QuantOut& o) {
  QuantEpi e;
  e.y = o.y; e.si = o.si; e.sj = o.sj; e.bstride = o.bstride; e.ohw = o.ohw; e.P = o.P; e.Q = o.Q;
  e.vec = o.vec; e.w_on_i = o.w_on_i; e.colsum = o.colsum; e.flip = o.flip; e.bias = o.bias; e.ca = o.ca;
  e.ca_rows = o.ca_rows; e.comb = o.comb; e.n_comb = o.n_comb; e.out_kind = o.out_kind;
  e.y_zp = o.y_zp; e.lo = o.lo; e.hi = o.hi;
  return e;
}

static DenseRows make_dense(const DenseOperand& d) {
  DenseRows r;
  r.base = reinterpret_cast<const char*>(d.base);
  r.ld = d.ld_bytes; r.rows = d.rows; r.kc = d.kc; r.kwrap = d.kwrap; r.xor_mask = d.xor_mask;
  r.pad = u32x4{d.pad, d.pad, d.pad, d.pad};
  return r;
}

static Im2colNHWC make_im2col(const Im2colOperand& c) {
  Im2colNHWC r;
  r.base = reinterpret_cast<const char*>(c.base);
  r.H = c.H; r.W = c.W; r.OH = c.OH; r.OW = c.OW; r.KW = c.KW; r.cpc = c.cpc;
  r.sh = c.sh; r.sw = c.sw; r.dh = c.dh; r.dw = c.dw; r.pt = c.pt; r.pl = c.pl;
  r.rows = c.rows; r.kc = c.kc; r.kwrap = c.kwrap; r.xor_mask = c.xor_mask;
  r.pad = u32x4{c.pad, c.pad, c.pad, c.pad};
  return r;
}

template <Op O, class OutT, class LX, class LY>
static hipError_t float_dispatch(const LX& lx, const LY& ly, const FloatOut& o, int kc, int tile, hipStream_t st) {
  return launch_any<O>(lx, ly, make_float_epi<OutT>(o), o.P, o.Q, kc, tile, st);
}

template <class LX, class LY>
static hipError_t float_by_dtype(int dtype, const LX& lx, const LY& ly, const FloatOut& o, int kc, int tile,
                                 hipStream_t st) {
  switch (dtype) {
    case DT_F32: return float_dispatch<Op::F32, float>(lx, ly, o, kc, tile, st);
    case DT_F16: return float_dispatch<Op::F16, _Float16>(lx, ly, o, kc, tile, st);
    case DT_BF16: return float_dispatch<Op::BF16, __bf16>(lx, ly, o, kc, tile, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_dense_float(int dtype, const DenseOperand& x, const DenseOperand& y, const FloatOut& o, int tile,
                           hipStream_t st) {
  return float_by_dtype(dtype, make_dense(x), make_dense(y), o, x.kc, tile, st);
}

hipError_t run_conv_float(int dtype, const Im2colOperand& col, const DenseOperand& w, bool col_on_x,
                          const FloatOut& o, int tile, hipStream_t st) {
  if (col_on_x) return float_by_dtype(dtype, make_im2col(col), make_dense(w), o, col.kc, tile, st);
  return float_by_dtype(dtype, make_dense(w), make_im2col(col), o, col.kc, tile, st);
}

hipError_t run_dense_quant(const DenseOperand& x, const DenseOperand& y, const QuantOut& o, int tile, hipStream_t st) {
  return launch_any<Op::I8>(make_dense(x), make_dense(y), make_quant_epi(o), o.P, o.Q, x.kc, tile, st);
}
// (x is always the packed weight for the integer GEMM, so x.kc is the full
// loop length, including the second half of a split weight.)

hipError_t run_conv_quant(const Im2colOperand& col, const DenseOperand& w, bool col_on_x, const QuantOut& o,
                          int tile, hipStream_t st) {
  if (col_on_x)
    return launch_any<Op::I8>(make_im2col(col), make_dense(w), make_quant_epi(o), o.P, o.Q, w.kc, tile, st);
  return launch_any<Op::I8>(make_dense(w), make_im2col(col), make_quant_epi(o), o.P, o.Q, w.kc, tile, st);
}

// ---------------------------------------------------------------- skinny GEMV
// y[m][n] = sum_k A[m][k] * W[n][k] for M <= kMaxGemvM.  Each wave owns one
// weight row and one K slice, streams the row with 16-byte loads, and writes
// one f32 partial per (slice, m, n); gemv_finish sums the slices in a fixed
// order (deterministic) and applies the epilogue.
template <class T> struct Vec16;
template <> struct Vec16<float> {
  static __device__ __forceinline__ void unpack(u32x4 v, float (&f)[4]) {
    f[0] = lane_f32(v.x); f[1] = lane_f32(v.y); f[2] = lane_f32(v.z); f[3] = lane_f32(v.w);
  }
  static constexpr int N = 4;
};
template <> struct Vec16<_Float16> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(u32x4 v, float (&f)[8]) {
    f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (float)h[e];
  }
};
template <> struct Vec16<__bf16> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(u32x4 v, float (&f)[8]) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = __builtin_bit_cast(float, w[e] << 16);
      f[2 * e + 1] = __builtin_bit_cast(float, w[e] & 0xffff0000u);
    }
  }
};

template <class T, int M>
__global__ void __launch_bounds__(256)
gemv_partial_kernel(const T* __restrict__ a, int64_t lda, const T* __restrict__ w, int64_t ldw, int N, int kc,
                    int chunks_per_split, float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int s = blockIdx.y;
  if (n >= N) return;
  const int c0 = s * chunks_per_split;
  const int c1 = min(kc, c0 + chunks_per_split);
  constexpr int E = Vec16<T>::N;
  const u32x4* wr = reinterpret_cast<const u32x4*>(w + (int64_t)n * ldw);
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  int c = c0 + lane;
  for (; c + 64 < c1; c += 128) {
    u32x4 w0 = __builtin_nontemporal_load(wr + c);
    u32x4 w1 = __builtin_nontemporal_load(wr + c + 64);
    float f0[E], f1[E];
    Vec16<T>::unpack(w0, f0);
    Vec16<T>::unpack(w1, f1);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u32x4* ar = reinterpret_cast<const u32x4*>(a + (int64_t)m * lda);
      float g0[E], g1[E];
      Vec16<T>::unpack(ar[c], g0);
      Vec16<T>::unpack(ar[c + 64], g1);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[m] += f0[e] * g0[e];
#pragma unroll
      for (int e = 0; e < E; ++e) acc[m] += f1[e] * g1[e];
    }
  }
  for (; c < c1; c += 64) {
    u32x4 w0 = __builtin_nontemporal_load(wr + c);
    float f0[E];
    Vec16<T>::unpack(w0, f0);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u32x4* ar = reinterpret_cast<const u32x4*>(a + (int64_t)m * lda);
      float g0[E];
      Vec16<T>::unpack(ar[c], g0);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[m] += f0[e] * g0[e];
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v = acc[m];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) part[((int64_t)s * M + m) * N + n] = v;
  }
}

template <class OutT>
__global__ void gemv_finish_kernel(const float* __restrict__ part, int splits, int M, int N, FloatEpi<OutT> epi) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx - (int64_t)m * N);
  float v = 0.0f;
  for (int s = 0; s < splits; ++s) v += part[((int64_t)s * M + m) * N + n];
  // GEMM orientation: i = n (weight row), j = m (activation row)
  epi.y[epi.index(n, m)] = from_f32<OutT>(epi.finish(v, n, m));
}

template <class T, class OutT>
static hipError_t gemv_t(const GemvArgs& g, const FloatOut& o, hipStream_t st) {
  constexpr int E = Vec16<T>::N;
  (void)E;
  const T* a = reinterpret_cast<const T*>(g.a);
  const T* w = reinterpret_cast<const T*>(g.w);
  dim3 grid((g.N + 3) / 4, g.splits);
  switch (g.M) {
#define OHIP_GEMV_CASE(MM)                                                                                   \
  case MM:                                                                                                   \
    hipLaunchKernelGGL((gemv_partial_kernel<T, MM>), grid, dim3(256), 0, st, a, g.lda, w, g.ldw, g.N, g.kc, \
                       g.chunks_per_split, g.partial);                                                       \
    break;
    OHIP_GEMV_CASE(1) OHIP_GEMV_CASE(2) OHIP_GEMV_CASE(3) OHIP_GEMV_CASE(4)
    OHIP_GEMV_CASE(5) OHIP_GEMV_CASE(6) OHIP_GEMV_CASE(7) OHIP_GEMV_CASE(8)
#undef OHIP_GEMV_CASE
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t total = (int64_t)g.M * g.N;
  hipLaunchKernelGGL((gemv_finish_kernel<OutT>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     g.partial, g.splits, g.M, g.N, make_float_epi<OutT>(o));
  return hipGetLastError();
}

hipError_t run_gemv(int dtype, const GemvArgs& g, const FloatOut& o, hipStream_t st) {
  switch (dtype) {
    case DT_F32: return gemv_t<float, float>(g, o, st);
    case DT_F16: return gemv_t<_Float16, _Float16>(g, o, st);
    case DT_BF16: return gemv_t<__bf16, __bf16>(g, o, st);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------- layout
// NCHW -> NHWC with the channel axis zero-padded to cp: per image a [C][HW]
// -> [HW][cp] transpose through a 32x33 LDS tile (coalesced on both sides).
template <class T>
__global__ void nchw_to_nhwc_kernel(const T* __restrict__ src, T* __restrict__ dst, int C, int HW, int cp) {
  __shared__ T tile[32][33];
  const int n = blockIdx.z;
  const int c0 = blockIdx.y * 32, s0 = blockIdx.x * 32;
  const T* s = src + (int64_t)n * C * HW;
  T* d = dst + (int64_t)n * HW * cp;
  for (int r = threadIdx.y; r < 32; r += blockDim.y) {
    const int c = c0 + r, sp = s0 + threadIdx.x;
    tile[r][threadIdx.x] = (c < C && sp < HW) ? s[(int64_t)c * HW + sp] : T(0);
  }
  __syncthreads();
  for (int r = threadIdx.y; r < 32; r += blockDim.y) {
    const int sp = s0 + r, c = c0 + threadIdx.x;
    if (sp < HW && c < cp) d[(int64_t)sp * cp + c] = tile[threadIdx.x][r];
  }
}

template <class T>
static hipError_t nchw_to_nhwc_t(const void* src, void* dst, int N, int C, int HW, int cp, hipStream_t st) {
  dim3 grid((HW + 31) / 32, (cp + 31) / 32, N), block(32, 8);
  hipLaunchKernelGGL(nchw_to_nhwc_kernel<T>, grid, block, 0, st, reinterpret_cast<const T*>(src),
                     reinterpret_cast<T*>(dst), C, HW, cp);
  return hipGetLastError();
}

hipError_t run_nchw_to_nhwc(int elem_bytes, const void* src, void* dst, int N, int C, int HW, int cp,
                            hipStream_t st) {
  switch (elem_bytes) {
    case 1: return nchw_to_nhwc_t<uint8_t>(src, dst, N, C, HW, cp, st);
    case 2: return nchw_to_nhwc_t<uint16_t>(src, dst, N, C, HW, cp, st);
    case 4: return nchw_to_nhwc_t<uint32_t>(src, dst, N, C, HW, cp, st);
    default: return hipErrorInvalidValue;
  }
}

// dst[r][c] = c < K ? src[r * rs + c * cs] : 0 for a [R][ld] destination: pads a
// row-major operand to whole 16-byte chunks, or materialises a transpose.
template <class T>
__global__ void gather2d_kernel(const T* __restrict__ src, int64_t rs, int64_t cs, T* __restrict__ dst, int R,
                                int K, int ld) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)R * ld) return;
  const int r = (int)(idx / ld), c = (int)(idx - (int64_t)r * ld);
  dst[idx] = c < K ? src[r * rs + c * cs] : T(0);
}

hipError_t run_gather2d(int elem_bytes, const void* src, int64_t rs, int64_t cs, void* dst, int R, int K, int ld,
                        hipStream_t st) {
  const int64_t total = (int64_t)R * ld;
  dim3 grid((unsigned)((total + 255) / 256)), block(256);
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL(gather2d_kernel<uint8_t>, grid, block, 0, st, reinterpret_cast<const uint8_t*>(src), rs,
                         cs, reinterpret_cast<uint8_t*>(dst), R, K, ld);
      break;
    case 2:
      hipLaunchKernelGGL(gather2d_kernel<uint16_t>, grid, block, 0, st, reinterpret_cast<const uint16_t*>(src),
                         rs, cs, reinterpret_cast<uint16_t*>(dst), R, K, ld);
      break;
    case 4:
      hipLaunchKernelGGL(gather2d_kernel<uint32_t>, grid, block, 0, st, reinterpret_cast<const uint32_t*>(src),
                         rs, cs, reinterpret_cast<uint32_t*>(dst), R, K, ld);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ohip
