// Dispatch by element type to the per-dtype contraction units, plus the
// skinny-M GEMV path and the layout kernels that feed the MFMA kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "launch.hpp"

namespace ohip {

hipError_t run_dense_f32(const DenseOperand&, const DenseOperand&, const FloatOut&, int, hipStream_t);
hipError_t run_dense_f16(const DenseOperand&, const DenseOperand&, const FloatOut&, int, hipStream_t);
hipError_t run_dense_bf16(const DenseOperand&, const DenseOperand&, const FloatOut&, int, hipStream_t);
hipError_t run_dense_i8(const DenseOperand&, const DenseOperand&, const QuantOut&, int, hipStream_t);
hipError_t run_conv_f32(const Im2colOperand&, const DenseOperand&, bool, const FloatOut&, int, hipStream_t);
hipError_t run_conv_f16(const Im2colOperand&, const DenseOperand&, bool, const FloatOut&, int, hipStream_t);
hipError_t run_conv_bf16(const Im2colOperand&, const DenseOperand&, bool, const FloatOut&, int, hipStream_t);
hipError_t run_conv_i8(const Im2colOperand&, const DenseOperand&, bool, const QuantOut&, int, hipStream_t);
hipError_t run_halo_f32(const HaloGeo&, bool, const FloatOut&, hipStream_t);
hipError_t run_halo_f16(const HaloGeo&, bool, const FloatOut&, hipStream_t);
hipError_t run_halo_bf16(const HaloGeo&, bool, const FloatOut&, hipStream_t);
hipError_t run_wk_f32(const HaloGeo&, bool, const FloatOut&, float*, hipStream_t);
hipError_t run_wk_f16(const HaloGeo&, bool, const FloatOut&, float*, hipStream_t);
hipError_t run_wk_bf16(const HaloGeo&, bool, const FloatOut&, float*, hipStream_t);

hipError_t run_dense_float(int dtype, const DenseOperand& x, const DenseOperand& y, const FloatOut& o, int tile,
                           hipStream_t st) {
  switch (dtype) {
    case DT_F32: return run_dense_f32(x, y, o, tile, st);
    case DT_F16: return run_dense_f16(x, y, o, tile, st);
    case DT_BF16: return run_dense_bf16(x, y, o, tile, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_conv_float(int dtype, const Im2colOperand& col, const DenseOperand& w, bool col_on_x,
                          const FloatOut& o, int tile, hipStream_t st) {
  switch (dtype) {
    case DT_F32: return run_conv_f32(col, w, col_on_x, o, tile, st);
    case DT_F16: return run_conv_f16(col, w, col_on_x, o, tile, st);
    case DT_BF16: return run_conv_bf16(col, w, col_on_x, o, tile, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_halo_float(int dtype, const HaloGeo& g, bool pix_on_x, const FloatOut& o, hipStream_t st) {
  switch (dtype) {
    case DT_F32: return run_halo_f32(g, pix_on_x, o, st);
    case DT_F16: return run_halo_f16(g, pix_on_x, o, st);
    case DT_BF16: return run_halo_bf16(g, pix_on_x, o, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_wk_float(int dtype, const HaloGeo& g, bool pix_on_x, const FloatOut& o, float* mom, hipStream_t st) {
  switch (dtype) {
    case DT_F32: return run_wk_f32(g, pix_on_x, o, mom, st);
    case DT_F16: return run_wk_f16(g, pix_on_x, o, mom, st);
    case DT_BF16: return run_wk_bf16(g, pix_on_x, o, mom, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_dense_quant(const DenseOperand& x, const DenseOperand& y, const QuantOut& o, int tile, hipStream_t st) {
  return run_dense_i8(x, y, o, tile, st);
}

hipError_t run_conv_quant(const Im2colOperand& col, const DenseOperand& w, bool col_on_x, const QuantOut& o,
                          int tile, hipStream_t st) {
  return run_conv_i8(col, w, col_on_x, o, tile, st);
}

// ---------------------------------------------------------------- skinny GEMV
// y[m][n] = sum_k A[m][k] * W[n][k] for M <= 8: the HBM-bound skinny path,
// which streams every weight byte exactly once with 16-byte loads.
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

// One block per weight row n: its 8 waves stride the row's 16-byte chunks
// together (coalesced, up to 16 loads in flight per lane), reduce through
// registers and LDS in a fixed order (deterministic), and thread 0 runs the
// epilogue for the M outputs of that row.
template <class T, int M>
__global__ void __launch_bounds__(512)
gemv_row_kernel(const T* __restrict__ a, int64_t lda, const T* __restrict__ w, int64_t ldw, int kc,
                FloatEpi<T> epi) {
  constexpr int E = Vec16<T>::N;
  constexpr int kWaves = 8;
  __shared__ float red[kWaves][M];
  const int n = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const u32x4* wr = reinterpret_cast<const u32x4*>(w + (int64_t)n * ldw);
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  auto fma_chunk = [&](u32x4 wv, int c) {
    float f[E];
    Vec16<T>::unpack(wv, f);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u32x4* ar = reinterpret_cast<const u32x4*>(a + (int64_t)m * lda);
      float g[E];
      Vec16<T>::unpack(ar[c], g);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[m] += f[e] * g[e];
    }
  };
  constexpr int S = kWaves * 64;
  // loads in flight per lane, issued together (guarded at the row's end):
  // config 2a's K = 25088 row is one round of them in f32 and f16
  // (10.0 -> 9.35 us f32 against four at a time)
  constexpr int U = sizeof(T) == 4 ? 16 : 8;
  for (int c = tid; c < kc; c += U * S) {
    u32x4 wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c + u * S < kc) wv[u] = __builtin_nontemporal_load(wr + c + u * S);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (c + u * S < kc) fma_chunk(wv[u], c + u * S);
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v = acc[m];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) red[wave][m] = v;
  }
  __syncthreads();
  if (tid < M) {
    float v = 0.0f;
#pragma unroll
    for (int q = 0; q < kWaves; ++q) v += red[q][tid];
    // GEMM orientation: i = n (weight row), j = m (activation row)
    epi.store_one(v, n, tid);
  }
}

// Rows of at most kWaveRowChunks 16-byte chunks: one wave per weight row
// (four rows per block), each lane striding the row's chunks, the partial
// sums reduced across the wave by a fixed butterfly (deterministic); lane 0
// runs the epilogue for the M outputs of the row.  A block per row would
// leave most of its waves without a chunk.
constexpr int kWaveRowChunks = 256;

template <class T, int M>
__global__ void __launch_bounds__(256)
gemv_wave_kernel(const T* __restrict__ a, int64_t lda, const T* __restrict__ w, int64_t ldw, int kc, int N,
                 FloatEpi<T> epi) {
  constexpr int E = Vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const u32x4* wr = reinterpret_cast<const u32x4*>(w + (int64_t)n * ldw);
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  for (int c = lane; c < kc; c += 64) {
    float f[E];
    Vec16<T>::unpack(__builtin_nontemporal_load(wr + c), f);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float g[E];
      Vec16<T>::unpack(reinterpret_cast<const u32x4*>(a + (int64_t)m * lda)[c], g);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[m] += f[e] * g[e];
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
  }
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < M; ++m) epi.store_one(acc[m], n, m);
  }
}

template <class T>
static hipError_t gemv_t(const GemvArgs& g, const FloatOut& o, hipStream_t st) {
  const T* a = reinterpret_cast<const T*>(g.a);
  const T* w = reinterpret_cast<const T*>(g.w);
  const FloatEpi<T> epi = make_float_epi<T>(o);
  const bool by_wave = g.kc <= kWaveRowChunks;
  const unsigned wave_blocks = (unsigned)((g.N + 3) / 4);
  switch (g.M) {
#define OHIP_GEMV_CASE(MM)                                                                                      \
  case MM:                                                                                                      \
    if (by_wave)                                                                                                \
      hipLaunchKernelGGL((gemv_wave_kernel<T, MM>), dim3(wave_blocks), dim3(256), 0, st, a, g.lda, w, g.ldw, \
                         g.kc, g.N, epi);                                                                       \
    else                                                                                                        \
      hipLaunchKernelGGL((gemv_row_kernel<T, MM>), dim3(g.N), dim3(512), 0, st, a, g.lda, w, g.ldw, g.kc, epi); \
    break;
    OHIP_GEMV_CASE(1) OHIP_GEMV_CASE(2) OHIP_GEMV_CASE(3) OHIP_GEMV_CASE(4)
    OHIP_GEMV_CASE(5) OHIP_GEMV_CASE(6) OHIP_GEMV_CASE(7) OHIP_GEMV_CASE(8)
#undef OHIP_GEMV_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t run_gemv(int dtype, const GemvArgs& g, const FloatOut& o, hipStream_t st) {
  switch (dtype) {
    case DT_F32: return gemv_t<float>(g, o, st);
    case DT_F16: return gemv_t<_Float16>(g, o, st);
    case DT_BF16: return gemv_t<__bf16>(g, o, st);
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

__device__ __forceinline__ int pad_map(int o, int begin, int len, int mode) {
  int s = o - begin;
  if (s >= 0 && s < len) return s;
  if (mode == 2 || len == 1) return s < 0 ? 0 : len - 1;
  const int period = 2 * (len - 1);
  s %= period;
  if (s < 0) s += period;
  return s < len ? s : period - s;
}

// Row-tiled staging, the fast form of both transposes above: a block takes
// one span of source pixels (a run of the flattened H x W axis, or one whole
// source row when a reflect / edge border is added) for up to 64 channels,
// reads it with 16-byte loads along the pixels, transposes it through LDS and
// writes whole 16-byte channel vectors of every output pixel it covers.
// Output pixel x of the span takes LDS column map(x): x itself, or
// pad_map(x) for a bordered row.  Channels from C up to cp are written as
// zero.  Needs the span and the row to be whole 16-byte chunks.
struct RowStage {
  int C, H, W, HW, cp, tc;    // tc: channels per block (a multiple of 16 / sizeof(T), <= 64)
  int span;                   // pixels per block (unbordered form)
  int Hp, Wp, pt, pl, mode;   // bordered form
};

template <class T, bool BORDER>
__global__ void __launch_bounds__(256) stage_rows_kernel(const T* __restrict__ src, T* __restrict__ dst, RowStage g) {
  constexpr int V = 16 / (int)sizeof(T);
  extern __shared__ u32x4 stage_lds[];
  T* tile = reinterpret_cast<T*>(stage_lds);
  const int RS = g.tc + V;   // LDS row stride in elements (keeps rows 16-byte aligned)
  const int n = blockIdx.z, c0 = blockIdx.y * g.tc;
  int64_t sbase, obase;
  int L, O;
  if (BORDER) {
    const int y = blockIdx.x;
    sbase = (int64_t)pad_map(y, g.pt, g.H, g.mode) * g.W;
    L = g.W;
    O = g.Wp;
    obase = (int64_t)y * g.Wp;
  } else {
    const int64_t p0 = (int64_t)blockIdx.x * g.span;
    L = O = (int)min((int64_t)g.span, (int64_t)g.HW - p0);
    sbase = obase = p0;
  }
  const T* s = src + (int64_t)n * g.C * g.HW + sbase;
  const int lc = L / V;
  for (int v = threadIdx.x; v < g.tc * lc; v += 256) {
    const int c = v / lc, q = v - c * lc;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (c0 + c < g.C) w = *reinterpret_cast<const u32x4*>(s + (int64_t)(c0 + c) * g.HW + q * V);
    T e[V];
    __builtin_memcpy(e, &w, 16);
#pragma unroll
    for (int k = 0; k < V; ++k) tile[(q * V + k) * RS + c] = e[k];
  }
  __syncthreads();
  const int oc = g.tc / V;
  const int64_t HWo = BORDER ? (int64_t)g.Hp * g.Wp : (int64_t)g.HW;
  T* d = dst + ((int64_t)n * HWo + obase) * g.cp + c0;
  for (int v = threadIdx.x; v < O * oc; v += 256) {
    const int x = v / oc, q = v - x * oc;
    if (c0 + q * V >= g.cp) continue;
    const int m = BORDER ? pad_map(x, g.pl, g.W, g.mode) : x;
    *reinterpret_cast<u32x4*>(d + (int64_t)x * g.cp + q * V) = *reinterpret_cast<const u32x4*>(tile + m * RS + q * V);
  }
}

// Launches the row-tiled form when its conditions hold; hipErrorNotSupported
// otherwise (the caller then uses the element-tiled kernels).
template <class T>
static hipError_t stage_rows_t(const void* src, void* dst, int N, int C, int H, int W, int cp, int pt, int pl, int pb,
                               int pr, int mode, hipStream_t st) {
  constexpr int V = 16 / (int)sizeof(T);
  const bool border = pt | pl | pb | pr;
  const int HW = H * W;
  if (cp % V != 0 || (uintptr_t)src % 16 != 0 || (uintptr_t)dst % 16 != 0) return hipErrorNotSupported;
  if (border ? W % V != 0 : HW % V != 0) return hipErrorNotSupported;
  RowStage g{};
  g.C = C; g.H = H; g.W = W; g.HW = HW; g.cp = cp;
  g.tc = cp < 64 ? cp : 64;
  g.Hp = H + pt + pb; g.Wp = W + pl + pr; g.pt = pt; g.pl = pl; g.mode = mode;
  const int ctiles = (cp + g.tc - 1) / g.tc;
  const size_t px_bytes = (size_t)(g.tc + V) * sizeof(T);
  dim3 grid;
  size_t lds;
  if (border) {
    lds = (size_t)W * px_bytes;
    if (lds > 48 * 1024) return hipErrorNotSupported;
    grid = dim3((unsigned)g.Hp, (unsigned)ctiles, (unsigned)N);
  } else {
    // about 1024 blocks, each span a whole number of chunks within 32 KB of LDS
    const int64_t lds_px = (int64_t)(32 * 1024 / px_bytes) / V * V;
    int64_t span = ((int64_t)HW * ctiles * N + 1023) / 1024;
    span = (span + V - 1) / V * V;
    span = std::max<int64_t>(span, 4 * V);
    span = std::min<int64_t>(span, std::min<int64_t>(lds_px, HW));
    g.span = (int)span;
    lds = (size_t)span * px_bytes;
    grid = dim3((unsigned)((HW + span - 1) / span), (unsigned)ctiles, (unsigned)N);
  }
  if (border)
    hipLaunchKernelGGL((stage_rows_kernel<T, true>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(src),
                       reinterpret_cast<T*>(dst), g);
  else
    hipLaunchKernelGGL((stage_rows_kernel<T, false>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(src),
                       reinterpret_cast<T*>(dst), g);
  return hipGetLastError();
}

template <class T>
static hipError_t nchw_to_nhwc_t(const void* src, void* dst, int N, int C, int HW, int cp, hipStream_t st) {
  dim3 grid((HW + 31) / 32, (cp + 31) / 32, N), block(32, 8);
  hipLaunchKernelGGL(nchw_to_nhwc_kernel<T>, grid, block, 0, st, reinterpret_cast<const T*>(src),
                     reinterpret_cast<T*>(dst), C, HW, cp);
  return hipGetLastError();
}

// The inverse: NHWC with a pixel pitch back to NCHW, through a 32 x 32 LDS
// tile (pixels x channels).
template <class T>
__global__ void nhwc_to_nchw_kernel(const T* __restrict__ src, T* __restrict__ dst, int C, int HW, int pitch) {
  __shared__ T tile[32][33];
  const int n = blockIdx.z;
  const int c0 = blockIdx.y * 32, s0 = blockIdx.x * 32;
  const T* s = src + (int64_t)n * HW * pitch;
  T* d = dst + (int64_t)n * C * HW;
  for (int r = threadIdx.y; r < 32; r += blockDim.y) {
    const int sp = s0 + r, c = c0 + threadIdx.x;
    tile[r][threadIdx.x] = (sp < HW && c < C) ? s[(int64_t)sp * pitch + c] : T(0);
  }
  __syncthreads();
  for (int r = threadIdx.y; r < 32; r += blockDim.y) {
    const int c = c0 + r, sp = s0 + threadIdx.x;
    if (c < C && sp < HW) d[(int64_t)c * HW + sp] = tile[threadIdx.x][r];
  }
}

hipError_t run_nhwc_to_nchw(int elem_bytes, const void* src, void* dst, int N, int C, int HW, int pitch,
                            hipStream_t st) {
  if (N <= 0 || C <= 0 || HW <= 0) return hipSuccess;
  dim3 grid((HW + 31) / 32, (C + 31) / 32, N), block(32, 8);
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL(nhwc_to_nchw_kernel<uint8_t>, grid, block, 0, st, (const uint8_t*)src, (uint8_t*)dst, C, HW, pitch);
      break;
    case 2:
      hipLaunchKernelGGL(nhwc_to_nchw_kernel<uint16_t>, grid, block, 0, st, (const uint16_t*)src, (uint16_t*)dst, C, HW,
                         pitch);
      break;
    case 4:
      hipLaunchKernelGGL(nhwc_to_nchw_kernel<uint32_t>, grid, block, 0, st, (const uint32_t*)src, (uint32_t*)dst, C, HW,
                         pitch);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t run_nchw_to_nhwc(int elem_bytes, const void* src, void* dst, int N, int C, int HW, int cp,
                            hipStream_t st) {
  hipError_t e = hipErrorNotSupported;
  switch (elem_bytes) {
    case 1: e = stage_rows_t<uint8_t>(src, dst, N, C, 1, HW, cp, 0, 0, 0, 0, 0, st); break;
    case 2: e = stage_rows_t<uint16_t>(src, dst, N, C, 1, HW, cp, 0, 0, 0, 0, 0, st); break;
    case 4: e = stage_rows_t<uint32_t>(src, dst, N, C, 1, HW, cp, 0, 0, 0, 0, 0, st); break;
  }
  if (e != hipErrorNotSupported) return e;
  switch (elem_bytes) {
    case 1: return nchw_to_nhwc_t<uint8_t>(src, dst, N, C, HW, cp, st);
    case 2: return nchw_to_nhwc_t<uint16_t>(src, dst, N, C, HW, cp, st);
    case 4: return nchw_to_nhwc_t<uint32_t>(src, dst, N, C, HW, cp, st);
    default: return hipErrorInvalidValue;
  }
}

// NCHW [C][H][W] -> NHWC [Hp][Wp][cp] with the spatial border filled by
// reflection (mode 1) or edge replication (mode 2): the Pad node in front of
// a convolution, fused into its staging transpose.  Padded pixel (y, x)
// reads source pixel (src_y, src_x) of the ONNX Pad mapping.

template <class T>
__global__ void nchw_to_nhwc_pad_kernel(const T* __restrict__ src, T* __restrict__ dst, int C, int H, int W, int cp,
                                        int Hp, int Wp, int pt, int pl, int mode) {
  __shared__ T tile[32][33];
  const int n = blockIdx.z;
  const int c0 = blockIdx.y * 32, s0 = blockIdx.x * 32;
  const int HWp = Hp * Wp;
  const T* s = src + (int64_t)n * C * H * W;
  T* d = dst + (int64_t)n * HWp * cp;
  for (int r = threadIdx.y; r < 32; r += blockDim.y) {
    const int c = c0 + r, sp = s0 + threadIdx.x;
    T v = T(0);
    if (c < C && sp < HWp) {
      const int y = sp / Wp, x = sp - y * Wp;
      v = s[(int64_t)c * H * W + pad_map(y, pt, H, mode) * W + pad_map(x, pl, W, mode)];
    }
    tile[r][threadIdx.x] = v;
  }
  __syncthreads();
  for (int r = threadIdx.y; r < 32; r += blockDim.y) {
    const int sp = s0 + r, c = c0 + threadIdx.x;
    if (sp < HWp && c < cp) d[(int64_t)sp * cp + c] = tile[threadIdx.x][r];
  }
}

template <class T>
static hipError_t nchw_to_nhwc_pad_t(const void* src, void* dst, int N, int C, int H, int W, int cp, int pt, int pl,
                                     int pb, int pr, int mode, hipStream_t st) {
  const int Hp = H + pt + pb, Wp = W + pl + pr;
  dim3 grid((Hp * Wp + 31) / 32, (cp + 31) / 32, N), block(32, 8);
  hipLaunchKernelGGL(nchw_to_nhwc_pad_kernel<T>, grid, block, 0, st, reinterpret_cast<const T*>(src),
                     reinterpret_cast<T*>(dst), C, H, W, cp, Hp, Wp, pt, pl, mode);
  return hipGetLastError();
}

hipError_t run_nchw_to_nhwc_pad(int elem_bytes, const void* src, void* dst, int N, int C, int H, int W, int cp,
                                int pt, int pl, int pb, int pr, int mode, hipStream_t st) {
  hipError_t e = hipErrorNotSupported;
  switch (elem_bytes) {
    case 1: e = stage_rows_t<uint8_t>(src, dst, N, C, H, W, cp, pt, pl, pb, pr, mode, st); break;
    case 2: e = stage_rows_t<uint16_t>(src, dst, N, C, H, W, cp, pt, pl, pb, pr, mode, st); break;
    case 4: e = stage_rows_t<uint32_t>(src, dst, N, C, H, W, cp, pt, pl, pb, pr, mode, st); break;
  }
  if (e != hipErrorNotSupported) return e;
  switch (elem_bytes) {
    case 1: return nchw_to_nhwc_pad_t<uint8_t>(src, dst, N, C, H, W, cp, pt, pl, pb, pr, mode, st);
    case 2: return nchw_to_nhwc_pad_t<uint16_t>(src, dst, N, C, H, W, cp, pt, pl, pb, pr, mode, st);
    case 4: return nchw_to_nhwc_pad_t<uint32_t>(src, dst, N, C, H, W, cp, pt, pl, pb, pr, mode, st);
    default: return hipErrorInvalidValue;
  }
}

// NCHW [C][H][W] -> NHWC [Hp][Wp][cpt] staging of a grouped convolution's
// input for the implicit-im2col loader.  The channel axis is laid out per group: slot g * cpg + ci holds
// channel g * cg + ci for ci < cg, and zero for the padding slots up to cpg
// (cpg a whole number of 16-byte chunks, cpt = groups * cpg).  The spatial
// border, if any, is filled by pad_map (a fused reflect / edge Pad).
struct StageGeo {
  int C, H, W, Hp, Wp, pt, pl, mode, cg, cpg, cpt;
  __device__ __forceinline__ int64_t src_off(int64_t px) const {   // -1 past the image
    const int y = (int)(px / Wp), x = (int)(px - (int64_t)y * Wp);
    return (int64_t)pad_map(y, pt, H, mode) * W + pad_map(x, pl, W, mode);
  }
  __device__ __forceinline__ int channel(int slot) const {         // -1 for a padding slot
    const int g = slot / cpg, ci = slot - g * cpg, c = g * cg + ci;
    return (ci < cg && c < C) ? c : -1;
  }
};

// A block moves 32 pixels x 64 slots through LDS, reading source rows along
// the pixels and writing whole 16-byte slot vectors.
template <class T>
__global__ void __launch_bounds__(256)
stage_nhwc_tile_kernel(const T* __restrict__ src, T* __restrict__ dst, StageGeo g) {
  constexpr int VE = 16 / (int)sizeof(T), PX = 32, SL = 64;
  __shared__ T tile[SL][PX + 1];
  const int n = blockIdx.z;
  const int s0 = blockIdx.y * SL;
  const int64_t p0 = (int64_t)blockIdx.x * PX;
  const int64_t HWp = (int64_t)g.Hp * g.Wp;
  const T* s = src + (int64_t)n * g.C * g.H * g.W;
  const int64_t plane = (int64_t)g.H * g.W;
  const int tx = threadIdx.x & (PX - 1), ty = threadIdx.x / PX;
  const int64_t px = p0 + tx;
  const int64_t off = px < HWp ? g.src_off(px) : -1;
  for (int r = ty; r < SL; r += 256 / PX) {
    const int slot = s0 + r;
    const int c = (off >= 0 && slot < g.cpt) ? g.channel(slot) : -1;
    tile[r][tx] = c >= 0 ? s[c * plane + off] : T(0);
  }
  __syncthreads();
  T* d = dst + (int64_t)n * HWp * g.cpt;
  for (int v = threadIdx.x; v < PX * (SL / VE); v += 256) {
    const int p = v / (SL / VE), q = v - p * (SL / VE);
    const int64_t pix = p0 + p;
    const int slot = s0 + q * VE;
    if (pix >= HWp || slot >= g.cpt) continue;
    T e[VE];
#pragma unroll
    for (int k = 0; k < VE; ++k) e[k] = tile[q * VE + k][p];
    *reinterpret_cast<u32x4*>(d + pix * g.cpt + slot) = __builtin_bit_cast(u32x4, e);
  }
}

template <class T>
static hipError_t stage_nhwc_t(const void* src, void* dst, int N, int C, int H, int W, int pt, int pl, int pb,
                               int pr, int mode, int cg, int cpg, int groups, hipStream_t st) {
  StageGeo g{C, H, W, H + pt + pb, W + pl + pr, pt, pl, mode, cg, cpg, groups * cpg};
  const int64_t HWp = (int64_t)g.Hp * g.Wp;
  if (g.cpt % (16 / (int)sizeof(T)) != 0 || (uintptr_t)dst % 16 != 0) return hipErrorInvalidValue;
  const T* s = reinterpret_cast<const T*>(src);
  T* d = reinterpret_cast<T*>(dst);
  hipLaunchKernelGGL(stage_nhwc_tile_kernel<T>,
                     dim3((unsigned)((HWp + 31) / 32), (unsigned)((g.cpt + 63) / 64), (unsigned)N), dim3(256), 0, st,
                     s, d, g);
  return hipGetLastError();
}

hipError_t run_stage_nhwc(int elem_bytes, const void* src, void* dst, int N, int C, int H, int W, int pt, int pl,
                          int pb, int pr, int mode, int cg, int cpg, int groups, hipStream_t st) {
  switch (elem_bytes) {
    case 1: return stage_nhwc_t<uint8_t>(src, dst, N, C, H, W, pt, pl, pb, pr, mode, cg, cpg, groups, st);
    case 2: return stage_nhwc_t<uint16_t>(src, dst, N, C, H, W, pt, pl, pb, pr, mode, cg, cpg, groups, st);
    case 4: return stage_nhwc_t<uint32_t>(src, dst, N, C, H, W, pt, pl, pb, pr, mode, cg, cpg, groups, st);
    default: return hipErrorInvalidValue;
  }
}

// (n, co, oy, ox) of flat output index idx; 32-bit divisions when the
// whole output indexes in 32 bits (64-bit division is a long instruction
// sequence, and these kernels do little else per output)
__device__ __forceinline__ void split_out_index(int64_t idx, int64_t total, int OW, int OH, int cout, int& ox, int& oy,
                                                int& co, int& n) {
  if (total <= 0x7fffffff) {
    int r = (int)idx;
    ox = r % OW; r /= OW;
    oy = r % OH; r /= OH;
    co = r % cout;
    n = r / cout;
  } else {
    int64_t r = idx;
    ox = (int)(r % OW); r /= OW;
    oy = (int)(r % OH); r /= OH;
    co = (int)(r % cout);
    n = (int)(r / cout);
  }
}

// ---------------------------------------------------------------- direct conv
// Convolution for channel groups too narrow for the MFMA engine (depthwise
// and other small groups): one thread per output element, f32 accumulation
// over the (ci, ky, kx) taps of its group in that order; NCHW input, NCHW or
// NHWC output.  The filter is the packed [Cout][KH][KW][cpg] form.  Zero
// padding skips the taps outside the image; a fused reflect / edge Pad maps
// them into it (pad_map), as the staging transpose does for the MFMA path.
template <class T>
__global__ void __launch_bounds__(256)
conv_direct_kernel(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias, T* __restrict__ y,
                   DirectConvArgs a) {
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    int ox, oy, co, n;
    split_out_index(idx, total, a.OW, a.OH, a.cout, ox, oy, co, n);
    const int g = co / a.coutg;
    const T* xg = x + ((int64_t)n * a.C + (int64_t)g * a.cg) * a.H * a.W;
    const T* wr = w + (int64_t)co * a.ldw;
    float acc = 0.0f;
    for (int ci = 0; ci < a.cg; ++ci) {
      const T* xc = xg + (int64_t)ci * a.H * a.W;
      for (int ky = 0; ky < a.KH; ++ky) {
        int iy = oy * a.sh + ky * a.dh;
        if (a.pad_mode == 0) {
          iy -= a.pt;
          if ((unsigned)iy >= (unsigned)a.H) continue;
        } else {
          iy = pad_map(iy, a.pt, a.H, a.pad_mode);
        }
        for (int kx = 0; kx < a.KW; ++kx) {
          int ix = ox * a.sw + kx * a.dw;
          if (a.pad_mode == 0) {
            ix -= a.pl;
            if ((unsigned)ix >= (unsigned)a.W) continue;
          } else {
            ix = pad_map(ix, a.pl, a.W, a.pad_mode);
          }
          acc += to_f32(xc[(int64_t)iy * a.W + ix]) * to_f32(wr[(ky * a.KW + kx) * a.cpg + ci]);
        }
      }
    }
    float v = acc;
    if (bias) v = v + to_f32(bias[co]);
    v = activate_t<T>(v, a.act, a.lo, a.hi);
    const int64_t o = a.nhwc_out ? (((int64_t)n * a.OH + oy) * a.OW + ox) * a.ldo + co
                                 : (((int64_t)n * a.cout + co) * a.OH + oy) * a.OW + ox;
    y[o] = from_f32<T>(v);
  }
}

// ---------------------------------------------------------------- few output channels
constexpr int kFewTile = 16;   // output tile edge; one thread per output pixel

int fewout_slice(const DirectConvArgs& a) {
  const int ih = (kFewTile - 1) * a.sh + (a.KH - 1) * a.dh + 1, iw = (kFewTile - 1) * a.sw + (a.KW - 1) * a.dw + 1;
  const int per = ih * iw + (a.cout <= 4 ? 4 : kFewOutMax) * a.KH * a.KW;   // floats per input channel
  const int cs = (48 * 1024 / 4) / per;
  return std::max(1, std::min(cs, a.C));
}

template <class T, int CO, int KWC>   // KWC: the filter width when known at compile time (0: a.KW)
__global__ void __launch_bounds__(256) conv_fewout_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                          float* __restrict__ ws, DirectConvArgs a, int cslice) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ f32x4 fsm4[];
  float* fsm = reinterpret_cast<float*>(fsm4);
  const int IH = (kFewTile - 1) * a.sh + (a.KH - 1) * a.dh + 1, IW = (kFewTile - 1) * a.sw + (a.KW - 1) * a.dw + 1;
  const int KK = a.KH * a.KW;
  const int tiles_x = (a.OW + kFewTile - 1) / kFewTile;
  const int ox0 = (int)(blockIdx.x % tiles_x) * kFewTile, oy0 = (int)(blockIdx.x / tiles_x) * kFewTile;
  const int ci0 = blockIdx.y * cslice, n = blockIdx.z;
  const int cs = min(cslice, a.C - ci0);
  // weights first, [ci][tap][CO] (CO consecutive floats: one broadcast read
  // per tap and 4 outputs), then the input patch [ci][IH][IW]
  f32x4* wsm = fsm4;
  float* xs = fsm + cslice * KK * CO;
  const T* xn = x + ((int64_t)n * a.C + ci0) * a.H * a.W;
  // Both staging loops issue their global loads in batches of 8 before any
  // LDS store, so a thread's loads overlap instead of each waiting a round
  // trip.
  constexpr int B = 8;
  const int nw = cs * KK * CO;
  for (int base = threadIdx.x; base < nw; base += 256 * B) {
    float v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int idx = base + u * 256;
      const int co = idx % CO, r = idx / CO;
      const int t = r % KK, ci = r / KK;
      v[u] = idx < nw && co < a.cout ? to_f32(w[(int64_t)co * a.ldw + t * a.cpg + ci0 + ci]) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (base + u * 256 < nw) fsm[base + u * 256] = v[u];
  }
  // the input patch of the tile (padded positions as the direct kernel reads them)
  const int nx = cs * IH * IW;
  for (int base = threadIdx.x; base < nx; base += 256 * B) {
    float v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int idx = base + u * 256;
      const int ci = idx / (IH * IW), r = idx - ci * (IH * IW);
      const int yy = r / IW, xx = r - yy * IW;
      int iy = oy0 * a.sh + yy, ix = ox0 * a.sw + xx;
      bool ok = idx < nx;
      if (a.pad_mode == 0) {
        iy -= a.pt;
        ix -= a.pl;
        ok = ok && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
      } else {
        iy = pad_map(iy, a.pt, a.H, a.pad_mode);
        ix = pad_map(ix, a.pl, a.W, a.pad_mode);
      }
      v[u] = ok ? to_f32(xn[((int64_t)ci * a.H + iy) * a.W + ix]) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (base + u * 256 < nx) xs[base + u * 256] = v[u];
  }
  __syncthreads();
  const int tx = threadIdx.x % kFewTile, ty = threadIdx.x / kFewTile;
  const int ox = ox0 + tx, oy = oy0 + ty;
  f32x4 acc[CO / 4];
#pragma unroll
  for (int q = 0; q < CO / 4; ++q) acc[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int ci = 0; ci < cs; ++ci) {
    const float* xc = xs + ci * IH * IW + (ty * a.sh) * IW + tx * a.sw;
    const f32x4* wc = wsm + ci * KK * (CO / 4);
    for (int ky = 0; ky < a.KH; ++ky) {
      const float* xr = xc + ky * a.dh * IW;
      const f32x4* wr = wc + ky * a.KW * (CO / 4);
      if constexpr (KWC > 0) {
        // a whole filter row: independent LDS reads, then the FMAs
        float v[KWC];
#pragma unroll
        for (int kx = 0; kx < KWC; ++kx) v[kx] = xr[kx * a.dw];
#pragma unroll
        for (int kx = 0; kx < KWC; ++kx)
#pragma unroll
          for (int q = 0; q < CO / 4; ++q) acc[q] += v[kx] * wr[kx * (CO / 4) + q];
      } else {
        for (int kx = 0; kx < a.KW; ++kx) {
          const float v = xr[kx * a.dw];
#pragma unroll
          for (int q = 0; q < CO / 4; ++q) acc[q] += v * wr[kx * (CO / 4) + q];
        }
      }
    }
  }
  if (ox < a.OW && oy < a.OH) {
    const int64_t plane = (int64_t)a.OH * a.OW;
    float* wp = ws + (((int64_t)blockIdx.y * a.N + n) * a.cout) * plane + (int64_t)oy * a.OW + ox;
#pragma unroll
    for (int co = 0; co < CO; ++co)
      if (co < a.cout) wp[co * plane] = acc[co / 4][co % 4];
  }
}

template <class T>
__global__ void __launch_bounds__(256) fewout_reduce_kernel(const float* __restrict__ ws, const T* __restrict__ bias,
                                                            T* __restrict__ y, DirectConvArgs a, int slices) {
  const int64_t plane = (int64_t)a.OH * a.OW, total = (int64_t)a.N * a.cout * plane;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    // each group of eight slices loaded before its adds (one round trip per
    // group); the adds stay in slice order, slice 0 starts the sum
    float v;
    for (int s0 = 0; s0 < slices; s0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < slices) t[u] = ws[(int64_t)(s0 + u) * total + idx];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < slices) v = s0 + u == 0 ? t[u] : v + t[u];
    }
    const int64_t p = idx % plane, nc = idx / plane;
    const int co = (int)(nc % a.cout), n = (int)(nc / a.cout);
    if (bias) v = v + to_f32(bias[co]);
    v = activate_t<T>(v, a.act, a.lo, a.hi);
    const int64_t o = a.nhwc_out ? ((int64_t)n * plane + p) * a.ldo + co : idx;
    y[o] = from_f32<T>(v);
  }
}

hipError_t run_conv_fewout(int dtype, const void* x, const void* w, const void* bias, void* y, float* ws,
                           const DirectConvArgs& a, int cslice, hipStream_t st) {
  if (a.cout > kFewOutMax || cslice < 1) return hipErrorInvalidValue;
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  if (total <= 0) return hipSuccess;
  const int slices = (a.C + cslice - 1) / cslice;
  const int IH = (kFewTile - 1) * a.sh + (a.KH - 1) * a.dh + 1, IW = (kFewTile - 1) * a.sw + (a.KW - 1) * a.dw + 1;
  const int co = a.cout <= 4 ? 4 : kFewOutMax;
  const size_t lds = (size_t)cslice * (IH * IW + co * a.KH * a.KW) * 4;
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(((a.OW + kFewTile - 1) / kFewTile) * ((a.OH + kFewTile - 1) / kFewTile)), (unsigned)slices,
                  (unsigned)a.N);
  const unsigned rgrid = (unsigned)std::min<int64_t>((total + 255) / 256, 65535 * 16);
#define OHIP_FEW_KW(T, CO)                                                                                             \
  switch (a.KW) {                                                                                                       \
    case 3: hipLaunchKernelGGL((conv_fewout_kernel<T, CO, 3>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(x), \
                               reinterpret_cast<const T*>(w), ws, a, cslice); break;                                  \
    case 5: hipLaunchKernelGGL((conv_fewout_kernel<T, CO, 5>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(x), \
                               reinterpret_cast<const T*>(w), ws, a, cslice); break;                                  \
    case 7: hipLaunchKernelGGL((conv_fewout_kernel<T, CO, 7>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(x), \
                               reinterpret_cast<const T*>(w), ws, a, cslice); break;                                  \
    default: hipLaunchKernelGGL((conv_fewout_kernel<T, CO, 0>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(x),\
                                reinterpret_cast<const T*>(w), ws, a, cslice); break;                                 \
  }
#define OHIP_FEW(T)                                                                                                    \
  if (co == 4) { OHIP_FEW_KW(T, 4) }                                                                                    \
  else { OHIP_FEW_KW(T, 8) }                                                                                            \
  hipLaunchKernelGGL(fewout_reduce_kernel<T>, dim3(rgrid), dim3(256), 0, st, ws, reinterpret_cast<const T*>(bias),   \
                     reinterpret_cast<T*>(y), a, slices)
  switch (dtype) {
    case DT_F32: OHIP_FEW(float); break;
    case DT_F16: OHIP_FEW(_Float16); break;
    case DT_BF16: OHIP_FEW(__bf16); break;
    default: return hipErrorInvalidValue;
  }
#undef OHIP_FEW
#undef OHIP_FEW_KW
  return hipGetLastError();
}

// Few output channels on the MFMA: an ungrouped stride-1 KH x KW
// convolution of an NHWC f16 / bf16 input (an RGB head) whose 1-4 output
// channels would fill a sliver of the engine's 64-column tiles, each tap
// re-gathering its pixels from global memory.  A block takes one output row
// (up to 128 pixels, a wave per 32) and a slice of input channels: per slab
// of 16 channels it stages the row's input patch once, KH rows of OW + KW -
// 1 pixels, with the zero / reflect / edge border applied by the loader, and
// every tap reads its A fragments (32 pixels x 16 channels) from the patch
// at pixel offset kx.  The slice's filter sits in LDS for the valid output
// channels only; the other B columns are zero registers.  The slice's sums
// go to the same partial-sum layout as the few-output kernel, whose
// reduction adds the slices in order and applies bias and activation.
constexpr int kFewCoMax = 4;        // output channels (B columns) kept
constexpr int kFewCoSlab = 16;      // channels per slab (one k-step of a tap)

template <Op O, class T, int KH, int KW>
__global__ void __launch_bounds__(256) fewco_mfma_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                         float* __restrict__ ws, DirectConvArgs a, int pitch,
                                                         int cslice) {
  constexpr int TAPS = KH * KW;
  extern __shared__ u32x4 fsm[];
  const int PW = a.OW + KW - 1;
  const int slabs = cslice / kFewCoSlab;
  u32x4* pat = fsm;                                 // [KH][PW][2] chunks
  u32x4* wl = fsm + KH * PW * 2;                    // [slab][tap][2][kFewCoMax]
  const int n = (int)blockIdx.x / a.OH, oy = (int)blockIdx.x % a.OH;
  const int c0 = (int)blockIdx.y * cslice;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int m = lane & 31, hh = lane >> 5;
  const int nw = slabs * TAPS * 2 * kFewCoMax;
  for (int base = t; base < nw; base += 256 * 4) {   // four loads in flight a thread
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = base + u * 256;
      const int co = i % kFewCoMax;
      int r = i / kFewCoMax;
      const int h = r & 1;
      r >>= 1;
      const int tap = r % TAPS, sl = r / TAPS;
      v[u] = i < nw && co < a.cout
                 ? *reinterpret_cast<const u32x4*>(w + co * a.ldw + (int64_t)tap * a.cpg + c0 + sl * kFewCoSlab + h * 8)
                 : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (base + u * 256 < nw) wl[base + u * 256] = v[u];
  }
  // taps alternate over kChains independent accumulators (one chain of
  // dependent MFMAs would wait out each one's latency)
  constexpr int kChains = 4;
  typename OpT<O>::Acc acc[kChains];
#pragma unroll
  for (int j = 0; j < kChains; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
  const int px0 = wave * 32;
  const T* xn = x + (int64_t)n * a.H * a.W * pitch;
  const int np = KH * PW * 2;
  for (int sl = 0; sl < slabs; ++sl) {
    __syncthreads();   // the previous slab's patch has been read (the filter written, for slab 0)
    const int cc = c0 + sl * kFewCoSlab;
    // the patch's loads are issued in batches of 8 before any LDS store, so
    // a thread's loads overlap instead of each waiting a round trip
    constexpr int B = 8;
    for (int base = t; base < np; base += 256 * B) {
      u32x4 v[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int i = base + u * 256;
        const int h = i & 1, r = i >> 1;
        const int px = r % PW, ky = r / PW;
        int iy = oy + ky, ix = px;   // padded coordinates
        bool ok = i < np;
        if (a.pad_mode == 0) {
          iy -= a.pt;
          ix -= a.pl;
          ok = ok && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
        } else {
          iy = pad_map(iy, a.pt, a.H, a.pad_mode);
          ix = pad_map(ix, a.pl, a.W, a.pad_mode);
        }
        v[u] = ok ? *reinterpret_cast<const u32x4*>(xn + ((int64_t)iy * a.W + ix) * pitch + cc + h * 8)
                  : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < B; ++u)
        if (base + u * 256 < np) pat[base + u * 256] = v[u];
    }
    __syncthreads();
    if (px0 < a.OW) {
      const u32x4* wsl = wl + sl * TAPS * 2 * kFewCoMax;
#pragma unroll
      for (int ky = 0; ky < KH; ++ky)
#pragma unroll
        for (int kx = 0; kx < KW; ++kx) {
          const u32x4 av = pat[((ky * PW) + px0 + m + kx) * 2 + hh];
          const u32x4 bv = m < a.cout ? wsl[((ky * KW + kx) * 2 + hh) * kFewCoMax + m] : u32x4{0u, 0u, 0u, 0u};
          acc[(ky * KW + kx) % kChains] = OpT<O>::mma(av, bv, acc[(ky * KW + kx) % kChains]);
        }
    }
  }
#pragma unroll
  for (int j = 1; j < kChains; ++j) acc[0] += acc[j];
  // lane: pixels px0 + 8g + 4hh + e (rows of A), output channel m (column of B)
  if (px0 < a.OW && m < a.cout) {
    const int64_t plane = (int64_t)a.OH * a.OW;
    float* dst = ws + (((int64_t)blockIdx.y * a.N + n) * a.cout + m) * plane + (int64_t)oy * a.OW;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int px = px0 + 8 * g + 4 * hh + e;
        if (px < a.OW) dst[px] = acc[0][4 * g + e];
      }
  }
}

int fewco_slice(const DirectConvArgs& a) {
  // enough slices to give every CU about two blocks, at least one slab each
  const int64_t rows = (int64_t)a.N * a.OH;
  int slabs = a.C / kFewCoSlab, s = 1;
  while (s < slabs && rows * s < 512 && slabs % (2 * s) == 0) s *= 2;
  return a.C / s;
}

bool fewco_supported(int dtype, const DirectConvArgs& a, int pitch) {
  if (dtype != DT_F16 && dtype != DT_BF16) return false;
  if (a.cout > kFewCoMax || a.cout < 1 || a.OW > 128 || a.sh != 1 || a.sw != 1 || a.dh != 1 || a.dw != 1) return false;
  if (a.KH != a.KW || (a.KH != 3 && a.KH != 5 && a.KH != 7)) return false;
  if (a.C % kFewCoSlab != 0 || pitch % 8 != 0 || a.cpg % 8 != 0 || a.ldw % 8 != 0) return false;
  const size_t lds = ((size_t)a.KH * (a.OW + a.KW - 1) * 2 + (size_t)(fewco_slice(a) / kFewCoSlab) * a.KH * a.KW * 2 * kFewCoMax) * 16;
  return lds <= 64 * 1024;
}

hipError_t run_conv_fewco(int dtype, const void* x, int pitch, const void* w, const void* bias, void* y, float* ws,
                          const DirectConvArgs& a, hipStream_t st) {
  if (!fewco_supported(dtype, a, pitch)) return hipErrorInvalidValue;
  const int cslice = fewco_slice(a);
  const int slices = a.C / cslice;
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  if (total <= 0) return hipSuccess;
  const size_t lds = ((size_t)a.KH * (a.OW + a.KW - 1) * 2 + (size_t)(cslice / kFewCoSlab) * a.KH * a.KW * 2 * kFewCoMax) * 16;
  const dim3 grid((unsigned)(a.N * a.OH), (unsigned)slices);
  const unsigned rgrid = (unsigned)std::min<int64_t>((total + 255) / 256, 65535 * 16);
#define OHIP_FEWCO(OP, T)                                                                                         \
  switch (a.KH) {                                                                                                 \
    case 3: hipLaunchKernelGGL((fewco_mfma_kernel<OP, T, 3, 3>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(x), \
                               reinterpret_cast<const T*>(w), ws, a, pitch, cslice); break;                         \
    case 5: hipLaunchKernelGGL((fewco_mfma_kernel<OP, T, 5, 5>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(x), \
                               reinterpret_cast<const T*>(w), ws, a, pitch, cslice); break;                         \
    default: hipLaunchKernelGGL((fewco_mfma_kernel<OP, T, 7, 7>), grid, dim3(256), lds, st, reinterpret_cast<const T*>(x), \
                                reinterpret_cast<const T*>(w), ws, a, pitch, cslice); break;                        \
  }                                                                                                               \
  hipLaunchKernelGGL(fewout_reduce_kernel<T>, dim3(rgrid), dim3(256), 0, st, ws, reinterpret_cast<const T*>(bias), \
                     reinterpret_cast<T*>(y), a, slices)
  if (dtype == DT_F16) { OHIP_FEWCO(Op::F16, _Float16); }
  else { OHIP_FEWCO(Op::BF16, __bf16); }
#undef OHIP_FEWCO
  return hipGetLastError();
}

// f32 stride-1 convolution straight from an NCHW input (config 1's shape):
// the f32 MFMA takes one element of each operand per lane, so a block can
// stage, per slab of 8 input channels, the channel-major input patch of its
// output row segment (KH rows of 64 + KW - 1 pixels, zero border) and the
// slab's filter ([64 output channels][taps x 8 channels]) in LDS and run every
// tap from the patch at pixel offset kx: no NHWC staging transpose, and the
// input is fetched once per slab instead of once per tap.  A block is one
// 64-pixel segment of an output row x 64 output channels, four waves of
// 32 x 32; the next slab's loads are issued into registers before the
// current slab's MFMAs and stored after them (two LDS buffers).  k runs
// (tap, channel): MFMA step j covers k = 2j, 2j + 1, one tap and channels
// 2j % 8 + {0, 1}, so both operands' addresses are a per-lane base plus a
// compile-time offset.
constexpr int kF32Seg = 64, kF32Co = 64, kF32Cs = 8;

template <int KH, int KW, bool MAPPED>
__global__ void __launch_bounds__(256) conv_nchw_f32_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            const float* __restrict__ bias, float* __restrict__ y,
                                                            DirectConvArgs a) {
  constexpr int TAPS = KH * KW, KS = TAPS * kF32Cs;           // k per slab
  constexpr int PWP = kF32Seg + KW - 1;                       // patch row
  constexpr int PATCH = kF32Cs * KH * PWP;                    // floats
  constexpr int FST = KS + 1;                                 // filter row stride (odd: no bank conflicts)
  constexpr int FILT = kF32Co * FST;
  constexpr int NP = (PATCH + 255) / 256, NF = (kF32Co * TAPS * 2 + 255) / 256;
  __shared__ float lds[2][PATCH + FILT];
  const int segs = (a.OW + kF32Seg - 1) / kF32Seg;
  const int seg = (int)blockIdx.x % segs;
  const int oy = ((int)blockIdx.x / segs) % a.OH, n = (int)blockIdx.x / segs / a.OH;
  const int co0 = (int)blockIdx.y * kF32Co, ox0 = seg * kF32Seg;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wp = wave & 1, wq = wave >> 1, m = lane & 31, kk = lane >> 5;
  const float* xn = x + (int64_t)n * a.C * a.H * a.W;
  const int slabs = (a.C + kF32Cs - 1) / kF32Cs;

  float pv[NP];
  f32x4 fv[NF];
  auto load = [&](int sl) __attribute__((always_inline)) {
    const int c0 = sl * kF32Cs;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int i = t + u * 256;
      const int px = i % PWP, r = i / PWP, ky = r % KH, c = r / KH;
      int iy = oy + ky, ix = ox0 + px;   // padded coordinates
      bool ok = i < PATCH && c0 + c < a.C;
      if constexpr (!MAPPED) {
        iy -= a.pt;
        ix -= a.pl;
        ok = ok && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W;
      } else {
        iy = pad_map(iy, a.pt, a.H, a.pad_mode);
        ix = pad_map(ix, a.pl, a.W, a.pad_mode);
      }
      pv[u] = ok ? xn[((int64_t)(c0 + c) * a.H + iy) * a.W + ix] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < NF; ++u) {
      const int i = t + u * 256;        // (co, tap, half)
      const int h = i & 1, r = i >> 1, tap = r % TAPS, co = r / TAPS;
      const bool ok = i < kF32Co * TAPS * 2 && co0 + co < a.cout && c0 + 4 * h < a.cpg;
      fv[u] = ok ? *reinterpret_cast<const f32x4*>(w + (int64_t)(co0 + co) * a.ldw + (int64_t)tap * a.cpg + c0 + 4 * h)
                 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  auto store = [&](int b) __attribute__((always_inline)) {
    float* pd = lds[b];
    float* fd = lds[b] + PATCH;
#pragma unroll
    for (int u = 0; u < NP; ++u)
      if (t + u * 256 < PATCH) pd[t + u * 256] = pv[u];
#pragma unroll
    for (int u = 0; u < NF; ++u) {
      const int i = t + u * 256;
      if (i < kF32Co * TAPS * 2) {
        const int h = i & 1, r = i >> 1, tap = r % TAPS, co = r / TAPS;
        float* d = fd + co * FST + tap * kF32Cs + 4 * h;
        d[0] = fv[u][0]; d[1] = fv[u][1]; d[2] = fv[u][2]; d[3] = fv[u][3];
      }
    }
  };

  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
  const int abase = kk * KH * PWP + wp * 32 + m;   // channel kk of the pair, this lane's pixel
  const int bbase = (wq * 32 + m) * FST + kk;
  load(0);
  store(0);
  __syncthreads();
  for (int sl = 0; sl < slabs; ++sl) {
    const int b = sl & 1;
    if (sl + 1 < slabs) load(sl + 1);
    const float* pa = lds[b] + abase;
    const float* pb = lds[b] + PATCH + bbase;
#pragma unroll
    for (int j = 0; j < KS / 2; ++j) {
      const int tap = (2 * j) / kF32Cs, cp2 = (2 * j) % kF32Cs;
      const int ky = tap / KW, kx = tap % KW;
      const float av = pa[(cp2 * KH + ky) * PWP + kx];
      const float bv = pb[2 * j];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
    }
    if (sl + 1 < slabs) store(b ^ 1);
    __syncthreads();
  }
  // lane: pixels wp * 32 + 8g + 4kk + e, output channel wq * 32 + m
  const int co = co0 + wq * 32 + m;
  if (co >= a.cout) return;
  const float bi = bias ? bias[co] : -0.0f;
  float* yr = y + (((int64_t)n * a.cout + co) * a.OH + oy) * a.OW;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int px = ox0 + wp * 32 + 8 * g + 4 * kk;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = activate(acc[4 * g + e] + bi, a.act, a.lo, a.hi);
    if (px + 3 < a.OW && (a.OW & 3) == 0) {
      *reinterpret_cast<f32x4*>(yr + px) = f32x4{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (px + e < a.OW) yr[px + e] = v[e];
    }
  }
}

bool conv_nchw_f32_supported(const DirectConvArgs& a) {
  return a.KH == a.KW && (a.KH == 3 || (a.KH == 1 && a.pad_mode == 0)) && a.sh == 1 && a.sw == 1 && a.dh == 1 && a.dw == 1 &&
         !a.nhwc_out && a.cpg % 4 == 0 && a.ldw % 4 == 0;
}

hipError_t run_conv_nchw_f32(const float* x, const float* w, const float* bias, float* y, const DirectConvArgs& a,
                             hipStream_t st) {
  if (!conv_nchw_f32_supported(a)) return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)a.N * a.OH * ((a.OW + kF32Seg - 1) / kF32Seg);
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks, (unsigned)((a.cout + kF32Co - 1) / kF32Co));
  if (a.KH == 3 && a.pad_mode != 0)
    hipLaunchKernelGGL((conv_nchw_f32_kernel<3, 3, true>), grid, dim3(256), 0, st, x, w, bias, y, a);
  else if (a.KH == 3)
    hipLaunchKernelGGL((conv_nchw_f32_kernel<3, 3, false>), grid, dim3(256), 0, st, x, w, bias, y, a);
  else
    hipLaunchKernelGGL((conv_nchw_f32_kernel<1, 1, false>), grid, dim3(256), 0, st, x, w, bias, y, a);
  return hipGetLastError();
}

// Depthwise 3x3 (one input channel per output channel, zero padding,
// stride 1 or 2, no dilation): a block takes a band of `rows` output rows of
// one plane, stages the band's input window in LDS as f32 (one coalesced
// read of each input row instead of nine cached reads per output), keeps
// the nine weights in registers, and finishes each output exactly as
// conv_direct_kernel does: taps in (ky, kx) order with the ones outside the
// image skipped, + bias, activation.
constexpr int kDwLds = 8192;   // floats of staged window per block (32 KiB)

// Divisions of the depthwise kernel by the window width and by the runs of
// four outputs a row (magic_div multipliers: a multiply-high and a shift).
struct DwDiv {
  uint32_t cw_mul, rpr_mul, cpr_mul;
  int cw_shift, rpr_shift, cpr_shift;
  int vec_in;   // image rows of whole 16-byte chunks, 16-byte aligned: chunk loads
};

template <class T, int S>
__global__ void __launch_bounds__(256)
conv_dw3_kernel(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias, T* __restrict__ y,
                DirectConvArgs a, int rows, DwDiv dd, int vec4) {
  extern __shared__ float win[];   // the band's window, RW x CW floats
  const int bands = (a.OH + rows - 1) / rows;
  const int band = (int)(blockIdx.x % bands);
  const int plane = (int)(blockIdx.x / bands);   // n * C + c
  const int co = plane % a.cout, n = plane / a.cout;
  const int oy0 = band * rows, nr = min(rows, a.OH - oy0);
  const int iy0 = oy0 * S - a.pt, ix0 = -a.pl;
  const int RW = (nr - 1) * S + 3, CW = (a.OW - 1) * S + 3;
  const T* xc = x + (int64_t)plane * a.H * a.W;
  auto udiv = [](int i, uint32_t mul, int shift) { return (int)(((uint64_t)(uint32_t)i * mul) >> shift); };
  // the window's loads issued in batches of B before their LDS stores, so
  // a thread's loads overlap instead of each waiting a round trip
  constexpr int B = 16;
  const int nw = RW * CW;
  if (dd.vec_in) {
    // the image part of each window row by 16-byte chunks (EPV elements),
    // the pad columns (and rows outside the image) as zeros
    constexpr int EPV = 16 / sizeof(T);
    typedef T tv __attribute__((ext_vector_type(EPV)));
    const int cpr = a.W / EPV, nc = RW * cpr;
    constexpr int BV = 4;
    for (int base = threadIdx.x; base < nc; base += 256 * BV) {
      tv v[BV];
#pragma unroll
      for (int u = 0; u < BV; ++u) {
        const int i = base + u * 256;
        const int r = udiv(i, dd.cpr_mul, dd.cpr_shift), k = i - r * cpr;
        const int iy = iy0 + r;
        v[u] = tv{};
        if (i < nc && (unsigned)iy < (unsigned)a.H)
          v[u] = *reinterpret_cast<const tv*>(xc + (int64_t)iy * a.W + k * EPV);
      }
#pragma unroll
      for (int u = 0; u < BV; ++u) {
        const int i = base + u * 256;
        if (i >= nc) break;
        const int r = udiv(i, dd.cpr_mul, dd.cpr_shift), k = i - r * cpr;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          const int c = a.pl + k * EPV + e;
          if (c < CW) win[r * CW + c] = to_f32(v[u][e]);
        }
      }
    }
    const int right = CW - a.pl - a.W > 0 ? CW - a.pl - a.W : 0, np = a.pl + right;
    for (int i = threadIdx.x; i < RW * np; i += 256) {
      const int r = i / np, j = i - r * np;
      win[r * CW + (j < a.pl ? j : a.W + j)] = 0.0f;
    }
  } else
  for (int base = threadIdx.x; base < nw; base += 256 * B) {
    float v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int i = base + u * 256;
      const int r = udiv(i, dd.cw_mul, dd.cw_shift), c = i - r * CW;
      const int iy = iy0 + r, ix = ix0 + c;
      v[u] = i < nw && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W
                 ? to_f32(xc[(int64_t)iy * a.W + ix]) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (base + u * 256 < nw) win[base + u * 256] = v[u];
  }
  float wk[9];
  const T* wr = w + (int64_t)co * a.ldw;
#pragma unroll
  for (int k = 0; k < 9; ++k) wk[k] = to_f32(wr[k * a.cpg]);
  const float bv = bias ? to_f32(bias[co]) : 0.0f;
  __syncthreads();
  // runs of four outputs of a row: one 3 x (3 S + 3) patch of the window,
  // each output's taps still summed in (ky, kx) order
  constexpr int PW = 3 * S + 3;
  const int rpr = (a.OW + 3) / 4;
  for (int i = threadIdx.x; i < nr * rpr; i += 256) {
    const int r = udiv(i, dd.rpr_mul, dd.rpr_shift), ox0 = (i - r * rpr) * 4, oy = oy0 + r;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool interior = ox0 * S - a.pl >= 0 && (ox0 + 3) * S + 2 - a.pl < a.W;
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
      const int iy = oy * S + ky - a.pt;
      if ((unsigned)iy >= (unsigned)a.H) continue;
      const float* wrow = win + (r * S + ky) * CW + ox0 * S;
      float pv[PW];
#pragma unroll
      for (int j = 0; j < PW; ++j) pv[j] = ox0 * S + j < CW ? wrow[j] : 0.0f;
      if (interior) {   // every tap of the run inside the image: no per-tap checks
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int kx = 0; kx < 3; ++kx) acc[e] += pv[e * S + kx] * wk[ky * 3 + kx];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int kx = 0; kx < 3; ++kx) {
            const int ix = (ox0 + e) * S + kx - a.pl;
            if ((unsigned)ix < (unsigned)a.W) acc[e] += pv[e * S + kx] * wk[ky * 3 + kx];
          }
      }
    }
    if (vec4 && ox0 + 3 < a.OW) {   // NCHW, four aligned outputs: one store
      typedef T t4 __attribute__((ext_vector_type(4)));
      t4 o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[e];
        if (bias) v = v + bv;
        o4[e] = from_f32<T>(activate_t<T>(v, a.act, a.lo, a.hi));
      }
      *reinterpret_cast<t4*>(y + (((int64_t)n * a.cout + co) * a.OH + oy) * a.OW + ox0) = o4;
      continue;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ox = ox0 + e;
      if (ox >= a.OW) break;
      float v = acc[e];
      if (bias) v = v + bv;
      v = activate_t<T>(v, a.act, a.lo, a.hi);
      const int64_t o = a.nhwc_out ? (((int64_t)n * a.OH + oy) * a.OW + ox) * a.ldo + co
                                   : (((int64_t)n * a.cout + co) * a.OH + oy) * a.OW + ox;
      y[o] = from_f32<T>(v);
    }
  }
}

// Output rows per band of the depthwise kernel (from 2^18 outputs): bands small enough for
// about five blocks per CU (a block is a short serial chain of window load,
// sums and stores; 128 blocks of 36 rows ran 9.6 us on 64 planes of 56x56),
// at most about eight outputs a thread, within the window's LDS budget;
// 0 when the geometry is not its.
inline int dw3_rows(const DirectConvArgs& a) {
  // OHIP_DW3=0 keeps these convolutions on conv_direct_kernel (a measurement switch)
  static const bool on = [] { const char* e = std::getenv("OHIP_DW3"); return !(e && e[0] == '0'); }();
  if (!on) return 0;
  if (!(a.cg == 1 && a.coutg == 1 && a.KH == 3 && a.KW == 3 && a.dh == 1 && a.dw == 1 && a.sh == a.sw &&
        (a.sh == 1 || a.sh == 2) && a.pad_mode == 0 && a.OW > 0 && a.OH > 0))
    return 0;
  // below about 2^18 outputs the one-thread-per-output kernel is faster
  // (64 planes of 56x56: 5.3 against 5.7 us, 256 of 28x28: 5.2 against 6.9;
  // 128 planes of 56x56: 6.9 against 5.9, 256: 10.2 against 6.3, 1024: 30.3
  // against 12.3, 256 of 224x224: 145 against 29)
  if ((int64_t)a.N * a.cout * a.OH * a.OW < (1 << 18)) return 0;
  const int CW = (a.OW - 1) * a.sh + 3;
  const int max_rows = (kDwLds / CW - 3) / a.sh + 1;
  if (max_rows < 1) return 0;
  const int64_t planes = (int64_t)a.N * a.cout;
  const int64_t fill = std::max<int64_t>(1, (int64_t)a.OH * planes / 1280);
  return (int)std::max<int64_t>(1, std::min<int64_t>({(int64_t)a.OH, (int64_t)max_rows, 2048 / a.OW, fill}));
}

hipError_t run_conv_direct(int dtype, const void* x, const void* w, const void* bias, void* y,
                           const DirectConvArgs& a, hipStream_t st) {
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  if (total <= 0) return hipSuccess;
  if (const int rows = dw3_rows(a)) {
    const int64_t blocks = (int64_t)a.N * a.cout * ((a.OH + rows - 1) / rows);
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const size_t lds = (size_t)((rows - 1) * a.sh + 3) * ((a.OW - 1) * a.sh + 3) * sizeof(float);
    DwDiv dd{};
    magic_div((a.OW - 1) * a.sh + 3, &dd.cw_mul, &dd.cw_shift);
    magic_div((a.OW + 3) / 4, &dd.rpr_mul, &dd.rpr_shift);
    const int epv = dtype == DT_F32 ? 4 : 8;
    dd.vec_in = a.W % epv == 0 && (uintptr_t)x % 16 == 0 && a.pl >= 0 && a.pl <= 2;
    magic_div(std::max(1, a.W / epv), &dd.cpr_mul, &dd.cpr_shift);
    // NCHW rows of whole runs of four, 4-element aligned: vector stores
    const int vec4 = !a.nhwc_out && a.OW % 4 == 0 && (uintptr_t)y % (4 * (dtype == DT_F32 ? 4 : 2)) == 0;
#define OHIP_DW(T, S)                                                                                            \
  hipLaunchKernelGGL((conv_dw3_kernel<T, S>), dim3((unsigned)blocks), dim3(256), lds, st,                        \
                     reinterpret_cast<const T*>(x), reinterpret_cast<const T*>(w), reinterpret_cast<const T*>(bias), \
                     reinterpret_cast<T*>(y), a, rows, dd, vec4)
#define OHIP_DW_S(T) if (a.sh == 1) OHIP_DW(T, 1); else OHIP_DW(T, 2)
    switch (dtype) {
      case DT_F32: OHIP_DW_S(float); break;
      case DT_F16: OHIP_DW_S(_Float16); break;
      case DT_BF16: OHIP_DW_S(__bf16); break;
      default: return hipErrorInvalidValue;
    }
#undef OHIP_DW_S
#undef OHIP_DW
    return hipGetLastError();
  }
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65535 * 16);
#define OHIP_DIRECT(T)                                                                                      \
  hipLaunchKernelGGL(conv_direct_kernel<T>, dim3(grid), dim3(256), 0, st, reinterpret_cast<const T*>(x), \
                     reinterpret_cast<const T*>(w), reinterpret_cast<const T*>(bias), reinterpret_cast<T*>(y), a)
  switch (dtype) {
    case DT_F32: OHIP_DIRECT(float); break;
    case DT_F16: OHIP_DIRECT(_Float16); break;
    case DT_BF16: OHIP_DIRECT(__bf16); break;
    default: return hipErrorInvalidValue;
  }
#undef OHIP_DIRECT
  return hipGetLastError();
}

// Integer counterpart for narrow groups: exact int32 sum of
// (x - x_zp) * (w - w_zp) over the group's taps (padding taps skipped, as in
// integer_conv), the packed filter decoded as stored (two int8 halves when
// the rows are split, negated for a flipped channel), + bias, then the
// output kind's epilogue: raw int32, or requantisation (f64 product with the
// f32 combined scale, + y_zp, round half to even, clamp), optionally mapped
// through the 256-entry byte table, stored as a byte or as an f32 lane.
__global__ void __launch_bounds__(256)
qconv_direct_kernel(const uint8_t* __restrict__ x, const int8_t* __restrict__ w, void* __restrict__ y,
                    DirectQConvArgs a) {
#pragma clang fp contract(off)
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    int ox, oy, co, n;
    split_out_index(idx, total, a.OW, a.OH, a.cout, ox, oy, co, n);
    const int g = co / a.coutg;
    const uint8_t* xg = x + ((int64_t)n * a.C + (int64_t)g * a.cg) * a.H * a.W;
    const int8_t* wr = w + (int64_t)co * a.ldw;
    int32_t acc = 0;
    for (int ci = 0; ci < a.cg; ++ci) {
      const uint8_t* xc = xg + (int64_t)ci * a.H * a.W;
      for (int ky = 0; ky < a.KH; ++ky) {
        const int iy = oy * a.sh - a.pt + ky * a.dh;
        if ((unsigned)iy >= (unsigned)a.H) continue;
        for (int kx = 0; kx < a.KW; ++kx) {
          const int ix = ox * a.sw - a.pl + kx * a.dw;
          if ((unsigned)ix >= (unsigned)a.W) continue;
          const uint8_t raw = xc[(int64_t)iy * a.W + ix];
          const int32_t xv = (a.x_signed ? (int32_t)(int8_t)raw : (int32_t)raw) - a.x_zp;
          const int64_t k = (int64_t)(ky * a.KW + kx) * a.cpg + ci;
          int32_t v = wr[k];
          if (a.half) v += wr[a.half + k];
          acc += xv * v;
        }
      }
    }
    if (a.flip && a.flip[co]) acc = -acc;
    if (a.bias) acc += a.bias[co];
    const int64_t o = a.nhwc_out ? (((int64_t)n * a.OH + oy) * a.OW + ox) * a.ldo + co
                                 : (((int64_t)n * a.cout + co) * a.OH + oy) * a.OW + ox;
    if (a.out_kind == QOUT_I32) {
      reinterpret_cast<int32_t*>(y)[o] = acc;
      continue;
    }
    double d = (double)acc * (double)a.comb[a.n_comb > 1 ? co : 0];
    d = d + (double)a.y_zp;
    d = __builtin_rint(d);
    d = d < (double)a.lo ? (double)a.lo : d;
    d = d > (double)a.hi ? (double)a.hi : d;
    const int32_t q = (int32_t)d;
    if (a.out_kind == QOUT_F32) {
      reinterpret_cast<float*>(y)[o] = (float)q;
    } else {
      reinterpret_cast<uint8_t*>(y)[o] = a.table ? a.table[q & 0xff] : (uint8_t)(q & 0xff);
    }
  }
}

// An ungrouped convolution with few taps x channels (an RGB stem: 3 channels
// x 3x3) on an NCHW byte image.  A block computes a kStemTH x kStemTW tile of
// output pixels, a thread one pixel and every output channel:
//   * the input patch the tile reads is staged in LDS with 4-byte loads (rows
//     of the image are 4-byte aligned), a padding position holding the zero
//     point byte, so that its (x - x_zp) term is exactly zero ("padding taps
//     are skipped");
//   * the filter sits in LDS as int16 in [tap][channel] order (the two halves
//     of a split row already summed, flipped channels negated), read as
//     16-byte broadcast vectors;
//   * the byte table of a fused tail is copied into LDS;
//   * the epilogue is qconv_direct_kernel's; sixteen byte channels of an NHWC
//     output leave as one 16-byte store.
constexpr int kStemTaps = 32, kStemCout = 64, kStemTH = 4, kStemTW = 64;
constexpr int kStemPatchBytes = 16384;

struct StemGeo {
  int PR, RB, ND;   // patch rows, bytes per staged row (ND dwords)
};

__global__ void __launch_bounds__(256)
qconv_stem_kernel(const uint8_t* __restrict__ x, const int8_t* __restrict__ w, void* __restrict__ y,
                  DirectQConvArgs a, StemGeo sg) {
#pragma clang fp contract(off)
  // filter as int16 pairs of consecutive taps: wl[(t / 2) * kStemCout + co]
  // holds taps t (low half) and t + 1 (high half) of channel co
  __shared__ __attribute__((aligned(16))) uint32_t wl[kStemTaps / 2 * kStemCout];
  __shared__ __attribute__((aligned(16))) uint32_t patch[kStemPatchBytes / 4];
  __shared__ int tap_off[kStemTaps];
  __shared__ uint8_t tab[256];
  __shared__ int32_t sbias[kStemCout];
  __shared__ float scomb[kStemCout];
  const int ntaps = a.cg * a.KH * a.KW;
  // per-channel epilogue terms in LDS: read from global memory inside the
  // channel loop they would be one scalar-load round trip per channel
  if (threadIdx.x < kStemCout) {
    const int co = threadIdx.x < a.cout ? threadIdx.x : 0;
    sbias[threadIdx.x] = a.bias ? a.bias[co] : 0;
    scomb[threadIdx.x] = a.out_kind == QOUT_I32 ? 0.0f : a.comb[a.n_comb > 1 ? co : 0];
  }
  const int kk = a.KH * a.KW;
  // filter staging: every load of the thread's eight entries is issued
  // before any is used (clamped addresses, masked afterwards), so the block
  // waits for one round trip, not eight
  {
    constexpr int PER = kStemTaps * kStemCout / 256;
    int8_t w0[PER], w1[PER], fl[PER];
    bool ok[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = threadIdx.x + j * 256;
      const int t = i / kStemCout, co = i - t * kStemCout;
      ok[j] = co < a.cout && t < ntaps;
      const int tt = ok[j] ? t : 0, cc = ok[j] ? co : 0;
      const int ci = tt / kk, r = tt - ci * kk, ky = r / a.KW, kx = r - ky * a.KW;
      const int8_t* wr = w + (int64_t)cc * a.ldw + (int64_t)(ky * a.KW + kx) * a.cpg + ci;
      w0[j] = wr[0];
      w1[j] = a.half ? wr[a.half] : (int8_t)0;
      fl[j] = a.flip ? a.flip[cc] : (int8_t)0;
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      int v = (int)w0[j] + (int)w1[j];
      if (fl[j]) v = -v;
      const int i = threadIdx.x + j * 256;
      const int t = i / kStemCout, co = i - t * kStemCout;
      reinterpret_cast<int16_t*>(wl)[2 * ((t >> 1) * kStemCout + co) + (t & 1)] = (int16_t)(ok[j] ? v : 0);
    }
  }
  if (threadIdx.x < kStemTaps) {
    const int t = threadIdx.x;
    int off = 0;
    if (t < ntaps) {
      const int ci = t / kk, r = t - ci * kk, ky = r / a.KW, kx = r - ky * a.KW;
      off = (ci * sg.PR + ky * a.dh) * sg.RB + kx * a.dw;
    }
    tap_off[t] = off;
  }
  if (a.table) tab[threadIdx.x] = a.table[threadIdx.x];

  // stage the input patch: rows iy0 .. iy0 + PR - 1 of every channel, image
  // columns A .. A + RB - 1 (A = the tile's first input column rounded down to
  // a multiple of 4)
  const int ox0 = blockIdx.x * kStemTW, oy0 = blockIdx.y * kStemTH, n = blockIdx.z;
  const int iy0 = oy0 * a.sh - a.pt, ixl = ox0 * a.sw - a.pl;
  const int A = ixl >= 0 ? (ixl & ~3) : -((-ixl + 3) & ~3);
  const uint8_t padb = (uint8_t)(a.x_zp & 0xff);
  const uint32_t pad4 = padb * 0x01010101u;
  const uint8_t* xn = x + (int64_t)n * a.C * a.H * a.W;
  const int total = a.C * sg.PR * sg.ND;
  // four dwords per thread and round, their loads issued together; a dword
  // that straddles the image's left or right edge is assembled bytewise
  for (int i0 = 0; i0 < total; i0 += 4 * 256) {
    uint32_t v[4];
    int slot[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * 256 + threadIdx.x;
      slot[j] = -1;
      v[j] = pad4;
      if (i < total) {
        const int d = i % sg.ND, cr = i / sg.ND, r = cr % sg.PR, c = cr / sg.PR;
        const int iy = iy0 + r, gx = A + 4 * d;
        slot[j] = (c * sg.PR + r) * (sg.RB / 4) + d;
        if ((unsigned)iy < (unsigned)a.H) {
          const uint8_t* row = xn + ((int64_t)c * a.H + iy) * a.W;
          if (gx >= 0 && gx + 3 < a.W) {
            v[j] = *reinterpret_cast<const uint32_t*>(row + gx);
          } else {
            uint32_t u = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              const int gxb = gx + b;
              const uint32_t byte = (gxb >= 0 && gxb < a.W) ? row[gxb] : padb;
              u |= byte << (8 * b);
            }
            v[j] = u;
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (slot[j] >= 0) patch[slot[j]] = v[j];
  }
  __syncthreads();

  const int ty = threadIdx.x / kStemTW, tx = threadIdx.x - ty * kStemTW;
  const int oy = oy0 + ty, ox = ox0 + tx;
  if (oy >= a.OH || ox >= a.OW) return;
  const uint8_t* pb = reinterpret_cast<const uint8_t*>(patch) + ty * a.sh * sg.RB + tx * a.sw + (ixl - A);
  // the taps as int16 pairs (|x - x_zp| <= 255), dotted with the filter pairs
  // by v_dot2 (two multiply-adds an instruction, exact in int32)
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  s16x2 xp[kStemTaps / 2];
#pragma unroll
  for (int t = 0; t < kStemTaps; t += 2) {
    const uint8_t r0 = t < ntaps ? pb[tap_off[t]] : padb;
    const uint8_t r1 = t + 1 < ntaps ? pb[tap_off[t + 1]] : padb;
    const int32_t x0 = (a.x_signed ? (int32_t)(int8_t)r0 : (int32_t)r0) - a.x_zp;
    const int32_t x1 = (a.x_signed ? (int32_t)(int8_t)r1 : (int32_t)r1) - a.x_zp;
    xp[t >> 1] = s16x2{(short)x0, (short)x1};
  }
  const int64_t p = ((int64_t)n * a.OH + oy) * a.OW + ox;
  const bool bytes = a.out_kind != QOUT_I32 && a.out_kind != QOUT_F32;
  for (int c0 = 0; c0 < a.cout; c0 += 16) {
    int32_t acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
    for (int tp = 0; tp < kStemTaps / 2; ++tp) {
      if (2 * tp < ntaps) {
        const uint32_t* wr = wl + tp * kStemCout + c0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 wv = *reinterpret_cast<const u32x4*>(wr + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t we = wv[e];   // by value: a bit_cast of the element expression itself reads lane 0
            acc[4 * q + e] = __builtin_amdgcn_sdot2(xp[tp], __builtin_bit_cast(s16x2, we), acc[4 * q + e], false);
          }
        }
      }
    }
    uint32_t words[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int co = c0 + e;
      if (co >= a.cout) break;
      const int32_t v = acc[e] + sbias[co];
      const int64_t o = a.nhwc_out ? p * a.ldo + co : (((int64_t)n * a.cout + co) * a.OH + oy) * a.OW + ox;
      if (a.out_kind == QOUT_I32) {
        reinterpret_cast<int32_t*>(y)[o] = v;
        continue;
      }
      double dd = (double)v * (double)scomb[co];
      dd = dd + (double)a.y_zp;
      dd = __builtin_rint(dd);
      dd = dd < (double)a.lo ? (double)a.lo : dd;
      dd = dd > (double)a.hi ? (double)a.hi : dd;
      const int32_t q = (int32_t)dd;
      if (a.out_kind == QOUT_F32) {
        reinterpret_cast<float*>(y)[o] = (float)q;
        continue;
      }
      const uint8_t b = a.table ? tab[q & 0xff] : (uint8_t)(q & 0xff);
      words[e >> 2] |= (uint32_t)b << (8 * (e & 3));
      if (!a.nhwc_out || c0 + 16 > a.cout) reinterpret_cast<uint8_t*>(y)[o] = b;
    }
    if (bytes && a.nhwc_out && c0 + 16 <= a.cout)
      *reinterpret_cast<u32x4*>(reinterpret_cast<uint8_t*>(y) + p * a.ldo + c0) =
          u32x4{words[0], words[1], words[2], words[3]};
  }
}

hipError_t run_qconv_direct(const void* x, const void* w, void* y, const DirectQConvArgs& a, hipStream_t st) {
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  if (total <= 0) return hipSuccess;
  if (a.cg == a.C && a.cg * a.KH * a.KW <= kStemTaps && a.cout <= kStemCout && a.W % 4 == 0 &&
      (int64_t)a.C * a.H * a.W < INT_MAX && (uintptr_t)x % 4 == 0 &&
      (!a.nhwc_out || ((uintptr_t)y % 16 == 0 && a.ldo % 16 == 0)) && a.N <= 65535) {
    StemGeo sg;
    sg.PR = (kStemTH - 1) * a.sh + (a.KH - 1) * a.dh + 1;
    const int pc = (kStemTW - 1) * a.sw + (a.KW - 1) * a.dw + 1;
    sg.ND = (pc + 3) / 4 + 1;   // the tile's first column may sit up to 3 bytes into its dword
    sg.RB = sg.ND * 4;
    if ((int64_t)a.C * sg.PR * sg.RB <= kStemPatchBytes) {
      dim3 grid((unsigned)((a.OW + kStemTW - 1) / kStemTW), (unsigned)((a.OH + kStemTH - 1) / kStemTH),
                (unsigned)a.N);
      if (grid.y <= 65535) {
        hipLaunchKernelGGL(qconv_stem_kernel, grid, dim3(256), 0, st, reinterpret_cast<const uint8_t*>(x),
                           reinterpret_cast<const int8_t*>(w), y, a, sg);
        return hipGetLastError();
      }
    }
  }
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65535 * 16);
  hipLaunchKernelGGL(qconv_direct_kernel, dim3(grid), dim3(256), 0, st, reinterpret_cast<const uint8_t*>(x),
                     reinterpret_cast<const int8_t*>(w), y, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- ConvTranspose
// Output-stationary form of the reference's scatter: output (n, co, oy, ox)
// gathers x[ci][iy][ix] * w[ci][oc][ky][kx] over the taps with
// iy * sh + ky * dh - pt == oy (and likewise for x).  Walking ci, then ky and
// kx downwards (iy and ix upwards) adds the contributions in the order the
// scatter delivers them to this output, from an f32 zero, and the bias comes
// last, so the f32 result is the reference's to the bit.
template <class T>
__global__ void __launch_bounds__(256)
convt_kernel(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias, T* __restrict__ y,
             ConvTArgs a) {
#pragma clang fp contract(off)
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    int ox, oy, co, n;
    split_out_index(idx, total, a.OW, a.OH, a.cout, ox, oy, co, n);
    const int g = co / a.coutg, oc = co - g * a.coutg;
    const int ty = oy + a.pt, tx = ox + a.pl;
    float acc = 0.0f;
    for (int ic = 0; ic < a.cg; ++ic) {
      const int ci = g * a.cg + ic;
      const T* xc = x + ((int64_t)n * a.C + ci) * a.H * a.W;
      const T* wc = w + ((int64_t)ci * a.coutg + oc) * a.KH * a.KW;
      for (int ky = a.KH - 1; ky >= 0; --ky) {
        const int sy = ty - ky * a.dh;
        if (sy < 0 || sy % a.sh) continue;
        const int iy = sy / a.sh;
        if (iy >= a.H) continue;
        for (int kx = a.KW - 1; kx >= 0; --kx) {
          const int sx = tx - kx * a.dw;
          if (sx < 0 || sx % a.sw) continue;
          const int ix = sx / a.sw;
          if (ix >= a.W) continue;
          acc += to_f32(xc[(int64_t)iy * a.W + ix]) * to_f32(wc[ky * a.KW + kx]);
        }
      }
    }
    if (bias) acc += to_f32(bias[co]);
    y[(((int64_t)n * a.cout + co) * a.OH + oy) * a.OW + ox] = from_f32<T>(acc);
  }
}

hipError_t run_conv_transpose(int dtype, const void* x, const void* w, const void* bias, void* y,
                              const ConvTArgs& a, hipStream_t st) {
  const int64_t total = (int64_t)a.N * a.cout * a.OH * a.OW;
  if (total <= 0) return hipSuccess;
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65535 * 16);
#define OHIP_CONVT(T)                                                                                \
  hipLaunchKernelGGL(convt_kernel<T>, dim3(grid), dim3(256), 0, st, reinterpret_cast<const T*>(x), \
                     reinterpret_cast<const T*>(w), reinterpret_cast<const T*>(bias), reinterpret_cast<T*>(y), a)
  switch (dtype) {
    case DT_F32: OHIP_CONVT(float); break;
    case DT_F16: OHIP_CONVT(_Float16); break;
    case DT_BF16: OHIP_CONVT(__bf16); break;
    default: return hipErrorInvalidValue;
  }
#undef OHIP_CONVT
  return hipGetLastError();
}

// ---------------------------------------------------------------- batched transpose
// dst[s][n][c] = c < K ? src[s][c][n] : 0 for the slices s of a batched [K][N]
// matrix (row stride ld elements in dst): MatMul's B operand brought into
// K-contiguous rows.  32 x 32 tiles through LDS, coalesced on both sides.
template <class T>
__global__ void __launch_bounds__(256)
transpose_batched_kernel(const T* __restrict__ src, T* __restrict__ dst, int K, int N, int ld) {
  __shared__ T tile[32][33];
  const int s = blockIdx.z;
  const int c0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const T* sp = src + (int64_t)s * K * N;
  T* dp = dst + (int64_t)s * N * ld;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int r = ty; r < 32; r += 8) {
    const int c = c0 + r, n = n0 + tx;
    tile[r][tx] = (c < K && n < N) ? sp[(int64_t)c * N + n] : T(0);
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int n = n0 + r, c = c0 + tx;
    if (n < N && c < ld) dp[(int64_t)n * ld + c] = tile[tx][r];
  }
}

hipError_t run_transpose_batched(int elem_bytes, const void* src, void* dst, int slices, int K, int N, int ld,
                                 hipStream_t st) {
  if (slices <= 0 || K <= 0 || N <= 0) return hipSuccess;
  if (slices > 65535) return hipErrorInvalidValue;
  dim3 grid((unsigned)((N + 31) / 32), (unsigned)((ld + 31) / 32), (unsigned)slices), block(256);
  switch (elem_bytes) {
    case 2:
      hipLaunchKernelGGL(transpose_batched_kernel<uint16_t>, grid, block, 0, st,
                         reinterpret_cast<const uint16_t*>(src), reinterpret_cast<uint16_t*>(dst), K, N, ld);
      break;
    case 4:
      hipLaunchKernelGGL(transpose_batched_kernel<uint32_t>, grid, block, 0, st,
                         reinterpret_cast<const uint32_t*>(src), reinterpret_cast<uint32_t*>(dst), K, N, ld);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
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

// ---------------------------------------------------------------- float conversion
template <int S, int D>
__global__ void __launch_bounds__(256) convert_float_kernel(const void* __restrict__ src, void* __restrict__ dst,
                                                            int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    float v;
    if constexpr (S == DT_F32) v = static_cast<const float*>(src)[i];
    else if constexpr (S == DT_F16) v = f16_bits_to_f32(static_cast<const uint16_t*>(src)[i]);
    else v = bf16_bits_to_f32(static_cast<const uint16_t*>(src)[i]);
    if constexpr (D == DT_F32) static_cast<float*>(dst)[i] = v;
    else if constexpr (D == DT_F16) static_cast<uint16_t*>(dst)[i] = f32_to_f16_bits(v);
    else static_cast<uint16_t*>(dst)[i] = f32_to_bf16_bits(v);
  }
}

hipError_t run_convert_float(int src_dt, int dst_dt, const void* src, void* dst, int64_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
  dim3 grid((unsigned)blocks), block(256);
#define OHIP_CONV_CASE(S, D)                                                                       \
  if (src_dt == S && dst_dt == D) {                                                                \
    hipLaunchKernelGGL((convert_float_kernel<S, D>), grid, block, 0, st, src, dst, n);             \
    return hipGetLastError();                                                                      \
  }
  OHIP_CONV_CASE(DT_F32, DT_F16) OHIP_CONV_CASE(DT_F32, DT_BF16) OHIP_CONV_CASE(DT_F16, DT_F32)
  OHIP_CONV_CASE(DT_F16, DT_BF16) OHIP_CONV_CASE(DT_BF16, DT_F32) OHIP_CONV_CASE(DT_BF16, DT_F16)
#undef OHIP_CONV_CASE
  return hipErrorInvalidValue;
}

}  // namespace ohip
