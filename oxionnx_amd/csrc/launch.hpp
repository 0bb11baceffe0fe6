// Epilogues, tile table and launch helpers shared by the per-dtype
// contraction translation units (contract_*.hip) and the GEMV path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "internal.hpp"
#include "mfma_core.hpp"

#include <type_traits>

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
    if (bstride == 0) return (int64_t)i * si + (int64_t)j * sj;
    const int n = i / ohw;
    return (int64_t)n * bstride + (int64_t)(i - n * ohw) * si + (int64_t)j * sj;
  }
  // LDS-staged epilogue (mfma_core.hpp): 1- and 2-byte outputs are written as
  // whole 16-byte row chunks when rows of i are contiguous and aligned.
  static constexpr int kStageBytes = sizeof(OutT) <= 2 ? (int)sizeof(OutT) : 0;
  __device__ __forceinline__ bool staged_ok(int bp) const {
    return vec && ((uintptr_t)y % 16 == 0) && ((sj * (int64_t)sizeof(OutT)) % 16 == 0) &&
           (bstride == 0 || ohw % bp == 0);
  }
  __device__ __forceinline__ char* out_ptr(int i, int j) const { return reinterpret_cast<char*>(y + index(i, j)); }
  // The four outputs (i0..i0+3, j) as packed bits; positions outside the
  // matrix give 0 and read nothing.
  __device__ __forceinline__ uint64_t pack4(int i0, int j, f32x4 acc) const {
    uint64_t bits = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool in = j < Q && i0 + r < P;
      const OutT o = from_f32<OutT>(in ? finish(acc[r], i0 + r, j) : 0.0f);
      uint64_t b;
      if constexpr (sizeof(OutT) == 2) b = __builtin_bit_cast(uint16_t, o);
      else b = __builtin_bit_cast(uint32_t, o);
      bits |= b << (r * 8 * sizeof(OutT));
    }
    return bits;
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
  const uint8_t* table;     // byte -> byte map applied after requantisation (may be null)

  __device__ __forceinline__ int64_t index(int i, int j) const {
    if (bstride == 0) return (int64_t)i * si + (int64_t)j * sj;
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
  static constexpr int kStageBytes = 1;
  __device__ __forceinline__ bool staged_ok(int bp) const {
    return (out_kind == QOUT_U8 || out_kind == QOUT_I8) && vec && ((uintptr_t)y % 16 == 0) && (sj % 16 == 0) &&
           (bstride == 0 || ohw % bp == 0);
  }
  __device__ __forceinline__ char* out_ptr(int i, int j) const { return reinterpret_cast<char*>(y) + index(i, j); }
  __device__ __forceinline__ uint64_t pack4(int i0, int j, i32x4 acc) const {
    uint64_t bits = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int32_t v = 0;
      if (j < Q && i0 + r < P) {
        v = requant(exact(acc[r], i0 + r, j), i0 + r, j);
        if (table) v = table[v & 0xff];
      }
      bits |= (uint64_t)(uint32_t)(v & 0xff) << (r * 8);
    }
    return bits;
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
      if (table) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = table[v[r] & 0xff];
      }
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
// Tile ids (ohip_set_tile_override): block tile BP x BQ, WP x WQ waves,
// LDS stages.
using T64 = Tile<64, 64, 2, 2, 2>;          // 1: 4 waves, 32x32 per wave
using T128 = Tile<128, 128, 2, 2, 3>;       // 2: 4 waves, 64x64 per wave
using T256x128 = Tile<256, 128, 4, 2, 3>;   // 3: 8 waves, 64x64 per wave
using T128x256 = Tile<128, 256, 2, 4, 3>;   // 4: 8 waves, 64x64 per wave
using T256w4 = Tile<256, 256, 2, 2, 2>;     // 5: 4 waves, 128x128 per wave
using T256 = Tile<256, 256, 2, 4, 2>;       // 6: 8 waves, 128x64 per wave
using T128s2 = Tile<128, 128, 2, 2, 2>;     // 7: 4 waves, 64x64 per wave, two blocks per CU
using T128w8 = Tile<128, 128, 2, 4, 2>;     // 8: 8 waves, 64x32 per wave, two blocks per CU
using T64s4 = Tile<64, 64, 2, 2, 4>;        // 9: 4 waves, 32x32 per wave, four stages
constexpr int kTileCount = 9;

template <Op O, bool XX, bool XY, class Tl, class LX, class LY, class Epi>
inline hipError_t launch_tile(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc, hipStream_t st) {
  const int nP = (P + Tl::BP - 1) / Tl::BP, nQ = (Q + Tl::BQ - 1) / Tl::BQ;
  const int64_t nb = (int64_t)nP * nQ;
  if (nb <= 0) return hipSuccess;
  if (nb > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((mfma_gemm_kernel<O, Tl, LX, LY, Epi, XX, XY>), dim3((unsigned)nb), dim3(Tl::kThreads),
                     0, st, lx, ly, epi, nP, nQ, kc, 1);
  return hipGetLastError();
}

// Split-K launch on the 64x64 four-stage tile: partial sums into the
// workspace, then the ordered reduction applies the real epilogue.
template <Op O, bool XX, bool XY, class LX, class LY, class Epi>
inline hipError_t launch_split(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc, int splits,
                               void* ws, hipStream_t st) {
  using Tl = Tile<64, 64, 2, 2, 4>;
  using T = typename std::conditional<O == Op::I8, int32_t, float>::type;
  using V = typename OpT<O>::Out4;
  const int nP = (P + Tl::BP - 1) / Tl::BP, nQ = (Q + Tl::BQ - 1) / Tl::BQ;
  const int64_t nb = (int64_t)nP * nQ;
  if (nb <= 0) return hipSuccess;
  if (nb > 0x7fffffff || splits > 65535 || !ws) return hipErrorInvalidValue;
  const int Pp = (P + 3) / 4 * 4;
  PartialEpi<T> pe{reinterpret_cast<T*>(ws), P, Pp, Q};
  hipLaunchKernelGGL((mfma_gemm_kernel<O, Tl, LX, LY, PartialEpi<T>, XX, XY>), dim3((unsigned)nb, (unsigned)splits),
                     dim3(Tl::kThreads), 0, st, lx, ly, pe, nP, nQ, kc, splits);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t groups = (int64_t)(Pp / 4) * Q;
  const unsigned grid = (unsigned)std::min<int64_t>((groups + 255) / 256, 65535 * 4);
  hipLaunchKernelGGL((split_reduce_kernel<T, V, Epi>), dim3(grid), dim3(256), 0, st, reinterpret_cast<const T*>(ws),
                     splits, P, Pp, Q, epi);
  return hipGetLastError();
}

// Automatic choice (split-K is decided beforehand, plan_splits).  The
// largest tile that still gives at least one block per CU (256 CUs); among
// the smaller tiles, the two-stage 128x128 tile keeps two blocks resident
// per CU and the four-stage 64x64 tile hides the load latency of the
// narrowest problems.  A short K loop (few 128-byte stages) is dominated by
// the prologue and the epilogue, which the resident 128x128 blocks overlap.
inline int pick_tile(int P, int Q, int kc, int forced) {
  if (forced >= 1 && forced <= kTileCount) return forced;
  auto blocks = [&](int bp, int bq) { return (int64_t)((P + bp - 1) / bp) * ((Q + bq - 1) / bq); };
  const int nk = (kc + 7) / 8;
  if (nk <= 16) return blocks(128, 128) >= 256 ? 8 : 9;
  if (blocks(256, 256) >= 256) return 6;
  if (blocks(256, 128) >= 256) return P >= Q ? 3 : 4;
  if (blocks(128, 128) >= 192) return 8;
  return 9;
}

// XX / XY: the X / Y operand holds u8 activations that the MFMA reads as
// int8 after XOR 0x80.
template <Op O, bool XX, bool XY, class LX, class LY, class Epi>
inline hipError_t launch_any(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc, int tile,
                             int splits, void* split_ws, hipStream_t st) {
  if (splits > 1) return launch_split<O, XX, XY>(lx, ly, epi, P, Q, kc, splits, split_ws, st);
  switch (pick_tile(P, Q, kc, tile)) {
    case 2: return launch_tile<O, XX, XY, T128>(lx, ly, epi, P, Q, kc, st);
    case 3: return launch_tile<O, XX, XY, T256x128>(lx, ly, epi, P, Q, kc, st);
    case 4: return launch_tile<O, XX, XY, T128x256>(lx, ly, epi, P, Q, kc, st);
    case 5: return launch_tile<O, XX, XY, T256w4>(lx, ly, epi, P, Q, kc, st);
    case 6: return launch_tile<O, XX, XY, T256>(lx, ly, epi, P, Q, kc, st);
    case 7: return launch_tile<O, XX, XY, T128s2>(lx, ly, epi, P, Q, kc, st);
    case 8: return launch_tile<O, XX, XY, T128w8>(lx, ly, epi, P, Q, kc, st);
    case 9: return launch_tile<O, XX, XY, T64s4>(lx, ly, epi, P, Q, kc, st);
    default: return launch_tile<O, XX, XY, T64>(lx, ly, epi, P, Q, kc, st);
  }
}

template <class OutT>
inline FloatEpi<OutT> make_float_epi(const FloatOut& o) {
  FloatEpi<OutT> e;
  e.y = reinterpret_cast<OutT*>(o.y);
  e.si = o.si; e.sj = o.sj; e.bstride = o.bstride; e.ohw = o.ohw; e.P = o.P; e.Q = o.Q;
  e.vec = o.vec; e.has_alpha = o.alpha != 1.0f; e.alpha = o.alpha; e.beta = o.beta;
  e.bias = reinterpret_cast<const OutT*>(o.bias); e.bias_mode = o.bias ? o.bias_mode : BIAS_NONE;
  e.act = o.act; e.lo = o.lo; e.hi = o.hi;
  return e;
}

inline QuantEpi make_quant_epi(const QuantOut& o) {
  QuantEpi e;
  e.y = o.y; e.si = o.si; e.sj = o.sj; e.bstride = o.bstride; e.ohw = o.ohw; e.P = o.P; e.Q = o.Q;
  e.vec = o.vec; e.w_on_i = o.w_on_i; e.colsum = o.colsum; e.flip = o.flip; e.bias = o.bias; e.ca = o.ca;
  e.ca_rows = o.ca_rows; e.comb = o.comb; e.n_comb = o.n_comb; e.out_kind = o.out_kind;
  e.y_zp = o.y_zp; e.lo = o.lo; e.hi = o.hi; e.table = o.table;
  return e;
}

inline DenseRows make_dense(const DenseOperand& d) {
  DenseRows r;
  r.base = reinterpret_cast<const char*>(d.base);
  r.ld = d.ld_bytes; r.rows = d.rows; r.kc = d.kc; r.kwrap = d.kwrap;
  return r;
}

inline Im2colNHWC make_im2col(const Im2colOperand& c) {
  Im2colNHWC r;
  r.base = reinterpret_cast<const char*>(c.base);
  r.H = c.H; r.W = c.W; r.OH = c.OH; r.OW = c.OW; r.KW = c.KW; r.cpc = c.cpc;
  r.sh = c.sh; r.sw = c.sw; r.dh = c.dh; r.dw = c.dw; r.pt = c.pt; r.pl = c.pl;
  r.rows = c.rows; r.kc = c.kc; r.kwrap = c.kwrap;
  r.pad = reinterpret_cast<const char*>(c.pad16);
  return r;
}

}  // namespace ohip
