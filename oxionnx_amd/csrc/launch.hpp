// Epilogues, tile table and launch helpers shared by the per-dtype
// contraction translation units (contract_*.hip) and the GEMV path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "internal.hpp"
#include "mfma_core.hpp"
#include "halo_conv.hpp"

#include <cstdlib>
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

// LeakyRelu is this provider's fusion: the reference keeps it a node of its
// own that reads the conv's stored output, so a 2-byte output is rounded to
// its type before the slope is applied (the unfused pair's two roundings).
// Relu commutes with the rounding and Clip is the reference's own fusion
// (applied before the conversion, conv_typed.rs:54-109).
template <class OutT> __device__ __forceinline__ float activate_t(float v, int act, float lo, float hi) {
  if (sizeof(OutT) == 2 && act == ACT_LEAKY_RELU) v = to_f32(from_f32<OutT>(v));
  return activate(v, act, lo, hi);
}

// Both epilogues read their per-position parameters (biases, column sums,
// scales) in batches before any output is formed: PreI for a group of four
// consecutive i positions (one vector load per array where aligned), PreJ
// for one j.  finish() then turns the group's four accumulators into output
// bit patterns with its mode switches outside the element loops: the
// epilogue runs once per block, and a per-element branch tree there costs
// more than a short K loop costs MFMA time.

// an index clamped into [0, n): positions past the edge read a valid element
// whose value is then discarded
__device__ __forceinline__ int clamp_index(int i, int n) { return i < n ? i : n - 1; }

// o[r] = p[i + r] for r < 4: one vector load when i is a multiple of 4, the
// run lies inside [0, n) and p is 16-byte aligned (vec), else clamped scalars
template <class T> __device__ __forceinline__ void load4(const T* p, int i, int n, bool vec, T (&o)[4]) {
  if (vec && (i & 3) == 0 && i + 3 < n) {
    if constexpr (sizeof(T) == 4) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p + i);
      const uint32_t w0 = v.x, w1 = v.y, w2 = v.z, w3 = v.w;   // lanes by value before the bit casts
      o[0] = __builtin_bit_cast(T, w0); o[1] = __builtin_bit_cast(T, w1);
      o[2] = __builtin_bit_cast(T, w2); o[3] = __builtin_bit_cast(T, w3);
    } else if constexpr (sizeof(T) == 2) {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 v = *reinterpret_cast<const u32x2*>(p + i);
      const uint32_t lo = v.x, hi = v.y;
      o[0] = __builtin_bit_cast(T, (uint16_t)lo); o[1] = __builtin_bit_cast(T, (uint16_t)(lo >> 16));
      o[2] = __builtin_bit_cast(T, (uint16_t)hi); o[3] = __builtin_bit_cast(T, (uint16_t)(hi >> 16));
    } else {
      const uint32_t v = *reinterpret_cast<const uint32_t*>(p + i);
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = __builtin_bit_cast(T, (uint8_t)(v >> (8 * r)));
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = p[clamp_index(i + r, n)];
  }
}

template <class T> __device__ __forceinline__ uint32_t out_bits(T v) {
  if constexpr (sizeof(T) == 2) return __builtin_bit_cast(uint16_t, v);
  else return __builtin_bit_cast(uint32_t, v);
}

// Float output: v = acc * alpha; v = v + beta * bias; act; round to OutT.
// alpha == 1 multiplies exactly, and a missing bias adds -0.0, the exact
// additive identity, so neither needs a branch.
template <class OutT> struct FloatEpi {
  OutAddr out;
  float alpha, beta;
  const OutT* bias;
  int64_t bias_z;     // batched launch: slice blockIdx.z reads bias + z * bias_z (BIAS_I / BIAS_J)
  int bias_mode;      // BIAS_*
  int bias_vec;       // bias is 16-byte aligned: runs of four load as one vector
  int act;
  float lo, hi;

  static constexpr int kStageBytes = sizeof(OutT) <= 2 ? (int)sizeof(OutT) : 0;
  static constexpr bool kStageWide = sizeof(OutT) == 4;   // f32 outputs stage as 4-byte elements
  // finish() reduces to acc + the row term: alpha is 1 (an exact multiply),
  // no column or full-matrix term (the column term would add -0.0, the exact
  // identity) and no activation
  // (either staging mode: f16 / bf16 outputs stage in mode 1, f32 in mode 2)
  static constexpr bool kHasSimple = true;
  static constexpr bool kSimpleTable = false;
  __device__ __forceinline__ int simple(int) const {
    return alpha == 1.0f && (bias_mode == BIAS_I || bias_mode == BIAS_SCALAR || bias_mode == BIAS_NONE) &&
           act == ACT_NONE;
  }
  __device__ __forceinline__ int out_bytes() const { return (int)sizeof(OutT); }
  __device__ __forceinline__ OutAddr addr() const { return out; }
  __device__ __forceinline__ bool staged_ok(int bp) const {
    return out.stage && out.vec && ((uintptr_t)out.y % 16 == 0) && ((out.sj * (int64_t)sizeof(OutT)) % 16 == 0) &&
           (out.bstride == 0 || out.ohw % bp == 0);
  }
  __device__ __forceinline__ bool staged_wide_ok(int bp) const { return sizeof(OutT) == 4 && staged_ok(bp); }

  struct PreI { float b[4]; };    // beta * bias per row (BIAS_I, BIAS_SCALAR), else -0
  struct PreJ { float b; };       // beta * bias per column (BIAS_J), else -0
  template <int EB, class A>
  __device__ __forceinline__ void finish_simple(const PreI& pi, A acc, uint32_t (&bits)[4]) const {
#pragma clang fp contract(off)
#pragma unroll
    for (int r = 0; r < 4; ++r) bits[r] = out_bits(from_f32<OutT>(acc[r] + pi.b[r]));
  }
  __device__ __forceinline__ void load_i(PreI& p, int i) const {
#pragma clang fp contract(off)
    if (bias_mode == BIAS_I) {
      OutT raw[4];
      load4(bias + (int64_t)blockIdx.z * bias_z, i, out.P, bias_vec, raw);
#pragma unroll
      for (int r = 0; r < 4; ++r) p.b[r] = i + r < out.P ? beta * to_f32(raw[r]) : 0.0f;
    } else {
      const float s = bias_mode == BIAS_SCALAR ? beta * to_f32(bias[0]) : -0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) p.b[r] = s;
    }
  }
  __device__ __forceinline__ void load_j(PreJ& p, int j) const {
#pragma clang fp contract(off)
    if (bias_mode == BIAS_J) {
      const float x = to_f32(bias[(int64_t)blockIdx.z * bias_z + clamp_index(j, out.Q)]);
      p.b = j < out.Q ? beta * x : 0.0f;
    } else {
      p.b = -0.0f;
    }
  }
  template <class A>
  __device__ __forceinline__ void finish(const PreI& pi, const PreJ& pj, int i, int j, A acc,
                                         uint32_t (&bits)[4]) const {
#pragma clang fp contract(off)
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = acc[r] * alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = v[r] + (pi.b[r] + pj.b);
    if (bias_mode == BIAS_FULL_JI) {
      OutT c[4];
      const int64_t cj = (int64_t)clamp_index(j, out.Q) * out.P;
#pragma unroll
      for (int r = 0; r < 4; ++r) c[r] = bias[cj + clamp_index(i + r, out.P)];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = v[r] + beta * to_f32(c[r]);
    }
    if (act == ACT_RELU) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = v[r] > 0.0f ? v[r] : 0.0f;   // f32::max(NaN, 0) == 0
    } else if (act == ACT_CLIP) {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = v[r] < lo ? lo : (v[r] > hi ? hi : v[r]);
    } else if (act == ACT_LEAKY_RELU) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (sizeof(OutT) == 2) v[r] = to_f32(from_f32<OutT>(v[r]));   // as activate_t
        v[r] = v[r] >= 0.0f ? v[r] : v[r] * lo;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) bits[r] = out_bits(from_f32<OutT>(v[r]));
  }
  // one output of a reduction that has no MFMA tile (the GEMV path)
  __device__ __forceinline__ void store_one(float acc, int i, int j) const {
    PreI pi;
    PreJ pj;
    load_i(pi, i);
    load_j(pj, j);
    f32x4 a = {acc, 0.0f, 0.0f, 0.0f};
    uint32_t bits[4];
    finish(pi, pj, i, j, a, bits);
    OutT* dst = reinterpret_cast<OutT*>(out.y) + out.row(i) + (int64_t)j * out.sj;
    *dst = __builtin_bit_cast(OutT, (typename std::conditional<sizeof(OutT) == 2, uint16_t, uint32_t>::type)bits[0]);
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
  OutAddr out;
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
  int vec_ok;               // every per-channel / per-row array is 16-byte aligned

  // simple(1): the common QLinearMatMul / QLinearConv form (weight channels
  // on i, a per-tensor correction factor, a u8 / i8 output, with or without the byte table), whose
  // finish needs only the row terms; the staged epilogue then runs
  // finish_simple, the same arithmetic with no uniform branches
  static constexpr bool kHasSimple = true;
  // Mode 2 (4-byte outputs): the raw int32 form (MatMulInteger) likewise.
  // Returns 1 for the plain form, 2 for a u8 / i8 form with the byte table
  // (a fused activation), 0 otherwise.
  static constexpr bool kSimpleTable = true;
  __device__ __forceinline__ int simple(int mode) const {
    if (!w_on_i || ca_rows != nullptr) return 0;
    if (mode == 2) return out_kind == QOUT_I32 ? 1 : 0;
    if (out_kind != QOUT_U8 && out_kind != QOUT_I8) return 0;
    return table == nullptr ? 1 : 2;
  }
  static constexpr int kStageBytes = 1;
  static constexpr bool kStageWide = true;   // int32 / f32 outputs stage as 4-byte elements
  __device__ __forceinline__ int out_bytes() const { return (out_kind == QOUT_U8 || out_kind == QOUT_I8) ? 1 : 4; }
  __device__ __forceinline__ OutAddr addr() const { return out; }
  __device__ __forceinline__ bool staged_ok(int bp) const {
    return out.stage && (out_kind == QOUT_U8 || out_kind == QOUT_I8) && out.vec && ((uintptr_t)out.y % 16 == 0) &&
           (out.sj % 16 == 0) && (out.bstride == 0 || out.ohw % bp == 0);
  }
  __device__ __forceinline__ bool staged_wide_ok(int bp) const {
    return out.stage && (out_kind == QOUT_I32 || out_kind == QOUT_F32) && out.vec && ((uintptr_t)out.y % 16 == 0) &&
           (out.sj % 4 == 0) && (out.bstride == 0 || out.ohw % bp == 0);
  }

  // Per-channel terms of a weight channel, prepared once per block: cs the
  // column sum, k = ca * cs when the correction factor is per tensor (so an
  // output adds it instead of multiplying), bi the int32 bias, fl the flip
  // mask (-1: the packed channel holds -(w - w_zp)), cb the combined scale
  // widened to f64.  Per activation row: the correction factor ca.
  struct Chan { int32_t cs, k, bi, fl; double cb; };
  // ch must be in range (callers clamp); the loads carry no branch
  __device__ __forceinline__ Chan chan(int ch) const {
    Chan c;
    c.cs = colsum[ch];
    c.k = (int32_t)((uint32_t)ca * (uint32_t)c.cs);
    c.bi = bias ? bias[ch] : 0;
    c.fl = (flip && flip[ch]) ? -1 : 0;
    c.cb = (double)comb[n_comb > 1 ? ch : 0];
    return c;
  }
  // Per group of four rows, 64 bytes (the epilogue reads them from LDS for
  // every group, so they are kept to four 16-byte reads): with the weight
  // channels on i, k = ca * cs (or cs itself when ca is per activation row),
  // the int32 bias, the combined scale as stored (f32, widened at use) and
  // the flip mask in x; with them on j, x holds the rows' correction factor.
  struct PreI { int32_t k[4]; int32_t bi[4]; float cb[4]; int32_t x[4]; };
  struct PreJ { Chan c; int32_t ca; };         // ca when w_on_i, else c
  __device__ __forceinline__ void load_i(PreI& p, int i) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) { p.k[r] = 0; p.bi[r] = 0; p.cb[r] = 0.0f; p.x[r] = 0; }
    if (w_on_i) {
      int32_t cs[4];
      int8_t fl[4] = {0, 0, 0, 0};
      load4(colsum, i, out.P, vec_ok, cs);
      if (bias) load4(bias, i, out.P, vec_ok, p.bi);
      if (flip) load4(flip, i, out.P, vec_ok, fl);
      if (n_comb > 1) {
        load4(comb, i, out.P, vec_ok, p.cb);
      } else {
        const float c0 = comb[0];
        p.cb[0] = p.cb[1] = p.cb[2] = p.cb[3] = c0;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p.k[r] = ca_rows ? cs[r] : (int32_t)((uint32_t)ca * (uint32_t)cs[r]);
        p.x[r] = fl[r] ? -1 : 0;
      }
    } else if (ca_rows) {
      load4(ca_rows, i, out.P, vec_ok, p.x);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) p.x[r] = ca;
    }
  }
  __device__ __forceinline__ void load_j(PreJ& p, int j) const {
    const int jj = clamp_index(j, out.Q);
    if (w_on_i) p.ca = ca_rows ? ca_rows[jj] : ca;
    else p.c = chan(jj);
  }
  // the exact int32 accumulator (modulo 2^32): acc + ca * cs, negated for a
  // flipped channel (fl = -1), + bias; `k` is ca * cs
  static __device__ __forceinline__ int32_t exact(int32_t acc, int32_t fl, int32_t bi, int32_t k) {
    uint32_t v = (uint32_t)acc + (uint32_t)k;
    v = (v ^ (uint32_t)fl) - (uint32_t)fl;   // fl = -1: two's complement negation
    v += (uint32_t)bi;
    return (int32_t)v;
  }
  // SatRange::requantize: f64 product with the combined scale, + zp, round
  // half to even, clamp (d is never NaN, so max / min clamp exactly)
  __device__ __forceinline__ int32_t requant(int32_t v, double cs) const {
#pragma clang fp contract(off)
    double d = (double)v * cs;
    d = d + (double)y_zp;
    d = __builtin_rint(d);
    d = __builtin_fmax(d, (double)lo);
    d = __builtin_fmin(d, (double)hi);
    return (int32_t)d;
  }
  template <int EB, class A>
  __device__ __forceinline__ void finish_simple(const PreI& pi, A acc, uint32_t (&bits)[4]) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int32_t v = exact(acc[r], pi.x[r], pi.bi[r], pi.k[r]);
      if constexpr (EB == 4) bits[r] = (uint32_t)v;
      else if constexpr ((EB & 16) != 0) bits[r] = table[requant(v, (double)pi.cb[r]) & 0xff];
      else bits[r] = (uint32_t)requant(v, (double)pi.cb[r]) & 0xff;
    }
  }
  template <class A>
  __device__ __forceinline__ void finish(const PreI& pi, const PreJ& pj, int, int, A acc,
                                         uint32_t (&bits)[4]) const {
    int32_t v[4];
    double cb[4];
    // a per-row correction factor multiplies per output; a per-tensor one
    // was folded into k (a uniform branch: the common path has no multiply)
    if (w_on_i) {
      const bool rowca = __builtin_expect(ca_rows != nullptr, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t a = acc[r];   // by value
        const int32_t k = rowca ? (int32_t)((uint32_t)pj.ca * (uint32_t)pi.k[r]) : pi.k[r];
        v[r] = exact(a, pi.x[r], pi.bi[r], k);
        cb[r] = (double)pi.cb[r];
      }
    } else {
      const bool rowca = __builtin_expect(ca_rows != nullptr, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t a = acc[r];
        const int32_t k = rowca ? (int32_t)((uint32_t)pi.x[r] * (uint32_t)pj.c.cs) : pj.c.k;
        v[r] = exact(a, pj.c.fl, pj.c.bi, k);
        cb[r] = pj.c.cb;
      }
    }
    if (out_kind == QOUT_I32) {
#pragma unroll
      for (int r = 0; r < 4; ++r) bits[r] = (uint32_t)v[r];
      return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = requant(v[r], cb[r]);
    if (out_kind == QOUT_F32) {
      // requantised lanes stored as f32, the reference Tensor's representation
#pragma unroll
      for (int r = 0; r < 4; ++r) bits[r] = __builtin_bit_cast(uint32_t, (float)v[r]);
      return;
    }
    if (table) {
#pragma unroll
      for (int r = 0; r < 4; ++r) bits[r] = table[v[r] & 0xff];
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) bits[r] = (uint32_t)v[r] & 0xff;
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
                                            // 10, 11: the split-K paths (launch_split_on)
using T128d4 = Tile<128, 128, 2, 4, 4>;     // 12: 8 waves, 64x32 per wave, four stages (one block per CU)
using T64d8 = Tile<64, 64, 2, 2, 8>;        // 13: 4 waves, 32x32 per wave, eight stages
using T128x4w4 = Tile<128, 128, 2, 2, 4>;   // 14: 4 waves, 64x64 per wave, four stages
using T256x3 = Tile<256, 256, 2, 4, 2, 8, 3>;  // 16: as 6 with a third X buffer, X loads two stages ahead
using T192x256 = Tile<192, 256, 2, 4, 2>;   // 18: 8 waves, 96x64 per wave (one block per CU)


// Tiles per XCD group along P in the engine's tile order (map_tile);
// OHIP_GP overrides the default of 8 (a measurement switch)
inline int tile_group_width() {
  static const int v = [] { const char* e = std::getenv("OHIP_GP"); return e ? std::max(1, std::atoi(e)) : 8; }();
  return v;
}

template <Op O, bool XX, bool XY, class Tl, class LX, class LY, class Epi>
inline hipError_t launch_tile(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc, hipStream_t st) {
  const int nP = (P + Tl::BP - 1) / Tl::BP, nQ = (Q + Tl::BQ - 1) / Tl::BQ;
  const int64_t nb = (int64_t)nP * nQ;
  const int batch = epi.out.batch > 1 ? epi.out.batch : 1;   // slices on blockIdx.z
  if (nb <= 0) return hipSuccess;
  if (nb > 0x7fffffff || batch > 65535) return hipErrorInvalidValue;
  // two dense operands of whole stages on the large tiles (and the int8
  // 128x128 ones): the loader without the K-tail select, one VALU select
  // less per load (f16 headline +1-2 %, config 2c +3 %, int8 FFN pair about
  // +5 %; the small f16 / f32 tiles gain nothing measurable and keep one
  // loader, which halves their instantiations)
  if constexpr ((Tl::XST != Tl::STAGES || Tl::BP * Tl::BQ >= 128 * 256 ||
                 (O == Op::I8 && Tl::BP * Tl::BQ >= 128 * 128)) &&
                std::is_same<LX, DenseRows>::value && std::is_same<LY, DenseRows>::value) {
    if (lx.kc == kc && ly.kc == kc && kc >= Tl::CH && kc % Tl::CH == 0 && lx.kwrap == 0 && ly.kwrap == 0) {
      hipLaunchKernelGGL((mfma_gemm_kernel<O, Tl, DenseRowsWhole, DenseRowsWhole, Epi, XX, XY>),
                         dim3((unsigned)nb, 1, (unsigned)batch), dim3(Tl::kThreads), 0, st, DenseRowsWhole(lx),
                         DenseRowsWhole(ly), epi, nP, nQ, kc, 1, tile_group_width());
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((mfma_gemm_kernel<O, Tl, LX, LY, Epi, XX, XY>), dim3((unsigned)nb, 1, (unsigned)batch),
                     dim3(Tl::kThreads), 0, st, lx, ly, epi, nP, nQ, kc, 1, tile_group_width());
  return hipGetLastError();
}

// The ordered reduction of `splits` partial-sum slices (PartialEpi layout),
// which applies the real epilogue.
template <Op O, class Epi>
inline hipError_t launch_reduce(const void* ws, int splits, int P, int Q, const Epi& epi, hipStream_t st) {
  using T = typename std::conditional<O == Op::I8, int32_t, float>::type;
  using V = typename OpT<O>::Out4;
  const int Pp = (P + 3) / 4 * 4;
  const int64_t groups = (int64_t)(Pp / 4) * Q;
  if (groups > 0x7fffffff) return hipErrorInvalidValue;   // the reduction indexes groups in 32 bits
  const unsigned grid = (unsigned)std::min<int64_t>((groups + 255) / 256, 65535 * 4);
  hipLaunchKernelGGL((split_reduce_kernel<T, V, Epi>), dim3(grid), dim3(256), 0, st, reinterpret_cast<const T*>(ws),
                     splits, P, Pp, Q, epi);
  return hipGetLastError();
}

// Split-K launch: partial sums of every K slice into the workspace, then the
// ordered reduction applies the real epilogue.
template <Op O, bool XX, bool XY, class Tl, class LX, class LY, class Epi>
inline hipError_t launch_split_on(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc, int splits,
                                  void* ws, hipStream_t st) {
  using T = typename std::conditional<O == Op::I8, int32_t, float>::type;
  const int nP = (P + Tl::BP - 1) / Tl::BP, nQ = (Q + Tl::BQ - 1) / Tl::BQ;
  const int64_t nb = (int64_t)nP * nQ;
  if (nb <= 0) return hipSuccess;
  if (nb > 0x7fffffff || splits > 65535 || !ws) return hipErrorInvalidValue;
  const int Pp = (P + 3) / 4 * 4;
  PartialEpi<T> pe{reinterpret_cast<T*>(ws), P, Pp, Q};
  hipLaunchKernelGGL((mfma_gemm_kernel<O, Tl, LX, LY, PartialEpi<T>, XX, XY>), dim3((unsigned)nb, (unsigned)splits),
                     dim3(Tl::kThreads), 0, st, lx, ly, pe, nP, nQ, kc, splits, tile_group_width());
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || epi.out.defer) return e;
  return launch_reduce<O>(ws, splits, P, Q, epi, st);
}

// Halo-patch convolution (halo_conv_kernel): 64 output channels x 256
// pixels per block, eight waves, four stages of two-chunk slabs.  Each XCD
// owns whole output-channel tiles (the filter is the operand that would be
// re-read), with every pixel tile of them.
template <Op O, bool PIXX, class Epi, int PIXMAX>
inline hipError_t launch_halo_px(const HaloGeo& g, const Epi& epi, int P, int Q, int splits, void* ws,
                                 hipStream_t st) {
  using Ht = HaloTile<PIXX ? kHaloBPix : 64, PIXX ? 64 : kHaloBPix, PIXX ? 4 : 2, PIXX ? 2 : 4, 2, 4, 3, 3,
                      PIXMAX, PIXX>;
  using T = typename std::conditional<O == Op::I8, int32_t, float>::type;
  const int nP = (P + Ht::BP - 1) / Ht::BP, nQ = (Q + Ht::BQ - 1) / Ht::BQ;
  const int64_t nb = (int64_t)nP * nQ;
  if (nb <= 0) return hipSuccess;
  if (nb > 0x7fffffff || splits < 1 || splits > 65535) return hipErrorInvalidValue;
  const int gp = PIXX ? nP : 1;
  if (splits == 1) {
    hipLaunchKernelGGL((halo_conv_kernel<O, Ht, Epi>), dim3((unsigned)nb, 1), dim3(Ht::kThreads), 0, st, g, epi, nP,
                       nQ, 1, gp);
    return hipGetLastError();
  }
  if (!ws) return hipErrorInvalidValue;
  const int Pp = (P + 3) / 4 * 4;
  PartialEpi<T> pe{reinterpret_cast<T*>(ws), P, Pp, Q};
  hipLaunchKernelGGL((halo_conv_kernel<O, Ht, PartialEpi<T>>), dim3((unsigned)nb, (unsigned)splits),
                     dim3(Ht::kThreads), 0, st, g, pe, nP, nQ, splits, gp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || epi.out.defer) return e;
  return launch_reduce<O>(ws, splits, P, Q, epi, st);
}
// 128-wide output rows (two rows a tile) stage a larger patch
template <Op O, bool PIXX, class Epi>
inline hipError_t launch_halo(const HaloGeo& g, const Epi& epi, int P, int Q, int splits, void* ws, hipStream_t st) {
  if (g.OW == 128) return launch_halo_px<O, PIXX, Epi, kHaloPixMaxWide>(g, epi, P, Q, splits, ws, st);
  return launch_halo_px<O, PIXX, Epi, kHaloPixMax>(g, epi, P, Q, splits, ws, st);
}

// Whole-K halo convolution (wk_conv_kernel): NPT * 32 pixels (whole output
// rows) x 32 output channels a block, eight-chunk (128-byte) slabs, two
// stages.  32-wide rows take two pixel tiles (eight waves), 16- and 64-wide
// rows four (sixteen waves: a 64-wide tile is two rows, a 16-wide one
// eight).
// A deferred epilogue (the fused conv -> norm node) leaves the raw f32 sums
// in `ws` instead, as one split-K slice, for the norm kernel that reads
// partial sums.  mom (with the conv's bias and channel count): the
// kernel also writes each 64-pixel segment's moments (wk_conv_kernel).
template <Op O, bool PIXX, class Epi>
inline hipError_t launch_wk(const HaloGeo& g, const Epi& epi, int P, int Q, void* ws, float* mom, const void* mbias,
                            hipStream_t st) {
  auto go = [&](auto wt, const auto& e) -> hipError_t {
    using Wt = decltype(wt);
    using E = std::decay_t<decltype(e)>;
    const int pix = PIXX ? P : Q, co = PIXX ? Q : P;
    const int nP = pix / (Wt::NPT * 32), nQ = (co + 31) / 32;
    if (nP <= 0 || nQ <= 0) return hipSuccess;
    if (pix % (Wt::NPT * 32) != 0 || (int64_t)nP * nQ > 0x7fffffff) return hipErrorInvalidValue;
    if (mom && (!PIXX || (g.OH * g.OW) % kNormSeg != 0)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((wk_conv_kernel<O, Wt, E>), dim3((unsigned)(nP * nQ)), dim3(Wt::kThreads), 0, st, g, e, nP,
                       nQ, mom, mbias, co);
    return hipGetLastError();
  };
  auto pick = [&](const auto& e) -> hipError_t {
    if (g.OW == 32) return go(WkTile<32, 2, 8, 2, PIXX>{}, e);
    if (g.OW == 64) return go(WkTile<64, 4, 8, 2, PIXX>{}, e);
    if (g.OW == 16) return go(WkTile<16, 4, 8, 2, PIXX>{}, e);
    return hipErrorInvalidValue;
  };
  if (!epi.out.defer) return pick(epi);
  if (!ws || !PIXX || O == Op::I8 || mom) return hipErrorInvalidValue;
  return pick(PartialEpi<float>{reinterpret_cast<float*>(ws), P, (P + 3) / 4 * 4, Q});
}

// Automatic choice (split-K is decided beforehand, plan_splits).  The
// largest tile that still gives at least one block per CU (256 CUs); among
// the smaller tiles, the two-stage 128x128 tile keeps two blocks resident
// per CU and the four-stage 64x64 tile hides the load latency of the
// narrowest problems.  A short K loop (few 128-byte stages) is dominated by
// the prologue and the epilogue, which the resident 128x128 blocks overlap.
inline int pick_tile(int P, int Q, int kc, int forced) {
  if (plain_tile_id(forced)) return forced;
  auto blocks = [&](int bp, int bq) { return (int64_t)((P + bp - 1) / bp) * ((Q + bq - 1) / bq); };
  const int nk = (kc + 7) / 8;
  if (nk <= 16) return blocks(128, 128) >= 256 ? 8 : 9;
  // a long K and about one round of 128x128 tiles (config 3's second FFN
  // GEMM, 4096x3072x768: 192 tiles): the four-stage eight-wave tile, one
  // block per CU with deeper prefetch (int8 21.1 against 22.1 us for the
  // two-stage tile; f16 1024x4096x4096 43.8 against 55.5, 768x4096x4096
  // 38.5 against 52.0; f32 within 3 %)
  if (blocks(128, 128) >= 192 && blocks(128, 128) < 320 && blocks(256, 256) < 256) return 12;
  // the 256x256 tile with the X operand's loads two stages ahead
  // (bit-identical; headline 312.0 -> 308.7 us, f16 8192^3 889.7 -> 868.6,
  // bf16 863.6 -> 844.9; int8 8192^3 2423-2429 -> 2496-2508 TOPS and f32
  // 4096x4096x11008 134.0 -> 136.1 TFLOP/s once its loop ran unrolled
  // without K-tail selects)
  if (blocks(256, 256) >= 256) return 16;
  if (blocks(256, 128) >= 256) return P >= Q ? 3 : 4;
  if (blocks(128, 128) >= 192) return 8;
  return 9;
}

// Byte outputs (u8 / i8 requantised) of a short-K grid of more than two
// rounds of 128x128 tiles (two blocks a CU) that the 192x256 tile covers in
// one round of one block a CU: config 3's first FFN GEMM (4096x768 ->
// 3072: 768 tiles of 128x128, 256 of 192x256) 22.6 -> 19.4 us.  Its
// staged byte outputs fit the stage buffers; 4-byte outputs would leave
// unstaged (MatMulInteger: 29.7 against 24.6 us) and keep the 128x128 tile.
template <class Epi> inline bool byte_outputs(const Epi&) { return false; }
inline bool byte_outputs(const QuantEpi& e) { return e.out_kind == QOUT_U8 || e.out_kind == QOUT_I8; }
inline bool prefer_192x256(int P, int Q, int kc) {
  auto blocks = [&](int bp, int bq) { return (int64_t)((P + bp - 1) / bp) * ((Q + bq - 1) / bq); };
  return (kc + 7) / 8 <= 16 && blocks(128, 128) > 512 && blocks(192, 256) <= 256;
}

// XX / XY: the X / Y operand holds u8 activations that the MFMA reads as
// int8 after XOR 0x80.
template <Op O, bool XX, bool XY, class LX, class LY, class Epi>
inline hipError_t launch_any(const LX& lx, const LY& ly, const Epi& epi, int P, int Q, int kc, int tile,
                             int splits, void* split_ws, hipStream_t st) {
  if (splits > 1 && epi.out.batch > 1) return hipErrorInvalidValue;   // one workspace: no split-K per slice
  if (splits > 1) {
    // OHIP_SPLIT_TILE=12/13/14 runs the slices on that deeper-pipelined tile (a measurement switch)
    static const int sv = [] { const char* e = std::getenv("OHIP_SPLIT_TILE"); return e ? std::atoi(e) : 0; }();
    if (sv == 12) return launch_split_on<O, XX, XY, T128d4>(lx, ly, epi, P, Q, kc, splits, split_ws, st);
    if (sv == 13) return launch_split_on<O, XX, XY, T64d8>(lx, ly, epi, P, Q, kc, splits, split_ws, st);
    if (sv == 14) return launch_split_on<O, XX, XY, T128x4w4>(lx, ly, epi, P, Q, kc, splits, split_ws, st);
    if (split_tile_size(P, Q, tile) == 128)
      return launch_split_on<O, XX, XY, T128w8>(lx, ly, epi, P, Q, kc, splits, split_ws, st);
    return launch_split_on<O, XX, XY, T64s4>(lx, ly, epi, P, Q, kc, splits, split_ws, st);
  }
  int choice = pick_tile(P, Q, kc, tile);
  if (tile == 0 && byte_outputs(epi) && prefer_192x256(P, Q, kc)) choice = 18;
  switch (choice) {
    case 2: return launch_tile<O, XX, XY, T128>(lx, ly, epi, P, Q, kc, st);
    case 3: return launch_tile<O, XX, XY, T256x128>(lx, ly, epi, P, Q, kc, st);
    case 4: return launch_tile<O, XX, XY, T128x256>(lx, ly, epi, P, Q, kc, st);
    case 5: return launch_tile<O, XX, XY, T256w4>(lx, ly, epi, P, Q, kc, st);
    case 6: return launch_tile<O, XX, XY, T256>(lx, ly, epi, P, Q, kc, st);
    case 7: return launch_tile<O, XX, XY, T128s2>(lx, ly, epi, P, Q, kc, st);
    case 8: return launch_tile<O, XX, XY, T128w8>(lx, ly, epi, P, Q, kc, st);
    case 9: return launch_tile<O, XX, XY, T64s4>(lx, ly, epi, P, Q, kc, st);
    case 12: return launch_tile<O, XX, XY, T128d4>(lx, ly, epi, P, Q, kc, st);
    case 13: return launch_tile<O, XX, XY, T64d8>(lx, ly, epi, P, Q, kc, st);
    case 14: return launch_tile<O, XX, XY, T128x4w4>(lx, ly, epi, P, Q, kc, st);
    case 16: return launch_tile<O, XX, XY, T256x3>(lx, ly, epi, P, Q, kc, st);
    case 18: return launch_tile<O, XX, XY, T192x256>(lx, ly, epi, P, Q, kc, st);
    default: return launch_tile<O, XX, XY, T64>(lx, ly, epi, P, Q, kc, st);
  }
}

// Per-slice pads (Im2colNHWC::zpt / zpl) hold four entries, indexed by the
// batch slice: a launch that uses them must have at most four slices and no
// more slices than entries.
inline bool zpads_fit(const Im2colOperand& col, const OutMap& o) {
  if (col.zpads <= 0) return true;
  const int batch = o.batch > 1 ? o.batch : 1;
  return col.zpads <= 4 && batch <= col.zpads;
}

// OHIP_STAGE=0 turns the LDS-staged epilogue off (a measurement switch)
inline int stage_allowed() {
  static const int v = [] {
    const char* e = std::getenv("OHIP_STAGE");
    return (e && e[0] == '0') ? 0 : 1;
  }();
  return v;
}

inline OutAddr make_out_addr(const OutMap& o) {
  OutAddr a{};
  a.stage = stage_allowed();
  a.y = reinterpret_cast<char*>(o.y);
  a.si = o.si; a.sj = o.sj; a.bstride = o.bstride; a.ohw = o.ohw > 0 ? o.ohw : 1;
  magic_div(a.ohw, &a.ohw_mul, &a.ohw_shift);
  a.P = o.P; a.Q = o.Q; a.vec = o.vec;
  a.batch = o.batch > 1 ? o.batch : 1; a.zstride = o.zstride;
  a.zsw = o.zsw; a.zrow = o.zrow;
  a.defer = o.defer_reduce;
  return a;
}

template <class OutT>
inline FloatEpi<OutT> make_float_epi(const FloatOut& o) {
  FloatEpi<OutT> e;
  e.out = make_out_addr(o);
  e.alpha = o.alpha; e.beta = o.beta;
  e.bias = reinterpret_cast<const OutT*>(o.bias); e.bias_mode = o.bias ? o.bias_mode : BIAS_NONE;
  e.bias_z = o.bias_z;
  e.bias_vec = ((uintptr_t)o.bias % 16) == 0 && (o.bias_z * (int64_t)sizeof(OutT)) % 16 == 0;
  e.act = o.act; e.lo = o.lo; e.hi = o.hi;
  return e;
}

inline QuantEpi make_quant_epi(const QuantOut& o) {
  QuantEpi e;
  e.out = make_out_addr(o);
  e.w_on_i = o.w_on_i; e.colsum = o.colsum; e.flip = o.flip; e.bias = o.bias; e.ca = o.ca;
  e.ca_rows = o.ca_rows; e.comb = o.comb; e.n_comb = o.n_comb; e.out_kind = o.out_kind;
  e.y_zp = o.y_zp; e.lo = o.lo; e.hi = o.hi; e.table = o.table;
  auto al = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
  e.vec_ok = al(o.colsum) && al(o.flip) && al(o.bias) && al(o.ca_rows) && al(o.comb);
  return e;
}

inline DenseRows make_dense(const DenseOperand& d) {
  DenseRows r;
  r.base = reinterpret_cast<const char*>(d.base);
  r.ld = d.ld_bytes; r.rows = d.rows; r.kc = d.kc; r.kwrap = d.kwrap;
  r.zmod = d.zmod; r.zstride = d.zstride;
  return r;
}

inline Im2colNHWC make_im2col(const Im2colOperand& c) {
  Im2colNHWC r;
  r.base = reinterpret_cast<const char*>(c.base);
  r.H = c.H; r.W = c.W; r.OH = c.OH; r.OW = c.OW; r.KW = c.KW; r.cpc = c.cpc;
  r.pstride = c.pstride > 0 ? c.pstride : c.cpc;
  r.sh = c.sh; r.sw = c.sw; r.dh = c.dh; r.dw = c.dw; r.pt = c.pt; r.pl = c.pl;
  r.rows = c.rows; r.kc = c.kc; r.kwrap = c.kwrap;
  r.pad = reinterpret_cast<const char*>(c.pad16);
  r.zstride = c.zstride;
  r.zpads = c.zpads;
  for (int i = 0; i < 4; ++i) { r.zpt[i] = c.zpt[i]; r.zpl[i] = c.zpl[i]; }
  magic_div(r.cpc, &r.cpc_mul, &r.cpc_shift);
  magic_div(r.KW, &r.kw_mul, &r.kw_shift);
  return r;
}

}  // namespace ohip
