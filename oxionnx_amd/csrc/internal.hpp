// Internal contract between the host policy (ops.cpp, runtime.cpp) and the
// device launchers (kernels.hip).  Plain structs, no HIP types beyond the
// stream and error code.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdlib>

namespace ohip {

// ONNX TensorProto element type codes (the public header uses the same).
enum { DT_F32 = 1, DT_U8 = 2, DT_I8 = 3, DT_I32 = 6, DT_F16 = 10, DT_BF16 = 16 };
enum { ACT_NONE = 0, ACT_RELU = 1, ACT_CLIP = 2, ACT_LEAKY_RELU = 3 };
enum { BIAS_NONE = 0, BIAS_SCALAR = 1, BIAS_I = 2, BIAS_J = 3, BIAS_FULL_JI = 4 };
enum { QOUT_U8 = 0, QOUT_I8 = 1, QOUT_I32 = 2, QOUT_F32 = 3 };

// ------------------------------------------------------------------ half conversions
// Bit-exact on host and device: round to nearest even, NaN kept quiet with
// its top payload bits, overflow to infinity, subnormals rounded.
__host__ __device__ inline uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  __builtin_memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(man ? (sign | 0x7e00u | (man >> 13)) : (sign | 0x7c00u));
  int e = (int)exp - 112;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t mm = man | 0x800000u;
    int sh = 14 - e;
    uint32_t h = mm >> sh, rem = mm & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)h;
}
__host__ __device__ inline float f16_bits_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, x;
  if (exp == 0) {
    if (!man) x = sign;
    else {
      int e = -1;
      do { man <<= 1; ++e; } while (!(man & 0x400u));
      x = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) x = sign | 0x7f800000u | (man << 13);
  else x = sign | ((exp + 112) << 23) | (man << 13);
  float f;
  __builtin_memcpy(&f, &x, 4);
  return f;
}
__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t x;
  __builtin_memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint16_t h) {
  uint32_t x = (uint32_t)h << 16;
  float f;
  __builtin_memcpy(&f, &x, 4);
  return f;
}

// Element conversion of a float array between F32 / F16 / BF16 (ONNX codes),
// with the rounding above.
hipError_t run_convert_float(int src_dt, int dst_dt, const void* src, void* dst, int64_t n, hipStream_t st);

// Rows of K-contiguous 16-byte chunks.
struct DenseOperand {
  const void* base;
  int64_t ld_bytes;
  int rows;
  int kc;             // 16-byte chunks per row that hold data
  int kwrap;          // > 0: loop chunk g >= kwrap reads chunk g - kwrap
  uint32_t xor_mask;  // applied after the LDS read: 0x80808080 turns u8 into (u8 - 128) as int8
  const void* pad16;  // device address of 16 bytes read for any chunk outside the matrix
  int zmod;           // batched launch: slice z reads matrix z % zmod (0 / 1: one matrix for all)
  int64_t zstride;    // bytes between those matrices
};

// Implicit im2col rows over an NHWC activation with channels padded to cpc
// 16-byte chunks.
struct Im2colOperand {
  const void* base;   // channel chunk 0 of this operand's channel group at pixel (0, 0)
  int H, W, OH, OW, KW, cpc;
  int pstride;        // 16-byte chunks between pixels (0: cpc)
  int sh, sw, dh, dw, pt, pl;
  int rows, kc, kwrap;
  uint32_t xor_mask;  // as DenseOperand::xor_mask
  const void* pad16;  // 16 bytes standing for a padding tap (stored before the XOR)
  int64_t zstride;    // batched launch: slice z starts z * zstride bytes past base (0: one operand)
  int zpads;          // > 0: slice z (< zpads <= 4) uses pads zpt[z], zpl[z]
  int zpt[4], zpl[4];
};

// Output mapping shared by both epilogues: element (i, j) lives at
// (i / ohw) * bstride + (i % ohw) * si + j * sj.
struct OutMap {
  void* y;
  int64_t si, sj, bstride;
  int ohw, P, Q;
  int vec;
  int splits;      // > 1: split-K over `splits` slices, partial sums in split_ws
  void* split_ws;  // splits * Q * round_up(P, 4) accumulators (4 bytes each)
  int batch;       // > 1: a batched launch of `batch` independent contractions (no split-K)
  int64_t zstride; // bytes between the batch slices' outputs
  int zsw;         // > 0: slice z's output starts at (z / zsw) * zrow + (z % zsw) * zstride
  int64_t zrow;
  int defer_reduce; // split-K: leave the partial sums in split_ws (the caller consumes them)
};

// Split-K plan.  The slices run on the 64x64 four-stage tile when its
// tiling leaves the 256 CUs short of blocks (under one block per CU with at
// least 16 stages of 128 bytes of K, or under two with at least 32); slices
// keep at least 8 stages each and aim at two blocks per CU.  forced_tile
// 10 / 11 force the split path on the 64x64 / 128x128 (eight-wave) tile; any
// other forced tile disables it.  (The 128x128 slices measured slower on the
// generator's resident NHWC convolutions, so the automatic plan keeps 64x64.)
// Tile ids that name one unsplit block tile (launch.hpp); 10 and 11 force
// split-K.
inline bool plain_tile_id(int t) { return (t >= 1 && t <= 9) || (t >= 12 && t <= 14) || t == 16 || t == 18; }
inline int split_tile_size(int, int, int forced_tile) { return forced_tile == 11 ? 128 : 64; }
// OHIP_SPLITS=n (2..16) forces that many split-K slices wherever a split
// plan is made (a measurement switch)
inline int forced_splits() {
  static const int v = [] {
    const char* e = std::getenv("OHIP_SPLITS");
    const int n = e ? std::atoi(e) : 0;
    return n >= 2 && n <= 16 ? n : 0;
  }();
  return v;
}
inline int plan_splits(int P, int Q, int kc, int forced_tile, int auto_bs = 64) {
  if (forced_tile != 0 && forced_tile != 10 && forced_tile != 11) return 1;
  if (forced_splits()) return forced_splits();
  const int64_t nk = (kc + 7) / 8;
  const int bs = forced_tile == 0 ? auto_bs : split_tile_size(P, Q, forced_tile);
  const int64_t nb = (int64_t)((P + bs - 1) / bs) * ((Q + bs - 1) / bs);
  if (forced_tile != 0) return (int)std::max<int64_t>(2, std::min<int64_t>(16, nk / 2 > 0 ? nk / 2 : 1));
  if (nb >= 512 || nk < 16 || (nb >= 256 && nk < 32)) return 1;
  int64_t s = (512 + nb - 1) / nb;
  s = std::min<int64_t>(s, nk / 8);
  s = std::min<int64_t>(s, 16);
  return (int)std::max<int64_t>(s, 1);
}
// The split plan and the tile id to launch it with.  f32 contractions are
// bound by the f32 MFMA rate, which the eight-wave 128x128 tile sustains
// better than the 64x64 one (two accumulator chains per wave instead of
// one), so their slices run on it (as forced tile 11) when that still gives
// the chip a block per CU.
struct SplitChoice {
  int splits, tile;
};
inline SplitChoice plan_split_tile(int P, int Q, int kc, int override_tile, bool mfma_f32) {
  int s64 = plan_splits(P, Q, kc, override_tile);
  // f32 on the 64x64 tile: slices of at least 12 k-stages (config 2b's
  // 128x768x3072, 24 stages: 2 slices 16.0 us against 3 slices 18.3)
  if (mfma_f32 && override_tile == 0 && !forced_splits() && s64 > 2)
    s64 = std::max(2, std::min(s64, (kc + 7) / 8 / 12));
  if (override_tile == 0 && mfma_f32 && s64 > 1) {   // only where the 64x64 plan splits too
    const int s = plan_splits(P, Q, kc, 0, 128);
    const int64_t nb = (int64_t)((P + 127) / 128) * ((Q + 127) / 128);
    if (s > 1 && nb * s >= 256) return {s, 11};
  }
  return {s64, override_tile};
}
inline size_t split_ws_bytes(int P, int Q, int splits) {
  return splits > 1 ? (size_t)splits * (size_t)Q * (size_t)((P + 3) / 4 * 4) * 4 : 0;
}

struct FloatOut : OutMap {
  float alpha, beta;
  const void* bias;  // same element type as the output
  int64_t bias_z;    // batched launch: slice z reads bias + z * bias_z elements (BIAS_I / BIAS_J)
  int bias_mode;
  int act;
  float lo, hi;
};

struct QuantOut : OutMap {
  int w_on_i;
  const int32_t* colsum;
  const int8_t* flip;
  const int32_t* bias;
  int32_t ca;
  const int32_t* ca_rows;
  const float* comb;
  int n_comb;
  int out_kind;
  int32_t y_zp, lo, hi;
  const uint8_t* table;  // device, 256 entries: applied to requantised bytes (may be null)
};

struct GemvArgs {
  const void* a;   // [M][lda] activations
  int64_t lda;     // elements
  const void* w;   // [N][ldw] packed weight rows
  int64_t ldw;     // elements
  int M, N, kc;
};

// Halo-patch convolution geometry (stride 1, dilation 1, one group, NHWC
// input, pixel tiles of whole output rows); see halo_conv_kernel.
struct HaloGeo {
  const char* x;      // NHWC input, image 0; pixels are `pstride` 16-byte chunks apart
  int64_t img_bytes;  // bytes between images
  int H, W, OH, OW;
  int pt, pl;         // padding (top, left) of the patch
  int pad_mode;       // 0: zeros outside the image; 1 / 2: reflect / edge (indices mapped into it)
  int pstride;
  int cpc;            // channel chunks per tap (the input's valid chunks and the filter's)
  int th;             // output rows per pixel tile
  int ow_shift;       // log2(OW)
  const char* w;      // filter rows [cout][KH * KW taps][cpc chunks]
  int64_t ldw;        // bytes between filter rows
  int cout;           // valid filter rows
};
hipError_t run_halo_float(int dtype, const HaloGeo& g, bool pix_on_x, const FloatOut& o, hipStream_t st);
// the whole-K variant (wk_conv_kernel): every block runs the whole
// reduction, no split-K partial sums (HaloGeo.th unused); mom: also the
// outputs' 64-pixel segment moments (pix_on_x, no activation)
hipError_t run_wk_float(int dtype, const HaloGeo& g, bool pix_on_x, const FloatOut& o, float* mom, hipStream_t st);
// pixel-tile extent and largest staged patch of the halo path
constexpr int kHaloBPix = 256;
constexpr int kHaloPixMax = 400;       // patch pixels of a 16-, 32- or 64-wide output row tile
constexpr int kHaloPixMaxWide = 520;   // of a 128-wide one: (2 + 2) x 130

hipError_t run_dense_float(int dtype, const DenseOperand& x, const DenseOperand& y, const FloatOut& o, int tile,
                           hipStream_t st);
hipError_t run_conv_float(int dtype, const Im2colOperand& col, const DenseOperand& w, bool col_on_x,
                          const FloatOut& o, int tile, hipStream_t st);
hipError_t run_dense_quant(const DenseOperand& x, const DenseOperand& y, const QuantOut& o, int tile,
                           hipStream_t st);
hipError_t run_conv_quant(const Im2colOperand& col, const DenseOperand& w, bool col_on_x, const QuantOut& o,
                          int tile, hipStream_t st);
hipError_t run_gemv(int dtype, const GemvArgs& g, const FloatOut& o, hipStream_t st);
// Direct (non-MFMA) grouped convolution; see conv_direct_kernel.
struct DirectConvArgs {
  int N, C, H, W, cout, cg, coutg, KH, KW;
  int sh, sw, dh, dw, pt, pl, pad_mode;  // pad_mode 0: zeros (pt, pl are the conv's pads); 1/2: reflect / edge
  int OH, OW;
  int64_t ldw;    // elements between filter rows
  int cpg;        // channel slots per tap in the packed filter
  int nhwc_out;
  int64_t ldo;    // NHWC output: elements between pixels
  int act;
  float lo, hi;
};
hipError_t run_conv_direct(int dtype, const void* x, const void* w, const void* bias, void* y,
                           const DirectConvArgs& a, hipStream_t st);

// Ungrouped convolution with at most 8 output channels over a long
// reduction (an RGB head): the input channels are cut into `cslice`-wide
// slices; a block stages one slice's input patch of a 16x16 output tile in
// LDS and writes its partial sums (f32) to ws[slice][n][co][oy][ox]; the
// reduction adds the slices in order and applies bias, activation and the
// output type as conv_direct_kernel does.  ws holds
// ceil(C / cslice) * N * cout * OH * OW floats.
constexpr int kFewOutMax = 8;
int fewout_slice(const DirectConvArgs& a);   // channels per slice for the LDS budget
// The same few-output convolution on the MFMA for an NHWC f16 / bf16 input
// (pitch: channel slots per pixel), stride and dilation 1, square 3 / 5 / 7
// filters, at most 4 output channels, output rows up to 128 pixels.
bool fewco_supported(int dtype, const DirectConvArgs& a, int pitch);
int fewco_slice(const DirectConvArgs& a);
hipError_t run_conv_fewco(int dtype, const void* x, int pitch, const void* w, const void* bias, void* y, float* ws,
                          const DirectConvArgs& a, hipStream_t st);
// f32, stride and dilation 1, zero padding, 3x3 or 1x1, NCHW input and output
// (the patch-staged MFMA kernel)
bool conv_nchw_f32_supported(const DirectConvArgs& a);
hipError_t run_conv_nchw_f32(const float* x, const float* w, const float* bias, float* y, const DirectConvArgs& a,
                             hipStream_t st);
hipError_t run_conv_fewout(int dtype, const void* x, const void* w, const void* bias, void* y, float* ws,
                           const DirectConvArgs& a, int cslice, hipStream_t st);

// Direct (non-MFMA) grouped integer convolution; see qconv_direct_kernel.
struct DirectQConvArgs {
  int N, C, H, W, cout, cg, coutg, KH, KW;
  int sh, sw, dh, dw, pt, pl;
  int OH, OW;
  int64_t ldw;       // bytes between packed filter rows
  int cpg;           // channel slots per tap in the packed filter
  int64_t half;      // bytes to a split row's second half (0: rows are not split)
  int x_signed;      // X is int8 (else uint8)
  int32_t x_zp;
  const int8_t* flip;    // per output channel, may be null
  const int32_t* bias;   // per output channel, may be null
  const float* comb;     // combined scales (n_comb == 1: per tensor)
  int n_comb;
  int out_kind;          // QOUT_*
  int32_t y_zp, lo, hi;
  const uint8_t* table;  // may be null
  int nhwc_out;
  int64_t ldo;
};
hipError_t run_qconv_direct(const void* x, const void* w, void* y, const DirectQConvArgs& a, hipStream_t st);

// dst[s][n][c] = c < K ? src[s][c][n] : 0, ld elements per dst row.
hipError_t run_transpose_batched(int elem_bytes, const void* src, void* dst, int slices, int K, int N, int ld,
                                 hipStream_t st);

// ConvTranspose as an output-stationary gather; see convt_kernel.
struct ConvTArgs {
  int N, C, H, W, cout, cg, coutg, KH, KW;
  int sh, sw, dh, dw, pt, pl;
  int OH, OW;
};
hipError_t run_conv_transpose(int dtype, const void* x, const void* w, const void* bias, void* y,
                              const ConvTArgs& a, hipStream_t st);

// NCHW -> NHWC staging with per-group channel slots and an optional
// reflect (1) / edge (2) spatial border; see stage_nhwc_kernel.
hipError_t run_stage_nhwc(int elem_bytes, const void* src, void* dst, int N, int C, int H, int W, int pt, int pl,
                          int pb, int pr, int mode, int cg, int cpg, int groups, hipStream_t st);
// NHWC [N][HW][pitch] (first C slots meaningful) -> NCHW [N][C][HW]
hipError_t run_nhwc_to_nchw(int elem_bytes, const void* src, void* dst, int N, int C, int HW, int pitch,
                            hipStream_t st);
hipError_t run_nchw_to_nhwc(int elem_bytes, const void* src, void* dst, int N, int C, int HW, int cp,
                            hipStream_t st);
hipError_t run_nchw_to_nhwc_pad(int elem_bytes, const void* src, void* dst, int N, int C, int H, int W, int cp,
                                int pt, int pl, int pb, int pr, int mode, hipStream_t st);
hipError_t run_gather2d(int elem_bytes, const void* src, int64_t rs, int64_t cs, void* dst, int R, int K, int ld,
                        hipStream_t st);

// ---------------------------------------------------------------- memory-bound nodes
enum { UN_IDENTITY = 0, UN_RELU = 1, UN_LEAKY_RELU = 2, UN_TANH = 3, UN_SIGMOID = 4, UN_SILU = 5 };
enum { BIN_ADD = 0, BIN_SUB = 1, BIN_MUL = 2, BIN_DIV = 3 };
enum { RZ_HALF_PIXEL = 0, RZ_ASYMMETRIC = 1, RZ_ALIGN_CORNERS = 2, RZ_PYTORCH_HALF_PIXEL = 3,
       RZ_TF_HALF_PIXEL_FOR_NN = 4 };
enum { RZ_ROUND_PREFER_FLOOR = 0, RZ_ROUND_PREFER_CEIL = 1, RZ_FLOOR = 2, RZ_CEIL = 3 };
enum { PAD_CONSTANT = 0, PAD_REFLECT = 1, PAD_EDGE = 2, PAD_WRAP = 3 };
constexpr int kMaxRank = 6;

// Output extents (right-aligned in kMaxRank slots) and the element strides of
// each operand along them (0 on a broadcast axis).
struct BcastPlan {
  int rank;
  int64_t shape[kMaxRank], sa[kMaxRank], sb[kMaxRank];
};

// Optional affine term and activation applied after the normalisation.
struct NormAffine {
  const void* scale;   // per channel, or per (n, c) when per_sample; f32 or the tensor's dtype
  const void* bias;
  int per_sample;      // scale / bias index n * stride + c
  int64_t stride;      // per-sample row stride (elements) of scale / bias
  int same_type;       // scale / bias are in the normalised tensor's dtype (else f32)
  int act;             // UN_NONE / UN_RELU / UN_LEAKY_RELU
  float alpha;
  const void* residual;   // added last (an Add of a same-shape tensor of the dtype), may be null
  int res_nhwc;           // the residual is NHWC with C elements per pixel (else NCHW)
};

struct ResizePlan {
  int ih, iw, oh, ow;
  float sh, sw;        // scales of the H and W axes
  int coord, rule;
};

struct PadPlan {
  int rank, mode;
  int64_t in[kMaxRank], out[kMaxRank], begin[kMaxRank];
  uint32_t value_bits;  // the constant fill as the element's bit pattern
};

struct PoolPlan {
  int ih, iw, oh, ow, kh, kw, sh, sw, pt, pl, dh, dw;
  int nhwc_c = 0;       // > 0: NHWC input of this many channels (output compact NHWC)
  int64_t pitch = 0;    // NHWC input: element slots between pixels
};

struct SlicePlan {
  int rank;
  int64_t out[kMaxRank], start[kMaxRank], step[kMaxRank], in_stride[kMaxRank];
};

hipError_t run_unary(int dt, const void* x, void* y, int64_t n, int op, float alpha, hipStream_t st);
hipError_t run_binary(int dt, const void* a, const void* b, void* y, int64_t n, const BcastPlan& p, bool same, int op,
                      hipStream_t st);
hipError_t run_instnorm(int dt, const void* x, void* y, int64_t planes, int64_t spatial, int C, float eps,
                        const NormAffine& aff, hipStream_t st);
// Instance normalisation of a split-K convolution's output straight from
// its partial sums (PartialEpi layout: slice s, channel c, pixel i at
// ws[(s * C + c) * Pp + i], images one after another along i): each output
// is the ordered slice sum + the conv bias rounded to the tensor's dtype, as
// the split reduction stores it, then normalised as run_instnorm does.  The
// output is NCHW, or NHWC with C elements per pixel (out_nhwc).
constexpr int64_t kNormPartialsMaxSpatial = 16384;
// the moments-fed norm's largest plane (64 segments a channel, merged in registers)
constexpr int64_t kNormMomMaxSpatial = 4096;
// f16 / f32 (dt) instance normalisation from the conv output x (NCHW) and
// its 64-pixel segment moments (wk_conv_kernel's mom); the residual, if any,
// in the output's layout; x, y and the residual aligned to eight elements
hipError_t run_instnorm_mom(int dt, const void* x, const float* mom, void* y, int64_t N, int C, int64_t spatial,
                            float eps, const NormAffine& aff, bool out_nhwc, hipStream_t st);
hipError_t run_instnorm_partials(int dt, const float* ws, int splits, int64_t Pp, const void* conv_bias, void* y,
                                 int64_t N, int64_t spatial, int C, float eps, const NormAffine& aff, bool out_nhwc,
                                 hipStream_t st);
hipError_t run_resize_nearest(int elem_bytes, const void* x, void* y, int64_t planes, const ResizePlan& p,
                              hipStream_t st);
// NHWC (C elements a pixel, C * elem_bytes a multiple of 16, 16-byte aligned)
hipError_t run_resize_nearest_nhwc(int elem_bytes, const void* x, void* y, int64_t images, int64_t C,
                                   const ResizePlan& p, hipStream_t st);
hipError_t run_pad(int elem_bytes, const void* x, void* y, int64_t n, const PadPlan& p, hipStream_t st);
hipError_t run_slice(int elem_bytes, const void* x, void* y, int64_t n, const SlicePlan& p, hipStream_t st);
hipError_t run_maxpool(int dt, const void* x, void* y, int64_t planes, const PoolPlan& p, hipStream_t st);
hipError_t run_quantize(const float* x, uint8_t* y, int64_t n, float scale, float zp, float lo, float hi,
                        hipStream_t st);
hipError_t run_dequantize(const uint8_t* x, bool is_signed, float* y, int64_t n, float scale, float zp,
                          hipStream_t st);
hipError_t run_byte_table(const uint8_t* x, uint8_t* y, int64_t n, const uint8_t* table, hipStream_t st);
// QLinearAdd parameters: operand scales / zero points, the output's scale,
// zero point and saturation range, and whether each operand is int8.
struct QAddArgs {
  float sa, za, sb, zb, sc, zc, lo, hi;
  int a_signed, b_signed;
};
hipError_t run_qadd(const uint8_t* a, const uint8_t* b, uint8_t* y, int64_t n, const BcastPlan& p, bool same,
                    const QAddArgs& q, hipStream_t st);

constexpr int kConcatMax = 8;
struct ConcatPlan {
  const void* src[kConcatMax];
  int64_t w[kConcatMax];     // row width of each input
  int64_t off[kConcatMax];   // where that input's part of an output row starts
  int64_t sp[kConcatMax];    // that input's row pitch (its width, or an NHWC pixel pitch)
  int n;
  void* dst;
};
hipError_t run_concat_rows(ConcatPlan p, int64_t row, int64_t rows, hipStream_t st);
hipError_t run_zero_fill(void* p, size_t bytes, hipStream_t st);
hipError_t run_copy2d(const void* src, int64_t src_pitch, void* dst, int64_t dst_pitch, int64_t width, int64_t rows,
                      hipStream_t st);

}  // namespace ohip
