// Shared MFMA tile engine for every dense contraction in the provider.
//
// One kernel skeleton computes D[i][j] = sum_k X[i][k] * Y[j][k] for the
// f32, f16, bf16 and int8 paths.  Both operands are staged in LDS as rows of
// K-contiguous 16-byte chunks, so the same skeleton serves
//   * Gemm / MatMul  (X = packed weight rows [N][K], Y = activation rows [M][K]),
//   * Conv NCHW out  (X = implicit im2col rows of an NHWC input, Y = weights),
//   * Conv NHWC out  (X = weights, Y = implicit im2col rows).
// Nothing is materialised for im2col: the loader gathers 16-byte channel
// chunks straight from the NHWC activation.
//
// Global -> LDS traffic uses the LDS DMA path (buffer_load / global_load
// dwordx4 ... lds): each wave writes 1 KiB of contiguous LDS per load, with no
// VGPR staging, and the operands run STAGES deep.  Dense operands go through
// a buffer resource: the per-lane row offset is fixed for the whole loop and
// the K position is a scalar offset, so a stage costs no vector address
// arithmetic, and rows past the matrix edge, the K tail and prefetches past
// the end read as zero through the resource's range check.  The implicit
// im2col operand redirects padding taps to a 16-byte pad source in global
// memory instead (its pad value is not always zero).
//
// The MFMAs are the 32x32 shapes, which gfx950 runs at about twice the rate
// of the 16x16 ones for f16 / bf16 and 1.4x for int8:
//   f16/bf16: v_mfma_f32_32x32x16_{f16,bf16}  (lane l: row l%32, k 8*(l/32)..+7)
//   int8    : v_mfma_i32_32x32x32_i8          (lane l: row l%32, k 16*(l/32)..+15)
//   f32     : four v_mfma_f32_32x32x2_f32     (element e of lane l's 16-byte
//             fragment is k = 4*(l/32)+e in both operands, so the sums agree)
// so a 16-byte fragment of a row is chunk 2*ks + (l/32) of the 128-byte
// stage, ks = 0..3.  The 32x32 result holds, in lane l, rows
// 8*g + 4*(l/32) .. +3 (g = 0..3) of column l%32: four runs of four
// P-consecutive outputs, which is why the side whose output index is
// memory-contiguous is always put on X.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace ohip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum class Op { F32, F16, BF16, I8 };

// Bit-cast one 32-bit lane to float.  Taking the lane by value matters:
// __builtin_bit_cast applied directly to a vector-element expression (v.y)
// reads from the start of the vector on this compiler.
__device__ __forceinline__ float lane_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

template <Op O> struct OpT;
template <> struct OpT<Op::F16> {
  using Acc = f32x16;
  using Out4 = f32x4;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
};
template <> struct OpT<Op::BF16> {
  using Acc = f32x16;
  using Out4 = f32x4;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
};
template <> struct OpT<Op::I8> {
  using Acc = i32x16;
  using Out4 = i32x4;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0,
                                                 0, 0);
  }
};
template <> struct OpT<Op::F32> {
  using Acc = f32x16;
  using Out4 = f32x4;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(lane_f32(a.x), lane_f32(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(lane_f32(a.y), lane_f32(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(lane_f32(a.z), lane_f32(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(lane_f32(a.w), lane_f32(b.w), c, 0, 0, 0);
    return c;
  }
};

// Block tile: BP x BQ outputs, WP x WQ waves, STAGES LDS buffers of one K
// slab each; a slab holds CH 16-byte chunks per row (CH = 8: 128-byte slabs,
// four MFMA k-steps; CH = 4: 64-byte slabs, two k-steps, so the same LDS
// holds twice the stages and the loads run further ahead of their use).
// static_for<N>(f): f(std::integral_constant<int, 0>{}) .. f(..N - 1), expanded
// at compile time.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F> __device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// XST > STAGES: the X operand keeps more buffers than Y and its loads run
// further ahead (XST = 3 over STAGES = 2: X two stages ahead, Y one), so a
// CU has more bytes in flight within the same LDS.
template <int BP_, int BQ_, int WP_, int WQ_, int STAGES_, int CH_ = 8, int XST_ = STAGES_> struct Tile {
  static constexpr int BP = BP_, BQ = BQ_, WP = WP_, WQ = WQ_, STAGES = STAGES_, CH = CH_, XST = XST_;
  static constexpr int KS = CH / 2;                               // MFMA k-steps per slab
  static constexpr int kWaves = WP * WQ;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int TP = BP / (WP * 32), TQ = BQ / (WQ * 32);  // 32x32 MFMA tiles per wave
  static constexpr int kRowStride = CH;                           // rows are CH * 16 bytes
  static constexpr int NX = BP * CH / kThreads;                   // DMA loads per thread per stage
  static constexpr int NY = BQ * CH / kThreads;
  static constexpr int kStage = (BP + BQ) * kRowStride;           // in u32x4 units
  // X buffers first (XST of BP rows), then the Y buffers (STAGES of BQ rows)
  static constexpr int kYBase = XST * BP * kRowStride;
  static constexpr int kStageArea = kYBase + STAGES * BQ * kRowStride;
  static_assert(CH == 8 || CH == 4, "slabs are 128 or 64 bytes");
  static_assert(TP >= 1 && TQ >= 1, "wave tile must hold at least one 32x32 MFMA tile");
  static_assert(NX * kThreads == BP * CH && NY * kThreads == BQ * CH, "loader split must be exact");
  static_assert(kWaves % 2 == 0, "the DMA swizzle phase relies on an even wave count");
  static_assert(STAGES >= 2 && kStageArea * 16 <= 160 * 1024, "LDS budget");
  static_assert(XST >= STAGES, "X runs at least as deep as Y");
};

// LDS slot of 16-byte chunk c (0..7) of staged row r.  Rows are 128 bytes
// with no padding; the slot is c ^ (r & 7) ^ ((r >> 3) & 1), which keeps
// every group of 8 consecutive rows on 8 distinct 16-byte bank groups (a
// 32-bank LDS serving 8 lanes of a b128 access per cycle) and every group of
// 16 rows on 16 distinct groups (64 banks serving 16 lanes), for both the
// row-major DMA writes and the MFMA fragment reads (rows at one chunk).
//
// For 64-byte rows (CH = 4) the slot is c ^ ((r >> 1) & 3) ^ ((r >> 3) & 1):
// the 16-byte bank group of (r, slot) is 4 * (r % 4) + slot modulo 16 (or
// 4 * (r % 2) + slot modulo 8), and this XOR makes both distinct over every
// aligned group of 16 (8) rows for each chunk c.
template <int CH> __device__ __forceinline__ int lds_slot(int r, int c) {
  if constexpr (CH == 8) return c ^ (r & 7) ^ ((r >> 3) & 1);
  else return c ^ ((r >> 1) & 3) ^ ((r >> 3) & 1);
}

// ---------------------------------------------------------------- loaders
// DMA load i of a thread (i < NR) writes 1 KiB of LDS: rows
// (i * W + w) * (64 / CH) + L / CH (W waves, w = wave, L = lane) at slot
// L % CH, so it fetches the global chunk lds_slot(r, L % CH) (the swizzle is
// its own inverse).  CH = 8: with W even, r & 7 = L / 8 and (r >> 3) & 1 =
// w & 1 for every i; CH = 4: r & 15 = L / 4.  Either way the chunk is a
// per-thread constant.
template <int CH> __device__ __forceinline__ int dma_chunk(int lane, int wave) {
  if constexpr (CH == 8) return (lane & 7) ^ (lane >> 3) ^ (wave & 1);
  else return (lane & 3) ^ ((lane >> 3) & 3) ^ ((lane >> 5) & 1);
}

__device__ __forceinline__ void dma16(const void* g, u32x4* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)(lds), 16, 0, 0);
}

// Offset that fails the range check of every dense operand's buffer
// resource (valid offsets stay below 2^31 - 1; the host checks the extent).
constexpr int kOobOffset = (int)0x80000000u;

__device__ __forceinline__ void buf16(__amdgpu_buffer_rsrc_t rs, int voff, int soff, u32x4* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(lds), 16, voff, soff, 0, 0);
}

struct DenseRows {
  const char* base;   // row 0
  int64_t ld;         // bytes between rows (multiple of 16)
  int rows;           // valid rows
  int kc;             // valid 16-byte chunks per row
  int kwrap;          // > 0: chunk g >= kwrap reads chunk g - kwrap (the operand is
                      // re-read against the second half of a split int8 weight);
                      // a multiple of 8, so a stage never straddles the wrap
  int zmod;           // batched launch: slice blockIdx.z reads matrix z % zmod
  int64_t zstride;    // bytes between those matrices

  template <int NR>
  struct State { __amdgpu_buffer_rsrc_t rs; int voff[NR]; int c; };

  template <int NR, int NW, int CH>
  __device__ __forceinline__ void init(State<NR>& s, int row0, int lane, int wave) const {
    s.c = dma_chunk<CH>(lane, wave);
    const char* b0 = zmod > 1 ? base + (int64_t)(blockIdx.z % zmod) * zstride : base;
    s.rs = __builtin_amdgcn_make_buffer_rsrc((void*)(b0 + (int64_t)row0 * ld), (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int r = (i * NW + wave) * (64 / CH) + lane / CH;
      s.voff[i] = row0 + r < rows ? (int)(r * ld) + s.c * 16 : kOobOffset;
    }
  }
  // Loads of stage kt: step() computes what the stage's loads share, load(i)
  // issues this thread's i-th 16-byte load (the kernel spreads them under its
  // MFMAs), issue() does all of them.
  struct Step { int soff; bool kin; };
  template <int NR, int NW, int CH>
  __device__ __forceinline__ Step step(const State<NR>& s, int kt) const {
    int g0 = kt * CH;                      // first chunk of the stage (uniform)
    if (kwrap > 0 && g0 >= kwrap) g0 -= kwrap;
    // K tail or past the end: chunks at or beyond kc read as zero (a select
    // per load, not a branch, so the K loop stays one basic block)
    return Step{g0 * 16, g0 + s.c < kc};
  }
  template <int NR, int NW, int CH>
  __device__ __forceinline__ void load(const State<NR>& s, const Step& st, int i, int wave, u32x4* lds_rows) const {
    buf16(s.rs, st.kin ? s.voff[i] : kOobOffset, st.soff, lds_rows + (i * NW + wave) * 64);
  }
  template <int NR, int NW, int CH>
  __device__ __forceinline__ void issue(const State<NR>& s, int kt, int wave, u32x4* lds_rows) const {
    const Step st = step<NR, NW, CH>(s, kt);
#pragma unroll
    for (int i = 0; i < NR; ++i) load<NR, NW, CH>(s, st, i, wave, lds_rows);
  }
};

// DenseRows whose rows hold whole stages (kc a multiple of the stage's CH
// chunks, no kwrap): no stage has a K tail, so no per-load select; a stage
// past the end re-reads the last one (its data is never used) and rows past
// the edge still read zero through the range check.
struct DenseRowsWhole : DenseRows {
  explicit DenseRowsWhole(const DenseRows& d) : DenseRows(d) {}
  template <int NR, int NW, int CH>
  __device__ __forceinline__ Step step(const State<NR>&, int kt) const {
    const int g0 = kt * CH < kc ? kt * CH : kc - CH;
    return Step{g0 * 16, true};
  }
  template <int NR, int NW, int CH>
  __device__ __forceinline__ void load(const State<NR>& s, const Step& st, int i, int wave, u32x4* lds_rows) const {
    buf16(s.rs, s.voff[i], st.soff, lds_rows + (i * NW + wave) * 64);
  }
  template <int NR, int NW, int CH>
  __device__ __forceinline__ void issue(const State<NR>& s, int kt, int wave, u32x4* lds_rows) const {
    const Step st = step<NR, NW, CH>(s, kt);
#pragma unroll
    for (int i = 0; i < NR; ++i) load<NR, NW, CH>(s, st, i, wave, lds_rows);
  }
};

// Implicit im2col over an NHWC activation whose channel count is padded to a
// whole number of 16-byte chunks (cpc chunks per pixel).  Row r is output
// pixel (n, oy, ox); K runs over (ky, kx, channel chunk).
struct Im2colNHWC {
  const char* base;    // x[0][0][0][0]
  int H, W, OH, OW;
  int KW;
  int cpc;             // 16-byte channel chunks per tap (the K extent of one pixel)
  int pstride;         // 16-byte chunks between pixels (>= cpc: grouped channels)
  int sh, sw, dh, dw, pt, pl;
  int rows;            // N * OH * OW
  int kc;              // KH * KW * cpc
  int kwrap;           // as DenseRows::kwrap
  const char* pad;     // 16 bytes that stand for a padding tap (and the K tail)
  int64_t zstride;     // batched launch: slice blockIdx.z reads base + z * zstride
  int zpads;           // > 0: slice z (< zpads <= 4) uses pads zpt[z], zpl[z] instead of pt, pl
  int zpt[4], zpl[4];
  uint32_t cpc_mul, kw_mul;   // g / cpc and tap / KW as (x * mul) >> shift (magic_div)
  int cpc_shift, kw_shift;

  template <int NR>
  struct State { const char* img[NR]; int iy0[NR], ix0[NR]; uint32_t okmask; int c; };

  template <int NR, int NW, int CH>
  __device__ __forceinline__ void init(State<NR>& s, int row0, int lane, int wave) const {
    s.c = dma_chunk<CH>(lane, wave);
    const int ohw = OH * OW;
    const int z = (int)blockIdx.z;
    const int pt_ = zpads > 0 ? zpt[z & 3] : pt, pl_ = zpads > 0 ? zpl[z & 3] : pl;
    s.okmask = 0;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int r = row0 + (i * NW + wave) * (64 / CH) + lane / CH;
      const bool ok = r < rows;
      s.okmask |= (ok ? 1u : 0u) << i;
      const int rr = ok ? r : 0;
      const int n = rr / ohw, rem = rr - n * ohw;
      const int oy = rem / OW, ox = rem - oy * OW;
      s.img[i] = base + (int64_t)blockIdx.z * zstride + (int64_t)n * H * W * pstride * 16;
      s.iy0[i] = oy * sh - pt_;
      s.ix0[i] = ox * sw - pl_;
    }
  }
  struct Step { int dy, dx, cc; bool kin; };
  template <int NR, int NW, int CH>
  __device__ __forceinline__ Step step(const State<NR>& s, int kt) const {
    int gk = kt * CH + s.c;
    if (kwrap > 0 && gk >= kwrap) gk -= kwrap;
    const bool kin = gk < kc;
    const int g = kin ? gk : 0;
    const int tap = (int)(((uint64_t)(uint32_t)g * cpc_mul) >> cpc_shift);
    const int cc = g - tap * cpc;
    const int ky = (int)(((uint64_t)(uint32_t)tap * kw_mul) >> kw_shift);
    const int kx = tap - ky * KW;
    return Step{ky * dh, kx * dw, cc, kin};
  }
  template <int NR, int NW, int CH>
  __device__ __forceinline__ void load(const State<NR>& s, const Step& st, int i, int wave, u32x4* lds_rows) const {
    const int iy = s.iy0[i] + st.dy, ix = s.ix0[i] + st.dx;
    const bool inside =
        st.kin && ((s.okmask >> i) & 1u) && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
    dma16(inside ? s.img[i] + ((int64_t)(iy * W + ix) * pstride + st.cc) * 16 : pad, lds_rows + (i * NW + wave) * 64);
  }
  template <int NR, int NW, int CH>
  __device__ __forceinline__ void issue(const State<NR>& s, int kt, int wave, u32x4* lds_rows) const {
    const Step st = step<NR, NW, CH>(s, kt);
#pragma unroll
    for (int i = 0; i < NR; ++i) load<NR, NW, CH>(s, st, i, wave, lds_rows);
  }
};

// Compile-time loop: f(I) for I in [0, N), always fully unrolled.
template <int I, int N> struct Unroll {
  template <class F> static __device__ __forceinline__ void run(F& f) {
    f(I);
    Unroll<I + 1, N>::run(f);
  }
};
template <int N> struct Unroll<N, N> {
  template <class F> static __device__ __forceinline__ void run(F&) {}
};

// XCD-aware tile order.  The dispatcher hands consecutive workgroup ids to
// the 8 XCDs in turn; remapping makes each XCD own a contiguous run of
// logical tiles, and the grouped order inside a run keeps GP P-tiles sharing
// the same Q-tile panel resident in that XCD's L2.
__device__ __forceinline__ void map_tile(int bid, int nb, int nP, int nQ, int gp, int& tp, int& tq) {
  int id = bid;
  if ((nb & 7) == 0) id = (bid & 7) * (nb >> 3) + (bid >> 3);
  const int per_group = gp * nQ;
  const int g = id / per_group;
  const int first = g * gp;
  const int gsz = min(nP - first, gp);
  const int within = id - g * per_group;
  tp = first + within % gsz;
  tq = within / gsz;
}

// s_waitcnt vmcnt(N) with the other counters left at their maximum (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(0) with the other counters at their maximum.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Workgroup barrier without the memory fences of __syncthreads (which would
// also wait for every outstanding LDS DMA load, draining the prefetch
// pipeline).  Callers order memory themselves: each wave waits (vmcnt) for
// its own DMA loads of the stage that the barrier publishes, and (lgkmcnt)
// for its LDS reads of the buffer that the next DMA overwrites.
__device__ __forceinline__ void barrier_only() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// XX / XY: XOR 0x80 into every byte of an X / Y fragment before the MFMA
// (turns u8 activations into u8 - 128 as int8; the pad source of such an
// operand holds its pad bytes un-XORed).
template <bool XOR> __device__ __forceinline__ u32x4 frag(u32x4 v) {
  if (XOR) v ^= 0x80808080u;
  return v;
}

// Main loop, per stage kt (STAGES LDS buffers, KS = CH / 2 MFMA k-steps a
// stage):
//   k-step 0 issues the DMA loads of stage kt + STAGES - 1 (into the buffer
//   of stage kt - 1, released by the previous stage's barrier), interleaved
//   with the MFMAs;
//   k-steps 0..KS-2 read the next k-step's fragments under the MFMAs;
//   k-step KS-1 waits until stage kt + 1 has landed, passes the barrier and
//   reads stage kt + 1's first fragments under its MFMAs,
// so the MFMA pipe is never left waiting on a barrier with no work queued.
// Where the outputs go: element (i, j) sits at
//   (i / ohw) * bstride + (i % ohw) * si + j * sj      (elements of `eb` bytes)
// with i / ohw computed as (i * ohw_mul) >> ohw_shift (exact for 0 <= i < 2^31,
// magic_div below).  vec: si == 1 and every aligned run of four i is
// contiguous and 4-element aligned in memory.
struct OutAddr {
  char* y;
  int64_t si, sj, bstride;
  int ohw;
  uint32_t ohw_mul;
  int ohw_shift;
  int P, Q;
  int vec;
  int stage;         // the staged epilogue may be used
  int batch;         // > 1: batched launch, slice blockIdx.z
  int64_t zstride;   // bytes between the slices' outputs
  int zsw;           // > 0: slice z starts (z / zsw) * zrow + (z % zsw) * zstride bytes in
  int64_t zrow;
  int defer;         // host side: a split-K launch leaves its partial sums for the caller
  __device__ __forceinline__ int64_t row(int i) const {
    if (bstride == 0) return (int64_t)i * si;
    const int n = (int)(((uint64_t)(uint32_t)i * ohw_mul) >> ohw_shift);
    return (int64_t)n * bstride + (int64_t)(i - n * ohw) * si;
  }
};

// Division by an invariant d >= 1 for dividends below 2^31: with
// s = ceil(log2 d) and m = ceil(2^(31+s) / d) (which fits 32 bits),
// floor(i * m / 2^(31+s)) == floor(i / d), because the rounding excess of m
// contributes less than i / 2^(31+s) * d / d < 2^-s <= 1/d.
inline void magic_div(int d, uint32_t* mul, int* shift) {
  int s = 0;
  while ((1ll << s) < d) ++s;
  const unsigned __int128 num = (unsigned __int128)1 << (31 + s);
  *mul = (uint32_t)((num + (unsigned)d - 1) / (unsigned)d);
  *shift = 31 + s;
}

// Stores the four outputs (rows i .. i+3, column j) whose bit patterns are
// bits[r]; row = out.row(i).
__device__ __forceinline__ void store_group(const OutAddr& out, int eb, int64_t row, int i, int j,
                                            const uint32_t (&v)[4]) {
  if (j >= out.Q) return;
  const int64_t cj = (int64_t)j * out.sj;
  if (out.vec && i + 3 < out.P) {
    char* dst = out.y + (row + cj) * eb;
    if (eb == 4) {
      *reinterpret_cast<u32x4*>(dst) = u32x4{v[0], v[1], v[2], v[3]};
    } else if (eb == 2) {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u32x2*>(dst) = u32x2{v[0] | (v[1] << 16), v[2] | (v[3] << 16)};
    } else {
      *reinterpret_cast<uint32_t*>(dst) = v[0] | (v[1] << 8) | (v[2] << 16) | (v[3] << 24);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (i + r >= out.P) break;
    char* dst = out.y + (out.row(i + r) + cj) * eb;
    if (eb == 4) *reinterpret_cast<uint32_t*>(dst) = v[r];
    else if (eb == 2) *reinterpret_cast<uint16_t*>(dst) = (uint16_t)v[r];
    else *reinterpret_cast<uint8_t*>(dst) = (uint8_t)v[r];
  }
}

#ifdef OHIP_KTIMING
// Diagnostic build only (never in the shipped library): per-block stamps of
// the 100 MHz real-time counter at kernel start, after the prologue, after
// the K loop and at the end.
extern __device__ uint64_t ohip_ktime[8 * 65536];
#define OHIP_STAMP(i) do { const uint32_t kt_b = blockIdx.y * gridDim.x + blockIdx.x; \
    if (threadIdx.x == 0 && blockIdx.z == 0 && kt_b < 65536) \
    ohip_ktime[(i) * 65536 + kt_b] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define OHIP_STAMP(i) do {} while (0)
#endif

// The block's epilogue: finishes the accumulators of the tile at (p0, q0)
// through `epi` (staged through `smem`, which holds at least
// Tl::STAGES * Tl::kStage + the row-term tail u32x4 slots, free once the
// K loop's loads have landed).  Shared by every contraction kernel.
template <Op O, class Tl, class Epi, class A>
__device__ __forceinline__ void tile_epilogue(const Epi& epi, A (&acc)[Tl::TP][Tl::TQ], u32x4* smem, int p0, int q0,
                                              int wp, int wq, int lane, int t, bool rows_ready = false) {
  using A4 = typename OpT<O>::Out4;
  const int ibase = p0 + wp * Tl::TP * 32 + (lane >> 5) * 4;
  const int jbase = q0 + wq * Tl::TQ * 32 + (lane & 31);
  OutAddr out = epi.addr();
  if (out.batch > 1) {
    const int z = (int)blockIdx.z;
    out.y += out.zsw > 0 ? (int64_t)(z / out.zsw) * out.zrow + (int64_t)(z % out.zsw) * out.zstride
                         : (int64_t)z * out.zstride;
  }

  // the per-column epilogue terms, loaded once for all of this lane's rows
  typename Epi::PreJ pj[Tl::TQ];
#pragma unroll
  for (int b = 0; b < Tl::TQ; ++b) epi.load_j(pj[b], jbase + b * 32);

  // Staged epilogue: the block's outputs go through LDS (the stage buffers
  // are free once the last loads have landed) and leave as whole 16-byte
  // chunks of output rows, instead of 4-element pieces of 32 rows per store.
  // Staged row `lj` holds outputs (p0.., q0 + lj); its 16-byte chunk c sits
  // at slot c ^ (lj % CPR) so the fragment writes spread over the banks.
  // Mode 1 stages the epilogue's narrow output (1 or 2 bytes); mode 2 stages
  // 4-byte outputs (int32, f32) when the tile's stage buffers hold them.
  constexpr int EBN = Epi::kStageBytes > 0 ? Epi::kStageBytes : 1;
  // the row terms sit past the stage buffers, or (when both do not fit the
  // LDS) at the end of them, written once every load has landed
  constexpr int kRowTerms = (int)((Tl::BP / 4 * sizeof(typename Epi::PreI) + 15) / 16);
  constexpr bool kRowsInside = (Tl::kStageArea + kRowTerms) * 16 > 160 * 1024;
  constexpr int kStageCap = (kRowsInside ? Tl::kStageArea - kRowTerms : Tl::kStageArea) * 16;
  constexpr bool kWide = Epi::kStageWide && Tl::BQ * Tl::BP * 4 <= kStageCap;
  static_assert(Epi::kStageBytes == 0 || Tl::BQ * Tl::BP * EBN <= kStageCap, "staging must fit the stage buffers");
  char* stg = reinterpret_cast<char*>(smem);
  int smode = 0;
  // the batch slice's own output must be 16-byte aligned too (the Epi checks slice 0's)
  const bool zaligned = ((uintptr_t)out.y % 16) == 0;
  if constexpr (Epi::kStageBytes > 0) smode = zaligned && epi.staged_ok(Tl::BP) ? 1 : 0;
  if constexpr (kWide) if (smode == 0 && zaligned && epi.staged_wide_ok(Tl::BP)) smode = 2;
  const bool staged = smode != 0;
  // The per-row epilogue terms of the block's BP rows, fetched once by the
  // first BP / 4 threads into LDS (one global round trip for the block; read
  // group by group from global memory they cost a round trip per group).
  // (rows_ready: the kernel stored them before its K loop)
  typename Epi::PreI* s_rows =
      reinterpret_cast<typename Epi::PreI*>(smem + (kRowsInside ? Tl::kStageArea - kRowTerms : Tl::kStageArea));
  if constexpr (kRowsInside) {
    wait_vmcnt<0>();
    wait_lgkm0();
    barrier_only();
  }
  if (!rows_ready && t < Tl::BP / 4) {
    typename Epi::PreI pr;
    epi.load_i(pr, p0 + 4 * t);
    s_rows[t] = pr;
  }
  wait_vmcnt<0>();
  wait_lgkm0();
  barrier_only();
  OHIP_STAMP(4);
  auto stage_write = [&](auto ebc, int lj, int ig, const uint32_t (&bits)[4]) __attribute__((always_inline)) {
    constexpr int EB = decltype(ebc)::value;
    constexpr int CPR = Tl::BP * EB / 16;
    const int byte = (ig - p0) * EB;
    constexpr int SWZ = (CPR & -CPR) - 1;   // XOR inside aligned power-of-two chunk groups of the row
    char* dst = stg + lj * (Tl::BP * EB) + (((byte >> 4) ^ (lj & SWZ)) << 4) + (byte & 15);
    if constexpr (EB == 4) {
      *reinterpret_cast<u32x4*>(dst) = u32x4{bits[0], bits[1], bits[2], bits[3]};
    } else if constexpr (EB == 2) {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u32x2*>(dst) = u32x2{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
    } else {
      *reinterpret_cast<uint32_t*>(dst) = bits[0] | (bits[1] << 8) | (bits[2] << 16) | (bits[3] << 24);
    }
  };

  // The lane's outputs are finished one group at a time (rows i0 + 8g .. +3
  // of every column b): the group's row terms are loaded, its four outputs per
  // column turned into bit patterns and staged or stored.  Working a group at
  // a time keeps the epilogue's live registers to a few per column, so the
  // epilogue does not set the kernel's register count (and occupancy).
  // (Compile-time loops: every accumulator index is a constant, so the
  // accumulators stay in registers however large the unrolled body is.)
  // SEB > 0: the staged path (SEB-byte staged elements: mode 1's narrow or
  // mode 2's 4-byte ones) of an epilogue whose finish reduces to a function
  // of the accumulators and the row terms alone (Epi::simple(mode), checked
  // once; branch-free groups)
  auto groups = [&](auto simple_c) __attribute__((always_inline)) {
  constexpr int SEB = decltype(simple_c)::value;   // staged bytes | 16 for the byte-table form
  constexpr int SB = SEB & 15;
  constexpr bool SIMPLE = SB > 0;
  static_for<Tl::TP * 4>([&](auto ag) __attribute__((always_inline)) {
    constexpr int a = decltype(ag)::value / 4, g = decltype(ag)::value % 4;
    const int ig = ibase + a * 32 + 8 * g;
    const typename Epi::PreI pi = s_rows[(ig - p0) >> 2];
    int64_t row = 0;
    if constexpr (!SIMPLE) if (!staged) row = out.row(ig);
    static_for<Tl::TQ>([&](auto bc) __attribute__((always_inline)) {
      constexpr int b = decltype(bc)::value;
      const int j = jbase + b * 32;
      A4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = acc[a][b][4 * g + e];
      uint32_t bits[4];
      if constexpr (SIMPLE) {
        epi.template finish_simple<SEB>(pi, v, bits);
        stage_write(std::integral_constant<int, SB>{}, j - q0, ig, bits);
        return;
      }
      epi.finish(pi, pj[b], ig, j, v, bits);
      if constexpr (Epi::kStageBytes > 0) {
        if (smode == 1) {
          stage_write(std::integral_constant<int, EBN>{}, j - q0, ig, bits);
          return;
        }
      }
      if constexpr (kWide) {
        if (smode == 2) {
          stage_write(std::integral_constant<int, 4>{}, j - q0, ig, bits);
          return;
        }
      }
      store_group(out, epi.out_bytes(), row, ig, j, bits);
    });
  });
  };
  bool done = false;
  if constexpr (Epi::kHasSimple && Epi::kStageBytes > 0) {
    if (smode == 1) {
      const int sm = epi.simple(1);   // 1: the plain form, 2: with the byte table
      if (sm == 1) { groups(std::integral_constant<int, EBN>{}); done = true; }
      if constexpr (Epi::kSimpleTable) {
        if (sm == 2) { groups(std::integral_constant<int, EBN | 16>{}); done = true; }
      }
    }
  }
  if constexpr (Epi::kHasSimple && kWide) {
    if (smode == 2 && epi.simple(2)) { groups(std::integral_constant<int, 4>{}); done = true; }
  }
  if (!done) groups(std::integral_constant<int, 0>{});

  OHIP_STAMP(5);
  auto flush = [&](auto ebc) __attribute__((always_inline)) {
    constexpr int EB = decltype(ebc)::value;
    constexpr int CPR = Tl::BP * EB / 16;   // 16-byte chunks per staged row
    constexpr int EPC = 16 / EB;            // outputs per chunk
    wait_lgkm0();
    barrier_only();
    for (int c = t; c < Tl::BQ * CPR; c += Tl::kThreads) {
      const int row = c / CPR, cc = c - row * CPR;
      const int j = q0 + row, i = p0 + cc * EPC;
      if (j >= out.Q || i >= out.P) continue;
      constexpr int SWZ = (CPR & -CPR) - 1;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + row * (Tl::BP * EB) + ((cc ^ (row & SWZ)) << 4));
      char* dst = out.y + (out.row(i) + (int64_t)j * out.sj) * EB;
      if (i + EPC <= out.P) {
        *reinterpret_cast<u32x4*>(dst) = v;
      } else {
        // the row's last, partial chunk: its bytes one at a time (shifts,
        // not a dynamically indexed copy of v, which would live in memory)
        const int nbytes = (out.P - i) * EB;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t word = v[w];
#pragma unroll
          for (int bb = 0; bb < 4; ++bb)
            if (4 * w + bb < nbytes) dst[4 * w + bb] = (char)(word >> (8 * bb));
        }
      }
    }
  };
  if constexpr (Epi::kStageBytes > 0) {
    if (smode == 1) flush(std::integral_constant<int, EBN>{});
  }
  if constexpr (kWide) {
    if (smode == 2) flush(std::integral_constant<int, 4>{});
  }
}

template <Op O, class Tl, class LX, class LY, class Epi, bool XX, bool XY>
__global__ void __launch_bounds__(Tl::kThreads)
mfma_gemm_kernel(const LX lx, const LY ly, const Epi epi, int nP, int nQ, int kc, int splits, int gp) {
  OHIP_STAMP(0);
  using A = typename OpT<O>::Acc;
  // the stage buffers, then (after the K loop) the block's per-row epilogue terms
  constexpr int kRowTerms = (int)((Tl::BP / 4 * sizeof(typename Epi::PreI) + 15) / 16);
  constexpr bool kRowsInside = (Tl::kStageArea + kRowTerms) * 16 > 160 * 1024;
  __shared__ u32x4 smem[kRowsInside ? Tl::kStageArea : Tl::kStageArea + kRowTerms];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wp = wave % Tl::WP, wq = wave / Tl::WP;
  int tp, tq;
  map_tile(blockIdx.x, gridDim.x, nP, nQ, gp, tp, tq);
  const int p0 = tp * Tl::BP, q0 = tq * Tl::BQ;

  typename LX::template State<Tl::NX> sx;
  typename LY::template State<Tl::NY> sy;
  lx.template init<Tl::NX, Tl::kWaves, Tl::CH>(sx, p0, lane, wave);
  ly.template init<Tl::NY, Tl::kWaves, Tl::CH>(sy, q0, lane, wave);

  A acc[Tl::TP][Tl::TQ];
#pragma unroll
  for (int a = 0; a < Tl::TP; ++a)
#pragma unroll
    for (int b = 0; b < Tl::TQ; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0;

  // K stages of this block: all of them, or slice blockIdx.y of `splits`
  const int nk_all = (kc + Tl::CH - 1) / Tl::CH;
  const int per = (nk_all + splits - 1) / splits;
  const int kbeg = (int)blockIdx.y * per;
  const int kend = min(kbeg + per, nk_all);
  constexpr int NL = Tl::NX + Tl::NY;     // DMA loads per thread per stage
  // Every stage issues all its loads (past the last stage they read zero or
  // the pad source), so the waits below are fixed counts of outstanding loads.
  // ring slots count stages from kbeg (so an unrolled loop knows them at
  // compile time)
  auto xbuf = [&](int kt) __attribute__((always_inline)) {
    return smem + ((kt - kbeg) % Tl::XST) * (Tl::BP * Tl::kRowStride);
  };
  auto ybuf = [&](int kt) __attribute__((always_inline)) {
    return smem + Tl::kYBase + ((kt - kbeg) % Tl::STAGES) * (Tl::BQ * Tl::kRowStride);
  };
  auto issue_x = [&](int kt) { lx.template issue<Tl::NX, Tl::kWaves, Tl::CH>(sx, kt, wave, xbuf(kt)); };
  auto issue_y = [&](int kt) { ly.template issue<Tl::NY, Tl::kWaves, Tl::CH>(sy, kt, wave, ybuf(kt)); };

  // Fragment slots of this lane: rows are tile bases (multiples of 32) plus
  // lane % 32, chunk 2 * ks + lane / 32.
  const int xr = wp * Tl::TP * 32 + (lane & 31);
  const int yr = wq * Tl::TQ * 32 + (lane & 31);
  int xslot[Tl::KS], yslot[Tl::KS];
#pragma unroll
  for (int ks = 0; ks < Tl::KS; ++ks) {
    xslot[ks] = xr * Tl::kRowStride + lds_slot<Tl::CH>(xr, 2 * ks + (lane >> 5));
    yslot[ks] = yr * Tl::kRowStride + lds_slot<Tl::CH>(yr, 2 * ks + (lane >> 5));
  }

  // The epilogue's per-row terms are loaded ahead of the first stages (their
  // round trip then overlaps the stages' instead of following the K loop)
  // and parked in LDS past the stage buffers.
  // Load order (the waits count outstanding loads): the prologue issues
  // X(kbeg), Y(kbeg), X(kbeg + 1), Y(kbeg + 1), ... up to each operand's
  // depth; stage kt issues Y(kt + STAGES - 1), then X(kt + XST - 1).  At the
  // end of stage kt, X and Y of stage kt + 1 have landed once at most
  // kAhead loads remain outstanding (the loads issued after Y(kt + 1) in the
  // steady state: that stage's X and every later stage's; earlier in the
  // loop more were, so the wait is stricter than needed, never looser);
  // after the prologue, once at most kAheadPro remain.
  constexpr int kAhead = (Tl::XST > Tl::STAGES ? Tl::NX : 0) + (Tl::STAGES - 2) * NL;
  constexpr int kAheadPro = (Tl::XST - 2) * Tl::NX + (Tl::STAGES - 2) * Tl::NY;
  {
    typename Epi::PreI pr;
    if constexpr (!kRowsInside) if (t < Tl::BP / 4) epi.load_i(pr, p0 + 4 * t);
#pragma unroll
    for (int s = 0; s < Tl::XST - 1; ++s) {
      issue_x(kbeg + s);
      if (s < Tl::STAGES - 1) issue_y(kbeg + s);
    }
    if constexpr (!kRowsInside)
      if (t < Tl::BP / 4) reinterpret_cast<typename Epi::PreI*>(smem + Tl::kStageArea)[t] = pr;
  }
  wait_vmcnt<kAheadPro>();
  barrier_only();
  OHIP_STAMP(1);

  u32x4 fx[2][Tl::TP], fy[2][Tl::TQ];
  {
    const u32x4* x0 = xbuf(kbeg);
    const u32x4* y0 = ybuf(kbeg);
#pragma unroll
    for (int a = 0; a < Tl::TP; ++a) fx[0][a] = x0[xslot[0] + a * 32 * Tl::kRowStride];
#pragma unroll
    for (int b = 0; b < Tl::TQ; ++b) fy[0][b] = y0[yslot[0] + b * 32 * Tl::kRowStride];
  }

  // One k-step in program order, fenced so the compiler keeps it: each MFMA
  // is followed by at most one fragment read for the next k-step (in the
  // order the next k-step consumes them, so the waits before its MFMAs are
  // partial) and, on k-step 0, by one DMA load of the stage STAGES - 1 ahead.
  // The last k-step reads the next stage: its first MFMAs go before the
  // stage barrier, which then overlaps them.
  constexpr int NM = Tl::TP * Tl::TQ;      // MFMAs per k-step
  constexpr int NRD = Tl::TP + Tl::TQ;     // fragment reads per k-step
  constexpr int PRE = NM >= 4 ? 2 : 0;     // MFMAs of the last k-step ahead of the barrier
  // one stage; phc: (kt - kbeg) modulo kUnroll as a compile-time constant,
  // or -1 (ring slots computed at run time)
  auto stage = [&](int kt, auto phc) __attribute__((always_inline)) {
    constexpr int ph = decltype(phc)::value;
    auto ring = [&](int d, auto isx) __attribute__((always_inline)) -> u32x4* {
      constexpr bool X = decltype(isx)::value;
      if constexpr (ph >= 0) {
        if constexpr (X) return smem + ((ph + d) % Tl::XST) * (Tl::BP * Tl::kRowStride);
        else return smem + Tl::kYBase + ((ph + d) % Tl::STAGES) * (Tl::BQ * Tl::kRowStride);
      } else {
        if constexpr (X) return xbuf(kt + d);
        else return ybuf(kt + d);
      }
    };
    const u32x4* sX = ring(0, std::true_type{});
    const u32x4* sY = ring(0, std::false_type{});
    const u32x4* snX = ring(1, std::true_type{});
    const u32x4* snY = ring(1, std::false_type{});
    u32x4* sdX = ring(Tl::XST - 1, std::true_type{});
    u32x4* sdY = ring(Tl::STAGES - 1, std::false_type{});
    const typename LX::Step stx = lx.template step<Tl::NX, Tl::kWaves, Tl::CH>(sx, kt + Tl::XST - 1);
    const typename LY::Step sty = ly.template step<Tl::NY, Tl::kWaves, Tl::CH>(sy, kt + Tl::STAGES - 1);
    // Y's loads first, then X's (the order the waits count on)
    auto dma = [&](int i) __attribute__((always_inline)) {
      if (i < Tl::NY) ly.template load<Tl::NY, Tl::kWaves, Tl::CH>(sy, sty, i, wave, sdY);
      else lx.template load<Tl::NX, Tl::kWaves, Tl::CH>(sx, stx, i - Tl::NY, wave, sdX);
    };
    static_for<Tl::KS>([&](auto ksc) __attribute__((always_inline)) {
      constexpr int ks = decltype(ksc)::value;
      constexpr bool last = ks == Tl::KS - 1;
      constexpr int cur = ks & 1, nxt = cur ^ 1;
      const u32x4* srcX = last ? snX : sX;
      const u32x4* srcY = last ? snY : sY;
      const int kr = last ? 0 : ks + 1;
      // read r of the next k-step: fx[0], fy[0 .. TQ-1], fx[1 .. TP-1]
      auto read = [&](auto rc) __attribute__((always_inline)) {
        constexpr int r = decltype(rc)::value;
        if constexpr (r == 0) fx[nxt][0] = srcX[xslot[kr]];
        else if constexpr (r <= Tl::TQ) fy[nxt][r - 1] = srcY[yslot[kr] + (r - 1) * 32 * Tl::kRowStride];
        else fx[nxt][r - Tl::TQ] = srcX[xslot[kr] + (r - Tl::TQ) * 32 * Tl::kRowStride];
      };
      static_for<NM>([&](auto mc) __attribute__((always_inline)) {
        constexpr int m = decltype(mc)::value;
        constexpr int a = m / Tl::TQ, b = m % Tl::TQ;
        if constexpr (last && m == PRE) {
          wait_vmcnt<kAhead>();
          wait_lgkm0();
          barrier_only();
        }
        acc[a][b] = OpT<O>::mma(frag<XX>(fx[cur][a]), frag<XY>(fy[cur][b]), acc[a][b]);
        __builtin_amdgcn_sched_barrier(0);
        constexpr int r = last ? m - PRE : m;
        if constexpr (r >= 0 && r < NRD) read(std::integral_constant<int, r>{});
        if constexpr (ks == 0 && m < NL) dma(m);
        __builtin_amdgcn_sched_barrier(0);
      });
      // the reads and loads that outnumber the MFMAs (small tiles)
      static_for<(NRD > NM - (last ? PRE : 0) ? NRD - (NM - (last ? PRE : 0)) : 0)>([&](auto rc) __attribute__((always_inline)) {
        constexpr int r = NM - (last ? PRE : 0) + decltype(rc)::value;
        read(std::integral_constant<int, r>{});
      });
      if constexpr (ks == 0) {
        static_for<(NL > NM ? NL - NM : 0)>([&](auto ic) __attribute__((always_inline)) { dma(NM + decltype(ic)::value); });
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // A ring of three (tile 16's X ring, the three-stage tiles' rings) would
  // take a division per ring slot per stage: such a loop runs lcm(XST,
  // STAGES) stages a trip with every slot a constant, the last part trip
  // stage by stage.  Power-of-two rings keep the plain loop (a mask).
  constexpr bool kPow2 = (Tl::XST & (Tl::XST - 1)) == 0 && (Tl::STAGES & (Tl::STAGES - 1)) == 0;
  constexpr int kLcm = Tl::XST == Tl::STAGES ? Tl::XST : Tl::XST * Tl::STAGES;
  constexpr int kUnroll = !kPow2 && kLcm <= 6 ? kLcm : 1;
  if constexpr (kUnroll > 1) {
    int kt = kbeg;
    for (; kt + kUnroll <= kend; kt += kUnroll)
      static_for<kUnroll>([&](auto u) __attribute__((always_inline)) { stage(kt + decltype(u)::value, u); });
    static_for<kUnroll - 1>([&](auto u) __attribute__((always_inline)) {
      if (kt + decltype(u)::value < kend) stage(kt + decltype(u)::value, u);
    });
  } else {
    for (int kt = kbeg; kt < kend; ++kt) stage(kt, std::integral_constant<int, -1>{});
  }

  OHIP_STAMP(2);
  tile_epilogue<O, Tl>(epi, acc, smem, p0, q0, wp, wq, lane, t, !kRowsInside);
  OHIP_STAMP(3);
}

// Split-K: slice s of the K loop stores its raw accumulators (f32, or i32
// modulo 2^32) at ws[(s * Q + j) * Pp + i]; the reduction adds the slices in
// slice order and hands each run of four sums to the real epilogue.
template <class T> struct PartialEpi {
  T* ws;
  int P, Pp, Q;
  static constexpr bool kHasSimple = false;   // (simple() / finish_simple() are never called)
  static constexpr bool kSimpleTable = false;
  __device__ __forceinline__ int simple(int) const { return 0; }
  struct PreI {};
  template <int EB, class A> __device__ __forceinline__ void finish_simple(const PreI&, A, uint32_t (&)[4]) const {}
  static constexpr int kStageBytes = 0;
  static constexpr bool kStageWide = false;
  __device__ __forceinline__ bool staged_ok(int) const { return false; }
  __device__ __forceinline__ bool staged_wide_ok(int) const { return false; }
  struct PreJ {};
  __device__ __forceinline__ void load_i(PreI&, int) const {}
  __device__ __forceinline__ void load_j(PreJ&, int) const {}
  __device__ __forceinline__ int out_bytes() const { return 4; }
  __device__ __forceinline__ OutAddr addr() const {
    OutAddr o{};
    o.y = reinterpret_cast<char*>(ws + (int64_t)blockIdx.y * Q * Pp);
    o.si = 1; o.sj = Pp; o.bstride = 0; o.ohw = 1; o.P = P; o.Q = Q; o.vec = 1;
    return o;
  }
  template <class A>
  __device__ __forceinline__ void finish(const PreI&, const PreJ&, int, int, A acc, uint32_t (&bits)[4]) const {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const auto e = acc[k];   // by value: a bit_cast of the element expression itself reads lane 0
      bits[k] = __builtin_bit_cast(uint32_t, e);
    }
  }
};

template <class T, class A, class Epi>
__global__ void __launch_bounds__(256) split_reduce_kernel(const T* __restrict__ ws, int splits, int P, int Pp, int Q,
                                                           const Epi epi) {
  const int groups = Pp / 4;
  const int64_t n = (int64_t)groups * Q;
  const int64_t slice = (int64_t)Q * Pp;   // elements per K slice
  const OutAddr out = epi.addr();
  for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < n; g += (int64_t)gridDim.x * 256) {
    // n < 2^31 for every workspace the host sizes, so the index split is 32-bit
    const int gi = (int)g;
    const int j = gi / groups, i0 = (gi - j * groups) * 4;
    typename Epi::PreI pi;
    typename Epi::PreJ pj;
    epi.load_i(pi, i0);
    epi.load_j(pj, j);
    const T* src = ws + (int64_t)j * Pp + i0;
    auto ld = [&](const T* p) __attribute__((always_inline)) { return *reinterpret_cast<const A*>(p); };
    // each group of four slices loaded before its adds (one round trip per
    // group, not per slice); the adds stay in slice order, slice 0 starts
    A acc;
    for (int s0 = 0; s0 < splits; s0 += 4) {
      A v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (s0 + u < splits) v[u] = ld(src + (s0 + u) * slice);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (s0 + u < splits) acc = s0 + u == 0 ? v[u] : acc + v[u];
    }
    uint32_t bits[4];
    epi.finish(pi, pj, i0, j, acc, bits);
    store_group(out, epi.out_bytes(), out.row(i0), i0, j, bits);
  }
}

}  // namespace ohip
