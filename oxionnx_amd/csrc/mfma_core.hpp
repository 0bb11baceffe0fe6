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
// Per 64-lane wave and per 16-byte fragment pair the engine issues
//   f16/bf16: one v_mfma_f32_16x16x32_{f16,bf16}
//   int8    : one v_mfma_i32_16x16x64_i8
//   f32     : four v_mfma_f32_16x16x4_f32 (lane group g supplies k = 4g+e for
//             the e-th instruction in both operands, so the sums agree)
// and the 16x16 result lands with lane l holding rows 4*(l/16)..+3 of column
// l%16: each lane owns four P-consecutive outputs, which is why the side whose
// output index is memory-contiguous is always put on X.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ohip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum class Op { F32, F16, BF16, I8 };

// Bit-cast one 32-bit lane to float.  Taking the lane by value matters:
// __builtin_bit_cast applied directly to a vector-element expression (v.y)
// reads from the start of the vector on this compiler.
__device__ __forceinline__ float lane_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

template <Op O> struct OpT;
template <> struct OpT<Op::F16> {
  using Acc = f32x4;
  static constexpr int kElemBytes = 2;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct OpT<Op::BF16> {
  using Acc = f32x4;
  static constexpr int kElemBytes = 2;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct OpT<Op::I8> {
  using Acc = i32x4;
  static constexpr int kElemBytes = 1;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                                 __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
  }
};
template <> struct OpT<Op::F32> {
  using Acc = f32x4;
  static constexpr int kElemBytes = 4;
  static __device__ __forceinline__ Acc mma(u32x4 a, u32x4 b, Acc c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(lane_f32(a.x), lane_f32(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(lane_f32(a.y), lane_f32(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(lane_f32(a.z), lane_f32(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(lane_f32(a.w), lane_f32(b.w), c, 0, 0, 0);
    return c;
  }
};

// Block tile: BP x BQ outputs, WP x WQ waves, one 128-byte K slab per stage.
template <int BP_, int BQ_, int WP_, int WQ_> struct Tile {
  static constexpr int BP = BP_, BQ = BQ_, WP = WP_, WQ = WQ_;
  static constexpr int kThreads = 64 * WP * WQ;
  static constexpr int TP = BP / (WP * 16), TQ = BQ / (WQ * 16);
  static constexpr int kChunks = 8;          // 16-byte chunks per row per stage
  static constexpr int kRowStride = 8;       // rows are 128 B; chunks are XOR-swizzled (lds_slot)
  static constexpr int NX = BP * kChunks / kThreads;
  static constexpr int NY = BQ * kChunks / kThreads;
  static constexpr int kStage = (BP + BQ) * kRowStride;  // in u32x4 units
  static_assert(TP >= 1 && TQ >= 1, "wave tile must hold at least one 16x16 MFMA tile");
  static_assert(NX >= 1 && NY >= 1 && NX * kThreads == BP * kChunks && NY * kThreads == BQ * kChunks,
                "loader split must be exact");
};

// ---------------------------------------------------------------- loaders
// A loader owns NR rows of one operand for the lifetime of the block.  Thread
// t loads chunk (t & 7) of rows (t >> 3) + i * (threads / 8), i < NR.
//
// load() only issues the 16-byte global loads -- every address is clamped
// into the operand, so no branch and no wait sits between them -- and returns
// a bit mask of which rows hold real data.  fix() runs after the MFMAs of the
// current stage, when the loads have landed: it applies the u8 -> int8 shift
// and substitutes the pad value for out-of-range rows, chunks and taps.
struct DenseRows {
  const char* base;   // row 0
  int64_t ld;         // bytes between rows (multiple of 16)
  int rows;           // valid rows
  int kc;             // valid 16-byte chunks per row
  int kwrap;          // > 0: chunk g >= kwrap reads chunk g - kwrap (the operand is
                      // re-read against the second half of a split int8 weight)
  uint32_t xor_mask;  // applied to every loaded dword (u8 -> int8 shift uses 0x80808080)
  u32x4 pad;          // value used outside the matrix

  template <int NR, int kThreads>
  struct State { const char* ptr[NR]; uint32_t okmask; };

  template <int NR, int kThreads>
  __device__ __forceinline__ void init(State<NR, kThreads>& s, int row0, int t) const {
    s.okmask = 0;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      int r = row0 + (t >> 3) + i * (kThreads / 8);
      const bool ok = r < rows;
      s.okmask |= (ok ? 1u : 0u) << i;
      s.ptr[i] = base + (int64_t)(ok ? r : 0) * ld;
    }
  }
  template <int NR, int kThreads>
  __device__ __forceinline__ uint32_t load(const State<NR, kThreads>& s, int kt, int t, u32x4 (&v)[NR]) const {
    int gk = kt * 8 + (t & 7);
    if (kwrap > 0 && gk >= kwrap) gk -= kwrap;
    const bool kin = gk < kc;
    const int64_t off = (int64_t)(kin ? gk : 0) * 16;
#pragma unroll
    for (int i = 0; i < NR; ++i) v[i] = *reinterpret_cast<const u32x4*>(s.ptr[i] + off);
    return kin ? s.okmask : 0u;
  }
  template <int NR>
  __device__ __forceinline__ void fix(u32x4 (&v)[NR], uint32_t valid) const {
    if (xor_mask) {
#pragma unroll
      for (int i = 0; i < NR; ++i) v[i] ^= xor_mask;
    }
    if (valid != (1u << NR) - 1u) {  // only edge tiles, K tails and padding taps
#pragma unroll
      for (int i = 0; i < NR; ++i) v[i] = ((valid >> i) & 1u) ? v[i] : pad;
    }
  }
};

// Implicit im2col over an NHWC activation whose channel count is padded to a
// whole number of 16-byte chunks (cpc chunks per pixel).  Row r is output
// pixel (n, oy, ox); K runs over (ky, kx, channel chunk).
struct Im2colNHWC {
  const char* base;    // x[0][0][0][0]
  int H, W, OH, OW;
  int KW;
  int cpc;             // 16-byte channel chunks per pixel
  int sh, sw, dh, dw, pt, pl;
  int rows;            // N * OH * OW
  int kc;              // KH * KW * cpc
  int kwrap;           // as DenseRows::kwrap
  uint32_t xor_mask;
  u32x4 pad;           // value of a padding tap (already in the shifted domain)

  template <int NR, int kThreads>
  struct State { const char* img[NR]; int iy0[NR], ix0[NR]; uint32_t okmask; };

  template <int NR, int kThreads>
  __device__ __forceinline__ void init(State<NR, kThreads>& s, int row0, int t) const {
    const int ohw = OH * OW;
    s.okmask = 0;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      int r = row0 + (t >> 3) + i * (kThreads / 8);
      const bool ok = r < rows;
      s.okmask |= (ok ? 1u : 0u) << i;
      int rr = ok ? r : 0;
      int n = rr / ohw, rem = rr - n * ohw;
      int oy = rem / OW, ox = rem - oy * OW;
      s.img[i] = base + (int64_t)n * H * W * cpc * 16;
      s.iy0[i] = oy * sh - pt;
      s.ix0[i] = ox * sw - pl;
    }
  }
  template <int NR, int kThreads>
  __device__ __forceinline__ uint32_t load(const State<NR, kThreads>& s, int kt, int t, u32x4 (&v)[NR]) const {
    int gk = kt * 8 + (t & 7);
    if (kwrap > 0 && gk >= kwrap) gk -= kwrap;
    const bool kin = gk < kc;
    const int g = kin ? gk : 0;
    const int tap = g / cpc;
    const int cc = g - tap * cpc;
    const int ky = tap / KW;
    const int kx = tap - ky * KW;
    const int dy = ky * dh, dx = kx * dw;
    uint32_t valid = 0;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int iy = s.iy0[i] + dy, ix = s.ix0[i] + dx;
      const bool inside = (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
      valid |= (inside ? 1u : 0u) << i;
      const int64_t off = inside ? ((int64_t)(iy * W + ix) * cpc + cc) * 16 : 0;
      v[i] = *reinterpret_cast<const u32x4*>(s.img[i] + off);
    }
    return kin ? (valid & s.okmask) : 0u;
  }
  template <int NR>
  __device__ __forceinline__ void fix(u32x4 (&v)[NR], uint32_t valid) const {
    if (xor_mask) {
#pragma unroll
      for (int i = 0; i < NR; ++i) v[i] ^= xor_mask;
    }
    if (valid != (1u << NR) - 1u) {  // only edge tiles, K tails and padding taps
#pragma unroll
      for (int i = 0; i < NR; ++i) v[i] = ((valid >> i) & 1u) ? v[i] : pad;
    }
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

// LDS slot of 16-byte chunk c (0..7) of staged row r.  Rows are 128 bytes
// with no padding; the slot is c ^ (r & 7) ^ ((r >> 3) & 1), which keeps
// every group of 8 consecutive rows on 8 distinct 16-byte bank groups (a
// 32-bank LDS serving 8 lanes of a b128 access per cycle) and every group of
// 16 rows on 16 distinct groups (64 banks serving 16 lanes), for both the
// row-major stores and the MFMA fragment reads (16 rows at one chunk).
__device__ __forceinline__ int lds_slot(int r, int c) { return c ^ (r & 7) ^ ((r >> 3) & 1); }

// XCD-aware tile order.  The dispatcher hands consecutive workgroup ids to
// the 8 XCDs in turn; remapping makes each XCD own a contiguous run of
// logical tiles, and the grouped order inside a run keeps GP P-tiles sharing
// the same Q-tile panel resident in that XCD's L2.
__device__ __forceinline__ void map_tile(int bid, int nb, int nP, int nQ, int& tp, int& tq) {
  int id = bid;
  if ((nb & 7) == 0) id = (bid & 7) * (nb >> 3) + (bid >> 3);
  constexpr int GP = 8;
  const int per_group = GP * nQ;
  const int g = id / per_group;
  const int first = g * GP;
  const int gsz = min(nP - first, GP);
  const int within = id - g * per_group;
  tp = first + within % gsz;
  tq = within / gsz;
}

template <Op O, class Tl, class LX, class LY, class Epi>
__global__ void __launch_bounds__(Tl::kThreads)
mfma_gemm_kernel(const LX lx, const LY ly, const Epi epi, int nP, int nQ, int kc) {
  using A = typename OpT<O>::Acc;
  __shared__ u32x4 smem[2 * Tl::kStage];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wp = wave % Tl::WP, wq = wave / Tl::WP;
  int tp, tq;
  map_tile(blockIdx.x, gridDim.x, nP, nQ, tp, tq);
  const int p0 = tp * Tl::BP, q0 = tq * Tl::BQ;

  typename LX::template State<Tl::NX, Tl::kThreads> sx;
  typename LY::template State<Tl::NY, Tl::kThreads> sy;
  lx.init(sx, p0, t);
  ly.init(sy, q0, t);

  u32x4 rx[Tl::NX], ry[Tl::NY];
  A acc[Tl::TP][Tl::TQ];
#pragma unroll
  for (int a = 0; a < Tl::TP; ++a)
#pragma unroll
    for (int b = 0; b < Tl::TQ; ++b) acc[a][b] = A{0, 0, 0, 0};

  const int nk = (kc + 7) >> 3;
  const int srow = t >> 3, schunk = t & 7;

  auto stash = [&](int stage, uint32_t vx, uint32_t vy) {
    lx.fix(rx, vx);
    ly.fix(ry, vy);
    u32x4* s = smem + stage * Tl::kStage;
#pragma unroll
    for (int i = 0; i < Tl::NX; ++i) {
      const int r = srow + i * (Tl::kThreads / 8);
      s[r * Tl::kRowStride + lds_slot(r, schunk)] = rx[i];
    }
#pragma unroll
    for (int i = 0; i < Tl::NY; ++i) {
      const int r = Tl::BP + srow + i * (Tl::kThreads / 8);
      s[r * Tl::kRowStride + lds_slot(r, schunk)] = ry[i];
    }
  };

  if (nk > 0) {
    const uint32_t vx = lx.load(sx, 0, t, rx);
    const uint32_t vy = ly.load(sy, 0, t, ry);
    stash(0, vx, vy);
  }
  __syncthreads();

  // Fragment rows of this lane; every 16-row tile starts at a multiple of 16,
  // so the slot pattern of (lane & 15) is the same for every tile.
  const int xr = wp * Tl::TP * 16 + (lane & 15);
  const int yr = Tl::BP + wq * Tl::TQ * 16 + (lane & 15);
  int xslot[2], yslot[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    xslot[kk] = xr * Tl::kRowStride + lds_slot(xr, kk * 4 + (lane >> 4));
    yslot[kk] = yr * Tl::kRowStride + lds_slot(yr, kk * 4 + (lane >> 4));
  }

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    uint32_t vx = 0, vy = 0;
    if (more) {
      vx = lx.load(sx, kt + 1, t, rx);
      vy = ly.load(sy, kt + 1, t, ry);
    }
    const u32x4* s = smem + cur * Tl::kStage;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 fx[Tl::TP], fy[Tl::TQ];
#pragma unroll
      for (int a = 0; a < Tl::TP; ++a) fx[a] = s[xslot[kk] + a * 16 * Tl::kRowStride];
#pragma unroll
      for (int b = 0; b < Tl::TQ; ++b) fy[b] = s[yslot[kk] + b * 16 * Tl::kRowStride];
#pragma unroll
      for (int a = 0; a < Tl::TP; ++a)
#pragma unroll
        for (int b = 0; b < Tl::TQ; ++b) acc[a][b] = OpT<O>::mma(fx[a], fy[b], acc[a][b]);
    }
    if (more) stash(cur ^ 1, vx, vy);
    __syncthreads();
  }

  const int ibase = p0 + wp * Tl::TP * 16 + (lane >> 4) * 4;
  const int jbase = q0 + wq * Tl::TQ * 16 + (lane & 15);
  auto out = [&](int ab) {
    const int a = ab / Tl::TQ, b = ab % Tl::TQ;
    epi.store(ibase + a * 16, jbase + b * 16, acc[a][b]);
  };
  Unroll<0, Tl::TP * Tl::TQ>::run(out);
}

}  // namespace ohip
