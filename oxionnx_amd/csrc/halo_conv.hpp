// Halo-patch convolution: stride 1, dilation 1, KH x KW taps, one group,
// NHWC input.  The engine's implicit-im2col loader fetches every tap's
// channel chunk of every output pixel from global memory (KH * KW reads of
// each input byte per output tile); here a block stages, per channel slab,
// the input patch its output rows need (TH + KH - 1 rows of OW + KW - 1
// pixels, padding read as zero) ONCE in LDS, and the KH * KW taps read their
// MFMA fragments from that patch at a pixel offset of ky * PW + kx.  The
// filter slab (the KH * KW taps of CC channel chunks for the block's output
// channels) is staged next to it.  Per FLOP the block then fetches the
// filter bytes plus about (TH + KH - 1)(OW + KW - 1) / (TH * OW * KH * KW)
// of the activation bytes the im2col gather would: on the 512-channel 3x3
// conv at 32x32 a stage is 29 KiB against the 72 KiB the engine's 64x64
// tiles fetch for the same MFMA work.  That matters because a CU's vector
// memory path delivers a fixed number of outstanding cache lines per L2
// round trip (about 40-50 GB/s per CU here), which is what bounds these
// mid-size convolutions, not the MFMA rate.
//
// A pixel tile is TH whole output rows of one image (TH * OW = the tile's
// pixel extent), so its outputs are a contiguous run of the GEMM's pixel
// index and the engine's epilogues (float, split-K partials) apply
// unchanged.  PIX_ON_X puts the pixels on the X side (P = pixels, NCHW
// output, contiguous along pixels), otherwise the filter rows are X
// (P = output channels, NHWC output).
//
// LDS: a stage is [filter rows x (taps x CC chunks)] then [patch pixels x CC
// chunks], 16-byte chunks XOR-swizzled within each row so that 16
// consecutive rows (filter rows, or patch pixels at any starting offset)
// read at one logical chunk fall on 16 distinct bank groups.  The DMA
// loads write 1 KiB of contiguous LDS each; load m of a stage belongs to
// wave m % waves, so the per-wave load count (and with it the vmcnt waits)
// is one of two compile-time values.
#pragma once
#include "internal.hpp"
#include "mfma_core.hpp"
#include "norm_stats.hpp"

namespace ohip {

template <int BP_, int BQ_, int WP_, int WQ_, int CC_, int STAGES_, int KH_, int KW_, int PIXMAX_, bool PIX_ON_X_>
struct HaloTile {
  static constexpr int BP = BP_, BQ = BQ_, WP = WP_, WQ = WQ_, CC = CC_, STAGES = STAGES_;
  static constexpr int KH = KH_, KW = KW_, TAPS = KH * KW, PIXMAX = PIXMAX_;
  static constexpr bool PIX_ON_X = PIX_ON_X_;
  static constexpr int kWaves = WP * WQ, kThreads = 64 * kWaves;
  static constexpr int TP = BP / (WP * 32), TQ = BQ / (WQ * 32);
  static constexpr int BPIX = PIX_ON_X ? BP : BQ, BCO = PIX_ON_X ? BQ : BP;
  static constexpr int RW = TAPS * CC;                    // chunks per staged filter row
  static constexpr int WI = BCO * RW / 64;                // filter DMA loads per stage
  static constexpr int PI = (PIXMAX * CC + 63) / 64;      // patch DMA loads per stage
  static constexpr int TI = WI + PI;
  static constexpr int kStage = TI * 64;                  // u32x4 slots per stage
  static constexpr int kStageArea = STAGES * kStage;
  static constexpr int NLO = TI / kWaves, NHI = (TI + kWaves - 1) / kWaves;
  static_assert(CC == 2 || CC == 4, "slabs of 2 or 4 chunks");
  static_assert(BCO * RW % 64 == 0, "filter slab must be whole DMA loads");
  static_assert(TP >= 1 && TQ >= 1, "wave tile must hold a 32x32 MFMA tile");
  static_assert(STAGES >= 2 && STAGES * kStage * 16 + 4096 <= 160 * 1024, "LDS budget");
  static_assert(2 * NHI < 64, "vmcnt range");
};

// bank-group swizzle of a row's chunks (row stride a multiple of CC chunks)
template <int CC> __device__ __forceinline__ int halo_swz(int r) {
  if constexpr (CC == 2) return (r >> 3) & 1;
  else return (r >> 2) & 3;
}

template <Op O, class Ht, class Epi>
__global__ void __launch_bounds__(Ht::kThreads)
halo_conv_kernel(const HaloGeo g, const Epi epi, int nP, int nQ, int splits, int gp) {
  OHIP_STAMP(0);
  using A = typename OpT<O>::Acc;
  constexpr int CC = Ht::CC;
  constexpr int kRowTerms = (int)((Ht::BP / 4 * sizeof(typename Epi::PreI) + 15) / 16);
  __shared__ u32x4 smem[Ht::STAGES * Ht::kStage + kRowTerms];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wp = wave % Ht::WP, wq = wave / Ht::WP;
  int tp, tq;
  map_tile(blockIdx.x, gridDim.x, nP, nQ, gp, tp, tq);
  const int p0 = tp * Ht::BP, q0 = tq * Ht::BQ;
  const int pix0 = Ht::PIX_ON_X ? p0 : q0;
  const int co0 = Ht::PIX_ON_X ? q0 : p0;
  const int ohw = g.OH * g.OW;
  const int n = pix0 / ohw;
  const int oy0 = (pix0 - n * ohw) >> g.ow_shift;
  const int PW = g.OW + Ht::KW - 1;
  const int npix = (g.th + Ht::KH - 1) * PW;

  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.w + (int64_t)co0 * g.ldw), (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.x + (int64_t)n * g.img_bytes), (short)0, 0x7fffffff, 0x00020000);

  // this thread's share of a stage's DMA loads: global offset at slab 0 and
  // the channel chunk within the slab (for the channel tail)
  int voff[Ht::NHI], sub[Ht::NHI];
#pragma unroll
  for (int i = 0; i < Ht::NHI; ++i) {
    const int m = i * Ht::kWaves + wave;
    voff[i] = kOobOffset;
    sub[i] = 0;
    if (m < Ht::WI) {
      const int slot = m * 64 + lane;
      const int row = slot / Ht::RW, phys = slot - row * Ht::RW;
      const int c = phys ^ halo_swz<CC>(row);
      const int tap = c / CC, s = c - tap * CC;
      sub[i] = s;
      if (co0 + row < g.cout) voff[i] = (int)(row * g.ldw) + (tap * g.cpc + s) * 16;
    } else if (m < Ht::TI) {
      const int slot = (m - Ht::WI) * 64 + lane;
      const int pix = slot / CC, phys = slot - pix * CC;
      const int c = phys ^ halo_swz<CC>(pix);
      const int py = pix / PW, px = pix - py * PW;
      int iy = oy0 + py - g.pt, ix = px - g.pl;
      if (g.pad_mode == 1) {          // reflect (pads below the extent; the host checks)
        iy = iy < 0 ? -iy : (iy >= g.H ? 2 * g.H - 2 - iy : iy);
        ix = ix < 0 ? -ix : (ix >= g.W ? 2 * g.W - 2 - ix : ix);
      } else if (g.pad_mode == 2) {   // edge
        iy = iy < 0 ? 0 : (iy >= g.H ? g.H - 1 : iy);
        ix = ix < 0 ? 0 : (ix >= g.W ? g.W - 1 : ix);
      }
      sub[i] = c;
      if (pix < npix && (unsigned)iy < (unsigned)g.H && (unsigned)ix < (unsigned)g.W)
        voff[i] = ((iy * g.W + ix) * g.pstride + c) * 16;
    }
  }

  const int nslab = (g.cpc + CC - 1) / CC;
  const int per = (nslab + splits - 1) / splits;
  const int sbeg = (int)blockIdx.y * per;
  const int send = min(sbeg + per, nslab);
  // Every stage issues the same loads (past the last slab, and in the
  // channel tail, they read zero through the range check), so the waits are
  // fixed counts.
  auto issue = [&](int s) __attribute__((always_inline)) {
    u32x4* base = smem + (s % Ht::STAGES) * Ht::kStage;
    const bool live = s < send;
    const int soff = s * CC * 16;
#pragma unroll
    for (int i = 0; i < Ht::NHI; ++i) {
      const int m = i * Ht::kWaves + wave;
      if (m < Ht::TI) {
        const int off = live && s * CC + sub[i] < g.cpc ? voff[i] : kOobOffset;
        buf16(m < Ht::WI ? rw : rx, off, soff, base + m * 64);
      }
    }
  };
  auto wait_stages = [&](auto kc) __attribute__((always_inline)) {
    constexpr int K = decltype(kc)::value;
    if (wave < Ht::TI % Ht::kWaves) wait_vmcnt<K * Ht::NHI>();
    else wait_vmcnt<K * Ht::NLO>();
  };

  // fragment slots: filter rows (chunk t * CC + 2u + lane / 32, swizzled),
  // patch pixels (tap offset added per tap)
  constexpr int TCO = Ht::PIX_ON_X ? Ht::TQ : Ht::TP;
  constexpr int TPX = Ht::PIX_ON_X ? Ht::TP : Ht::TQ;
  const int wco = Ht::PIX_ON_X ? wq : wp, wpx = Ht::PIX_ON_X ? wp : wq;
  const int hi = lane >> 5;
  int wslot[TCO][CC / 2];
#pragma unroll
  for (int c = 0; c < TCO; ++c) {
    const int row = wco * TCO * 32 + c * 32 + (lane & 31);
#pragma unroll
    for (int u = 0; u < CC / 2; ++u) wslot[c][u] = row * Ht::RW + ((2 * u + hi) ^ halo_swz<CC>(row));
  }
  int pbase[TPX];
#pragma unroll
  for (int b = 0; b < TPX; ++b) {
    const int ql = wpx * TPX * 32 + b * 32 + (lane & 31);
    const int qy = ql >> g.ow_shift, qx = ql & (g.OW - 1);
    pbase[b] = qy * PW + qx;
  }

  A acc[Ht::TP][Ht::TQ];
#pragma unroll
  for (int a = 0; a < Ht::TP; ++a)
#pragma unroll
    for (int b = 0; b < Ht::TQ; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0;

#pragma unroll
  for (int s = 0; s < Ht::STAGES - 1; ++s) issue(sbeg + s);
  wait_stages(std::integral_constant<int, Ht::STAGES - 2>{});
  barrier_only();
  OHIP_STAMP(1);

  for (int s = sbeg; s < send; ++s) {
    issue(s + Ht::STAGES - 1);
    const u32x4* S = smem + (s % Ht::STAGES) * Ht::kStage;
    const u32x4* SP = S + Ht::WI * 64;
    static_for<Ht::TAPS>([&](auto tc) __attribute__((always_inline)) {
      constexpr int tap = decltype(tc)::value;
      constexpr int ky = tap / Ht::KW, kx = tap % Ht::KW;
      const int toff = ky * PW + kx;
      static_for<CC / 2>([&](auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
        u32x4 wf[TCO], pf[TPX];
#pragma unroll
        for (int c = 0; c < TCO; ++c) wf[c] = S[wslot[c][u] + tap * CC];
#pragma unroll
        for (int b = 0; b < TPX; ++b) {
          const int pix = pbase[b] + toff;
          pf[b] = SP[pix * CC + ((2 * u + hi) ^ halo_swz<CC>(pix))];
        }
#pragma unroll
        for (int a = 0; a < Ht::TP; ++a)
#pragma unroll
          for (int b = 0; b < Ht::TQ; ++b) {
            if constexpr (Ht::PIX_ON_X) acc[a][b] = OpT<O>::mma(pf[a], wf[b], acc[a][b]);
            else acc[a][b] = OpT<O>::mma(wf[a], pf[b], acc[a][b]);
          }
      });
    });
    wait_stages(std::integral_constant<int, Ht::STAGES - 2>{});
    wait_lgkm0();
    barrier_only();
  }
  OHIP_STAMP(2);
  tile_epilogue<O, Ht>(epi, acc, smem, p0, q0, wp, wq, lane, t);
  OHIP_STAMP(3);
}

}  // namespace ohip

namespace ohip {

// Whole-K halo convolution (wk_conv_kernel): 3x3, stride 1, one group, NHWC
// input, for mid-size convolutions whose output (pixels x channels) is too
// small to give every CU a block of the halo kernel's 256 x 64 tiles
// without splitting K.  A block takes NPT * 32 pixels (TH whole output rows
// of one image) x 32 output channels over the whole reduction, so nothing
// leaves the block but its outputs (no split-K partial sums, no reduction
// launch): with 32 x 32 images and 512 channels that is 16 x 16 = 256
// blocks.  Per stage (a slab of CC 16-byte channel chunks) the block DMA-
// loads the 32 filter rows' slab (9 taps x CC chunks a row) and the input
// patch of its rows ((TH + 2) x (OW + 2) pixels x CC chunks) into LDS with
// the halo kernel's layout and swizzle (whole 128-byte lines at CC = 8).
// The block's waves split the MFMA work instead of the output: wave
// (pt, ks) takes pixel tile pt (32 pixels) and k-step ks of every slab, for
// all nine taps, so each wave holds one 32 x 32 accumulator; after the K
// loop the partial tiles meet in LDS and are added in k-step order (a fixed
// order: the result does not depend on timing), and waves 0 .. NPT - 1 run
// the float epilogue on their pixel tile.
template <int OW_, int NPT_, int CC_, int STAGES_, bool PIX_ON_X_>
struct WkTile {
  static constexpr int OW = OW_, NPT = NPT_, CC = CC_, STAGES = STAGES_;
  static constexpr bool PIX_ON_X = PIX_ON_X_;
  static constexpr int TH = NPT * 32 / OW, PW = OW + 2, NPIX = (TH + 2) * PW;
  static constexpr int KSN = CC / 2, kWaves = NPT * KSN, kThreads = kWaves * 64;
  static constexpr int RW = 9 * CC;                  // chunks per staged filter row
  static constexpr int WI = 32 * RW / 64;            // filter DMA loads per stage
  static constexpr int PI = (NPIX * CC + 63) / 64;   // patch DMA loads per stage
  static constexpr int TI = WI + PI, kStage = TI * 64;
  static constexpr int NLO = TI / kWaves, NHI = (TI + kWaves - 1) / kWaves;
  static_assert(CC == 4 || CC == 8, "slabs of 4 or 8 chunks");
  static_assert(TH * OW == NPT * 32 && (OW & (OW - 1)) == 0, "whole output rows of a power-of-two width");
  static_assert(kThreads <= 1024, "block size");
  static_assert(STAGES >= 2 && STAGES * kStage * 16 <= 160 * 1024, "LDS budget");
  static_assert(kWaves * 64 * 4 <= STAGES * kStage, "the partial tiles fit the stage buffers");
  static_assert(2 * NHI < 64, "vmcnt range");
};

template <int CC> __device__ __forceinline__ int wk_swz(int r) {
  if constexpr (CC == 4) return (r >> 2) & 3;
  else return (r >> 1) & 7;
}

// mom != null (a conv under an instance norm, no activation): the kernel
// also writes the moments of each 64-pixel segment of every output plane
// (norm_stats.hpp) at mom[((n * C + c) * S + segment) * 2] = (mean, M2), S =
// OH * OW / 64, from the values the epilogue stores, T(sum + bias).
template <Op O, class Wt, class Epi>
__global__ void __launch_bounds__(Wt::kThreads) wk_conv_kernel(const HaloGeo g, const Epi epi, int nP, int nQ,
                                                               float* __restrict__ mom, const void* mbias, int C) {
  using A = typename OpT<O>::Acc;
  constexpr int CC = Wt::CC;
  __shared__ u32x4 smem[Wt::STAGES * Wt::kStage];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int pt = wave % Wt::NPT, ks = wave / Wt::NPT;
  int tp, tq;
  // each XCD owns whole output-channel tiles (the filter is the operand
  // that would otherwise be re-read from every XCD)
  map_tile(blockIdx.x, gridDim.x, nP, nQ, nP, tp, tq);
  const int pix0 = tp * (Wt::NPT * 32), co0 = tq * 32;
  const int ohw = g.OH * g.OW;
  const int n = pix0 / ohw;
  const int oy0 = (pix0 - n * ohw) >> g.ow_shift;

  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.w + (int64_t)co0 * g.ldw), (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)(g.x + (int64_t)n * g.img_bytes), (short)0, 0x7fffffff, 0x00020000);

  // this thread's share of a stage's DMA loads (load m of a stage belongs
  // to wave m % waves): global offset at slab 0 and the channel chunk
  int voff[Wt::NHI], sub[Wt::NHI];
#pragma unroll
  for (int i = 0; i < Wt::NHI; ++i) {
    const int m = i * Wt::kWaves + wave;
    voff[i] = kOobOffset;
    sub[i] = 0;
    if (m < Wt::WI) {
      const int slot = m * 64 + lane;
      const int row = slot / Wt::RW, phys = slot - row * Wt::RW;
      const int tap = phys / CC, c = (phys - tap * CC) ^ wk_swz<CC>(row);
      sub[i] = c;
      if (co0 + row < g.cout) voff[i] = (int)(row * g.ldw) + (tap * g.cpc + c) * 16;
    } else if (m < Wt::TI) {
      const int slot = (m - Wt::WI) * 64 + lane;
      const int pix = slot / CC, c = (slot - pix * CC) ^ wk_swz<CC>(pix);
      const int py = pix / Wt::PW, px = pix - py * Wt::PW;
      int iy = oy0 + py - g.pt, ix = px - g.pl;
      if (g.pad_mode == 1) {          // reflect (pads below the extent; the host checks)
        iy = iy < 0 ? -iy : (iy >= g.H ? 2 * g.H - 2 - iy : iy);
        ix = ix < 0 ? -ix : (ix >= g.W ? 2 * g.W - 2 - ix : ix);
      } else if (g.pad_mode == 2) {   // edge
        iy = iy < 0 ? 0 : (iy >= g.H ? g.H - 1 : iy);
        ix = ix < 0 ? 0 : (ix >= g.W ? g.W - 1 : ix);
      }
      sub[i] = c;
      if (pix < Wt::NPIX && (unsigned)iy < (unsigned)g.H && (unsigned)ix < (unsigned)g.W)
        voff[i] = ((iy * g.W + ix) * g.pstride + c) * 16;
    }
  }
  const int nslab = (g.cpc + CC - 1) / CC;
  // every stage issues the same loads (past the last slab, and in the
  // channel tail, they read zero through the range check), so the waits
  // are fixed counts
  auto issue = [&](int s) __attribute__((always_inline)) {
    u32x4* base = smem + (s % Wt::STAGES) * Wt::kStage;
    const bool live = s < nslab;
    const int soff = s * CC * 16;
#pragma unroll
    for (int i = 0; i < Wt::NHI; ++i) {
      const int m = i * Wt::kWaves + wave;
      if (m < Wt::TI) {
        const int off = live && s * CC + sub[i] < g.cpc ? voff[i] : kOobOffset;
        buf16(m < Wt::WI ? rw : rx, off, soff, base + m * 64);
      }
    }
  };
  auto wait_stages = [&](auto kc) __attribute__((always_inline)) {
    constexpr int K = decltype(kc)::value;
    if (wave < Wt::TI % Wt::kWaves) wait_vmcnt<K * Wt::NHI>();
    else wait_vmcnt<K * Wt::NLO>();
  };

  // fragment slots: filter row lane % 32, chunk 2 ks + lane / 32 of each
  // tap; patch pixel of this lane's output pixel, shifted per tap
  const int hi = lane >> 5;
  const int cc = 2 * ks + hi;
  const int wrow = lane & 31;
  const int wbase = wrow * Wt::RW + (cc ^ wk_swz<CC>(wrow));
  const int ql = pt * 32 + (lane & 31);
  const int pbase = (ql >> g.ow_shift) * Wt::PW + (ql & (Wt::OW - 1));

  A acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0;
#pragma unroll
  for (int s = 0; s < Wt::STAGES - 1; ++s) issue(s);
  wait_stages(std::integral_constant<int, Wt::STAGES - 2>{});
  barrier_only();
  for (int s = 0; s < nslab; ++s) {
    issue(s + Wt::STAGES - 1);
    const u32x4* S = smem + (s % Wt::STAGES) * Wt::kStage;
    const u32x4* SP = S + Wt::WI * 64;
    u32x4 wf[9], pf[9];
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      const int ky = tap / 3, kx = tap - ky * 3;
      wf[tap] = S[wbase + tap * CC];
      const int pix = pbase + ky * Wt::PW + kx;
      pf[tap] = SP[pix * CC + (cc ^ wk_swz<CC>(pix))];
    }
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) {
      if constexpr (Wt::PIX_ON_X) acc = OpT<O>::mma(pf[tap], wf[tap], acc);
      else acc = OpT<O>::mma(wf[tap], pf[tap], acc);
    }
    wait_stages(std::integral_constant<int, Wt::STAGES - 2>{});
    wait_lgkm0();
    barrier_only();
  }

  // the waves' partial tiles meet in LDS (the stage buffers, free once every
  // load has landed: past the last slab they read zero but still land)
  wait_vmcnt<0>();
  barrier_only();
  f32x4* red = reinterpret_cast<f32x4*>(smem);
#pragma unroll
  for (int gq = 0; gq < 4; ++gq)
    red[(wave * 4 + gq) * 64 + lane] = f32x4{acc[4 * gq], acc[4 * gq + 1], acc[4 * gq + 2], acc[4 * gq + 3]};
  __syncthreads();
  // the finished tile of pixel tile pt: its k-steps' partial tiles added in
  // k-step order (group gq: the lane's rows 8 gq + 4 (lane / 32) .. + 3)
  auto tile_sum = [&](int gq) __attribute__((always_inline)) {
    f32x4 v = red[(pt * 4 + gq) * 64 + lane];
#pragma unroll
    for (int k2 = 1; k2 < Wt::KSN; ++k2) v += red[((pt + k2 * Wt::NPT) * 4 + gq) * 64 + lane];
    return v;
  };
  // the moments of this lane's channel over its pixel tile (lanes 0 .. 31)
  const int co = co0 + (lane & 31);
  Moments tm{0.0f, 0.0f, 0.0f};
  if constexpr (Wt::PIX_ON_X && O != Op::I8) {
    if (mom) {
      // runs of four pixels (group gq of half-wave hi is run 2 gq + hi of
      // the tile) merge as a tree into the tile's moments; the odd tile of
      // each pair hands its moments to the even one through LDS
      static_assert(Wt::NPT % 2 == 0, "pixel tiles pair into 64-pixel segments");
      static_assert(Wt::kWaves * 4 * 64 + Wt::NPT / 2 * 32 / 2 <= Wt::STAGES * Wt::kStage, "LDS");
      using OutT = typename std::conditional<O == Op::F32, float,
                   typename std::conditional<O == Op::F16, _Float16, __bf16>::type>::type;
      float2* odd = reinterpret_cast<float2*>(smem + Wt::kWaves * 4 * 64);   // [pair][channel]
      if (wave < Wt::NPT) {
        const float b = mbias && co < C ? (float)static_cast<const OutT*>(mbias)[co] : -0.0f;
        Moments r[4];
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const f32x4 v = tile_sum(gq);
          float h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = (float)(OutT)(v[e] + b);
          const Moments own = run_moments4(h[0], h[1], h[2], h[3]);
          // every run holds four values: the counts are constants and the
          // merges' count ratios fold
          r[gq] = own;
          chan_merge(r[gq], Moments{4.0f, __shfl_xor(own.m, 32), __shfl_xor(own.m2, 32)});
        }
        chan_merge(r[0], r[1]);
        chan_merge(r[2], r[3]);
        chan_merge(r[0], r[2]);
        tm = r[0];
        if ((pt & 1) && hi == 0) odd[(pt >> 1) * 32 + (lane & 31)] = float2{tm.m, tm.m2};
      }
      __syncthreads();
    }
  }
  if (wave >= Wt::NPT) return;
  // wave pt adds the partial tiles of k-steps 0 .. KSN - 1 in that order and
  // finishes its 32 pixels x 32 channels
  const OutAddr out = epi.addr();
  const int pixl = pix0 + pt * 32;
  const int jl = Wt::PIX_ON_X ? co0 + (lane & 31) : pixl + (lane & 31);
  typename Epi::PreJ pj;
  epi.load_j(pj, jl);
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const f32x4 v = tile_sum(gq);
    const int i = (Wt::PIX_ON_X ? pixl : co0) + 8 * gq + 4 * hi;
    typename Epi::PreI pi;
    epi.load_i(pi, i);
    typename OpT<O>::Out4 a4;
#pragma unroll
    for (int e = 0; e < 4; ++e) a4[e] = v[e];
    uint32_t bits[4];
    epi.finish(pi, pj, i, jl, a4, bits);
    store_group(out, epi.out_bytes(), out.row(i), i, jl, bits);
  }
  // the even tile's lanes complete their segment (after the stores are
  // issued: the merge overlaps their write-back)
  if constexpr (Wt::PIX_ON_X && O != Op::I8) {
    if (mom) {
      const float2* odd = reinterpret_cast<const float2*>(smem + Wt::kWaves * 4 * 64);
      if (!(pt & 1) && hi == 0 && co < C) {
        const float2 o = odd[(pt >> 1) * 32 + (lane & 31)];
        chan_merge(tm, Moments{32.0f, o.x, o.y});
        const int seg = (pix0 - n * ohw + pt * 32) / kNormSeg;
        *reinterpret_cast<float2*>(mom + (((int64_t)n * C + co) * (ohw / kNormSeg) + seg) * 2) =
            float2{tm.m, tm.m2};
      }
    }
  }
}

}  // namespace ohip
