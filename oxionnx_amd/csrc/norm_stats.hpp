// Instance-norm statistics in one fixed order, shared by every kernel that
// normalises a plane (the plain norm node, the split-K partial-sum reader,
// and the whole-K conv whose epilogue takes its tiles' moments for the
// moments-fed norm kernel), so that a fused Conv -> norm node and the
// unfused pair give the same bits.
//
// A plane of n values is cut into runs of 4 consecutive values and
// segments of 16 runs (64 values; the last run and segment may be
// shorter), and segments into groups of 256 (16384 values).  A run's
// moments are its mean m = (((x0 + x1) + x2) + x3) / len and M2 = sum
// (x - m)^2 (in order).  A segment's runs merge as a pairwise tree, and so
// do a group's segments: each level merges items 2i and 2i + 1 into item
// i, a last unpaired item moving up as it is.  The groups' results merge
// in group order.  Each merge is Chan, Golub and LeVeque's pairwise update
// (delta = m_b - m_a; m += delta * (n_b / n_ab); M2 += M2_b + delta^2 *
// (n_a * n_b / n_ab)).  Then var = M2 / n and the plane is normalised as
// (x - mean) * (1 / sqrt(var + eps)), like the reference's
// normalize_plane, whose single two-pass sum over the plane this replaces
// by a numerically equivalent, parallel one.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ohip {

// The affine tail's storage roundings: v is first materialised as an f32
// value (the operation's own rounding), then rounded to T, so that the
// compiler cannot fold the f32 operation and the narrowing into one
// mixed-precision FMA with a single rounding -- every norm kernel then
// rounds twice, the same way, whatever its surrounding code.
__device__ __forceinline__ float opaque(float v) {
  __asm__("" : "+v"(v));
  return v;
}
template <class T>
__device__ __forceinline__ float round_to(float v) {
  return (float)(T)opaque(v);
}

constexpr int kNormRun = 4;
constexpr int kNormSeg = 64;      // 16 runs
constexpr int kNormGroup = 256;   // segments merged as one tree

struct Moments {
  float n, m, m2;
};

// A run's moments from its first len (1 .. 4) values (the rest unused);
// scalar arguments, so no array lives in private memory.
__device__ __forceinline__ Moments run_moments_n(float x0, float x1, float x2, float x3, int len) {
#pragma clang fp contract(off)
  float s = x0;
  if (len > 1) s += x1;
  if (len > 2) s += x2;
  if (len > 3) s += x3;
  // s / 4 is s * 0.25 exactly (one rounding of the same real number)
  const float m = len == kNormRun ? s * 0.25f : s / (float)len;
  float d = x0 - m;
  float q = d * d;
  if (len > 1) d = x1 - m, q += d * d;
  if (len > 2) d = x2 - m, q += d * d;
  if (len > 3) d = x3 - m, q += d * d;
  return Moments{(float)len, m, q};
}

__device__ __forceinline__ Moments run_moments4(float x0, float x1, float x2, float x3) {
  return run_moments_n(x0, x1, x2, x3, kNormRun);
}

// Merges b into a.
// Equal counts (every merge of whole runs or segments inside a pairwise
// tree) take n_b / n_ab = 0.5 and n_a n_b / n_ab = n_a / 2: the same
// values the divisions round to (n is 4 or 64 times a power of two, so
// n_a n_b and n_a / 2 are exact).
__device__ __forceinline__ void chan_merge(Moments& a, const Moments& b) {
#pragma clang fp contract(off)
  const float nab = a.n + b.n;
  const float delta = b.m - a.m;
  float rb, rab;
  if (a.n == b.n) {
    rb = 0.5f;
    rab = a.n * 0.5f;
  } else {
    rb = b.n / nab;
    rab = a.n * b.n / nab;
  }
  a.m = a.m + delta * rb;
  a.m2 = a.m2 + b.m2 + delta * delta * rab;
  a.n = nab;
}

__device__ __forceinline__ int norm_segments(int64_t n) { return (int)((n + kNormSeg - 1) / kNormSeg); }

// The pairwise tree over the first cnt of N items (N a power of two), in
// place in registers: item 0 ends with the result.  Level w merges item i
// into item i - w for every i that is an odd multiple of w (items 2k and
// 2k + 1 of that level).
template <int N>
__device__ __forceinline__ void tree_regs(Moments (&r)[N], int cnt) {
#pragma unroll
  for (int w = 1; w < N; w *= 2)
#pragma unroll
    for (int i = 0; i + w < N; i += 2 * w)
      if (i + w < cnt) chan_merge(r[i], r[i + w]);
}

// The moments of segments s0 .. s0 + cnt - 1 of a plane of n values read
// by ld(i), into segm[0 .. cnt - 1]; s0 a multiple of 256.  The 256
// threads of a group call it together (lt = 0 .. 255): each thread takes a
// run per pass, and the 16 runs of a segment (16 neighbouring lanes) merge
// by shuffles as a pairwise tree.
template <class LD>
__device__ __forceinline__ void group_segments(const LD& ld, int64_t n, int s0, int cnt, float2* segm, int lt) {
  const int64_t nruns = (n + kNormRun - 1) / kNormRun;
  const int64_t r0 = (int64_t)s0 * (kNormSeg / kNormRun);
  const int64_t r1 = r0 + (int64_t)cnt * (kNormSeg / kNormRun) < nruns ? r0 + (int64_t)cnt * (kNormSeg / kNormRun)
                                                                         : nruns;
  const int q = lt & 15;   // run index in its segment
  for (int64_t base = r0; base < r1; base += 256) {
    const int64_t j = base + lt;
    Moments m{1.0f, 0.0f, 0.0f};
    if (j < r1) {
      const int64_t i = j * kNormRun;
      const int len = i + kNormRun <= n ? kNormRun : (int)(n - i);
      m = run_moments_n(ld(i), len > 1 ? ld(i + 1) : 0.0f, len > 2 ? ld(i + 2) : 0.0f, len > 3 ? ld(i + 3) : 0.0f,
                        len);
    }
    const int64_t seg = (j - r0) >> 4;
    const int64_t left = r1 - (r0 + seg * 16);
    const int cnt_seg = left < 16 ? (int)left : 16;
#pragma unroll
    for (int w = 1; w < 16; w *= 2) {
      const Moments o{__shfl_down(m.n, w), __shfl_down(m.m, w), __shfl_down(m.m2, w)};
      if ((q & (2 * w - 1)) == 0 && q + w < cnt_seg) chan_merge(m, o);
    }
    if (q == 0 && j < r1) segm[seg] = float2{m.m, m.m2};
  }
}

// The pairwise tree over a group's cnt0 <= 256 segments, run by one wave:
// lane l holds segments 4 l .. 4 l + 3 ((mean, M2) in v; segments of 64
// values, the last of n_last).  Levels 1 and 2 merge inside a lane, the
// wider ones across lanes (lane l takes lane l + s's item at level 4 s).
// Every lane of the wave calls it; lane 0 returns the result.
__device__ __forceinline__ Moments wave_tree(const float2 (&v)[4], int cnt0, int n_last, int lane) {
  Moments it[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    it[j] = Moments{4 * lane + j == cnt0 - 1 ? (float)n_last : (float)kNormSeg, v[j].x, v[j].y};
  const int k = 4 * lane;
  if (k + 1 < cnt0) chan_merge(it[0], it[1]);
  if (k + 3 < cnt0) chan_merge(it[2], it[3]);
  if (k + 2 < cnt0) chan_merge(it[0], it[2]);
  for (int sl = 1; 4 * sl < cnt0; sl *= 2) {
    const Moments o{__shfl_down(it[0].n, sl), __shfl_down(it[0].m, sl), __shfl_down(it[0].m2, sl)};
    if ((lane & (2 * sl - 1)) == 0 && 4 * (lane + sl) < cnt0) chan_merge(it[0], o);
  }
  return it[0];
}

}  // namespace ohip
