// Instance-norm statistics in one fixed order, shared by every kernel that
// normalises a plane (the plain norm node, the split-K partial-sum reader,
// and the whole-K conv whose epilogue takes its tiles' moments for the
// moments-fed norm kernel), so that a fused Conv -> norm node and the
// unfused pair give the same bits.
//
// A plane of n values is cut into runs of 4 consecutive values and
// segments of 16 runs (64 values; the last run and segment may be
// shorter).  A run's moments are its mean m = (((x0 + x1) + x2) + x3) / len
// and M2 = sum (x - m)^2 (in order).  A segment's moments are its runs'
// merged in run order.  Segments form groups of 256 (16384 values); within
// a group they merge as a pairwise tree (each level merges items 2i and
// 2i + 1 into item i, a last unpaired item moves up as it is), and the
// groups' results merge in group order.  Each merge is Chan, Golub and
// LeVeque's pairwise update (delta = m_b - m_a; m += delta * (n_b / n_ab);
// M2 += M2_b + delta^2 * (n_a * n_b / n_ab)).
// Then var = M2 / n and the plane is normalised as (x - mean) *
// (1 / sqrt(var + eps)), like the reference's normalize_plane, whose single
// two-pass sum over the plane this replaces by a numerically equivalent,
// parallel one.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ohip {

constexpr int kNormRun = 4;
constexpr int kNormSeg = 64;      // 16 runs
constexpr int kNormGroup = 256;   // segments merged as one tree

struct Moments {
  float n, m, m2;
};

__device__ __forceinline__ Moments run_moments(const float* x, int len) {
#pragma clang fp contract(off)
  float s = x[0];
  for (int i = 1; i < len; ++i) s += x[i];
  const float m = s / (float)len;
  float q = 0.0f;
  for (int i = 0; i < len; ++i) {
    const float d = x[i] - m;
    q += d * d;
  }
  return Moments{(float)len, m, q};
}

__device__ __forceinline__ Moments run_moments4(float x0, float x1, float x2, float x3) {
  const float x[4] = {x0, x1, x2, x3};
  return run_moments(x, 4);
}

// Merges b into a.
__device__ __forceinline__ void chan_merge(Moments& a, const Moments& b) {
#pragma clang fp contract(off)
  const float nab = a.n + b.n;
  const float delta = b.m - a.m;
  a.m = a.m + delta * (b.n / nab);
  a.m2 = a.m2 + b.m2 + delta * delta * (a.n * b.n / nab);
  a.n = nab;
}

__device__ __forceinline__ int norm_segments(int64_t n) { return (int)((n + kNormSeg - 1) / kNormSeg); }

// Moments of segment s of a plane of n values read by ld(i).
template <class LD>
__device__ __forceinline__ Moments segment_moments(const LD& ld, int64_t n, int s) {
  const int64_t b = (int64_t)s * kNormSeg, e = b + kNormSeg < n ? b + kNormSeg : n;
  Moments acc{0.0f, 0.0f, 0.0f};
  for (int64_t r = b; r < e; r += kNormRun) {
    float x[kNormRun];
    const int len = r + kNormRun <= e ? kNormRun : (int)(e - r);
    for (int i = 0; i < len; ++i) x[i] = ld(r + i);
    const Moments rm = run_moments(x, len);
    if (r == b) acc = rm;
    else chan_merge(acc, rm);
  }
  return acc;
}

// Item i of tree level L + 1 over cnt0 segments (the last holding n_last
// values): items 2i and 2i + 1 of level L (cnt items, (mean, M2) at src)
// merged, or item 2i alone when it is the last.
__device__ __forceinline__ float2 tree_pair(const float2* src, int i, int cnt, int L, int cnt0, int n_last) {
  const float2 a = src[2 * i];
  if (2 * i + 1 >= cnt) return a;
  const float2 b = src[2 * i + 1];
  const int lo = (2 * i) << L, mid = (2 * i + 1) << L;
  const int hi = (2 * i + 2) << L < cnt0 ? (2 * i + 2) << L : cnt0;
  Moments ma{(float)((mid - lo) * kNormSeg), a.x, a.y};
  const Moments mb{(float)((hi - mid - 1) * kNormSeg + (hi == cnt0 ? n_last : kNormSeg)), b.x, b.y};
  chan_merge(ma, mb);
  return float2{ma.m, ma.m2};
}

// The pairwise tree over `lists` independent lists of cnt0 segments each
// ((mean, M2) at a + l * stride, level 0), run by nthreads threads of the
// block with a barrier per level; b (same stride) is scratch.  Every thread
// of the block calls it; returns the buffer whose element l * stride holds
// list l's result.
__device__ __forceinline__ float2* tree_merge(float2* a, float2* b, int stride, int lists, int cnt0, int n_last,
                                              int t, int nthreads) {
  int L = 0;
  for (int cnt = cnt0; cnt > 1; cnt = (cnt + 1) / 2, ++L) {
    const int nc = (cnt + 1) / 2;
    for (int idx = t; idx < lists * nc; idx += nthreads) {
      const int l = idx / nc, i = idx - l * nc;
      b[l * stride + i] = tree_pair(a + l * stride, i, cnt, L, cnt0, n_last);
    }
    __syncthreads();
    float2* tmp = a;
    a = b;
    b = tmp;
  }
  return a;
}

}  // namespace ohip
