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
// merged in run order, the plane's its segments' merged in segment order,
// each merge Chan, Golub and LeVeque's pairwise update (delta = m_b - m_a;
// m += delta * (n_b / n_ab); M2 += M2_b + delta^2 * (n_a * n_b / n_ab)).
// Then var = M2 / n and the plane is normalised as (x - mean) *
// (1 / sqrt(var + eps)), like the reference's normalize_plane, whose single
// two-pass sum over the plane this replaces by a numerically equivalent,
// parallel one.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ohip {

constexpr int kNormRun = 4;
constexpr int kNormSeg = 64;   // 16 runs

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

// Mean and 1 / sqrt(var + eps) from a plane's segments seg(s), in order.
template <class SEG>
__device__ __forceinline__ void plane_stats(const SEG& seg, int64_t n, float eps, float& mean, float& inv) {
#pragma clang fp contract(off)
  const int S = norm_segments(n);
  Moments acc = seg(0);
  for (int s = 1; s < S; ++s) chan_merge(acc, seg(s));
  mean = acc.m;
  inv = 1.0f / sqrtf(acc.m2 / (float)n + eps);
}

}  // namespace ohip
