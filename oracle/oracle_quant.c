/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, integer half.
 * Restates oxionnx-ops/src/registry/quant_ops/{mod.rs,qlinear_matmul.rs,
 * qlinear_conv.rs,conv_kernel.rs} and oxionnx-ops/src/conv/spatial.rs.
 * Built with -ffp-contract=off: the reference (rustc) never fuses a*b+c.
 */
#include "oracle.h"
#include <math.h>
#include <unistd.h>

/* quant_ops/mod.rs:51-65 -- floor, then step up past the midpoint or at an
 * exact tie when floor is odd. */
double orc_round_ties_even_f64(double v) {
    if (!isfinite(v)) return v;
    double fl = floor(v);
    double diff = v - fl;
    int odd = fmod(fl, 2.0) != 0.0;
    if (diff > 0.5 || (diff == 0.5 && odd)) return fl + 1.0;
    return fl;
}

/* SatRange::infer (quant_ops/mod.rs:188-200): y_zp lanes first, then x_zp. */
void orc_satrange_infer(const int32_t* yzp, int ny, const int32_t* xzp, int nx,
                        int32_t* lo, int32_t* hi) {
    const int32_t* lanes[2] = {yzp, xzp};
    int counts[2] = {ny, nx};
    for (int s = 0; s < 2; ++s) {
        for (int i = 0; i < counts[s]; ++i) if (lanes[s][i] > 127) { *lo = 0; *hi = 255; return; }
        for (int i = 0; i < counts[s]; ++i) if (lanes[s][i] < 0) { *lo = -128; *hi = 127; return; }
    }
    *lo = -128; *hi = 255;
}

/* SatRange::requantize (quant_ops/mod.rs:229-233): f64 product, then + zp,
 * ties-to-even, clamp. */
float orc_requantize(int64_t acc, float combined, int32_t zp, int32_t lo, int32_t hi) {
    double scaled = (double)acc * (double)combined;
    scaled = scaled + (double)zp;
    double r = orc_round_ties_even_f64(scaled);
    if (r < (double)lo) r = (double)lo;
    if (r > (double)hi) r = (double)hi;
    return (float)r;
}

/* saturate_i32 (quant_ops/mod.rs:243-245). */
float orc_saturate_i32(int64_t acc) {
    if (acc < INT32_MIN) acc = INT32_MIN;
    if (acc > INT32_MAX) acc = INT32_MAX;
    return (float)acc;
}

/* zp_at (qlinear_matmul.rs:94-101) */
static inline int32_t zp_at(const int32_t* lanes, int len, int64_t idx) {
    if (len == 1) return lanes[0];
    return idx < len ? lanes[idx] : 0;
}

/* integer_matmul (qlinear_matmul.rs:106-133).  Loop order i-p-j: for every
 * (i,j) the i64 sum is exact, so the order cannot change the result. */
int orc_integer_matmul(const int32_t* a, const int32_t* b,
                       const int32_t* a_zp, int n_azp, const int32_t* b_zp, int n_bzp,
                       int64_t batch, int a_bcast, int b_bcast,
                       int64_t m, int64_t k, int64_t n, int64_t* out) {
    for (int64_t bi = 0; bi < batch; ++bi) {
        const int32_t* ab = a + (a_bcast ? 0 : bi * m * k);
        const int32_t* bb = b + (b_bcast ? 0 : bi * k * n);
        int64_t* ob = out + bi * m * n;
        for (int64_t i = 0; i < m; ++i) {
            int64_t* orow = ob + i * n;
            for (int64_t j = 0; j < n; ++j) orow[j] = 0;
            int64_t azp = zp_at(a_zp, n_azp, i);
            for (int64_t p = 0; p < k; ++p) {
                int64_t av = (int64_t)ab[i * k + p] - azp;
                const int32_t* brow = bb + p * n;
                if (n_bzp == 1) {
                    int64_t bzp = b_zp[0];
                    for (int64_t j = 0; j < n; ++j) orow[j] += av * ((int64_t)brow[j] - bzp);
                } else {
                    for (int64_t j = 0; j < n; ++j)
                        orow[j] += av * ((int64_t)brow[j] - zp_at(b_zp, n_bzp, j));
                }
            }
        }
    }
    return 0;
}

/* QLinearMatMulOp::run tail (qlinear_matmul.rs:243-253). */
void orc_qlinear_requant(const int64_t* acc, int64_t count, float combined,
                         int32_t y_zp, int32_t lo, int32_t hi, float* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = orc_requantize(acc[i], combined, y_zp, lo, hi);
}

/* integer_conv, rank 2 (conv_kernel.rs:134-254).  A tap that lands in the
 * padding is skipped, i.e. contributes exactly 0. */
int orc_integer_conv2d(const int32_t* x, int64_t n, int64_t c, int64_t h, int64_t w,
                       const int32_t* wt, int64_t cout, int64_t cpg, int64_t kh, int64_t kw,
                       int32_t x_zp, const int32_t* w_zp, int n_wzp, const int32_t* bias,
                       const int64_t strides[2], const int64_t pads[4], const int64_t dils[2],
                       int64_t group, int64_t oh, int64_t ow, int64_t* out) {
    if (n_wzp != 1 && n_wzp != cout) return -1;
    int64_t coutpg = cout / group;
    int64_t kvol = kh * kw;
    for (int64_t b = 0; b < n; ++b)
        for (int64_t oc = 0; oc < cout; ++oc) {
            int64_t g = oc / coutpg;
            int64_t wzp = n_wzp == 1 ? w_zp[0] : w_zp[oc];
            const int32_t* wbase = wt + oc * cpg * kvol;
            int64_t bterm = bias ? (int64_t)bias[oc] : 0;
            for (int64_t oy = 0; oy < oh; ++oy)
                for (int64_t ox = 0; ox < ow; ++ox) {
                    int64_t sum = bterm;
                    for (int64_t ky = 0; ky < kh; ++ky) {
                        int64_t iy = oy * strides[0] + ky * dils[0] - pads[0];
                        if (iy < 0 || iy >= h) continue;
                        for (int64_t kx = 0; kx < kw; ++kx) {
                            int64_t ix = ox * strides[1] + kx * dils[1] - pads[1];
                            if (ix < 0 || ix >= w) continue;
                            for (int64_t ic = 0; ic < cpg; ++ic) {
                                int64_t inc = g * cpg + ic;
                                int64_t xv = x[((b * c + inc) * h + iy) * w + ix];
                                int64_t wv = wbase[(ic * kh + ky) * kw + kx];
                                sum += (xv - x_zp) * (wv - wzp);
                            }
                        }
                    }
                    out[((b * cout + oc) * oh + oy) * ow + ox] = sum;
                }
        }
    return 0;
}

/* QLinearConvOp::run tail (qlinear_conv.rs:83-101): per-channel combined
 * scale formed in f32 as x_s * w_s / y_s. */
void orc_qlinear_conv_requant(const int64_t* acc, int64_t batch, int64_t cout, int64_t spatial,
                              float x_s, const float* w_s, int n_ws, float y_s,
                              int32_t y_zp, int32_t lo, int32_t hi, float* out) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t oc = 0; oc < cout; ++oc) {
            float ws = n_ws > 1 ? w_s[oc] : w_s[0];
            volatile float prod = x_s * ws;
            float combined = prod / y_s;
            const int64_t* a = acc + (b * cout + oc) * spatial;
            float* o = out + (b * cout + oc) * spatial;
            for (int64_t s = 0; s < spatial; ++s) o[s] = orc_requantize(a[s], combined, y_zp, lo, hi);
        }
}

/* same_pad_split / resolve_pads (conv/spatial.rs:204-257). */
void orc_resolve_pads2d(int auto_pad, const int64_t in_hw[2], const int64_t k_hw[2],
                        const int64_t strides[2], const int64_t dils[2],
                        const int64_t explicit_pads[4], int64_t out_pads[4]) {
    if (auto_pad == 0) { for (int i = 0; i < 4; ++i) out_pads[i] = explicit_pads[i]; return; }
    if (auto_pad == 1) { for (int i = 0; i < 4; ++i) out_pads[i] = 0; return; }
    for (int ax = 0; ax < 2; ++ax) {
        int64_t s = strides[ax] < 1 ? 1 : strides[ax];
        int64_t out_dim = (in_hw[ax] + s - 1) / s;
        int64_t eff_k = (k_hw[ax] > 0 ? k_hw[ax] - 1 : 0) * dils[ax] + 1;
        int64_t needed = (out_dim > 0 ? out_dim - 1 : 0) * s + eff_k - in_hw[ax];
        if (needed < 0) needed = 0;
        int64_t half = needed / 2;
        if (auto_pad == 3) { out_pads[ax] = needed - half; out_pads[ax + 2] = half; }
        else { out_pads[ax] = half; out_pads[ax + 2] = needed - half; }
    }
}

/* conv_out_dim -> pool_out_dim with ceil_mode=false (conv/spatial.rs:272-330).
 * Returns -1 where the reference returns a ShapeMismatch error. */
int64_t orc_conv_out_dim(int64_t in, int64_t pb, int64_t pe, int64_t k, int64_t d, int64_t s) {
    if (s <= 0 || k <= 0 || d <= 0) return -1;
    int64_t eff_k = (k - 1) * d + 1;
    int64_t padded = in + pb + pe;
    if (padded < eff_k) return -1;
    return (padded - eff_k) / s + 1;
}

int orc_hardware_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}
