/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle, floating-point half.
 * Restates oxionnx-ops/src/math_typed.rs (f16/bf16/f32 GEMM),
 * oxionnx-ops/src/math/matmul.rs (alpha / beta passes),
 * oxionnx-ops/src/conv/{conv2d.rs,im2col.rs} (f32 Conv) and
 * oxionnx-ops/src/registry/conv_ops/conv.rs (fused activation).
 * Built with -ffp-contract=off: rustc never fuses a*b+c.  The sgemm itself
 * lives in oracle_sgemm.c (the reference's matrixmultiply uses FMA there).
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* half::f16::from_f32, round to nearest even. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(man ? (sign | 0x7e00u | (man >> 13)) : (sign | 0x7c00u));
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t mm = man | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = mm >> shift, rem = mm & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, x;
    if (exp == 0) {
        if (man == 0) x = sign;
        else {
            int e = -1;
            do { man <<= 1; ++e; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) x = sign | 0x7f800000u | (man << 13);
    else x = sign | ((exp - 15 + 127) << 23) | (man << 13);
    float f; memcpy(&f, &x, 4); return f;
}

/* half::bf16::from_f32, round to nearest even, NaN kept quiet. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t r = x + 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(r >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t x = (uint32_t)h << 16; float f; memcpy(&f, &x, 4); return f;
}

void orc_f32_to_f16_n(const float* s, uint16_t* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_f32_to_f16(s[i]); }
void orc_f16_to_f32_n(const uint16_t* s, float* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_f16_to_f32(s[i]); }
void orc_f32_to_bf16_n(const float* s, uint16_t* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_f32_to_bf16(s[i]); }
void orc_bf16_to_f32_n(const uint16_t* s, float* d, int64_t n) { for (int64_t i = 0; i < n; ++i) d[i] = orc_bf16_to_f32(s[i]); }

/* resolve_bias_f32 (math_typed.rs:444-455). */
static inline float bias_at(const float* c, int c_kind, int64_t row, int64_t col, int64_t n) {
    switch (c_kind) {
        case 1: return c[0];
        case 2: return c[col % n];
        case 3: return c[row * n + col];
        default: return 0.0f;
    }
}

/* gemm_f16 / gemm_bf16 (math_typed.rs:589-686).  The reference runs i-j-k
 * with an f32 accumulator summed in ascending p; this runs i-p-j with one
 * accumulator per (i,j), which visits every (i,j) in the same ascending-p
 * order, so each output element is bit-identical.  The f16 x f16 product is
 * exact in f32, so fused or not makes no difference there either. */
void orc_gemm_half(int is_bf16, const uint16_t* a, const uint16_t* b,
                   int64_t m, int64_t k, int64_t n, int trans_a, int trans_b,
                   float alpha, float beta, const uint16_t* c, int c_kind,
                   uint16_t* out, int64_t row0, int64_t row1) {
    float (*cvt)(uint16_t) = is_bf16 ? orc_bf16_to_f32 : orc_f16_to_f32;
    uint16_t (*back)(float) = is_bf16 ? orc_f32_to_bf16 : orc_f32_to_f16;
    if (row1 < 0 || row1 > m) row1 = m;
    float* bf = (float*)malloc(sizeof(float) * (size_t)(k * n));
    for (int64_t p = 0; p < k; ++p)
        for (int64_t j = 0; j < n; ++j)
            bf[p * n + j] = cvt(trans_b ? b[j * k + p] : b[p * n + j]);
    int64_t c_len = c_kind == 1 ? 1 : c_kind == 2 ? n : c_kind == 3 ? m * n : 0;
    float* cf = c_len ? (float*)malloc(sizeof(float) * (size_t)c_len) : NULL;
    for (int64_t i = 0; i < c_len; ++i) cf[i] = cvt(c[i]);
    float* acc = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t i = row0; i < row1; ++i) {
        for (int64_t j = 0; j < n; ++j) acc[j] = 0.0f;
        for (int64_t p = 0; p < k; ++p) {
            float av = cvt(trans_a ? a[p * m + i] : a[i * k + p]);
            const float* brow = bf + p * n;
            for (int64_t j = 0; j < n; ++j) acc[j] += av * brow[j];
        }
        for (int64_t j = 0; j < n; ++j) {
            float bias = bias_at(cf, c_kind, i, j, n);
            float t = acc[j] * alpha;
            float u = beta * bias;
            out[i * n + j] = back(t + u);
        }
    }
    free(acc); free(cf); free(bf);
}

/* gemm_f32 (math_typed.rs:759-788): one sgemm, alpha pass, beta*C pass with
 * C broadcast to [m,n] (math::broadcast_to). */
void orc_gemm_f32(const float* a, const float* b, int64_t m, int64_t k, int64_t n,
                  int trans_a, int trans_b, float alpha, float beta,
                  const float* c, int64_t c_rows, int64_t c_cols, float* out, int nthreads) {
    int64_t rsa = trans_a ? 1 : k, csa = trans_a ? m : 1;
    int64_t rsb = trans_b ? 1 : n, csb = trans_b ? k : 1;
    orc_sgemm(m, k, n, a, rsa, csa, b, rsb, csb, out, n, nthreads);
    if (alpha != 1.0f) for (int64_t i = 0; i < m * n; ++i) out[i] *= alpha;
    if (c) {
        for (int64_t i = 0; i < m; ++i)
            for (int64_t j = 0; j < n; ++j) {
                float cv = c[(c_rows == 1 ? 0 : i) * c_cols + (c_cols == 1 ? 0 : j)];
                float t = beta * cv;
                out[i * n + j] += t;
            }
    }
}

/* im2col (conv/im2col.rs:12-60): rows (ic, ky, kx), columns (oy, ox). */
static void im2col(const float* in, int64_t h, int64_t w, int64_t cpg, int64_t kh, int64_t kw,
                   const int64_t s[2], const int64_t p[4], const int64_t d[2],
                   int64_t oh, int64_t ow, float* col) {
    int64_t cols = oh * ow, row = 0;
    for (int64_t ic = 0; ic < cpg; ++ic) {
        const float* plane = in + ic * h * w;
        for (int64_t ky = 0; ky < kh; ++ky)
            for (int64_t kx = 0; kx < kw; ++kx, ++row)
                for (int64_t oy = 0; oy < oh; ++oy) {
                    float* dst = col + row * cols + oy * ow;
                    int64_t iy = oy * s[0] + ky * d[0] - p[0];
                    if (iy < 0 || iy >= h) { for (int64_t ox = 0; ox < ow; ++ox) dst[ox] = 0.0f; continue; }
                    for (int64_t ox = 0; ox < ow; ++ox) {
                        int64_t ix = ox * s[1] + kx * d[1] - p[1];
                        dst[ox] = (ix >= 0 && ix < w) ? plane[iy * w + ix] : 0.0f;
                    }
                }
    }
}

/* conv2d_into_slices_capped (conv/conv2d.rs:246-547) without the Winograd
 * branch (never taken at the configured shapes, conv2d.rs:88,325-346):
 * 1x1/stride-1/no-pad goes straight to sgemm (conv2d.rs:306-322,1071-1114),
 * everything else is im2col + sgemm + bias (conv2d.rs:354-448). */
int orc_conv2d_f32(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                   const float* wt, int64_t cout, int64_t cpg, int64_t kh, int64_t kw,
                   const float* bias, const int64_t strides[2], const int64_t pads[4],
                   const int64_t dils[2], int64_t group, int64_t oh, int64_t ow,
                   float* out, int nthreads) {
    if (group <= 0 || cpg * group != c || cout % group) return -1;
    int64_t coutpg = cout / group, rows = cpg * kh * kw, cols = oh * ow;
    int direct = kh == 1 && kw == 1 && strides[0] == 1 && strides[1] == 1 && dils[0] == 1 &&
                 dils[1] == 1 && !pads[0] && !pads[1] && !pads[2] && !pads[3];
    float* col = direct ? NULL : (float*)malloc(sizeof(float) * (size_t)(rows * cols));
    for (int64_t b = 0; b < n; ++b)
        for (int64_t g = 0; g < group; ++g) {
            const float* in = x + (b * c + g * cpg) * h * w;
            const float* wg = wt + g * coutpg * rows;
            float* o = out + (b * cout + g * coutpg) * cols;
            const float* rhs = in;
            if (!direct) { im2col(in, h, w, cpg, kh, kw, strides, pads, dils, oh, ow, col); rhs = col; }
            orc_sgemm(coutpg, rows, cols, wg, rows, 1, rhs, cols, 1, o, cols, nthreads);
            if (bias)
                for (int64_t oc = 0; oc < coutpg; ++oc) {
                    float bv = bias[g * coutpg + oc];
                    for (int64_t j = 0; j < cols; ++j) o[oc * cols + j] += bv;
                }
        }
    free(col);
    return 0;
}

/* apply_fused_activation (registry/conv_ops/conv.rs:124-156). */
void orc_apply_activation(float* data, int64_t count, int act, float lo, float hi) {
    if (act == 1) {
        for (int64_t i = 0; i < count; ++i) data[i] = data[i] > 0.0f ? data[i] : 0.0f; /* f32::max(NaN, 0) is 0 */
    } else if (act == 2) {
        if (isnan(lo)) lo = -INFINITY;
        if (isnan(hi)) hi = INFINITY;
        if (lo <= hi)
            for (int64_t i = 0; i < count; ++i) {
                float v = data[i];
                if (v < lo) v = lo;
                if (v > hi) v = hi;
                data[i] = v;
            }
    }
}

/* ---------------------------------------------------------------- elementwise nodes
 * Unary activations, element by element in f32 with the C library's
 * functions (the reference's f32::exp / f32::tanh lower to the same libm
 * expf / tanhf on this platform):
 *   op 0 LeakyRelu  nn/activations.rs:87-95      v >= 0 ? v : alpha * v
 *   op 1 Tanh       nn/activations.rs:52-56      tanhf(v)
 *   op 2 Sigmoid    nn/activations.rs:35-40      1 / (1 + expf(-v))
 *   op 3 Silu       registry/nn_ops/activations.rs:477-479   v / (1 + expf(-v))
 *   op 4 Relu       nn/activations.rs:16-21      v.max(0) (NaN -> 0) */
void orc_unary_f32(float* data, int64_t count, int op, float alpha) {
    for (int64_t i = 0; i < count; ++i) {
        const float v = data[i];
        switch (op) {
            case 0: data[i] = v >= 0.0f ? v : alpha * v; break;
            case 1: data[i] = tanhf(v); break;
            case 2: data[i] = 1.0f / (1.0f + expf(-v)); break;
            case 3: data[i] = v / (1.0f + expf(-v)); break;
            default: data[i] = v > 0.0f ? v : 0.0f; break;
        }
    }
}

/* OxiInstanceNorm normalize_plane (registry/oxi_instance_norm.rs:56-65): per
 * (n, c) plane, mean as an ascending f32 sum / count, variance about it the
 * same way, then (v - mean) * (1 / sqrt(var + eps)). */
void orc_instance_norm_f32(float* data, int64_t planes, int64_t spatial, float eps) {
    for (int64_t p = 0; p < planes; ++p) {
        float* x = data + p * spatial;
        const float count = (float)spatial;
        float s = 0.0f;
        for (int64_t i = 0; i < spatial; ++i) s += x[i];
        const float mean = s / count;
        float q = 0.0f;
        for (int64_t i = 0; i < spatial; ++i) q += (x[i] - mean) * (x[i] - mean);
        const float var = q / count;
        const float inv = 1.0f / sqrtf(var + eps);
        for (int64_t i = 0; i < spatial; ++i) x[i] = (x[i] - mean) * inv;
    }
}

/* ConvTranspose, rank 2, f32: conv_transpose_into + scatter_rank2
 * (oxionnx-ops/src/conv/transpose.rs:78-214, 233-309).  The output is zeroed,
 * every input element scatters in_val * w[ci][oc][ky][kx] to
 * (iy * s + ky * d - pad_begin, ...) when that lands inside the cropped
 * output, visiting batch, group, input channel, input position, output
 * channel, kernel offset in that order; the bias is added afterwards. */
int orc_conv_transpose2d_f32(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                             const float* wt, int64_t coutpg, int64_t kh, int64_t kw, const float* bias,
                             const int64_t strides[2], const int64_t pads[4], const int64_t dils[2],
                             int64_t group, int64_t oh, int64_t ow, float* out) {
    if (group <= 0 || c % group) return -1;
    const int64_t cpg = c / group, cout = coutpg * group;
    memset(out, 0, (size_t)(n * cout * oh * ow) * sizeof(float));
    for (int64_t ni = 0; ni < n; ++ni)
        for (int64_t g = 0; g < group; ++g)
            for (int64_t ic = 0; ic < cpg; ++ic) {
                const int64_t ci = g * cpg + ic;
                for (int64_t iy = 0; iy < h; ++iy)
                    for (int64_t ix = 0; ix < w; ++ix) {
                        const float v = x[((ni * c + ci) * h + iy) * w + ix];
                        for (int64_t oc = 0; oc < coutpg; ++oc) {
                            const int64_t co = g * coutpg + oc;
                            const float* wb = wt + (ci * coutpg + oc) * kh * kw;
                            float* ob = out + (ni * cout + co) * oh * ow;
                            for (int64_t ky = 0; ky < kh; ++ky) {
                                const int64_t oyr = iy * strides[0] + ky * dils[0];
                                if (oyr < pads[0] || oyr - pads[0] >= oh) continue;
                                for (int64_t kx = 0; kx < kw; ++kx) {
                                    const int64_t oxr = ix * strides[1] + kx * dils[1];
                                    if (oxr < pads[1] || oxr - pads[1] >= ow) continue;
                                    ob[(oyr - pads[0]) * ow + (oxr - pads[1])] += v * wb[ky * kw + kx];
                                }
                            }
                        }
                    }
            }
    if (bias)
        for (int64_t ni = 0; ni < n; ++ni)
            for (int64_t co = 0; co < cout; ++co) {
                float* ob = out + (ni * cout + co) * oh * ow;
                for (int64_t i = 0; i < oh * ow; ++i) ob[i] += bias[co];
            }
    return 0;
}
