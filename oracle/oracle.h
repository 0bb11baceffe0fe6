/*
 * CPU oracle for the OxiONNX dense-contraction hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates the reference's CPU
 * kernels (cool-japan/oxionnx v0.1.7, Rust) in plain C so that the HIP
 * execution provider can be checked against them.  Only tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg may load it, and only as the
 * checker / the CPU baseline -- never as a product path.
 *
 * Every function cites the reference file:line it follows.  The reference's
 * own Rust toolchain is absent from this image, so nothing is imported from
 * it; the restatement is pinned by the reference's inline golden vectors and
 * by closed-form checks in tests/test_oracle.py.
 */
#ifndef OXIONNX_ORACLE_H
#define OXIONNX_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- quant_ops/mod.rs ------------------------------------------------- */
double orc_round_ties_even_f64(double v);                       /* mod.rs:51-65 */
void orc_satrange_infer(const int32_t* yzp, int ny, const int32_t* xzp, int nx,
                        int32_t* lo, int32_t* hi);               /* mod.rs:188-200 */
float orc_requantize(int64_t acc, float combined, int32_t zp, int32_t lo, int32_t hi); /* mod.rs:229-233 */
float orc_saturate_i32(int64_t acc);                            /* mod.rs:243-245 */

/* ---- quant_ops/qlinear_matmul.rs -------------------------------------- */
/* integer_matmul (qlinear_matmul.rs:106-133): sum_p (a-a_zp[i])(b-b_zp[j]) in i64. */
int orc_integer_matmul(const int32_t* a, const int32_t* b,
                       const int32_t* a_zp, int n_azp, const int32_t* b_zp, int n_bzp,
                       int64_t batch, int a_bcast, int b_bcast,
                       int64_t m, int64_t k, int64_t n, int64_t* out);
/* QLinearMatMulOp::run requant tail (qlinear_matmul.rs:243-253). */
void orc_qlinear_requant(const int64_t* acc, int64_t count, float combined,
                         int32_t y_zp, int32_t lo, int32_t hi, float* out);

/* ---- quant_ops/conv_kernel.rs ----------------------------------------- */
/* integer_conv restricted to rank 2 (conv_kernel.rs:134-254); bias may be NULL. */
int orc_integer_conv2d(const int32_t* x, int64_t n, int64_t c, int64_t h, int64_t w,
                       const int32_t* wt, int64_t cout, int64_t cpg, int64_t kh, int64_t kw,
                       int32_t x_zp, const int32_t* w_zp, int n_wzp, const int32_t* bias,
                       const int64_t strides[2], const int64_t pads[4], const int64_t dils[2],
                       int64_t group, int64_t oh, int64_t ow, int64_t* out);
/* QLinearConvOp::run requant tail (qlinear_conv.rs:83-101). */
void orc_qlinear_conv_requant(const int64_t* acc, int64_t batch, int64_t cout, int64_t spatial,
                              float x_s, const float* w_s, int n_ws, float y_s,
                              int32_t y_zp, int32_t lo, int32_t hi, float* out);

/* ---- conv/spatial.rs -------------------------------------------------- */
/* auto_pad: 0 NOTSET, 1 VALID, 2 SAME_UPPER, 3 SAME_LOWER; pads [t,l,b,r] */
void orc_resolve_pads2d(int auto_pad, const int64_t in_hw[2], const int64_t k_hw[2],
                        const int64_t strides[2], const int64_t dils[2],
                        const int64_t explicit_pads[4], int64_t out_pads[4]); /* spatial.rs:204-257 */
int64_t orc_conv_out_dim(int64_t in, int64_t pb, int64_t pe, int64_t k, int64_t d, int64_t s); /* spatial.rs:272-330 */

/* ---- half crate conversions (RNE) ------------------------------------- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n);
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n);
void orc_f32_to_bf16_n(const float* src, uint16_t* dst, int64_t n);
void orc_bf16_to_f32_n(const uint16_t* src, float* dst, int64_t n);

/* ---- math_typed.rs: f16 / bf16 GEMM ----------------------------------- */
/* gemm_f16 / gemm_bf16 (math_typed.rs:589-686).  c_kind: 0 none, 1 scalar,
 * 2 row vector [n], 3 full [m,n].  Rows [row0,row1) only (row1<0 = all). */
void orc_gemm_half(int is_bf16, const uint16_t* a, const uint16_t* b,
                   int64_t m, int64_t k, int64_t n, int trans_a, int trans_b,
                   float alpha, float beta, const uint16_t* c, int c_kind,
                   uint16_t* out, int64_t row0, int64_t row1);

/* ---- math/matmul.rs + math_typed.rs: f32 GEMM ------------------------- */
/* C[m,n] = A·B with element strides (math_typed.rs:45-79, sgemm_strided). */
void orc_sgemm(int64_t m, int64_t k, int64_t n,
               const float* a, int64_t rsa, int64_t csa,
               const float* b, int64_t rsb, int64_t csb,
               float* c, int64_t rsc, int nthreads);
/* gemm_f32 (math_typed.rs:759-788): sgemm, then *=alpha, then += beta*C
 * (C broadcast from [c_rows, c_cols], each 1 or m / n). */
void orc_gemm_f32(const float* a, const float* b, int64_t m, int64_t k, int64_t n,
                  int trans_a, int trans_b, float alpha, float beta,
                  const float* c, int64_t c_rows, int64_t c_cols, float* out, int nthreads);

/* ---- conv/conv2d.rs: f32 Conv ----------------------------------------- */
/* conv2d_into_slices_capped (conv2d.rs:246-547): im2col + sgemm + bias. */
int orc_conv2d_f32(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                   const float* wt, int64_t cout, int64_t cpg, int64_t kh, int64_t kw,
                   const float* bias, const int64_t strides[2], const int64_t pads[4],
                   const int64_t dils[2], int64_t group, int64_t oh, int64_t ow,
                   float* out, int nthreads);
/* apply_fused_activation (registry/conv_ops/conv.rs:124-156): act 0 none,
 * 1 relu, 2 clip(lo,hi) with NaN bound = unbounded and inverted = no-op. */
void orc_apply_activation(float* data, int64_t count, int act, float lo, float hi);

int orc_conv_transpose2d_f32(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                             const float* wt, int64_t coutpg, int64_t kh, int64_t kw, const float* bias,
                             const int64_t strides[2], const int64_t pads[4], const int64_t dils[2],
                             int64_t group, int64_t oh, int64_t ow, float* out);
int orc_hardware_threads(void);

/* elementwise nodes (oracle_float.c) */
void orc_unary_f32(float* data, int64_t count, int op, float alpha);
void orc_instance_norm_f32(float* data, int64_t planes, int64_t spatial, float eps);

#ifdef __cplusplus
}
#endif
#endif
