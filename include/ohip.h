/*
 * ohip.h -- C ABI of the MI355X (gfx950) execution provider for OxiONNX's
 * dense-contraction hot path: Conv (implicit GEMM), Gemm / MatMul, and the
 * INT8 family MatMulInteger / QLinearMatMul / ConvInteger / QLinearConv.
 *
 * Everything here is plain C: pointers, sizes and POD structs.  No exception
 * crosses the boundary.  Every entry point returns an int status:
 *     OHIP_OK (0)         success
 *     OHIP_DECLINED (1)   configuration not handled; the caller runs its CPU
 *                         kernel (the reference's Ok(None) contract,
 *                         oxionnx-cuda/src/lib.rs:336-352)
 *     < 0                 failure; ohip_last_error() holds the message
 *                         (the reference's Err -> CPU fallback,
 *                         src/session/run/sequential.rs:1019-1031)
 *
 * Device pointers passed to the ohip_gemm / ohip_conv2d family must live on
 * the context's device; work is ordered on the context's single stream.
 * All citations are into cool-japan/oxionnx v0.1.7.
 */
#ifndef OXIONNX_OHIP_H
#define OXIONNX_OHIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OHIP_OK 0
#define OHIP_DECLINED 1
#define OHIP_E_INVALID (-1)
#define OHIP_E_HIP (-2)
#define OHIP_E_SHAPE (-3)
#define OHIP_E_NOMEM (-4)
#define OHIP_E_NODEVICE (-5)

/* Element types use ONNX TensorProto codes (oxionnx-core/src/dtype.rs:8). */
enum ohip_dtype { OHIP_F32 = 1, OHIP_U8 = 2, OHIP_I8 = 3, OHIP_I32 = 6, OHIP_F16 = 10, OHIP_BF16 = 16 };

/* Fused activation, the optimizer's attribute contract `activation` /
 * `activation_min` / `activation_max` (oxionnx-ops/src/registry/conv_ops/conv.rs:124-156).
 * LEAKY_RELU takes its slope in act_lo (oxionnx-gpu/src/shaders/conv2d.rs:134-232). */
enum ohip_act { OHIP_ACT_NONE = 0, OHIP_ACT_RELU = 1, OHIP_ACT_CLIP = 2, OHIP_ACT_LEAKY_RELU = 3 };

/* Gemm C operand shapes (oxionnx-ops/src/math_typed.rs:444-455, 718-727). */
enum ohip_bias_kind { OHIP_C_NONE = 0, OHIP_C_SCALAR = 1, OHIP_C_ROW = 2, OHIP_C_FULL = 3 };

enum ohip_layout { OHIP_NCHW = 0, OHIP_NHWC = 1 };
enum ohip_pad_mode { OHIP_PAD_ZEROS = 0, OHIP_PAD_REFLECT = 1, OHIP_PAD_EDGE = 2 };

/* Output kinds of the integer family: requantised u8 / i8 bytes, the raw int32
 * accumulator (MatMulInteger / ConvInteger), or requantised values stored as
 * f32 lanes -- the reference Tensor's own representation, which also carries
 * the union saturation range [-128, 255] that no 8-bit type holds
 * (quant_ops/mod.rs:188-200). */
enum ohip_qout { OHIP_QOUT_U8 = 0, OHIP_QOUT_I8 = 1, OHIP_QOUT_I32 = 2, OHIP_QOUT_F32 = 3 };

/* Performance classes for the dispatch gate (oxionnx-gpu/src/context/tuning.rs:271-611). */
enum ohip_perf_class { OHIP_CLASS_MI355X = 0, OHIP_CLASS_PARITY = 1, OHIP_CLASS_NEVER = 2, OHIP_CLASS_LEGACY = 3 };

typedef struct ohip_ctx ohip_ctx;
typedef struct ohip_weight ohip_weight;

/* ------------------------------------------------------------------ context */
/* Replaces CudaContext::try_new (oxionnx-cuda/src/context.rs:467-481).  The
 * context is Send + Sync: every entry point re-activates its device on the
 * calling thread (activate_context, oxionnx-cuda/src/lib.rs:277-332). */
int ohip_ctx_create(int device, ohip_ctx** out);
void ohip_ctx_destroy(ohip_ctx* ctx);
/* Adopt a caller stream (e.g. torch.cuda.current_stream()); NULL restores the
 * context's own stream. */
int ohip_ctx_set_stream(ohip_ctx* ctx, void* hip_stream);
void* ohip_ctx_stream(ohip_ctx* ctx);
int ohip_sync(ohip_ctx* ctx);

/* ------------------------------------------------------------------ graphs
 * Capture of a whole forward into one HIP graph (the reference's CUDA-graph
 * cache, oxionnx-cuda/src/graph_cache.rs): ohip_graph_begin opens a capture
 * on the context's stream; every dispatch until ohip_graph_end is recorded,
 * not run.  Dispatches must already be warm (weights, constants and output
 * tables cached), because uploads and synchronisations cannot be captured.
 * While a capture is open, freed device buffers are parked for the graph,
 * which keeps them until ohip_graph_destroy; a replay writes the same
 * buffers, so the caller keeps the captured inputs and outputs alive and
 * refills / reads them around ohip_graph_launch.  ohip_pool_parking(ctx, 1)
 * parks buffers without a capture (a dry run that leaves every buffer the
 * forward needs in the pool); ohip_pool_parking(ctx, 0) releases them. */
typedef struct ohip_graph ohip_graph;
int ohip_pool_parking(ohip_ctx* ctx, int on);
int ohip_graph_begin(ohip_ctx* ctx);
int ohip_graph_end(ohip_ctx* ctx, ohip_graph** out);
int ohip_graph_launch(ohip_graph* g);
void ohip_graph_destroy(ohip_graph* g);
int ohip_device_count(int* count);
const char* ohip_last_error(void);
const char* ohip_version(void);
/* Env truthiness used by OXIONNX_HIP / OXIONNX_HIP_VERIFY / OXIONNX_HIP_STRICT /
 * OXIONNX_HIP_RESIDENCY (same rule as oxionnx-cuda/src/context.rs:165-193). */
int ohip_env_flag(const char* name);

/* ------------------------------------------------------------------ memory */
int ohip_malloc(ohip_ctx* ctx, size_t bytes, void** dptr);
int ohip_free(ohip_ctx* ctx, void* dptr);
int ohip_memcpy_h2d(ohip_ctx* ctx, void* dst, const void* src, size_t bytes);  /* stream-ordered */
int ohip_memcpy_d2h(ohip_ctx* ctx, void* dst, const void* src, size_t bytes);  /* synchronous */
int ohip_memcpy_d2d(ohip_ctx* ctx, void* dst, const void* src, size_t bytes);  /* stream-ordered */

/* ------------------------------------------------------------------ gate */
/* GpuTuning (oxionnx-gpu/src/context/tuning.rs:271-611) recalibrated for
 * MI355X.  All of these are device-free. */
typedef struct {
    int perf_class;
    uint64_t gemm_min_mac;          /* B uploaded per dispatch */
    uint64_t gemm_min_mac_cached;   /* B resident in the weight cache */
    uint64_t gemm_min_intensity;    /* FLOP per transferred element, per-dispatch B only */
    uint64_t conv_min_mac;          /* implied GEMM of a Conv */
} ohip_tuning;
int ohip_tuning_for_class(int perf_class, ohip_tuning* out);
int ohip_set_tuning(ohip_ctx* ctx, const ohip_tuning* t);
int ohip_get_tuning(ohip_ctx* ctx, ohip_tuning* out);
/* gemm_mac / gemm_intensity / gemm_admits / conv_admits (tuning.rs:500-611). */
uint64_t ohip_gemm_mac(int64_t m, int64_t k, int64_t n);
uint64_t ohip_gemm_intensity(int64_t m, int64_t k, int64_t n);
int ohip_gemm_admits(const ohip_tuning* t, int64_t m, int64_t k, int64_t n, int b_cached);
int ohip_conv_admits(const ohip_tuning* t, int64_t m, int64_t k, int64_t n);

/* ------------------------------------------------------------------ weights */
/* Session-lifetime weight residency keyed like ResidentWeights / WeightId
 * (oxionnx-cuda/src/residency.rs:677-723) and initializer_key
 * (src/session/gpu_dispatch.rs:614-624): (name, label, packed form, dtype,
 * byte length).  key == NULL (or name == NULL) uploads transiently: the
 * weight is freed by ohip_weight_release.  A cached weight is owned by the
 * context; releasing it is a no-op.  Weights are packed on upload into the
 * kernels' K-contiguous row layout, so no per-call transpose ever runs. */
typedef struct {
    const char* name;   /* initializer name */
    const char* label;  /* operator slot, e.g. "Gemm.B" */
} ohip_weight_key;

/* Float GEMM operand B: host [K,N] (trans_b = 0) or [N,K] (trans_b = 1) of
 * src_dtype (F32/F16/BF16), converted to dtype (F32/F16/BF16, RNE). */
int ohip_weight_gemm(ohip_ctx* ctx, const ohip_weight_key* key, int src_dtype, const void* host,
                     int64_t k, int64_t n, int trans_b, int dtype, ohip_weight** out);
/* Float Conv filter: host [Cout, Cin/group, KH, KW]. */
int ohip_weight_conv(ohip_ctx* ctx, const ohip_weight_key* key, int src_dtype, const void* host,
                     int64_t cout, int64_t cin, int64_t kh, int64_t kw, int dtype, ohip_weight** out);
/* Integer GEMM operand B of MatMulInteger / QLinearMatMul
 * (oxionnx-ops/src/registry/quant_ops/qlinear_matmul.rs:106-133): host u8/i8
 * [K,N] (or [N,K] with trans_b), per-tensor or per-column zero point, and the
 * weight scale(s) (1 or N entries; NULL for MatMulInteger). */
int ohip_weight_qgemm(ohip_ctx* ctx, const ohip_weight_key* key, int src_dtype, const void* host,
                      int64_t k, int64_t n, int trans_b, const int32_t* zp, int n_zp,
                      const float* scale, int n_scale, ohip_weight** out);
/* Integer Conv filter of ConvInteger / QLinearConv
 * (oxionnx-ops/src/registry/quant_ops/conv_kernel.rs:134-254): host u8/i8
 * [Cout, Cin, KH, KW], per-tensor or per-output-channel zero point and scale. */
int ohip_weight_qconv(ohip_ctx* ctx, const ohip_weight_key* key, int src_dtype, const void* host,
                      int64_t cout, int64_t cin, int64_t kh, int64_t kw, const int32_t* zp, int n_zp,
                      const float* scale, int n_scale, ohip_weight** out);
/* Float ConvTranspose filter: host [Cin, Cout/group, KH, KW] of src_dtype,
 * converted to dtype (conv/transpose.rs:78-214).  The node's strides, top /
 * left pads, dilations and group select its form: for group 1, dilation 1
 * and a kernel at least as wide as the stride, the sub-pixel phase filters
 * of the MFMA path are packed as well. */
int ohip_weight_conv_transpose(ohip_ctx* ctx, const ohip_weight_key* key, int src_dtype, const void* host,
                               int64_t cin, int64_t cout_per_group, int64_t kh, int64_t kw, int64_t stride_h,
                               int64_t stride_w, int64_t pad_t, int64_t pad_l, int64_t dil_h, int64_t dil_w,
                               int64_t group, int dtype, ohip_weight** out);
void ohip_weight_release(ohip_weight* w);
size_t ohip_weight_bytes(const ohip_weight* w);

/* ------------------------------------------------------------------ float ops */
/* Gemm / MatMul (oxionnx-ops/src/registry/math_ops/matmul_gemm.rs:9-355,
 * math_typed.rs:589-788): Y[M,N] = act(alpha * A' B + beta * C).  A is a
 * device [M,K] row-major matrix (or [K,M] with trans_a) of `dtype`; B is a
 * packed weight of the same dtype; C / Y are `dtype`.  A batched MatMul whose
 * B is shared collapses to M = batch * rows (oxionnx-cuda/src/matmul.rs:189-252). */
typedef struct {
    int64_t m, k, n;
    int dtype;
    int trans_a;
    float alpha, beta;
    int c_kind;            /* ohip_bias_kind */
    int act;               /* ohip_act (OHIP_ACT_NONE for ONNX Gemm) */
    float act_lo, act_hi;
    int64_t lda, ldy;      /* row strides in elements; 0 = packed */
} ohip_gemm_desc;
int ohip_gemm(ohip_ctx* ctx, const ohip_gemm_desc* d, const void* a, const ohip_weight* b,
              const void* c, void* y);

/* MatMul with both operands on the device (MatMulOp, matmul_gemm.rs:9-126;
 * matmul_f32_into / typed_matmul_batch_info, math_typed.rs:85-115,334-423):
 * A [a_batches][M][K] and B [b_batches][K][N] row-major of `dtype`, Y
 * [batch][M][N]; slice s reads A slice s % a_batches and B slice
 * s % b_batches, like the reference's strided batch (oxionnx-cuda/src/matmul.rs:189-252).
 * B is brought into K-contiguous rows in scratch on every call. */
typedef struct {
    int64_t m, k, n;
    int64_t batch, a_batches, b_batches;
    int dtype;                     /* F32 / F16 / BF16 */
} ohip_matmul_desc;
int ohip_matmul(ohip_ctx* ctx, const ohip_matmul_desc* d, const void* a, const void* b, void* y);

/* Conv, rank 2, any group (oxionnx-ops/src/registry/conv_ops/conv.rs:163-323
 * and conv_typed.rs:54-153): Y = act(conv(X, W) + bias).  Groups run one
 * MFMA launch each, or a direct kernel when a group is too narrow for an
 * MFMA tile (depthwise).  Pads are
 * [top, left, bottom, right], already resolved from auto_pad
 * (conv/spatial.rs:228-257); asymmetric pads are supported.  NCHW inputs are
 * transposed on the device into a channel-padded NHWC staging buffer; NHWC
 * inputs must already carry channels padded to a multiple of 16 bytes. */
typedef struct {
    int64_t n, c, h, w;
    int64_t cout, kh, kw, group;
    int64_t stride_h, stride_w, dil_h, dil_w;
    int64_t pad_t, pad_l, pad_b, pad_r;
    int dtype;                     /* F32 / F16 / BF16 */
    int in_layout, out_layout;     /* ohip_layout */
    int act;
    float act_lo, act_hi;
    /* OHIP_PAD_ZEROS: the pads are ONNX Conv zero padding.  OHIP_PAD_REFLECT /
     * OHIP_PAD_EDGE: they are a reflect / edge Pad node fused in front of the
     * convolution (ONNX Pad semantics), applied while the NCHW input is
     * staged (in_layout must be NCHW). */
    int pad_mode;
} ohip_conv_desc;
int ohip_conv2d(ohip_ctx* ctx, const ohip_conv_desc* d, const void* x, const ohip_weight* w,
                const void* bias, void* y);
/* ohip_conv2d without device allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * kernels and results as ohip_conv2d; the NCHW staging copy and the split-K
 * partial sums live in a static 32 MiB device array per GPU instead of the
 * context's growable scratch.  A call needing more scratch than that returns
 * OHIP_E_NOMEM and launches nothing.  Every call on one GPU shares the array,
 * so calls that overlap on one GPU (other streams or contexts) race. */
int ohip_conv2d_noalloc(ohip_ctx* ctx, const ohip_conv_desc* d, const void* x, const ohip_weight* w,
                        const void* bias, void* y);

/* Conv followed by instance normalisation, one node of this provider's graph
 * fusion (Conv -> OxiInstanceNorm [-> Mul(gamma) -> Add(beta)] [-> Relu]).
 * No counterpart in the reference, whose session runs the two nodes:
 * y = InstanceNorm(conv(x)) with the conv output rounded to its dtype first,
 * exactly as the unfused pair computes it.  When the convolution splits K,
 * the normalisation reads the partial sums directly (no reduction launch).
 * The conv must be ungrouped and without activation, of dtype F32 or F16
 * (BF16 declines); out_layout may be OHIP_NHWC (cout elements per pixel,
 * whole 16-byte pixels). */
typedef struct {
    float epsilon;
    const void* scale;     /* gamma per channel (or per (n, c) when per_sample); may be null */
    const void* bias;      /* beta, same indexing; may be null */
    int per_sample;        /* scale / bias element n * stride + c */
    int64_t stride;
    int same_type;         /* scale / bias in the tensor's dtype (else f32) */
    int act;               /* OHIP_ACT_NONE, OHIP_ACT_RELU or OHIP_ACT_LEAKY_RELU */
    float alpha;           /* leaky slope */
    const void* residual;  /* added after the activation: a tensor of the output's shape and dtype
                              (a fused residual Add), may be null */
    int residual_layout;   /* OHIP_NCHW, or OHIP_NHWC with cout elements per pixel */
} ohip_norm_desc;
int ohip_conv2d_instnorm(ohip_ctx* ctx, const ohip_conv_desc* d, const void* x, const ohip_weight* w,
                         const void* bias, const ohip_norm_desc* norm, void* y);
/* Output extent per conv_out_dim (conv/spatial.rs:272-330); -1 if invalid. */
int64_t ohip_conv_out_dim(int64_t in, int64_t pad_begin, int64_t pad_end, int64_t k, int64_t dil,
                          int64_t stride);

/* ConvTranspose, rank 2 (ConvTransposeOp, oxionnx-ops/src/registry/conv_ops/conv.rs:556-710,
 * conv/transpose.rs:78-309, conv_typed.rs:159-222): Y = scatter(X, W) + bias with
 * W [Cin, Cout/group, KH, KW]; the caller resolves output_shape / auto_pad into
 * pads (conv.rs:412-470).  X and Y are NCHW of `dtype`.  With phase filters
 * (see ohip_weight_conv_transpose) every output phase runs as a stride-1
 * implicit-GEMM convolution on the MFMA engine (f32 accumulation, results
 * within the reference's tolerance); otherwise an output-stationary gather
 * accumulates each output in the reference's scatter order, equal to the
 * reference's result (f16 / bf16 rounded once, RNE). */
typedef struct {
    int64_t n, c, h, w;
    int64_t cout, kh, kw, group;
    int64_t stride_h, stride_w, dil_h, dil_w;
    int64_t pad_t, pad_l, pad_b, pad_r;
    int64_t out_pad_h, out_pad_w;
    int dtype;                     /* F32 / F16 / BF16 */
} ohip_convt_desc;
int ohip_conv_transpose2d(ohip_ctx* ctx, const ohip_convt_desc* d, const void* x, const ohip_weight* w,
                          const void* bias, void* y);
/* Output extent stride * (in - 1) + out_pad + (k - 1) * dil + 1 - pads
 * (conv/spatial.rs:346-407); -1 if invalid. */
int64_t ohip_conv_transpose_out_dim(int64_t in, int64_t stride, int64_t out_pad, int64_t k, int64_t dil,
                                    int64_t pad_begin, int64_t pad_end);

/* ------------------------------------------------------------------ integer ops */
/* MatMulInteger / QLinearMatMul (qlinear_matmul.rs:174-254).  A is a device
 * u8/i8 [M,K] matrix; a_zp holds 1 or M host entries.  For QOUT_U8/QOUT_I8
 * the accumulator is requantised exactly like SatRange::requantize
 * (quant_ops/mod.rs:229-233): combined = a_scale * w_scale / y_scale in f32,
 * f64 product, + y_zp, round half to even, clamp to [lo, hi].  QOUT_I32 emits
 * the raw accumulator (MatMulInteger).  The caller resolves [lo, hi]
 * (SatRange::infer / for_dtype, mod.rs:188-221). */
typedef struct {
    int64_t m, k, n;
    int a_dtype;                   /* U8 or I8 */
    const int32_t* a_zp; int n_azp;
    int out_kind;                  /* ohip_qout */
    float a_scale, y_scale;
    int32_t y_zp, lo, hi;
    int64_t lda, ldy;              /* 0 = packed */
} ohip_qgemm_desc;
int ohip_qgemm(ohip_ctx* ctx, const ohip_qgemm_desc* d, const void* a, const ohip_weight* b, void* y);

/* ConvInteger / QLinearConv (qlinear_conv.rs:34-203): padding taps contribute
 * exactly zero, bias is int32 added into the accumulator, the weight scale
 * may be per output channel. */
typedef struct {
    int64_t n, c, h, w;
    int64_t cout, kh, kw, group;
    int64_t stride_h, stride_w, dil_h, dil_w;
    int64_t pad_t, pad_l, pad_b, pad_r;
    int x_dtype;                   /* U8 or I8 */
    int32_t x_zp;
    int out_kind;
    float x_scale, y_scale;
    int32_t y_zp, lo, hi;
    int in_layout, out_layout;
    /* Optional host table of 256 bytes applied to every requantised byte
     * (QOUT_U8 / QOUT_I8 only), indexed by the byte's bit pattern; NULL for
     * none.  It carries a fused elementwise tail that maps quantised bytes
     * to quantised bytes, e.g. DequantizeLinear -> Silu -> QuantizeLinear
     * (indexing/quantize.rs:96-190, registry/nn_ops/activations.rs:477). */
    const uint8_t* out_table;
    /* NHWC input only: channel slots between consecutive pixels (a multiple
     * of 16, at least c rounded up to 16); 0 means c rounded up to 16.  A
     * larger pitch reads a channel range of a wider NHWC tensor in place. */
    int64_t in_pitch;
} ohip_qconv_desc;
int ohip_qconv2d(ohip_ctx* ctx, const ohip_qconv_desc* d, const void* x, const ohip_weight* w,
                 const int32_t* bias_dev, void* y);

/* ------------------------------------------------------------------ device tensors */
/* A run-scoped device activation (HipDeviceTensor; the DeviceActivation
 * contract of src/session/gpu_activations.rs:117-189 and
 * oxionnx-cuda/src/activation.rs).  Layout NCHW means plain row-major in the
 * ONNX shape; NHWC means channels-last (the conv kernels' native layout)
 * with a pixel pitch of at least the channel count: the channel count
 * padded to 16 bytes for an allocated tensor, the source's pitch for a
 * channel range of another NHWC tensor.  The shape is always the ONNX
 * (N, C, H, W) shape. */
typedef struct ohip_dtensor ohip_dtensor;
int ohip_dtensor_alloc(ohip_ctx* ctx, int dtype, int rank, const int64_t* shape, int layout, ohip_dtensor** out);
/* Take ownership of a device buffer of the context (NCHW layout). */
int ohip_dtensor_wrap(ohip_ctx* ctx, void* dptr, int dtype, int rank, const int64_t* shape, ohip_dtensor** out);
int ohip_dtensor_upload(ohip_ctx* ctx, ohip_dtensor* t, const void* host);      /* NCHW only */
int ohip_dtensor_download(ohip_ctx* ctx, const ohip_dtensor* t, void* host);    /* NCHW bytes, synchronous */
void* ohip_dtensor_ptr(const ohip_dtensor* t);
int ohip_dtensor_layout(const ohip_dtensor* t);
int ohip_dtensor_info(const ohip_dtensor* t, int* dtype, int* rank, int64_t* shape8, size_t* bytes);
void ohip_dtensor_free(ohip_dtensor* t);
/* The NCHW form of a resident tensor as a new tensor, enqueued on the
 * context's stream (an NCHW tensor is shared, not copied).  No counterpart in
 * the reference, whose device activations always hold the ONNX layout: this
 * provider keeps convolution outputs NHWC between convolutions, and a
 * session converts its graph outputs with this call inside the forward (so
 * a captured forward includes the conversion). */
int ohip_dtensor_to_nchw(ohip_ctx* ctx, const ohip_dtensor* t, ohip_dtensor** out);

/* ------------------------------------------------------------------ node dispatch */
/* The drop-in boundary for the session's per-node provider chain
 * (src/session/run/sequential.rs:614-665 -> dispatch_to_cuda :940-1034):
 * is_supported_op / accepts_resident_slot / try_cuda_dispatch[_resident]
 * (oxionnx-cuda/src/lib.rs:217, 419, 354, 561). */
enum ohip_attr_kind { OHIP_ATTR_INT = 0, OHIP_ATTR_FLOAT = 1, OHIP_ATTR_INTS = 2, OHIP_ATTR_STRING = 3 };
typedef struct {
    const char* name;
    int kind;
    int64_t i;
    float f;
    const int64_t* ints;
    int n_ints;
    const char* s;
} ohip_attr;

/* One node operand: a host tensor (data) or a resident device tensor
 * (device); both NULL marks an absent optional input.  dtype is the element
 * type of data -- F32 lanes for the engine's untyped Tensor -- and
 * declared_dtype the ONNX type a typed run knows (0 = unknown), which pins
 * the QLinear* saturation range like SatRange::for_dtype. */
typedef struct {
    const char* name;
    int dtype;
    int declared_dtype;
    int rank;
    const int64_t* shape;
    const void* data;
    const ohip_dtensor* device;
    int is_initializer;
} ohip_tensor;

typedef struct {
    const char* op_type;
    const char* name;
    int n_inputs;
    const ohip_tensor* inputs;
    int n_attrs;
    const ohip_attr* attrs;
} ohip_node;

enum ohip_placement { OHIP_PLACE_HOST = 0, OHIP_PLACE_DEVICE = 1 };

/* A node result: host data (malloc'd by the library) or a device tensor. */
typedef struct {
    int dtype;
    int rank;
    int64_t shape[8];
    void* data;
    ohip_dtensor* device;
} ohip_output;

int ohip_is_supported_op(const char* op_type);
int ohip_accepts_resident_slot(const char* op_type, int index);
/* OHIP_OK: claimed, *out filled.  OHIP_DECLINED: run the CPU operator.
 * < 0: failure (the caller logs it and falls back to the CPU). */
int ohip_try_dispatch(ohip_ctx* ctx, const ohip_node* node, int placement, ohip_output* out);
void ohip_output_free(ohip_output* out);
/* Context creation gated by OXIONNX_HIP like CudaContext::try_new
 * (oxionnx-cuda/src/context.rs:467-481): OHIP_DECLINED when not opted in. */
int ohip_ctx_try_new(ohip_ctx** out);
/* Record a decline reason in the counters (used by the dispatcher). */
void ohip_note_declined(ohip_ctx* ctx, const char* why);
const char* ohip_last_decline(ohip_ctx* ctx);

/* ------------------------------------------------------------------ counters */
/* CacheCounters (oxionnx-cuda/src/residency.rs:141-238) plus dispatch counts,
 * device allocations (hipMalloc calls for the context's weights, pool,
 * scratch and constants; a steady-state forward makes none), host fences
 * (stream synchronisations for a read-back or ohip_sync), as a gauge not
 * reset by ohip_reset_counters, the pool buffers currently handed out, and
 * the contraction launches issued (one per MFMA-engine, halo, GEMV or
 * integer contraction launch; a split-K reduction belongs to its launch). */
typedef struct {
    uint64_t weight_hits, weight_misses, weight_transient;
    uint64_t weight_uploaded_bytes, weight_resident_bytes;
    uint64_t h2d_bytes, d2h_bytes;
    uint64_t dispatches, declined;
    uint64_t device_allocs;
    uint64_t stream_syncs;
    uint64_t pool_live;
    uint64_t contraction_launches;
} ohip_counters;
int ohip_get_counters(ohip_ctx* ctx, ohip_counters* out);
int ohip_reset_counters(ohip_ctx* ctx);

/* Testing / tuning knob: force the MFMA block tile, 0 = automatic.
 * 1: 64x64 (4 waves)   2: 128x128 (4)   3: 256x128 (8)   4: 128x256 (8)
 * 5: 256x256 (4)       6: 256x256 (8)   7: 128x128 (4, two LDS stages)
 * 8: 128x128 (8, two LDS stages)           9: 64x64 (4, four LDS stages)
 * 10: split-K over 64x64 (4, four LDS stages) tiles with an ordered reduction.
 * 11: split-K over 128x128 (8, two LDS stages) tiles with an ordered reduction.
 * 12: 128x128 (8, four stages)   13: 64x64 (4, eight stages)   14: 128x128 (4, four stages)
 * 15: 3x3 stride-1 convolutions take the halo-patch kernel wherever its
 *     geometry allows (automatically only from 3 GFLOP up).
 * 16: 256x256 (8) with a third LDS buffer for the X operand, whose loads run
 *     two stages ahead (the automatic choice where 6 would be).
 * 17: 3x3 stride-1 f16 / bf16 / f32 convolutions with 16-, 32- or 64-wide output
 *     rows take the whole-K halo kernel (no split-K) wherever its geometry
 *     allows (automatically from 256 blocks and 1.5 GFLOP up).
 * 18: 192x256 (8, two LDS stages, one block per CU).
 * The automatic choice splits K (on 64x64 tiles) when the 64x64 tiling gives
 * fewer than 256 blocks and K is at least 16 stages of 128 bytes. */
int ohip_set_tile_override(ohip_ctx* ctx, int tile_id);

#ifdef __cplusplus
}
#endif
#endif
