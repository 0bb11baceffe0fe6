"""Write tests/golden/reference_vectors.json.

The vectors are transcribed by hand from the reference's own test files
(cool-japan/oxionnx v0.1.7); each case names the file:line it comes from.
The reference generated its expected values with onnx.reference / numpy and
inlined them as literals; inputs given there as closed forms
(e.g. ``(0..18).map(|i| ((i % 7) - 3) * 0.5)``) are re-evaluated here from the
same closed form.  Nothing from the reference is imported or executed.

Run:  python tests/golden/make_reference_vectors.py
"""
import json
import os


def seq(n, mod, off, scale):
    return [((i % mod) - off) * scale for i in range(n)]


def iota(n):
    return [float(i) for i in range(n)]


CASES = []


def case(name, source, op, inputs, attrs, expected, shape, **extra):
    d = dict(name=name, source=source, op=op, inputs=inputs, attrs=attrs,
             expected=expected, shape=shape)
    d.update(extra)
    CASES.append(d)


def T(data, shape):
    return {"data": data, "shape": shape}


# ---- tests/w2_quantized_ops_e2e.rs ---------------------------------------
case("matmul_integer_u8_with_zero_point", "tests/w2_quantized_ops_e2e.rs:119-145",
     "MatMulInteger",
     {"a": T([11, 7, 3, 10, 6, 2, 9, 5, 1, 8, 4, 0], [4, 3]),
      "b": T([1, 4, 2, 5, 3, 6], [3, 2]), "a_zp": T([12], [1]), "b_zp": T([0], [1])},
     {}, [-38, -83, -44, -98, -50, -113, -56, -128], [4, 2], dtypes={"a": "u8", "b": "u8"})
case("matmul_integer_i8_without_zero_points", "tests/w2_quantized_ops_e2e.rs:147-165",
     "MatMulInteger",
     {"a": T([1, 2, 3, 4, 5, 6], [2, 3]), "b": T([-1, 2, 3, -4, 5, 6], [3, 2])},
     {}, [20, 12, 41, 24], [2, 2], dtypes={"a": "i8", "b": "i8"})
case("qlinear_matmul_u8_node_test", "tests/w2_quantized_ops_e2e.rs:169-202", "QLinearMatMul",
     {"a": T([208, 236, 0, 238, 3, 214, 255, 29], [2, 4]), "a_scale": T([0.0066], [1]),
      "a_zp": T([113], [1]),
      "b": T([152, 51, 244, 60, 26, 255, 0, 127, 246, 127, 254, 247], [4, 3]),
      "b_scale": T([0.00705], [1]), "b_zp": T([114], [1]), "y_scale": T([0.0107], [1]),
      "y_zp": T([118], [1])},
     {}, [168, 115, 255, 1, 66, 151], [2, 3], dtypes={"a": "u8", "b": "u8", "y": "u8"})
case("qlinear_matmul_i8_symmetric_keeps_negative_outputs",
     "tests/w2_quantized_ops_e2e.rs:206-232", "QLinearMatMul",
     {"a": T([1, -2, 3, 4, 5, -6], [2, 3]), "a_scale": T([0.5], [1]), "a_zp": T([0], [1]),
      "b": T([-1, 2, 3, -4, 5, 6], [3, 2]), "b_scale": T([0.5], [1]), "b_zp": T([0], [1]),
      "y_scale": T([1.0], [1]), "y_zp": T([3], [1])},
     {}, [5, 10, -2, -9], [2, 2], dtypes={"a": "i8", "b": "i8"})
case("conv_integer_with_padding_pads0", "tests/w2_quantized_ops_e2e.rs:236-255", "ConvInteger",
     {"x": T([2, 3, 4, 5, 6, 7, 8, 9, 10], [1, 1, 3, 3]), "w": T([1, 1, 1, 1], [1, 1, 2, 2]),
      "x_zp": T([1], [1])},
     {"pads": [0, 0, 0, 0]}, [12, 16, 24, 28], [1, 1, 2, 2], dtypes={"x": "u8", "w": "u8"})
case("conv_integer_with_padding_pads1", "tests/w2_quantized_ops_e2e.rs:257-274", "ConvInteger",
     {"x": T([2, 3, 4, 5, 6, 7, 8, 9, 10], [1, 1, 3, 3]), "w": T([1, 1, 1, 1], [1, 1, 2, 2]),
      "x_zp": T([1], [1])},
     {"pads": [1, 1, 1, 1]}, [1, 3, 5, 3, 5, 12, 16, 9, 11, 24, 28, 15, 7, 15, 17, 9],
     [1, 1, 4, 4], dtypes={"x": "u8", "w": "u8"})
case("conv_integer_mixed_sign_zero_points", "tests/w2_quantized_ops_e2e.rs:278-304",
     "ConvInteger",
     {"x": T([2, 3, 4, 5, 6, 7, 8, 9, 10], [1, 1, 3, 3]), "w": T([1, -1, 2, 3], [1, 1, 2, 2]),
      "x_zp": T([3], [1]), "w_zp": T([1], [1])},
     {"pads": [0, 0, 0, 0]}, [8, 9, 11, 12], [1, 1, 2, 2], dtypes={"x": "u8", "w": "i8"})
case("qlinear_conv_node_test", "tests/w2_quantized_ops_e2e.rs:308-350", "QLinearConv",
     {"x": T([255, 174, 162, 25, 203, 168, 58, 15, 59, 237, 95, 129, 0, 64, 56, 242, 153, 221,
              168, 12, 166, 232, 178, 186, 195, 237, 162, 237, 188, 39, 124, 77, 80, 102, 43,
              127, 230, 21, 83, 41, 40, 134, 255, 154, 92, 141, 42, 148, 247], [1, 1, 7, 7]),
      "x_scale": T([0.003692047], [1]), "x_zp": T([132], [1]), "w": T([0], [1, 1, 1, 1]),
      "w_scale": T([0.0017279458], [1]), "w_zp": T([255], [1]),
      "y_scale": T([0.0016268126], [1]), "y_zp": T([123], [1])},
     {}, [0, 81, 93, 230, 52, 87, 197, 240, 196, 18, 160, 126, 255, 191, 199, 13, 102, 34, 87,
          243, 89, 23, 77, 69, 60, 18, 93, 18, 67, 216, 131, 178, 175, 153, 212, 128, 25, 234,
          172, 214, 215, 121, 0, 101, 163, 114, 213, 107, 8], [1, 1, 7, 7],
     dtypes={"x": "u8", "w": "u8", "y": "u8"})
case("qlinear_conv_per_channel_scale_and_int32_bias", "tests/w2_quantized_ops_e2e.rs:356-397",
     "QLinearConv",
     {"x": T([float(v) for v in range(1, 33)], [1, 2, 4, 4]), "x_scale": T([0.02], [1]),
      "x_zp": T([16], [1]),
      "w": T([1, -2, 3, 0, 2, 1, -1, 1, 0, 1, 2, -3, 1, 1, 1, 1], [2, 2, 2, 2]),
      "w_scale": T([0.5, 0.25], [2]), "w_zp": T([0, 0], [2]), "y_scale": T([0.05], [1]),
      "y_zp": T([100], [1]), "b": T([50, -60], [2])},
     {"strides": [1, 1], "pads": [0, 0, 0, 0]},
     [107, 108, 109, 111, 112, 113, 115, 116, 117, 95, 95, 96, 96, 97, 97, 98, 98, 99],
     [1, 2, 3, 3], dtypes={"x": "u8", "w": "i8"})
case("qlinear_conv_depthwise_same_upper", "tests/w2_quantized_ops_e2e.rs:401-442", "QLinearConv",
     {"x": T([float(v) for v in range(1, 37)], [1, 4, 3, 3]), "x_scale": T([0.05], [1]),
      "x_zp": T([10], [1]),
      "w": T([130, 120, 140, 126, 128, 132, 124, 129, 127, 131, 125, 133, 135, 121, 138, 122],
             [4, 1, 2, 2]),
      "w_scale": T([0.4], [1]), "w_zp": T([128], [1]), "y_scale": T([0.1], [1]),
      "y_zp": T([50], [1])},
     {"group": 4, "auto_pad": "SAME_UPPER", "kernel_shape": [2, 2]},
     [47, 48, 38, 49, 50, 46, 52, 51, 50, 49, 49, 46, 50, 50, 44, 56, 56, 50, 60, 61, 39, 62,
      63, 37, 57, 57, 47, 64, 65, 124, 67, 67, 134, 49, 49, 86], [1, 4, 3, 3],
     dtypes={"x": "u8", "w": "u8"})
case("qlinear_conv_int8_with_dilations", "tests/w2_quantized_ops_e2e.rs:446-480", "QLinearConv",
     {"x": T([-5, 3, 7, -2, 0, 9, 4, -8, 6, 1, -3, 2, 8, -6, 5, 0], [1, 1, 4, 4]),
      "x_scale": T([0.5], [1]), "x_zp": T([0], [1]), "w": T([2, -1, 1, 3], [1, 1, 2, 2]),
      "w_scale": T([0.5], [1]), "w_zp": T([0], [1]), "y_scale": T([0.25], [1]),
      "y_zp": T([-5], [1])},
     {"dilations": [2, 2], "pads": [0, 0, 0, 0]}, [-25, 10, 14, 15], [1, 1, 2, 2],
     dtypes={"x": "i8", "w": "i8", "y": "i8"})
case("qlinear_matmul_ambiguous_zero_points_use_the_union_range",
     "tests/w2_quantized_ops_e2e.rs:686-713", "QLinearMatMul",
     {"a": T([10, 0, 0, 10], [2, 2]), "a_scale": T([1.0], [1]), "a_zp": T([0], [1]),
      "b": T([10, -15, 0, 0], [2, 2]), "b_scale": T([1.0], [1]), "b_zp": T([0], [1]),
      "y_scale": T([1.0], [1]), "y_zp": T([100], [1])},
     {}, [200, -50, 100, 100], [2, 2], dtypes={"a": "u8", "b": "i8"})

# ---- oxionnx-ops/tests/w2_perf_matmul.rs ---------------------------------
A = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0]
AT = [1.0, 3.0, 5.0, 2.0, 4.0, 6.0]
B = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0]
BT = [1.0, 5.0, 2.0, 6.0, 3.0, 7.0, 4.0, 8.0]
for ta in (0, 1):
    for tb in (0, 1):
        case(f"gemm_stride_table_ta{ta}_tb{tb}", "oxionnx-ops/tests/w2_perf_matmul.rs:110-160",
             "Gemm", {"a": T(AT if ta else A, [2, 3] if ta else [3, 2]),
                      "b": T(BT if tb else B, [4, 2] if tb else [2, 4])},
             {"alpha": 1.0, "beta": 0.0, "transA": ta, "transB": tb},
             [11.0, 14.0, 17.0, 20.0, 23.0, 30.0, 37.0, 44.0, 35.0, 46.0, 57.0, 68.0], [3, 4],
             tol=1e-5)
case("matmul_m1_matches_numpy", "oxionnx-ops/tests/w2_perf_matmul.rs:265-280", "MatMul",
     {"a": T([-1.486, -0.003, 0.406, -1.885, -1.408], [1, 5]),
      "b": T([1.713, -1.718, -1.481, 1.793, 0.488, -0.524, 0.046, 0.651, -0.899, -1.448, 1.152,
              0.681, 0.05, 1.267, 0.196], [5, 3])},
     {}, [0.126859, -1.139666, 0.277691], [1, 3], tol=1e-4)

# ---- tests/conformance_conv.rs -------------------------------------------
case("conformance_conv2d_1x1", "tests/conformance_conv.rs:15-55", "Conv",
     {"x": T([1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0], [1, 2, 2, 2]),
      "w": T([1.0, 0.0, 0.0, 1.0, 1.0, 1.0], [3, 2, 1, 1])},
     {"strides": [1, 1], "pads": [0, 0, 0, 0], "dilations": [1, 1], "group": 1},
     [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0, 6.0, 8.0, 10.0, 12.0], [1, 3, 2, 2], tol=1e-5)
case("conformance_conv2d_3x3_pad1", "tests/conformance_conv.rs:58-90", "Conv",
     {"x": T([1.0] * 9, [1, 1, 3, 3]), "w": T([1.0] * 9, [1, 1, 3, 3])},
     {"strides": [1, 1], "pads": [1, 1, 1, 1], "dilations": [1, 1], "group": 1},
     [4.0, 6.0, 4.0, 6.0, 9.0, 6.0, 4.0, 6.0, 4.0], [1, 1, 3, 3], tol=1e-5)

# ---- oxionnx-ops/tests/w1_conv_pool.rs (iota inputs start at 0) ----------
case("conv_auto_pad_same_upper_preserves_spatial_size",
     "oxionnx-ops/tests/w1_conv_pool.rs:88-106", "Conv",
     {"x": T(iota(25), [1, 1, 5, 5]), "w": T([1.0] * 9, [1, 1, 3, 3])},
     {"auto_pad": "SAME_UPPER"},
     [12.0, 21.0, 27.0, 33.0, 24.0, 33.0, 54.0, 63.0, 72.0, 51.0, 63.0, 99.0, 108.0, 117.0,
      81.0, 93.0, 144.0, 153.0, 162.0, 111.0, 72.0, 111.0, 117.0, 123.0, 84.0], [1, 1, 5, 5],
     tol=1e-4)
case("conv_auto_pad_same_upper_stride2", "oxionnx-ops/tests/w1_conv_pool.rs:108-127", "Conv",
     {"x": T(iota(36), [1, 1, 6, 6]), "w": T([1.0] * 9, [1, 1, 3, 3])},
     {"auto_pad": "SAME_UPPER", "strides": [2, 2]},
     [63.0, 81.0, 63.0, 171.0, 189.0, 135.0, 168.0, 180.0, 126.0], [1, 1, 3, 3], tol=1e-4)
case("conv_auto_pad_same_lower_stride2", "oxionnx-ops/tests/w1_conv_pool.rs:128-137", "Conv",
     {"x": T(iota(36), [1, 1, 6, 6]), "w": T([1.0] * 9, [1, 1, 3, 3])},
     {"auto_pad": "SAME_LOWER", "strides": [2, 2]},
     [14.0, 30.0, 42.0, 75.0, 126.0, 144.0, 147.0, 234.0, 252.0], [1, 1, 3, 3], tol=1e-4)
case("conv_auto_pad_valid_overrides_explicit_pads", "oxionnx-ops/tests/w1_conv_pool.rs:140-155",
     "Conv", {"x": T(iota(25), [1, 1, 5, 5]), "w": T([1.0] * 9, [1, 1, 3, 3])},
     {"auto_pad": "VALID", "pads": [1, 1, 1, 1]},
     [54.0, 63.0, 72.0, 99.0, 108.0, 117.0, 144.0, 153.0, 162.0], [1, 1, 3, 3], tol=1e-4)

# ---- oxionnx-ops/tests/w2_conv_nd.rs: Conv1D cases, run as [N,C,1,W] ------
X18 = seq(18, 7, 3, 0.5)
W18 = seq(18, 5, 2, 0.25)
c1 = "oxionnx-ops/tests/w2_conv_nd.rs"
case("conv1d_basic_with_bias", c1 + ":93-118", "Conv1D",
     {"x": T(X18, [1, 2, 9]), "w": T(W18, [3, 2, 3]), "b": T(seq(3, 3, 1, 0.5), [3])},
     {"kernel_shape": [3]},
     [0.125, -0.125, -0.375, 1.125, -0.875, -2.0, -1.375, -0.125, -0.25, -0.375, 0.375, 2.0,
      -0.75, -0.875, 0.25, 0.25, 0.25, 0.25, 1.125, 1.125, 0.25], [1, 3, 7], tol=1e-5)
case("conv1d_stride2_pads", c1 + ":121-143", "Conv1D",
     {"x": T(X18, [1, 2, 9]), "w": T(W18, [3, 2, 3])},
     {"kernel_shape": [3], "strides": [2], "pads": [2, 1]},
     [0.25, 0.625, 0.125, -0.375, -0.875, -0.25, -0.125, -0.375, 2.0, -0.875, -0.75, -0.25,
      -0.25, 0.625, -0.25], [1, 3, 5], tol=1e-5)
case("conv1d_dilation3", c1 + ":146-166", "Conv1D",
     {"x": T(X18, [1, 2, 9]), "w": T(W18, [3, 2, 3])},
     {"kernel_shape": [3], "dilations": [3]},
     [1.625, 1.375, -0.625, 0.25, -0.75, 0.875, 0.75, -1.0, -0.125], [1, 3, 3], tol=1e-5)
case("conv1d_auto_pad_same_upper", c1 + ":169-191", "Conv1D",
     {"x": T(X18, [1, 2, 9]), "w": T(W18, [3, 2, 3])},
     {"kernel_shape": [3], "strides": [2], "auto_pad": "SAME_UPPER"},
     [0.125, 0.375, 1.625, -1.5, 0.875, 0.0, -0.25, 0.375, -0.75, 0.125, -0.75, -0.25, -0.25,
      0.625, 0.0], [1, 3, 5], tol=1e-5)
case("conv1d_auto_pad_same_lower", c1 + ":194-217", "Conv1D",
     {"x": T(X18, [1, 2, 9]), "w": T(W18, [3, 2, 3])},
     {"kernel_shape": [3], "strides": [2], "dilations": [2], "auto_pad": "SAME_LOWER"},
     [-0.125, 0.25, 1.5, -0.75, -0.75, 0.0, -0.375, 0.25, 0.875, -0.875, -0.5, 0.25, 0.25,
      -0.625, 0.25], [1, 3, 5], tol=1e-5)
case("conv1d_auto_pad_valid", c1 + ":220-243", "Conv1D",
     {"x": T(X18, [1, 2, 9]), "w": T(W18, [3, 2, 3])},
     {"kernel_shape": [3], "strides": [2], "auto_pad": "VALID"},
     [0.625, 0.125, -0.375, -0.875, -0.125, -0.375, 2.0, -0.875, -0.25, -0.25, 0.625, -0.25],
     [1, 3, 4], tol=1e-5)
case("conv1d_group2", c1 + ":246-270", "Conv1D",
     {"x": T(seq(28, 6, 2, 0.5), [1, 4, 7]), "w": T(seq(24, 7, 3, 0.25), [4, 2, 3])},
     {"kernel_shape": [3], "pads": [1, 1], "group": 2},
     [0.5, 1.25, 0.875, 0.5, -1.375, -1.75, -0.75, 1.0, -0.125, -0.375, -0.625, -1.625, -0.375,
      2.125, -0.5, -0.875, -1.0, 1.875, 1.0, -0.625, -0.375, -0.125, -0.25, 0.5, -0.25, 0.5,
      -0.25, -0.375], [1, 4, 7], tol=1e-5)
case("conv1d_batch2_stride_dilation", c1 + ":273-312", "Conv1D",
     {"x": T(seq(66, 9, 4, 0.5), [2, 3, 11]), "w": T(seq(36, 11, 5, 0.25), [4, 3, 3]),
      "b": T(seq(4, 4, 2, 0.5), [4])},
     {"kernel_shape": [3], "strides": [2], "pads": [2, 2], "dilations": [2]},
     [2.75, 5.0, -0.625, -5.125, -4.0, -1.0, -0.75, -2.75, -5.125, -4.125, 4.75, 1.625, -1.5,
      -5.0, -4.125, 2.375, 6.625, -1.25, -2.25, -1.75, 2.375, 2.0, 1.625, -1.375, -5.125, -4.0,
      0.5, 0.5, -4.0, -4.375, -2.625, 4.75, 2.375, -4.5, -3.5, 2.375, 2.625, 6.625, -2.625,
      -4.0, 2.5, 7.75, 3.75, 1.625, -2.125, 2.0, 1.625, 3.5], [2, 4, 6], tol=1e-5)

# ---- oxionnx-ops/tests/gemm_native_dtype_test.rs:320-380 ------------------
# The reference compares the typed f16 Gemm against its own f32 Gemm with an
# absolute tolerance of 1e-2; the f32 expectation below is that closed form
# (A@B*0.5 + 0.5*bias) evaluated exactly, every value being a short dyadic.
GA = [1.0, 0.5, -0.5, 0.25, 0.25, 1.0, 0.5, -0.5, -0.5, 0.25, 1.0, 0.5, 0.5, -0.5, 0.25, 1.0]
GB = [1.0, 0.0, 0.5, -0.5, 0.0, 1.0, -0.5, 0.5, 0.5, -0.5, 1.0, 0.0, -0.5, 0.5, 0.0, 1.0]
GC = [0.1, 0.2, 0.3, 0.4]
exp = []
for i in range(4):
    for j in range(4):
        s = sum(GA[i * 4 + p] * GB[p * 4 + j] for p in range(4))
        exp.append(s * 0.5 + 0.5 * GC[j])
case("test_gemm_f16_parity", "oxionnx-ops/tests/gemm_native_dtype_test.rs:320-380", "GemmF16",
     {"a": T(GA, [4, 4]), "b": T(GB, [4, 4]), "c": T(GC, [4])},
     {"alpha": 0.5, "beta": 0.5, "transA": 0, "transB": 0}, exp, [4, 4], tol=1e-2)


# ---- graph nodes of the end-to-end workloads (oracle/graph_ref.py) --------
# Nearest Resize: oxionnx-ops/tests/w1_resize.rs:144-151 (inputs d14 / d22 /
# d45), :8-23 (expected rows), :200-263, :590-611, :613-637.
D14 = T([1.0, 2.0, 3.0, 4.0], [1, 1, 1, 4])
D22 = T([1.0, 2.0, 3.0, 4.0], [1, 1, 2, 2])
rz = "oxionnx-ops/tests/w1_resize.rs"
for mode, exp in [("round_prefer_floor", [1.0, 1.0, 2.0, 2.0, 3.0, 3.0, 4.0, 4.0]),
                  ("round_prefer_ceil", [1.0, 1.0, 2.0, 2.0, 3.0, 3.0, 4.0, 4.0]),
                  ("floor", [1.0, 1.0, 1.0, 2.0, 2.0, 3.0, 3.0, 4.0]),
                  ("ceil", [1.0, 2.0, 2.0, 3.0, 3.0, 4.0, 4.0, 4.0])]:
    case(f"resize_nearest_half_pixel_{mode}", rz + ":8-11,219-233", "Resize",
         {"x": D14, "scales": T([1.0, 1.0, 1.0, 2.0], [4])},
         {"mode": "nearest", "coordinate_transformation_mode": "half_pixel", "nearest_mode": mode},
         exp, [1, 1, 1, 8])
case("resize_nearest_asymmetric_prefer_floor", rz + ":14-17,236-248", "Resize",
     {"x": D22, "scales": T([1.0, 1.0, 2.0, 2.0], [4])},
     {"mode": "nearest", "coordinate_transformation_mode": "asymmetric", "nearest_mode": "round_prefer_floor"},
     [1.0, 1.0, 2.0, 2.0, 1.0, 1.0, 2.0, 2.0, 3.0, 3.0, 4.0, 4.0, 3.0, 3.0, 4.0, 4.0], [1, 1, 4, 4])
case("resize_nearest_asymmetric_prefer_ceil", rz + ":19-23,250-262", "Resize",
     {"x": D22, "scales": T([1.0, 1.0, 2.0, 2.0], [4])},
     {"mode": "nearest", "coordinate_transformation_mode": "asymmetric", "nearest_mode": "round_prefer_ceil"},
     [1.0, 2.0, 2.0, 2.0, 3.0, 4.0, 4.0, 4.0, 3.0, 4.0, 4.0, 4.0, 3.0, 4.0, 4.0, 4.0], [1, 1, 4, 4])
case("resize_nearest_tf_half_pixel_for_nn", rz + ":590-611", "Resize",
     {"x": D14, "scales": T([1.0, 1.0, 1.0, 2.0], [4])},
     {"mode": "nearest", "coordinate_transformation_mode": "tf_half_pixel_for_nn",
      "nearest_mode": "round_prefer_floor"},
     [1.0, 2.0, 2.0, 3.0, 3.0, 4.0, 4.0, 4.0], [1, 1, 1, 8])
for sc, hw in [(0.5, [2, 2]), (0.6, [2, 3]), (1.3, [5, 6]), (2.7, [10, 13])]:
    case(f"resize_output_shape_floor_{sc}", rz + ":613-637", "ResizeShape",
         {"x": T(iota(20), [1, 1, 4, 5]), "scales": T([1.0, 1.0, sc, sc], [4])},
         {"mode": "nearest", "coordinate_transformation_mode": "half_pixel"}, None, [1, 1] + hw)
# Upsample-9 (scales input): the asymmetric mapping, tests/w2_vision_ops_e2e.rs:578-608
case("upsample_nearest_scales_input_is_asymmetric", "tests/w2_vision_ops_e2e.rs:578-608", "Resize",
     {"x": D22, "scales": T([1.0, 1.0, 2.0, 2.0], [4])},
     {"mode": "nearest", "coordinate_transformation_mode": "asymmetric", "nearest_mode": "floor"},
     [1., 1., 2., 2., 1., 1., 2., 2., 3., 3., 4., 4., 3., 3., 4., 4.], [1, 1, 4, 4])
case("upsample_nearest_scales_attribute", "tests/w2_vision_ops_e2e.rs:610-640", "Resize",
     {"x": D22, "scales": T([1.0, 1.0, 2.0, 3.0], [4])},
     {"mode": "nearest", "coordinate_transformation_mode": "asymmetric", "nearest_mode": "floor"},
     [1., 1., 1., 2., 2., 2., 1., 1., 1., 2., 2., 2., 3., 3., 3., 4., 4., 4., 3., 3., 3., 4., 4., 4.],
     [1, 1, 4, 6])

# MaxPool (floor mode): tests/conformance_conv.rs:94-126, tests/op_conv_tests.rs:111-141,
# oxionnx-ops/tests/w1_conv_pool.rs:276-328
case("conformance_maxpool_2x2", "tests/conformance_conv.rs:94-126", "MaxPool",
     {"x": T([float(v) for v in range(1, 17)], [1, 1, 4, 4])},
     {"kernel_shape": [2, 2], "strides": [2, 2], "pads": [0, 0, 0, 0]}, [6.0, 8.0, 14.0, 16.0], [1, 1, 2, 2])
case("test_maxpool", "tests/op_conv_tests.rs:111-141", "MaxPool",
     {"x": T([float(v) for v in range(1, 17)], [1, 1, 4, 4])},
     {"kernel_shape": [2, 2], "strides": [2, 2], "pads": [0, 0, 0, 0]}, [6.0, 8.0, 14.0, 16.0], [1, 1, 2, 2])
case("max_pool_floor_5x5_k2_s2", "oxionnx-ops/tests/w1_conv_pool.rs:294-303", "MaxPool",
     {"x": T(iota(25), [1, 1, 5, 5])}, {"kernel_shape": [2, 2], "strides": [2, 2]},
     [6.0, 8.0, 16.0, 18.0], [1, 1, 2, 2])
case("max_pool_floor_4x4_k3_s2", "oxionnx-ops/tests/w1_conv_pool.rs:323-328", "MaxPool",
     {"x": T(iota(16), [1, 1, 4, 4])}, {"kernel_shape": [3, 3], "strides": [2, 2]}, [10.0], [1, 1, 1, 1])

# Pad: oxionnx-ops/src/shape/tests.rs:187-199 (reflect), oxionnx-ops/tests/stitch_s2_shape.rs:154-167
# (an empty constant_value falls back to 0)
case("test_pad_reflect", "oxionnx-ops/src/shape/tests.rs:187-199", "Pad",
     {"x": T([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], [2, 3]), "pads": T([0, 1, 0, 1], [4])},
     {"mode": "reflect"}, [2.0, 1.0, 2.0, 3.0, 2.0, 5.0, 4.0, 5.0, 6.0, 5.0], [2, 5])
case("pad_constant_default_zero", "oxionnx-ops/tests/stitch_s2_shape.rs:154-167", "Pad",
     {"x": T([1.0, 2.0], [2]), "pads": T([1, 1], [2])}, {"mode": "constant"}, [0.0, 1.0, 2.0, 0.0], [4])

# QuantizeLinear / DequantizeLinear (per tensor): tests/conformance_quant.rs:13-62,
# oxionnx-ops/tests/w1_indexing_quant.rs:420-476 (each per-axis row there taken as a per-tensor case)
qsrc = "oxionnx-ops/tests/w1_indexing_quant.rs"
case("conformance_quantize", "tests/conformance_quant.rs:13-62", "QuantizeLinear",
     {"x": T([0.0, 1.0, 2.0, 3.0, 4.0], [5]), "scale": T([0.1], [1]), "zp": T([0.0], [1])}, {},
     [0.0, 10.0, 20.0, 30.0, 40.0], [5])
case("conformance_dequantize", "tests/conformance_quant.rs:13-62", "DequantizeLinear",
     {"x": T([0.0, 10.0, 20.0, 30.0, 40.0], [5]), "scale": T([0.1], [1]), "zp": T([0.0], [1])}, {},
     [0.0, 1.0, 2.0, 3.0, 4.0], [5], tol=0.1)
case("quantize_ties_to_even_row1", qsrc + ":421-439", "QuantizeLinear",
     {"x": T([4.0, 5.0, 6.0], [3]), "scale": T([10.0], [1])}, {}, [0.0, 0.0, 1.0], [3])
case("quantize_ties_to_even_columns", qsrc + ":441-453", "QuantizeLinear",
     {"x": T([2.0, 5.0], [2]), "scale": T([2.0], [1])}, {}, [1.0, 2.0], [2])
case("quantize_zero_point_row1", qsrc + ":455-465", "QuantizeLinear",
     {"x": T([7.0, 3.0], [2]), "scale": T([1.0], [1]), "zp": T([100.0], [1])}, {}, [107.0, 103.0], [2])
case("dequantize_row0", qsrc + ":467-476", "DequantizeLinear",
     {"x": T([10.0, 20.0], [2]), "scale": T([2.0], [1]), "zp": T([1.0], [1])}, {}, [18.0, 38.0], [2], tol=0.0)
case("dequantize_row1", qsrc + ":467-476", "DequantizeLinear",
     {"x": T([30.0, 40.0], [2]), "scale": T([0.5], [1]), "zp": T([2.0], [1])}, {}, [14.0, 19.0], [2], tol=0.0)

# Unary activations: tests/w3_simd_scalar_reference_equivalence.rs:61-63 (input A),
# :156-173 (Sigmoid), :176-193 (Tanh), :227-244 (SiLU); tests/op_nn_tests.rs:404-421 (LeakyRelu)
UA = [-3.0, -1.5, -0.5, -0.001, 0.0, 0.001, 0.25, 0.5, 1.0, 1.5, 2.0, 4.5]
us = "tests/w3_simd_scalar_reference_equivalence.rs"
case("sigmoid_matches_numpy_reference", us + ":156-173", "Sigmoid", {"x": T(UA, [12])}, {},
     [0.047425873, 0.18242553, 0.37754068, 0.49975, 0.5, 0.50025, 0.5621765, 0.62245935, 0.7310586,
      0.8175745, 0.8807971, 0.9890131], [12], tol=1e-6)
case("tanh_matches_numpy_reference", us + ":176-193", "Tanh", {"x": T(UA, [12])}, {},
     [-0.9950548, -0.90514827, -0.46211717, -0.0009999997, 0.0, 0.0009999997, 0.24491866, 0.46211717,
      0.7615942, 0.90514827, 0.9640276, 0.99975324], [12], tol=1e-6)
case("silu_matches_numpy_reference", us + ":227-244", "Silu", {"x": T(UA, [12])}, {},
     [-0.14227762, -0.27363828, -0.18877034, -0.00049975, 0.0, 0.00050025, 0.14054413, 0.31122968,
      0.7310586, 1.2263618, 1.7615942, 4.4505587], [12], tol=1e-6)
case("test_leaky_relu", "tests/op_nn_tests.rs:404-421", "LeakyRelu", {"x": T([-10.0, -1.0, 0.0, 1.0, 10.0], [5])},
     {"alpha": 0.1}, [-1.0, -0.1, 0.0, 1.0, 10.0], [5], tol=1e-5)

if __name__ == "__main__":
    here = os.path.dirname(os.path.abspath(__file__))
    with open(os.path.join(here, "reference_vectors.json"), "w") as f:
        json.dump({"generator": "tests/golden/make_reference_vectors.py", "cases": CASES}, f,
                  indent=1)
    print(len(CASES), "cases")
