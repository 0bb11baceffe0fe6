"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked three ways where the domain allows:
  * the reference's own golden vectors (tests/golden/reference_vectors.json);
  * a closed form computed independently (numpy int64 brute force, numpy
    float64 / torch float64 convolution, numpy's IEEE float16 cast);
  * special cases that a plausible mistake would break (ties in rounding,
    transposed operands with m != k != n, asymmetric pads).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests import _golden as G


# ------------------------------------------------------------ golden vectors
@pytest.mark.parametrize("c", G.cases("MatMulInteger"), ids=lambda c: c["name"])
def test_matmul_integer_golden(c):
    y = O.matmul_integer(G.arr(c, "a"), G.arr(c, "b"), G.arr(c, "a_zp"), G.arr(c, "b_zp"))
    assert list(y.shape) == c["shape"]
    assert y.ravel().tolist() == c["expected"]


@pytest.mark.parametrize("c", G.cases("QLinearMatMul"), ids=lambda c: c["name"])
def test_qlinear_matmul_golden(c):
    g = lambda n: G.arr(c, n)
    y = O.qlinear_matmul(g("a"), g("a_scale"), g("a_zp"), g("b"), g("b_scale"), g("b_zp"),
                         g("y_scale"), g("y_zp"))
    assert list(y.shape) == c["shape"]
    assert y.ravel().tolist() == c["expected"]


@pytest.mark.parametrize("c", G.cases("ConvInteger"), ids=lambda c: c["name"])
def test_conv_integer_golden(c):
    y = O.conv_integer(G.arr(c, "x"), G.arr(c, "w"), G.arr(c, "x_zp"), G.arr(c, "w_zp"),
                       **G.conv_attrs(c))
    assert list(y.shape) == c["shape"]
    assert y.ravel().tolist() == c["expected"]


@pytest.mark.parametrize("c", G.cases("QLinearConv"), ids=lambda c: c["name"])
def test_qlinear_conv_golden(c):
    g = lambda n: G.arr(c, n)
    y = O.qlinear_conv(g("x"), g("x_scale"), g("x_zp"), g("w"), g("w_scale"), g("w_zp"),
                       g("y_scale"), g("y_zp"), bias=g("b"), **G.conv_attrs(c))
    assert list(y.shape) == c["shape"]
    assert y.ravel().tolist() == c["expected"]


@pytest.mark.parametrize("c", G.cases("Conv") + G.cases("Conv1D"), ids=lambda c: c["name"])
def test_conv_f32_golden(c):
    x, w, b = G.conv_inputs(c)
    y = O.conv(x, w, b, **G.conv_attrs(c))
    assert int(np.prod(y.shape)) == int(np.prod(c["shape"]))
    np.testing.assert_allclose(y.ravel(), np.asarray(c["expected"], np.float32), atol=c["tol"])


@pytest.mark.parametrize("c", G.cases("Gemm") + G.cases("MatMul"), ids=lambda c: c["name"])
def test_gemm_f32_golden(c):
    at = c["attrs"]
    y = O.gemm(G.arr(c, "a"), G.arr(c, "b"), None, at.get("alpha", 1.0), at.get("beta", 1.0),
               at.get("transA", 0), at.get("transB", 0))
    assert list(y.shape) == c["shape"]
    np.testing.assert_allclose(y.ravel(), c["expected"], atol=c["tol"])


@pytest.mark.parametrize("c", G.cases("GemmF16"), ids=lambda c: c["name"])
def test_gemm_f16_golden(c):
    at = c["attrs"]
    h = lambda n: O.f32_to_half_bits(G.arr(c, n))
    y = O.gemm_half(h("a"), h("b"), h("c"), at["alpha"], at["beta"], at["transA"], at["transB"])
    np.testing.assert_allclose(O.half_bits_to_f32(y).ravel(), c["expected"], atol=c["tol"])


# ------------------------------------------------------------- closed forms
def test_round_ties_even_special_cases():
    cases = {2.5: 2.0, 3.5: 4.0, -2.5: -2.0, -3.5: -4.0, 0.5: 0.0, -0.5: -0.0, 1.5: 2.0,
             2.4999999: 2.0, 2.5000001: 3.0, -127.49999: -127.0, 7.0: 7.0}
    for v, want in cases.items():
        assert O.round_ties_even(v) == want, v
    rng = np.random.default_rng(0)
    v = rng.uniform(-1e6, 1e6, 5000)
    v[::3] = np.floor(v[::3]) + 0.5
    got = np.array([O.round_ties_even(x) for x in v])
    np.testing.assert_array_equal(got, np.rint(v))


def test_satrange_cascade():
    assert O.satrange_infer([200], [0]) == (0, 255)
    assert O.satrange_infer([-3], [200]) == (-128, 127)
    assert O.satrange_infer([0], [130]) == (0, 255)
    assert O.satrange_infer([5], [-1]) == (-128, 127)
    assert O.satrange_infer([0], [0]) == (-128, 255)


def _brute_qmm(a, b, az, bz):
    return (a.astype(np.int64) - np.asarray(az, np.int64).reshape(-1, 1)) @ (
        b.astype(np.int64) - np.asarray(bz, np.int64).reshape(1, -1))


def test_integer_matmul_matches_int64_brute_force():
    rng = np.random.default_rng(1)
    for (m, k, n) in [(1, 1, 1), (7, 13, 5), (33, 64, 17), (64, 300, 48)]:
        a = rng.integers(0, 256, (m, k))
        b = rng.integers(-128, 128, (k, n))
        az = rng.integers(0, 256, m)          # per-row a_zp (ONNX allows [M])
        bz = rng.integers(-128, 128, n)       # per-column b_zp
        got = O.matmul_integer(a, b, az, bz)
        np.testing.assert_array_equal(got, _brute_qmm(a, b, az, bz))
        got = O.matmul_integer(a, b, az[:1], bz[:1])
        np.testing.assert_array_equal(got, _brute_qmm(a, b, az[:1], bz[:1]))


def test_qlinear_requant_matches_numpy_rint_f64():
    rng = np.random.default_rng(2)
    m, k, n = 16, 96, 24
    a = rng.integers(0, 256, (m, k))
    b = rng.integers(-127, 128, (k, n))
    a_s, b_s, y_s = np.float32(0.02), np.float32(0.0037), np.float32(0.05)
    y = O.qlinear_matmul(a, a_s, 128, b, b_s, 0, y_s, 128)
    comb = np.float32(np.float32(a_s * b_s) / y_s)
    acc = _brute_qmm(a, b, [128], [0]).astype(np.float64)
    want = np.clip(np.rint(acc * np.float64(comb) + 128.0), 0, 255)
    np.testing.assert_array_equal(y, want)


def test_qlinear_matmul_reads_only_first_b_scale():
    """Reference quirk: scale_input reads data.first() (quant_ops/mod.rs:100-118)."""
    rng = np.random.default_rng(3)
    a = rng.integers(0, 256, (4, 8))
    b = rng.integers(-127, 128, (8, 6))
    bs = np.linspace(0.001, 0.01, 6).astype(np.float32)
    y1 = O.qlinear_matmul(a, 0.02, 128, b, bs, 0, 0.05, 128)
    y2 = O.qlinear_matmul(a, 0.02, 128, b, bs[:1], 0, 0.05, 128)
    np.testing.assert_array_equal(y1, y2)


def _brute_int_conv(x, w, xzp, wzp, bias, s, p, d, g):
    n, c, h, wd = x.shape
    co, cpg, kh, kw = w.shape
    xp = np.full((n, c, h + p[0] + p[2], wd + p[1] + p[3]), xzp, np.int64)
    xp[:, :, p[0]:p[0] + h, p[1]:p[1] + wd] = x
    oh = (h + p[0] + p[2] - ((kh - 1) * d[0] + 1)) // s[0] + 1
    ow = (wd + p[1] + p[3] - ((kw - 1) * d[1] + 1)) // s[1] + 1
    wz = np.broadcast_to(np.asarray(wzp, np.int64).reshape(-1), (co,))
    out = np.zeros((n, co, oh, ow), np.int64)
    copg = co // g
    for oc in range(co):
        gi = oc // copg
        wv = w[oc].astype(np.int64) - wz[oc]
        for ky in range(kh):
            for kx in range(kw):
                patch = xp[:, gi * cpg:(gi + 1) * cpg, ky * d[0]:ky * d[0] + s[0] * (oh - 1) + 1:s[0],
                           kx * d[1]:kx * d[1] + s[1] * (ow - 1) + 1:s[1]] - xzp
                out[:, oc] += np.einsum("ncij,c->nij", patch, wv[:, ky, kx])
        if bias is not None:
            out[:, oc] += int(bias[oc])
    return out


def test_integer_conv_matches_padded_brute_force():
    """Padding taps are skipped (conv_kernel.rs:216-229), which equals padding
    x with x_zp -- an independent formulation."""
    rng = np.random.default_rng(4)
    for (shape, wshape, s, p, d, g) in [
        ((1, 3, 9, 11), (5, 3, 3, 3), (1, 1), (1, 2, 0, 1), (1, 1), 1),
        ((2, 4, 8, 8), (4, 2, 3, 3), (2, 2), (1, 1, 1, 1), (1, 1), 2),
        ((1, 6, 7, 9), (6, 1, 3, 2), (1, 2), (2, 0, 1, 1), (2, 1), 6),
        ((1, 16, 10, 10), (8, 16, 1, 1), (1, 1), (0, 0, 0, 0), (1, 1), 1),
    ]:
        x = rng.integers(0, 256, shape)
        w = rng.integers(-127, 128, wshape)
        wz = rng.integers(-5, 6, wshape[0])
        bias = rng.integers(-1000, 1000, wshape[0])
        got, _ = O.integer_conv(x, w, 77, wz, bias, strides=s, pads=p, dilations=d, group=g)
        want = _brute_int_conv(x, w, 77, wz, bias, s, p, d, g)
        np.testing.assert_array_equal(got.reshape(want.shape), want)


def test_conv_f32_matches_torch_float64():
    rng = np.random.default_rng(5)
    for (shape, wshape, s, p, d, g) in [
        ((1, 8, 17, 13), (6, 8, 3, 3), (1, 1), (1, 1, 1, 1), (1, 1), 1),
        ((2, 4, 12, 12), (8, 2, 3, 3), (2, 2), (1, 1, 1, 1), (1, 1), 2),
        ((1, 3, 20, 20), (16, 3, 7, 7), (1, 1), (3, 3, 3, 3), (1, 1), 1),
        ((1, 16, 9, 9), (4, 16, 1, 1), (1, 1), (0, 0, 0, 0), (1, 1), 1),
        ((1, 5, 11, 10), (3, 5, 3, 2), (2, 1), (2, 0, 2, 0), (2, 3), 1),
    ]:
        x = rng.uniform(-1, 1, shape).astype(np.float32)
        w = rng.normal(0, 0.05, wshape).astype(np.float32)
        b = rng.normal(0, 0.01, wshape[0]).astype(np.float32)
        got = O.conv(x, w, b, strides=s, pads=p, dilations=d, group=g)
        xt = torch.nn.functional.pad(torch.from_numpy(x).double(), (p[1], p[3], p[0], p[2]))
        want = torch.nn.functional.conv2d(xt, torch.from_numpy(w).double(),
                                          torch.from_numpy(b).double(), stride=s, dilation=d,
                                          groups=g).numpy()
        assert got.shape == want.shape
        assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))


def test_fused_activation_semantics():
    v = np.array([-2.0, -0.5, 0.0, 0.5, 2.0, np.nan], np.float32)
    np.testing.assert_array_equal(O.apply_activation(v.copy(), "relu"),
                                  [0.0, 0.0, 0.0, 0.5, 2.0, 0.0])
    got = O.apply_activation(v.copy(), "clip", -1.0, 1.0)
    np.testing.assert_array_equal(got[:5], [-1.0, -0.5, 0.0, 0.5, 1.0])
    assert np.isnan(got[5])
    # inverted range is a no-op; NaN bound is unbounded on that side
    np.testing.assert_array_equal(O.apply_activation(v.copy(), "clip", 1.0, -1.0)[:5], v[:5])
    np.testing.assert_array_equal(O.apply_activation(v.copy(), "clip", float("nan"), 1.0)[:5],
                                  [-2.0, -0.5, 0.0, 0.5, 1.0])


def test_gemm_f32_transposes_and_bias_broadcast():
    rng = np.random.default_rng(6)
    m, k, n = 5, 7, 3
    a = rng.normal(size=(m, k)).astype(np.float32)
    b = rng.normal(size=(k, n)).astype(np.float32)
    for c in [None, rng.normal(size=(n,)), rng.normal(size=(m, 1)), rng.normal(size=(m, n)),
              np.float32(0.5)]:
        for ta in (0, 1):
            for tb in (0, 1):
                aa = a.T.copy() if ta else a
                bb = b.T.copy() if tb else b
                got = O.gemm(aa, bb, c, 0.75, 1.25, ta, tb)
                want = 0.75 * (a.astype(np.float64) @ b)
                if c is not None:
                    want = want + 1.25 * np.broadcast_to(np.asarray(c, np.float64), (m, n))
                np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_half_conversions_match_ieee():
    rng = np.random.default_rng(7)
    v = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 5000),
                        rng.normal(0, 3e4, 5000), [65504.0, 65520.0, 65519.99, 1e-8, -0.0,
                                                   np.inf, -np.inf, 6.1e-5, 5.96e-8, 2.98e-8]])
    v = v.astype(np.float32)
    h = O.f32_to_half_bits(v)
    np.testing.assert_array_equal(h, v.astype(np.float16).view(np.uint16))
    back = O.half_bits_to_f32(h)
    np.testing.assert_array_equal(back, h.view(np.float16).astype(np.float32))
    # bf16: round-to-nearest-even on the top 16 bits, checked on exact ties
    bits = np.array([0x3f808000, 0x3f818000, 0x3f80c000, 0x3f804000, 0x7f7fffff], np.uint32)
    got = O.f32_to_half_bits(bits.view(np.float32), bf16=True)
    np.testing.assert_array_equal(got, [0x3f80, 0x3f82, 0x3f81, 0x3f80, 0x7f80])
    t = torch.from_numpy(v[np.isfinite(v)]).to(torch.bfloat16).view(torch.int16).numpy()
    np.testing.assert_array_equal(O.f32_to_half_bits(v[np.isfinite(v)], bf16=True),
                                  t.view(np.uint16))


def test_gemm_half_matches_ascending_f32_accumulation():
    """gemm_f16's per-element order is ascending p with an f32 accumulator;
    checked against an explicit numpy loop in that order."""
    rng = np.random.default_rng(8)
    m, k, n = 6, 37, 9
    a = rng.uniform(-1, 1, (m, k)).astype(np.float16)
    b = rng.normal(0, 0.3, (k, n)).astype(np.float16)
    c = rng.normal(0, 0.1, n).astype(np.float16)
    for ta, tb in [(0, 0), (1, 1)]:
        aa = a.T.copy() if ta else a
        bb = b.T.copy() if tb else b
        got = O.gemm_half(aa.view(np.uint16), bb.view(np.uint16), c.view(np.uint16), 0.5, 2.0,
                          ta, tb)
        acc = np.zeros((m, n), np.float32)
        for p in range(k):
            acc = acc + a[:, p:p + 1].astype(np.float32) * b[p:p + 1, :].astype(np.float32)
        want = (acc * np.float32(0.5) + np.float32(2.0) * c.astype(np.float32)).astype(np.float16)
        np.testing.assert_array_equal(got, want.view(np.uint16))


def test_conv_geometry_same_pads():
    s, p, d, out = O.conv_geometry([1, 1, 6, 6], [1, 1, 3, 3], [2, 2], None, None, 1, "SAME_UPPER")
    assert p == [0, 0, 1, 1] and out == [1, 1, 3, 3]
    s, p, d, out = O.conv_geometry([1, 1, 6, 6], [1, 1, 3, 3], [2, 2], None, None, 1, "SAME_LOWER")
    assert p == [1, 1, 0, 0]
    with pytest.raises(ValueError):
        O.conv_geometry([1, 1, 2, 2], [1, 1, 5, 5])


# ------------------------------------------------------------------ ConvTranspose
def test_conv_transpose_known_answers():
    """oxionnx-ops/src/conv/tests.rs:137-253 (test_conv_transpose_basic / _upsample /
    _with_bias / _with_padding / _multi_channel)."""
    x = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 2, 2)
    assert O.conv_transpose(x, np.ones((1, 1, 1, 1), np.float32)).ravel().tolist() == [1, 2, 3, 4]
    up = O.conv_transpose(np.ones((1, 1, 1, 1), np.float32), np.ones((1, 1, 2, 2), np.float32), strides=[2, 2])
    assert up.shape == (1, 1, 2, 2) and up.ravel().tolist() == [1, 1, 1, 1]
    yb = O.conv_transpose(np.ones((1, 1, 1, 1), np.float32), np.full((1, 1, 1, 1), 2, np.float32),
                          np.array([3], np.float32))
    assert yb.ravel().tolist() == [5.0]
    yp = O.conv_transpose(x, np.ones((1, 1, 3, 3), np.float32), pads=[1, 1, 1, 1])
    # pads 1 crop the 4x4 scatter of a 3x3 ones kernel to its centre: every
    # output sums all four inputs
    assert yp.shape == (1, 1, 2, 2) and yp.ravel().tolist() == [10, 10, 10, 10]
    xm = np.array([1, 1, 1, 1, 2, 2, 2, 2], np.float32).reshape(1, 2, 2, 2)
    assert O.conv_transpose(xm, np.ones((2, 1, 1, 1), np.float32)).ravel().tolist() == [3, 3, 3, 3]


def test_conv_transpose_output_shape_rules():
    """tests/s4_engine_stitch.rs:277-325: the 4-entry output_shape form, SAME_UPPER
    (in * stride) and the natural extent stride * (in - 1) + k."""
    g = lambda **a: O.conv_transpose_geometry((1, 1, 3, 3), (1, 2, 3, 3), strides=[2, 2], **a)[3]
    assert g(output_shape=[1, 2, 6, 6]) == [1, 2, 6, 6]
    assert g(auto_pad="SAME_UPPER") == [1, 2, 6, 6]
    assert g() == [1, 2, 7, 7]
    # SAME_UPPER crops the odd pixel from the end, SAME_LOWER from the start
    assert O.conv_transpose_geometry((1, 1, 3, 3), (1, 1, 3, 3), [2, 2], auto_pad="SAME_UPPER")[1] == [0, 0, 1, 1]
    assert O.conv_transpose_geometry((1, 1, 3, 3), (1, 1, 3, 3), [2, 2], auto_pad="SAME_LOWER")[1] == [1, 1, 0, 0]


@pytest.mark.parametrize("case", [
    ((1, 4, 5, 6), (4, 3, 3, 3), dict(strides=[2, 2], pads=[1, 0, 0, 1], output_padding=[1, 0])),
    ((2, 6, 4, 4), (6, 2, 4, 4), dict(strides=[2, 2], pads=[1, 1, 1, 1], group=3)),
    ((1, 3, 5, 5), (3, 5, 3, 2), dict(strides=[1, 3], dilations=[2, 1])),
    ((1, 8, 3, 3), (8, 1, 3, 3), dict(strides=[2, 2], group=8, output_padding=[1, 1])),
])
def test_conv_transpose_matches_torch(case):
    """Against torch's float64 conv_transpose2d as an independent library
    routine (pads here are symmetric per axis where torch needs them)."""
    import torch
    xs, ws, attrs = case
    rng = np.random.default_rng(sum(xs) + sum(ws))
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.3, ws).astype(np.float32)
    b = rng.normal(0, 0.1, ws[1] * attrs.get("group", 1)).astype(np.float32)
    got = O.conv_transpose(x, w, b, **attrs)
    s, p, d, shape = O.conv_transpose_geometry(x.shape, w.shape, attrs.get("strides"), attrs.get("pads"),
                                               attrs.get("dilations"), attrs.get("group", 1),
                                               attrs.get("output_padding"))
    # torch crops symmetrically: run it uncropped and without the bias, append
    # the output_padding rows / columns (which no input reaches), add the bias,
    # then crop [begin, end) per axis
    full = torch.nn.functional.conv_transpose2d(
        torch.from_numpy(x).double(), torch.from_numpy(w).double(), None,
        stride=tuple(s), padding=0, output_padding=0, groups=attrs.get("group", 1), dilation=tuple(d)).numpy()
    op = attrs.get("output_padding", [0, 0])
    full = np.pad(full, [(0, 0), (0, 0), (0, op[0]), (0, op[1])]) + b.astype(np.float64).reshape(1, -1, 1, 1)
    want = full[:, :, p[0]:full.shape[2] - p[2], p[1]:full.shape[3] - p[3]]
    assert got.shape == want.shape == tuple(shape)
    np.testing.assert_allclose(got, want, atol=1e-5 * max(1.0, np.abs(want).max()))


def test_conv_transpose_is_the_adjoint_of_conv():
    """<Conv(z, W), x> == <z, ConvTranspose(x, W)>: the scatter is the exact
    adjoint of the gather with the same weights, strides, pads and dilations."""
    rng = np.random.default_rng(5)
    z = rng.normal(size=(1, 3, 9, 8)).astype(np.float32)
    w = rng.normal(size=(4, 3, 3, 3)).astype(np.float32)          # Conv: [Cout, Cin, k, k]
    attrs = dict(strides=[2, 2], pads=[1, 1, 1, 1], dilations=[1, 1])
    y = O.conv(z, w, None, **attrs)                                 # [1, 4, 5, 4]
    x = rng.normal(size=y.shape).astype(np.float32)
    zt = O.conv_transpose(x, w, None, strides=[2, 2], pads=[1, 1, 1, 1],
                          output_shape=list(z.shape[2:]))           # ConvTranspose W: [C_in=4, C_out=3]
    assert zt.shape == z.shape
    lhs = float(np.dot(y.astype(np.float64).ravel(), x.astype(np.float64).ravel()))
    rhs = float(np.dot(z.astype(np.float64).ravel(), zt.astype(np.float64).ravel()))
    assert abs(lhs - rhs) <= 1e-4 * max(1.0, abs(lhs))


def test_batched_matmul_slice_rule():
    """typed_matmul_batch_info + the s % batches slice pairing (math_typed.rs:85-115,
    352-369): where the batch prefixes are whole, it agrees with numpy's
    broadcast matmul; where one prefix is partial it follows the modulo rule."""
    rng = np.random.default_rng(3)
    a = rng.normal(size=(2, 3, 4, 5)).astype(np.float32)
    b = rng.normal(size=(3, 5, 6)).astype(np.float32)
    np.testing.assert_allclose(O.matmul_batched(a, b), np.matmul(a.astype(np.float64), b), atol=1e-12)
    a = rng.normal(size=(4, 1, 2, 3)).astype(np.float32)
    b = rng.normal(size=(3, 3, 2)).astype(np.float32)
    got = O.matmul_batched(a, b)
    assert got.shape == (4, 3, 2, 2)
    a3, b3 = a.reshape(4, 2, 3).astype(np.float64), b.astype(np.float64)
    for s in range(12):
        np.testing.assert_allclose(got.reshape(12, 2, 2)[s], a3[s % 4] @ b3[s % 3], atol=1e-12)
    # the half path: per slice the f16 Gemm loop, rounded once
    ah, bh = O.f32_to_half_bits(a), O.f32_to_half_bits(b)
    hb = O.matmul_batched_half(ah, bh)
    assert hb.shape == (4, 3, 2, 2)
    np.testing.assert_array_equal(hb.reshape(12, 2, 2)[5], O.gemm_half(ah.reshape(4, 2, 3)[1], bh[2], None))
