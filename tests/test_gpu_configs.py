"""Parity at the configured workloads (the benchmark shapes), through the C
ABI, against the CPU oracle:

* config 1: Conv f32 [1,64,128,128] x [64,64,3,3] pad 1 + Relu, whole output;
* config 2: Gemm f32 and f16 at (M,K,N) in {(1,25088,512), (128,768,3072),
  (2048,4096,4096), (4096,4096,11008)}, B as an initializer in both layouts
  (transB=0 and the gemm_nt transB=1), bias [N].  The oracle's f32 sgemm and
  its f16 i-p-j loop run on row bands of the two big shapes (first, middle
  and last rows: the first and last tiles of the grid and an interior one);
  the two small shapes are compared whole;
* config 3: the INT8 FFN pair at M=4096 (u8 A, zero point 128, scale 0.02;
  B1 [768,3072] and B2 [3072,768] int8 with per-output-channel scales
  ~U(0.001,0.01); output u8 scale 0.05 zero point 128), once through the
  QLinearMatMul node as the reference computes it (b_scale[0] only,
  qlinear_matmul.rs:230) and once with the per-column scales, plus
  MatMulInteger with int32 output; all bit-exact against an exact integer
  accumulator (float64 products and sums of 8-bit values are exact below 2^53).

Bars: f32 1e-4 and f16 1e-2 of max |reference|; integer paths bit-exact.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
HALF_TOL = 1e-2


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


@pytest.fixture(scope="module")
def ctx(torch):
    from oxionnx_amd.ep import HipContext
    c = HipContext(0)
    yield c
    c.close()


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bands(m):
    if m <= 128:
        return [(0, m)]
    return [(0, 16), (m // 2 - 8, m // 2 + 8), (m - 16, m)]


# ------------------------------------------------------------------ config 1
def test_config1_conv_f32_relu(torch, ctx):
    from oxionnx_amd import _lib as L
    rng = np.random.default_rng(1)
    x = rng.uniform(-1, 1, (1, 64, 128, 128)).astype(np.float32)
    w = rng.normal(0, 0.05, (64, 64, 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.01, 64).astype(np.float32)
    y = ctx.conv2d(_dev(torch, x), ctx.weight_conv(w), _dev(torch, b), pads=(1, 1, 1, 1),
                   act=L.ACT_RELU).cpu().numpy()
    want = O.conv(x, w, b, activation="relu", pads=[1, 1, 1, 1], nthreads=8)
    assert y.shape == want.shape == (1, 64, 128, 128)
    scale = float(np.abs(O.conv(x, w, b, pads=[1, 1, 1, 1], nthreads=8)).max())
    assert float(np.abs(y.astype(np.float64) - want).max()) <= F32_TOL * scale


# ------------------------------------------------------------------ config 2
CFG2 = [(1, 25088, 512), (128, 768, 3072), (2048, 4096, 4096), (4096, 4096, 11008)]


def _cfg2_operands(mkn):
    m, k, n = mkn
    rng = np.random.default_rng(m + k + n)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1 / np.sqrt(k), (k, n)).astype(np.float32)
    c = rng.normal(0, 0.01, n).astype(np.float32)
    return a, b, c


@pytest.mark.parametrize("trans_b", [0, 1], ids=["gemm", "gemm_nt"])
@pytest.mark.parametrize("mkn", CFG2, ids=str)
def test_config2_gemm_f32(torch, ctx, mkn, trans_b):
    m, k, n = mkn
    a, b, c = _cfg2_operands(mkn)
    bb = np.ascontiguousarray(b.T) if trans_b else b
    y = ctx.gemm(_dev(torch, a), ctx.weight_gemm(bb, trans_b=bool(trans_b)), _dev(torch, c)).cpu().numpy()
    assert y.shape == (m, n)
    for r0, r1 in _bands(m):
        want = O.gemm(a[r0:r1], bb, c, trans_b=trans_b)
        err = float(np.abs(y[r0:r1].astype(np.float64) - want).max())
        assert err <= F32_TOL * float(np.abs(want).max()), (r0, err)


@pytest.mark.parametrize("trans_b", [0, 1], ids=["gemm", "gemm_nt"])
@pytest.mark.parametrize("mkn", CFG2, ids=str)
def test_config2_gemm_f16(torch, ctx, mkn, trans_b):
    from oxionnx_amd import _lib as L
    m, k, n = mkn
    a, b, c = _cfg2_operands(mkn)
    bb = np.ascontiguousarray(b.T) if trans_b else b
    ah, bh, ch = (O.f32_to_half_bits(v) for v in (a, bb, c))
    w = ctx.weight_gemm(O.half_bits_to_f32(bh), trans_b=bool(trans_b), dtype=L.F16)
    at = torch.from_numpy(ah.view(np.int16)).cuda().view(torch.float16)
    ct = torch.from_numpy(ch.view(np.int16)).cuda().view(torch.float16)
    y = ctx.gemm(at, w, ct).view(torch.int16).cpu().numpy().view(np.uint16)
    got = O.half_bits_to_f32(y)
    for r0, r1 in _bands(m):
        want = O.half_bits_to_f32(O.gemm_half(ah, bh, ch, trans_b=trans_b, rows=(r0, r1)))[r0:r1]
        err = float(np.abs(got[r0:r1] - want).max())
        assert err <= HALF_TOL * float(np.abs(want).max()), (r0, err)


# ------------------------------------------------------------------ config 3
M3, D, F = 4096, 768, 3072


def _exact_acc(a, a_zp, b):
    """Σ (a - a_zp) · b, exact (float64 sums of 8-bit products stay below 2^53)."""
    return (a.astype(np.float64) - a_zp) @ b.astype(np.float64)


def _requant(acc, comb, y_zp=128):
    return np.clip(np.rint(acc * np.asarray(comb, np.float32).astype(np.float64) + y_zp), 0, 255)


@pytest.fixture(scope="module")
def ffn():
    rng = np.random.default_rng(3)
    a = rng.integers(0, 256, (M3, D)).astype(np.uint8)
    b1 = rng.integers(-127, 128, (D, F)).astype(np.int8)
    b2 = rng.integers(-127, 128, (F, D)).astype(np.int8)
    s1 = rng.uniform(0.001, 0.01, F).astype(np.float32)
    s2 = rng.uniform(0.001, 0.01, D).astype(np.float32)
    return a, b1, b2, s1, s2


def test_config3_ffn_pair_reference_node(ctx, ffn):
    """Both QLinearMatMul nodes through the drop-in boundary, the first one's
    output lanes feeding the second; each applies b_scale[0] only, as the
    reference does."""
    from oxionnx_amd import ep
    a, b1, b2, s1, s2 = ffn
    f = lambda v: np.array([v], np.float32)
    w = {"as": f(0.02), "azp": f(128), "b1": b1.astype(np.float32), "s1": s1, "bzp": f(0), "ys": f(0.05),
         "yzp": f(128), "b2": b2.astype(np.float32), "s2": s2}
    n1 = ep.Node("QLinearMatMul", ["a", "as", "azp", "b1", "s1", "bzp", "ys", "yzp"], ["h"])
    n2 = ep.Node("QLinearMatMul", ["h", "ys", "yzp", "b2", "s2", "bzp", "ys", "yzp"], ["y"])
    # QLinearMatMul has no resident slot (accepts_resident_slot, lib.rs:419-480):
    # a resident operand is declined, and the session passes host lanes
    assert ep.try_hip_dispatch_resident(n1, w, {"a": ep.DeviceTensor.from_host(ctx, a)}, ctx) is None
    assert "host-read slot 0" in ctx.last_decline()
    h = ep.try_hip_dispatch(n1, w, {"a": a.astype(np.float32)}, ctx)
    assert h is not None, ctx.last_decline()
    h = h[0]
    y = ep.try_hip_dispatch(n2, w, {"h": h}, ctx)
    assert y is not None, ctx.last_decline()
    y = y[0]
    want_h = _requant(_exact_acc(a, 128, b1), (np.float32(0.02) * s1[0]) / np.float32(0.05))
    np.testing.assert_array_equal(np.asarray(h, np.float64), want_h)
    want_y = _requant(_exact_acc(want_h, 128, b2), (np.float32(0.05) * s2[0]) / np.float32(0.05))
    np.testing.assert_array_equal(np.asarray(y, np.float64), want_y)
    # the oracle's restatement agrees on a row band of the second GEMM
    o = O.qlinear_matmul(want_h[:8].astype(np.uint8), 0.05, 128, b2, s2[0], 0, 0.05, 128, sat_range=(0, 255))
    np.testing.assert_array_equal(o, want_y[:8])


def test_config3_ffn_pair_per_column_scales(torch, ctx, ffn):
    from oxionnx_amd import _lib as L
    a, b1, b2, s1, s2 = ffn
    w1 = ctx.weight_qgemm(b1, zp=0, scale=s1)
    w2 = ctx.weight_qgemm(b2, zp=0, scale=s2)
    h = ctx.qgemm(_dev(torch, a), w1, a_zp=128, out_kind=L.QOUT_U8, a_scale=0.02, y_scale=0.05, y_zp=128)
    y = ctx.qgemm(h, w2, a_zp=128, out_kind=L.QOUT_U8, a_scale=0.05, y_scale=0.05, y_zp=128)
    want_h = _requant(_exact_acc(a, 128, b1), (np.float32(0.02) * s1) / np.float32(0.05))
    np.testing.assert_array_equal(h.cpu().numpy().astype(np.float64), want_h)
    want_y = _requant(_exact_acc(want_h, 128, b2), (np.float32(0.05) * s2) / np.float32(0.05))
    np.testing.assert_array_equal(y.cpu().numpy().astype(np.float64), want_y)


def test_config3_matmul_integer_int32(torch, ctx, ffn):
    from oxionnx_amd import _lib as L
    a, b1, _, _, _ = ffn
    y = ctx.qgemm(_dev(torch, a), ctx.weight_qgemm(b1, zp=0), a_zp=128, out_kind=L.QOUT_I32).cpu().numpy()
    np.testing.assert_array_equal(y.astype(np.float64), _exact_acc(a, 128, b1))
    acc, _ = O.integer_matmul(a[:4], b1, 128, 0)
    np.testing.assert_array_equal(y[:4].ravel(), np.asarray(acc).ravel())
