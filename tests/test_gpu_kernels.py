"""Parity of the HIP kernels against the CPU oracle, through the C ABI.

Tolerances follow the north-star contract: integer paths bit-exact; f32 max
|gpu - cpu| <= 1e-4 * max|cpu| (relative to the output's magnitude, the rule
of oxionnx-gpu/tests/c3_conv2d_parity.rs:47-50); f16/bf16 <= 1e-2 of the
magnitude.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import _golden as G

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
    from oxionnx_amd import _lib as L
    from oxionnx_amd.device import HipContext
    c = HipContext(0)
    yield c
    c.close()


def _rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(1e-30, float(np.max(np.abs(want))))
    return float(np.max(np.abs(got - want))) / scale


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# ------------------------------------------------------------------ float GEMM
GEMM_SHAPES = [(1, 64, 32), (3, 100, 17), (8, 256, 64), (2, 5000, 40), (9, 64, 40), (33, 70, 45), (64, 64, 64),
               (128, 256, 384), (200, 136, 72), (256, 512, 520), (300, 1000, 129)]


@pytest.mark.parametrize("mkn", GEMM_SHAPES, ids=str)
@pytest.mark.parametrize("tile", list(range(12)) + [16, 18])
def test_gemm_f32_matches_oracle(torch, ctx, mkn, tile):
    from oxionnx_amd import _lib as L
    m, k, n = mkn
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1 / np.sqrt(k), (k, n)).astype(np.float32)
    c = rng.normal(0, 0.1, n).astype(np.float32)
    ctx.set_tile(tile)
    try:
        w = ctx.weight_gemm(b)
        y = ctx.gemm(_dev(torch, a), w, _dev(torch, c)).cpu().numpy()
    finally:
        ctx.set_tile(0)
    want = O.gemm(a, b, c)
    assert _rel_err(y, want) <= F32_TOL


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_gemm_many_tiles_matches_float64(torch, ctx, dt):
    """A Gemm of 280 tiles of 256x256 (one whole round of the 256 CUs and a
    part-filled one) with a row bias, against torch float64 on the device at
    the dtype's tolerance (the CPU oracle would take minutes at this size)."""
    from oxionnx_amd import _lib as L
    m, k, n = 1024, 1152, 17920
    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.rand((m, k), generator=g, device="cuda", dtype=torch.float32) * 2 - 1
    b = torch.randn((k, n), generator=g, device="cuda", dtype=torch.float32) / np.sqrt(k)
    c = torch.randn((n,), generator=g, device="cuda", dtype=torch.float32) * 0.1
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dt]
    ldt = {"f32": L.F32, "f16": L.F16, "bf16": L.BF16}[dt]
    a, b, c = a.to(tdt), b.to(tdt), c.to(tdt)
    w = ctx.weight_gemm(b.float().cpu().numpy(), dtype=ldt)
    y = ctx.gemm(a, w, c).double()
    want = a.double() @ b.double() + c.double()
    err = float((y - want).abs().max() / want.abs().max())
    assert err <= (F32_TOL if dt == "f32" else HALF_TOL), err


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("ckind", ["none", "scalar", "row", "full"])
def test_gemm_f32_transposes_alpha_beta_bias(torch, ctx, ta, tb, ckind):
    m, k, n = 37, 52, 29
    rng = np.random.default_rng(11)
    a = rng.normal(size=(m, k)).astype(np.float32)
    b = rng.normal(size=(k, n)).astype(np.float32)
    c = {"none": None, "scalar": np.float32([0.5]), "row": rng.normal(size=n).astype(np.float32),
         "full": rng.normal(size=(m, n)).astype(np.float32)}[ckind]
    aa = a.T.copy() if ta else a
    bb = b.T.copy() if tb else b
    w = ctx.weight_gemm(bb, trans_b=bool(tb))
    y = ctx.gemm(_dev(torch, aa), w, None if c is None else _dev(torch, c), alpha=0.75, beta=1.5,
                 trans_a=bool(ta)).cpu().numpy()
    want = O.gemm(aa, bb, None if c is None else (c.reshape(()) if ckind == "scalar" else c), 0.75, 1.5, ta, tb)
    assert _rel_err(y, want) <= F32_TOL


@pytest.mark.parametrize("c", G.cases("Gemm") + G.cases("MatMul"), ids=lambda c: c["name"])
def test_gemm_golden_vectors(torch, ctx, c):
    at = c["attrs"]
    a, b = G.arr(c, "a"), G.arr(c, "b")
    w = ctx.weight_gemm(b, trans_b=bool(at.get("transB", 0)))
    y = ctx.gemm(_dev(torch, a), w, alpha=at.get("alpha", 1.0), beta=at.get("beta", 1.0),
                 trans_a=bool(at.get("transA", 0))).cpu().numpy()
    np.testing.assert_allclose(y.ravel(), c["expected"], atol=c["tol"])


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
# (257, 832, 300): 13 whole K stages (two six-stage trips of tile 16's
# unrolled loop and a one-stage tail) with ragged rows and columns
@pytest.mark.parametrize("mkn", [(1, 128, 64), (5, 96, 40), (64, 64, 64), (130, 264, 200), (512, 768, 384),
                                 (257, 832, 300)], ids=str)
@pytest.mark.parametrize("tile", [0, 6, 16, 18])
def test_gemm_half_matches_oracle(torch, ctx, bf16, mkn, tile):
    from oxionnx_amd import _lib as L
    m, k, n = mkn
    rng = np.random.default_rng(m + k + n)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1 / np.sqrt(k), (k, n)).astype(np.float32)
    c = rng.normal(0, 0.1, n).astype(np.float32)
    ah, bh, ch = (O.f32_to_half_bits(v, bf16) for v in (a, b, c))
    tdt = torch.bfloat16 if bf16 else torch.float16
    dt = L.BF16 if bf16 else L.F16
    w = ctx.weight_gemm(O.half_bits_to_f32(bh, bf16), dtype=dt)
    at = torch.from_numpy(ah.view(np.int16)).cuda().view(tdt)
    ct = torch.from_numpy(ch.view(np.int16)).cuda().view(tdt)
    ctx.set_tile(tile)
    try:
        y = ctx.gemm(at, w, ct, alpha=1.0, beta=1.0)
    finally:
        ctx.set_tile(0)
    got = O.half_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    want = O.half_bits_to_f32(O.gemm_half(ah, bh, ch, 1.0, 1.0, bf16=bf16), bf16)
    assert _rel_err(got, want) <= HALF_TOL


def test_gemm_f16_golden(torch, ctx):
    from oxionnx_amd import _lib as L
    c = G.cases("GemmF16")[0]
    at = c["attrs"]
    a, b, cc = G.arr(c, "a"), G.arr(c, "b"), G.arr(c, "c")
    w = ctx.weight_gemm(b, dtype=L.F16)
    y = ctx.gemm(_dev(torch, a.astype(np.float16)), w, _dev(torch, cc.astype(np.float16)),
                 alpha=at["alpha"], beta=at["beta"])
    np.testing.assert_allclose(y.float().cpu().numpy().ravel(), c["expected"], atol=c["tol"])


# ------------------------------------------------------------------ float Conv
CONV_CASES = [
    # (x shape, w shape, strides, pads [t,l,b,r], dilations)
    ((1, 64, 32, 32), (64, 64, 3, 3), (1, 1), (1, 1, 1, 1), (1, 1)),
    ((1, 3, 40, 40), (32, 3, 7, 7), (1, 1), (3, 3, 3, 3), (1, 1)),
    ((2, 16, 17, 19), (24, 16, 3, 3), (2, 2), (1, 1, 1, 1), (1, 1)),
    ((1, 8, 15, 15), (8, 8, 3, 3), (1, 1), (2, 0, 1, 2), (2, 1)),
    ((1, 32, 12, 12), (16, 32, 1, 1), (1, 1), (0, 0, 0, 0), (1, 1)),
    ((1, 128, 16, 16), (3, 128, 7, 7), (1, 1), (3, 3, 3, 3), (1, 1)),
    ((3, 5, 9, 11), (7, 5, 3, 2), (1, 2), (0, 1, 1, 0), (1, 1)),
    # row-tiled staging: a partial last channel tile, several images
    ((2, 70, 8, 16), (8, 70, 3, 3), (1, 1), (1, 1, 1, 1), (1, 1)),
    # an RGB stem (27 taps x channels: the direct kernel); few output
    # channels over a long reduction (the few-output kernel): an RGB head,
    # stride 2 with uneven pads over two images, dilation 2
    ((1, 3, 64, 64), (16, 3, 3, 3), (2, 2), (1, 1, 1, 1), (1, 1)),
    ((1, 64, 96, 96), (3, 64, 3, 3), (1, 1), (1, 1, 1, 1), (1, 1)),
    ((2, 40, 90, 90), (8, 40, 5, 5), (2, 2), (2, 1, 2, 1), (1, 1)),
    ((1, 32, 80, 80), (5, 32, 3, 3), (1, 1), (2, 2, 2, 2), (2, 2)),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"{c[0]}x{c[1]}s{c[2]}p{c[3]}d{c[4]}")
@pytest.mark.parametrize("act", ["none", "relu", "clip"])
def test_conv_f32_matches_oracle(torch, ctx, case, act):
    from oxionnx_amd import _lib as L
    xs, ws, s, p, d = case
    rng = np.random.default_rng(sum(xs) + sum(ws))
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.05, ws).astype(np.float32)
    b = rng.normal(0, 0.01, ws[0]).astype(np.float32)
    code = {"none": L.ACT_NONE, "relu": L.ACT_RELU, "clip": L.ACT_CLIP}[act]
    wt = ctx.weight_conv(w)
    y = ctx.conv2d(_dev(torch, x), wt, _dev(torch, b), strides=s, pads=p, dilations=d, act=code,
                   act_lo=-0.05, act_hi=0.05).cpu().numpy()
    want = O.conv(x, w, b, activation=None if act == "none" else act, act_min=-0.05, act_max=0.05,
                  strides=s, pads=p, dilations=d)
    assert y.shape == want.shape
    # the tolerance is relative to the conv output's magnitude; a clip caps the
    # activation's magnitude, not the accumulation's, so scale by the unclipped output
    scale = np.max(np.abs(O.conv(x, w, b, strides=s, pads=p, dilations=d)))
    assert np.max(np.abs(y.astype(np.float64) - want)) <= F32_TOL * scale


# Grouped convolutions: (x shape, w shape, group, strides, pads, dilations).
# Depthwise and narrow groups take the direct kernel, wide groups one MFMA
# launch with the group on the grid's z (channel slots per group padded to 16
# bytes); groups whose bias or output starts off 16-byte alignment included.
GROUP_CASES = [
    ((1, 32, 4, 5), (34, 16, 3, 3), 2, (1, 1), (1, 1, 1, 1), (1, 1)),       # 17 outputs a group: odd offsets
    ((1, 60, 7, 9), (60, 20, 3, 3), 3, (1, 1), (1, 1, 1, 1), (1, 1)),       # 20 a group, 63 pixels
    ((2, 48, 6, 6), (48, 16, 1, 1), 3, (1, 1), (0, 0, 0, 0), (1, 1)),       # 1x1, aligned groups
    ((2, 8, 11, 13), (8, 1, 3, 3), 8, (1, 1), (1, 1, 1, 1), (1, 1)),        # depthwise
    ((1, 6, 9, 9), (12, 1, 5, 5), 6, (2, 2), (2, 1, 2, 1), (1, 1)),         # depthwise, multiplier 2
    # depthwise 3x3 on the band kernel (from 2^18 outputs): bands of 56x56
    # planes, stride 2 with odd extents, uneven pads, a valid conv, 2000-wide
    # rows (four-row windows); the same geometries below 2^18 outputs take
    # the one-thread-per-output kernel; rows of whole 16-byte chunks are
    # staged by chunk loads
    ((2, 96, 56, 56), (96, 1, 3, 3), 96, (1, 1), (1, 1, 1, 1), (1, 1)),
    ((1, 288, 115, 63), (288, 1, 3, 3), 288, (2, 2), (1, 1, 1, 1), (1, 1)),
    ((1, 256, 66, 129), (256, 1, 3, 3), 256, (2, 2), (0, 1, 1, 0), (1, 1)),
    ((1, 96, 76, 76), (96, 1, 3, 3), 96, (1, 1), (0, 0, 0, 0), (1, 1)),
    ((1, 16, 17, 2000), (16, 1, 3, 3), 16, (1, 1), (1, 1, 1, 1), (1, 1)),
    ((1, 16, 57, 31), (16, 1, 3, 3), 16, (2, 2), (1, 1, 1, 1), (1, 1)),
    ((1, 128, 56, 56), (128, 1, 3, 3), 128, (1, 1), (1, 1, 1, 1), (1, 1)),     # just above the gate
    ((1, 256, 96, 112), (256, 1, 3, 3), 256, (2, 2), (1, 1, 1, 1), (1, 1)),   # 16-byte row chunks, stride 2
    ((1, 416, 64, 80), (416, 1, 3, 3), 416, (2, 2), (0, 2, 1, 0), (1, 1)),    # chunks, window narrower than the row
    ((1, 6, 10, 10), (4, 3, 3, 3), 2, (1, 1), (1, 1, 1, 1), (2, 2)),        # narrow groups, dilated
    ((2, 64, 12, 12), (64, 16, 3, 3), 4, (1, 1), (1, 1, 1, 1), (1, 1)),     # MFMA per group, aligned
    ((1, 40, 9, 9), (48, 20, 3, 3), 2, (2, 2), (0, 1, 1, 0), (1, 1)),       # MFMA per group, padded slots
]


@pytest.mark.parametrize("case", GROUP_CASES, ids=lambda c: f"{c[0]}x{c[1]}g{c[2]}")
@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_grouped_conv_matches_oracle(torch, ctx, case, dt):
    from oxionnx_amd import _lib as L
    xs, ws, grp, s, p, d = case
    rng = np.random.default_rng(sum(xs) + sum(ws) + grp)
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.2, ws).astype(np.float32)
    b = rng.normal(0, 0.1, ws[0]).astype(np.float32)
    if dt == "f32":
        wt = ctx.weight_conv(w)
        y = ctx.conv2d(_dev(torch, x), wt, _dev(torch, b), strides=s, pads=p, dilations=d, group=grp,
                       act=L.ACT_RELU).cpu().numpy()
        want = O.conv(x, w, b, activation="relu", strides=s, pads=p, dilations=d, group=grp)
        scale = max(1.0, float(np.max(np.abs(want))))
        assert y.shape == want.shape
        assert np.max(np.abs(y.astype(np.float64) - want)) <= F32_TOL * scale
    else:
        xh, wh, bh = (O.f32_to_half_bits(v) for v in (x, w, b))
        wt = ctx.weight_conv(O.half_bits_to_f32(wh), dtype=L.F16)
        xt = torch.from_numpy(xh.view(np.int16)).cuda().view(torch.float16)
        bt = torch.from_numpy(bh.view(np.int16)).cuda().view(torch.float16)
        y = ctx.conv2d(xt, wt, bt, strides=s, pads=p, dilations=d, group=grp)
        got = O.half_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16))
        want = O.half_bits_to_f32(O.conv_half(xh, wh, bh, strides=s, pads=p, dilations=d, group=grp))
        assert _rel_err(got, want) <= HALF_TOL


# bf16 depthwise 3x3 on both sides of the band kernel's 2^18-output gate,
# against torch's f32 conv of the same bf16-rounded operands (the oracle has
# no bf16 conv): (x shape, stride, pads [t, l, b, r]).
DW_BF16_CASES = [((1, 96, 76, 76), 1, (1, 1, 1, 1)), ((1, 288, 115, 63), 2, (1, 1, 1, 1)),
                 ((2, 8, 12, 10), 1, (0, 1, 1, 0))]


@pytest.mark.parametrize("case", DW_BF16_CASES, ids=lambda c: f"{c[0]}s{c[1]}")
def test_depthwise_bf16_matches_torch_f32(torch, ctx, case):
    from oxionnx_amd import _lib as L
    xs, s, p = case
    c = xs[1]
    g = torch.Generator(device="cuda").manual_seed(c + xs[2])
    x = (torch.rand(xs, generator=g, device="cuda") * 2 - 1).to(torch.bfloat16)
    w = (torch.randn((c, 1, 3, 3), generator=g, device="cuda") * 0.3).to(torch.bfloat16)
    b = (torch.randn((c,), generator=g, device="cuda") * 0.1).to(torch.bfloat16)
    wt = ctx.weight_conv(w.float().cpu().numpy(), dtype=L.BF16)
    y = ctx.conv2d(x, wt, b, strides=(s, s), pads=p, group=c, act=L.ACT_RELU).float()
    xp = torch.nn.functional.pad(x.float(), (p[1], p[3], p[0], p[2]))
    want = torch.relu(torch.nn.functional.conv2d(xp, w.float(), b.float(), stride=s, groups=c))
    assert y.shape == want.shape
    err = float((y - want).abs().max() / want.abs().max())
    assert err <= HALF_TOL, err


# Batched MatMul with both operands on the device: (A shape, B shape).  The
# slice rule is the reference's (s % a_batches, s % b_batches), which is not
# numpy's broadcast for every shape (the [4,1,..] x [3,..] case below).
BMM_CASES = [
    ((3, 37, 52), (3, 52, 29)),
    ((2, 3, 64, 64), (3, 64, 48)),
    ((4, 1, 5, 7), (3, 7, 4)),
    ((8, 128, 96), (96, 160)),
    ((1, 33, 21), (6, 21, 70)),
    ((4, 5, 64), (64, 36)),      # 2-byte slices start 8 bytes off a 16-byte boundary
    ((2, 37, 96), (96, 12)),
]


@pytest.mark.parametrize("case", BMM_CASES, ids=lambda c: f"{c[0]}x{c[1]}")
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_batched_matmul_matches_oracle(torch, ctx, case, dt):
    ash, bsh = case
    rng = np.random.default_rng(sum(ash) + sum(bsh))
    a = rng.uniform(-1, 1, ash).astype(np.float32)
    b = rng.normal(0, 1 / np.sqrt(bsh[-2]), bsh).astype(np.float32)
    if dt == "f32":
        y = ctx.matmul(_dev(torch, a), _dev(torch, b)).cpu().numpy()
        want = O.matmul_batched(a, b)
        assert y.shape == want.shape
        assert _rel_err(y, want) <= F32_TOL
    else:
        bf = dt == "bf16"
        tdt = torch.bfloat16 if bf else torch.float16
        ah, bh = O.f32_to_half_bits(a, bf), O.f32_to_half_bits(b, bf)
        at = torch.from_numpy(ah.view(np.int16)).cuda().view(tdt)
        bt = torch.from_numpy(bh.view(np.int16)).cuda().view(tdt)
        got = O.half_bits_to_f32(ctx.matmul(at, bt).view(torch.int16).cpu().numpy().view(np.uint16), bf)
        want = O.half_bits_to_f32(O.matmul_batched_half(ah, bh, bf), bf)
        assert got.shape == want.shape
        assert _rel_err(got, want) <= HALF_TOL


# ConvTranspose: (x shape, w shape [Cin, Cout/g, kh, kw], attrs with resolved pads).
# Group 1 / dilation 1 / kernel >= stride runs the sub-pixel phases on the
# MFMA engine (within the tolerances); the rest runs the gather kernel, which
# adds every output's contributions in the reference's order (bit-exact).
CONVT_CASES = [
    ((1, 8, 7, 9), (8, 6, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1], output_padding=[1, 1])),
    ((2, 6, 5, 5), (6, 4, 4, 4), dict(strides=[2, 2], pads=[1, 1, 1, 1], group=2)),
    ((1, 4, 6, 5), (4, 3, 3, 2), dict(strides=[1, 3], pads=[0, 1, 2, 0], dilations=[2, 1])),
    ((1, 16, 4, 4), (16, 1, 3, 3), dict(strides=[2, 2], group=16)),
    ((1, 64, 8, 8), (64, 32, 4, 4), dict(strides=[2, 2], pads=[1, 1, 1, 1])),
    ((2, 32, 5, 6), (32, 24, 2, 2), dict(strides=[2, 2], pads=[0, 0, 0, 0])),          # phases in one launch
    ((1, 128, 16, 16), (128, 64, 4, 4), dict(strides=[2, 2], pads=[1, 2, 1, 2])),      # one launch, uneven pads
    ((2, 24, 5, 7), (24, 40, 3, 3), dict(strides=[1, 1], pads=[1, 0, 0, 2])),
    ((1, 32, 6, 5), (32, 16, 5, 3), dict(strides=[3, 2], pads=[2, 1, 1, 0], output_padding=[2, 1])),
    # two phases in one launch: (2, 1) and (1, 2) strides (the z / zsw output offsets)
    ((1, 32, 8, 8), (32, 16, 4, 3), dict(strides=[2, 1], pads=[1, 1, 1, 1])),
    ((2, 16, 6, 8), (16, 24, 3, 4), dict(strides=[1, 2], pads=[1, 1, 1, 1])),
]

# (case, contraction launches one forward must take): one launch per image
# when every phase fits one grid, a launch per phase and image otherwise
# (an odd output extent: the phases' grids differ).
CONVT_LAUNCHES = [
    (((1, 32, 8, 8), (32, 16, 4, 3), dict(strides=[2, 1], pads=[1, 1, 1, 1])), 1),
    (((2, 16, 6, 8), (16, 24, 3, 4), dict(strides=[1, 2], pads=[1, 1, 1, 1])), 2),
    (((2, 32, 5, 6), (32, 24, 2, 2), dict(strides=[2, 2], pads=[0, 0, 0, 0])), 2),
    (((1, 8, 7, 9), (8, 6, 3, 3), dict(strides=[2, 2], pads=[1, 1, 1, 1])), 4),
]


def _convt_uses_gather(ws, attrs):
    s = attrs.get("strides", [1, 1])
    return (attrs.get("group", 1) != 1 or attrs.get("dilations", [1, 1]) != [1, 1]
            or ws[2] < s[0] or ws[3] < s[1])


@pytest.mark.parametrize("case", CONVT_CASES, ids=lambda c: f"{c[0]}x{c[1]}")
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_conv_transpose_matches_oracle(torch, ctx, case, dt):
    from oxionnx_amd import _lib as L
    xs, ws, attrs = case
    rng = np.random.default_rng(sum(xs) + sum(ws))
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.3, ws).astype(np.float32)
    b = rng.normal(0, 0.1, ws[1] * attrs.get("group", 1)).astype(np.float32)
    geo = dict(strides=attrs.get("strides", [1, 1]), pads=attrs.get("pads", [0, 0, 0, 0]),
               dilations=attrs.get("dilations", [1, 1]), group=attrs.get("group", 1))
    exact = _convt_uses_gather(ws, attrs)
    if dt == "f32":
        wt = ctx.weight_conv_transpose(w, **geo)
        y = ctx.conv_transpose2d(_dev(torch, x), wt, _dev(torch, b),
                                 output_padding=attrs.get("output_padding", [0, 0]), **geo).cpu().numpy()
        want = O.conv_transpose(x, w, b, **attrs)
        assert y.shape == want.shape
        if exact:
            np.testing.assert_array_equal(y.view(np.uint32), want.view(np.uint32))
        else:
            assert np.max(np.abs(y.astype(np.float64) - want)) <= F32_TOL * max(1.0, float(np.abs(want).max()))
    else:
        bf = dt == "bf16"
        tdt = torch.bfloat16 if bf else torch.float16
        xh, wh, bh = (O.f32_to_half_bits(v, bf) for v in (x, w, b))
        wt = ctx.weight_conv_transpose(O.half_bits_to_f32(wh, bf), dtype=L.BF16 if bf else L.F16, **geo)
        xt = torch.from_numpy(xh.view(np.int16)).cuda().view(tdt)
        bt = torch.from_numpy(bh.view(np.int16)).cuda().view(tdt)
        y = ctx.conv_transpose2d(xt, wt, bt, output_padding=attrs.get("output_padding", [0, 0]), **geo)
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        want = O.conv_transpose_half(xh, wh, bh, bf16=bf, **attrs)
        if exact:
            np.testing.assert_array_equal(got, want)
        else:
            assert _rel_err(O.half_bits_to_f32(got, bf), O.half_bits_to_f32(want, bf)) <= HALF_TOL


@pytest.mark.parametrize("case,launches", CONVT_LAUNCHES, ids=lambda c: str(c))
def test_conv_transpose_launch_count(torch, ctx, case, launches):
    xs, ws, attrs = case
    rng = np.random.default_rng(7 + sum(xs))
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.3, ws).astype(np.float32)
    geo = dict(strides=attrs["strides"], pads=attrs["pads"], dilations=[1, 1], group=1)
    wt = ctx.weight_conv_transpose(w, **geo)
    xd = _dev(torch, x)
    ctx.conv_transpose2d(xd, wt, None, **geo)
    ctx.sync()
    ctx.reset_counters()
    y = ctx.conv_transpose2d(xd, wt, None, **geo).cpu().numpy()
    assert ctx.counters()["contraction_launches"] == launches
    want = O.conv_transpose(x, w, None, **attrs)
    assert np.max(np.abs(y.astype(np.float64) - want)) <= F32_TOL * max(1.0, float(np.abs(want).max()))


@pytest.mark.parametrize("c", G.cases("Conv") + G.cases("Conv1D"), ids=lambda c: c["name"])
def test_conv_golden_vectors(torch, ctx, c):
    x, w, b = G.conv_inputs(c)
    attrs = G.conv_attrs(c)
    grp = c["attrs"].get("group", 1)
    s, p, d, out_shape = O.conv_geometry(x.shape, w.shape, attrs.get("strides"), attrs.get("pads"),
                                         attrs.get("dilations"), grp, attrs.get("auto_pad", "NOTSET"))
    wt = ctx.weight_conv(w)
    y = ctx.conv2d(_dev(torch, x), wt, None if b is None else _dev(torch, b), strides=s, pads=p,
                   dilations=d, group=grp).cpu().numpy()
    np.testing.assert_allclose(y.ravel(), np.asarray(c["expected"], np.float32), atol=c["tol"])


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", CONV_CASES[:4], ids=lambda c: f"{c[0]}x{c[1]}")
def test_conv_half_matches_oracle(torch, ctx, bf16, case):
    from oxionnx_amd import _lib as L
    xs, ws, s, p, d = case
    rng = np.random.default_rng(3 + sum(xs))
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.05, ws).astype(np.float32)
    b = rng.normal(0, 0.01, ws[0]).astype(np.float32)
    xh, wh, bh = (O.f32_to_half_bits(v, bf16) for v in (x, w, b))
    tdt = torch.bfloat16 if bf16 else torch.float16
    wt = ctx.weight_conv(O.half_bits_to_f32(wh, bf16), dtype=L.BF16 if bf16 else L.F16)
    xt = torch.from_numpy(xh.view(np.int16)).cuda().view(tdt)
    bt = torch.from_numpy(bh.view(np.int16)).cuda().view(tdt)
    y = ctx.conv2d(xt, wt, bt, strides=s, pads=p, dilations=d, act=L.ACT_RELU)
    got = O.half_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    want = O.half_bits_to_f32(O.conv_half(xh, wh, bh, bf16=bf16, activation="relu", strides=s, pads=p,
                                          dilations=d), bf16)
    assert _rel_err(got, want) <= HALF_TOL


def test_conv_nhwc_output_matches_nchw(torch, ctx):
    from oxionnx_amd import _lib as L
    rng = np.random.default_rng(5)
    x = rng.uniform(-1, 1, (2, 24, 13, 13)).astype(np.float32)
    w = rng.normal(0, 0.05, (20, 24, 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.01, 20).astype(np.float32)
    wt = ctx.weight_conv(w)
    y1 = ctx.conv2d(_dev(torch, x), wt, _dev(torch, b), pads=(1, 1, 1, 1))
    y2 = ctx.conv2d(_dev(torch, x), wt, _dev(torch, b), pads=(1, 1, 1, 1), out_layout=L.NHWC)
    # NCHW out runs the patch-staged f32 kernel, NHWC out the engine: equal to
    # f32 rounding, not bit for bit
    got = y2[..., :20].permute(0, 3, 1, 2).cpu().numpy()
    assert _rel_err(got, y1.cpu().numpy()) <= 1e-5
    assert _rel_err(got, O.conv(x, w, b, pads=(1, 1, 1, 1))) <= F32_TOL


# Halo-patch path (3x3, stride 1, 256-pixel tiles of whole output rows):
# (x shape, cout, pads).  A channel tail inside the last slab, partial
# output-channel tiles, two images, an uneven top pad, a valid (unpadded)
# conv, 64-wide rows, 128-wide rows (two rows a tile, the larger patch), and
# the 512-channel residual conv (split-K).
HALO_CASES = [
    ((2, 24, 16, 16), 40, (1, 1, 1, 1)),
    ((1, 8, 15, 16), 24, (2, 1, 1, 1)),
    ((1, 16, 34, 34), 64, (0, 0, 0, 0)),
    ((1, 128, 16, 64), 96, (1, 1, 1, 1)),
    ((2, 40, 6, 128), 72, (1, 1, 1, 1)),
    ((1, 512, 32, 32), 512, (1, 1, 1, 1)),
]


@pytest.mark.parametrize("case", HALO_CASES, ids=lambda c: f"{c[0]}x{c[1]}p{c[2]}")
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("nhwc_out", [False, True], ids=["nchw", "nhwc"])
def test_halo_conv_matches_oracle(torch, ctx, case, dt, nhwc_out):
    from oxionnx_amd import _lib as L
    xs, cout, p = case
    rng = np.random.default_rng(11 + sum(xs) + cout)
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.05, (cout, xs[1], 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.01, cout).astype(np.float32)
    lay = L.NHWC if nhwc_out else L.NCHW

    def run(xd, wt, bd):
        ctx.set_tile(15)   # the halo-patch kernel wherever the geometry allows
        try:
            y = ctx.conv2d(xd, wt, bd, pads=p, act=L.ACT_RELU, out_layout=lay)
        finally:
            ctx.set_tile(0)
        if nhwc_out:
            y = y[..., :cout].permute(0, 3, 1, 2)
        return y

    if dt == "f32":
        y = run(_dev(torch, x), ctx.weight_conv(w), _dev(torch, b)).cpu().numpy()
        want = O.conv(x, w, b, activation="relu", pads=p)
        scale = np.max(np.abs(O.conv(x, w, b, pads=p)))
        assert np.max(np.abs(y.astype(np.float64) - want)) <= F32_TOL * scale
        return
    bf16 = dt == "bf16"
    xh, wh, bh = (O.f32_to_half_bits(v, bf16) for v in (x, w, b))
    tdt = torch.bfloat16 if bf16 else torch.float16
    wt = ctx.weight_conv(O.half_bits_to_f32(wh, bf16), dtype=L.BF16 if bf16 else L.F16)
    xt = torch.from_numpy(xh.view(np.int16)).cuda().view(tdt)
    bt = torch.from_numpy(bh.view(np.int16)).cuda().view(tdt)
    y = run(xt, wt, bt).contiguous()
    got = O.half_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    want = O.half_bits_to_f32(O.conv_half(xh, wh, bh, bf16=bf16, activation="relu", pads=p), bf16)
    assert _rel_err(got, want) <= HALF_TOL


# Whole-K halo path (3x3, stride 1, 64- or 128-pixel tiles of whole output
# rows x 32 channels, every block over the whole reduction): (x shape, cout,
# pads).  The 512-channel residual conv of config 4, channel tails inside the
# eight-chunk slab (24, 72 and 40 channels), partial 32-channel tiles, two
# images, 16- and 64-wide rows, a valid (unpadded) conv and uneven pads.
WK_CASES = [
    ((1, 512, 32, 32), 512, (1, 1, 1, 1)),
    ((2, 24, 32, 32), 40, (1, 1, 1, 1)),
    ((1, 72, 16, 64), 96, (1, 1, 1, 1)),
    ((1, 40, 16, 16), 33, (1, 1, 1, 1)),
    ((1, 16, 34, 34), 64, (0, 0, 0, 0)),
    ((1, 8, 33, 32), 24, (2, 1, 1, 1)),
]


@pytest.mark.parametrize("case", WK_CASES, ids=lambda c: f"{c[0]}x{c[1]}p{c[2]}")
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("nhwc_out", [False, True], ids=["nchw", "nhwc"])
def test_wk_conv_matches_oracle(torch, ctx, case, dt, nhwc_out):
    from oxionnx_amd import _lib as L
    xs, cout, p = case
    rng = np.random.default_rng(17 + sum(xs) + cout)
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.05, (cout, xs[1], 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.01, cout).astype(np.float32)
    lay = L.NHWC if nhwc_out else L.NCHW
    bf16 = dt == "bf16"
    xh, wh, bh = (O.f32_to_half_bits(v, bf16) for v in (x, w, b))
    tdt = torch.bfloat16 if bf16 else torch.float16
    wt = ctx.weight_conv(O.half_bits_to_f32(wh, bf16), dtype=L.BF16 if bf16 else L.F16)
    xt = torch.from_numpy(xh.view(np.int16)).cuda().view(tdt)
    bt = torch.from_numpy(bh.view(np.int16)).cuda().view(tdt)
    ctx.set_tile(17)   # the whole-K halo kernel wherever the geometry allows
    try:
        y = ctx.conv2d(xt, wt, bt, pads=p, act=L.ACT_RELU, out_layout=lay)
    finally:
        ctx.set_tile(0)
    if nhwc_out:
        y = y[..., :cout].permute(0, 3, 1, 2)
    y = y.contiguous()
    got = O.half_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    want = O.half_bits_to_f32(O.conv_half(xh, wh, bh, bf16=bf16, activation="relu", pads=p), bf16)
    assert _rel_err(got, want) <= HALF_TOL
    # the automatic plan takes it for the 512-channel conv (256 blocks)
    if xs[1] == 512:
        y2 = ctx.conv2d(xt, wt, bt, pads=p, act=L.ACT_RELU, out_layout=lay)
        if nhwc_out:
            y2 = y2[..., :cout].permute(0, 3, 1, 2)
        assert torch.equal(y2.contiguous(), y)


# ------------------------------------------------------------------ few output channels on the MFMA
FEWCO_CASES = [
    # (N, C, H, W, cout, k, pad mode)
    (1, 128, 20, 24, 3, 7, "reflect"),
    (2, 32, 9, 16, 4, 5, "edge"),
    (1, 16, 7, 128, 1, 3, "zeros"),
    (1, 64, 12, 100, 3, 7, "zeros"),
]


@pytest.mark.parametrize("case", FEWCO_CASES, ids=str)
@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_fewout_mfma_conv_matches_oracle(torch, ctx, case, bf16):
    """An NHWC f16 / bf16 conv with at most 4 output channels (the few-output
    MFMA kernel: a row's input patch staged per 16-channel slab, the border
    applied by its loader) against the oracle conv of the padded image."""
    import ctypes

    from oxionnx_amd import _lib as L
    n, c, h, wd, cout, k, mode = case
    p = k // 2
    rng = np.random.default_rng(c + cout + k + h)
    x = rng.uniform(-1, 1, (n, c, h, wd)).astype(np.float32)
    w = rng.normal(0, 0.05, (cout, c, k, k)).astype(np.float32)
    b = rng.normal(0, 0.01, cout).astype(np.float32)
    xh, wh, bh = (O.f32_to_half_bits(v, bf16) for v in (x, w, b))
    tdt = torch.bfloat16 if bf16 else torch.float16
    ldt = L.BF16 if bf16 else L.F16
    wt = ctx.weight_conv(O.half_bits_to_f32(wh, bf16), dtype=ldt)
    xn = torch.from_numpy(xh.view(np.int16)).cuda().view(tdt).permute(0, 2, 3, 1).contiguous()
    bt = torch.from_numpy(bh.view(np.int16)).cuda().view(tdt)
    y = torch.empty((n, cout, h, wd), dtype=tdt, device="cuda")
    pm = {"zeros": L.PAD_ZEROS, "reflect": L.PAD_REFLECT, "edge": L.PAD_EDGE}[mode]
    d = L.ConvDesc(n, c, h, wd, cout, k, k, 1, 1, 1, 1, 1, p, p, p, p, ldt, L.NHWC, L.NCHW, L.ACT_NONE, 0.0, 0.0, pm)
    L.check(L.lib().ohip_conv2d(ctx.h, ctypes.byref(d), ctypes.c_void_p(xn.data_ptr()), wt.handle,
                                ctypes.c_void_p(bt.data_ptr()), ctypes.c_void_p(y.data_ptr())))
    got = O.half_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16), bf16)
    if mode == "zeros":
        want = O.conv_half(xh, wh, bh, bf16=bf16, pads=(p, p, p, p))
    else:
        xp = np.pad(xh, ((0, 0), (0, 0), (p, p), (p, p)), mode="reflect" if mode == "reflect" else "edge")
        want = O.conv_half(xp, wh, bh, bf16=bf16, pads=(0, 0, 0, 0))
    assert _rel_err(got, O.half_bits_to_f32(want, bf16)) <= HALF_TOL


# ------------------------------------------------------------------ fused conv + instance norm
CONV_NORM_KERNEL_CASES = [
    ((1, 64, 32, 32), 128, "f32", True, True),
    ((1, 16, 20, 20), 16, "f32", False, False),
    ((2, 32, 16, 16), 64, "f16", False, True),
    ((1, 512, 32, 32), 512, "f16", True, True),     # split K: the norm reads the partial sums
    ((1, 32, 24, 24), 48, "bf16", True, True),      # declined: the norm kernels are f32 / f16
]


@pytest.mark.parametrize("case", CONV_NORM_KERNEL_CASES, ids=str)
def test_conv2d_instnorm_entry_point(torch, ctx, case):
    """ohip_conv2d_instnorm against the oracle's conv (rounded to the dtype,
    as the node chain stores it) followed by a float64 instance norm with
    the chain's roundings: normalised value, gamma product, beta sum."""
    from oxionnx_amd import _lib as L
    xs, cout, dt, adain, relu = case
    n = xs[0]
    rng = np.random.default_rng(xs[1] + cout + n)
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.05, (cout, xs[1], 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.01, cout).astype(np.float32)
    ab = rng.normal(1, 0.3, (n, 2 * cout)).astype(np.float32)   # AdaIN rows: gamma then beta
    half = dt != "f32"
    bf16 = dt == "bf16"
    if half:
        xh, wh, bh, abh = (O.f32_to_half_bits(v, bf16) for v in (x, w, b, ab))
        tdt = torch.bfloat16 if bf16 else torch.float16
        dev = lambda v: torch.from_numpy(v.view(np.int16)).cuda().view(tdt)   # noqa: E731
        wt = ctx.weight_conv(O.half_bits_to_f32(wh, bf16), dtype=L.BF16 if bf16 else L.F16)
        xt, bt, abt = dev(xh), dev(bh), dev(abh)
        conv = O.half_bits_to_f32(O.conv_half(xh, wh, bh, bf16=bf16, pads=(1, 1, 1, 1)), bf16).astype(np.float64)
        g64 = O.half_bits_to_f32(abh, bf16).astype(np.float64)
        rnd = lambda v: O.half_bits_to_f32(O.f32_to_half_bits(v.astype(np.float32), bf16), bf16).astype(np.float64)  # noqa: E731
    else:
        wt = ctx.weight_conv(w)
        xt, bt, abt = _dev(torch, x), _dev(torch, b), _dev(torch, ab)
        conv = O.conv(x, w, b, pads=(1, 1, 1, 1)).astype(np.float32).astype(np.float64)
        g64 = ab.astype(np.float64)
        rnd = lambda v: v.astype(np.float32).astype(np.float64)  # noqa: E731
    call = lambda: ctx.conv2d_instnorm(xt, wt, bt, pads=(1, 1, 1, 1), eps=1e-5,  # noqa: E731
                                       gamma=abt if adain else None, beta=abt if adain else None,
                                       scale_offset=0, bias_offset=cout, relu=relu)
    if bf16:
        with pytest.raises(L.OhipDeclined):
            call()
        return
    y = call()
    got = (O.half_bits_to_f32(y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16), bf16)
           if half else y.cpu().numpy()).astype(np.float64)
    mean = conv.mean(axis=(2, 3), keepdims=True)
    var = ((conv - mean) ** 2).mean(axis=(2, 3), keepdims=True)
    want = (conv - mean) / np.sqrt(var + 1e-5)
    if adain:
        want = rnd(rnd(rnd(want) * g64[:, :cout, None, None]) + g64[:, cout:, None, None])
    if relu:
        want = np.maximum(want, 0.0)
    assert got.shape == want.shape
    assert _rel_err(got, want) <= (HALF_TOL if half else F32_TOL)


# (x shape, cout, tile): config 4's residual conv (the automatic plan), a
# 16-wide image pair with a partial 32-channel tile, a channel tail inside
# the eight-chunk slab (tile 17 forces the whole-K kernel; these planes take
# the segment-moments norm), and a 128 x 64 plane (8192 values, past the
# moments norm's 4096: the whole-K sums go to the norm as one slice)
WK_NORM_CASES = [
    ((1, 512, 32, 32), 512, 0),
    ((2, 64, 16, 16), 96, 17),
    ((1, 40, 32, 32), 72, 17),
    ((1, 32, 128, 64), 64, 17),
]


@pytest.mark.parametrize("case", WK_NORM_CASES, ids=str)
@pytest.mark.parametrize("residual", [False, True], ids=["plain", "residual"])
def test_conv_instnorm_nhwc_matches_nchw(torch, ctx, case, residual):
    """f16 conv -> AdaIN norm -> Relu [-> residual] on the whole-K kernel with
    NHWC input, output and residual (the norm reader writes four channels of
    each pixel as one run) equals the NCHW call bit for bit, twice in a row,
    and both are within the f16 bar of the oracle."""
    from oxionnx_amd import _lib as L
    xs, cout, tile = case
    n, c, h, w_ = xs
    rng = np.random.default_rng(c + cout + n)
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = rng.normal(0, 0.05, (cout, c, 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.01, cout).astype(np.float32)
    ab = rng.normal(1, 0.3, (n, 2 * cout)).astype(np.float32)
    res = rng.uniform(-1, 1, (n, cout, h, w_)).astype(np.float32)
    xh, wh, bh, abh, rh = (O.f32_to_half_bits(v) for v in (x, w, b, ab, res))
    dev = lambda v: torch.from_numpy(v.view(np.int16)).cuda().view(torch.float16)   # noqa: E731
    wt = ctx.weight_conv(O.half_bits_to_f32(wh), dtype=L.F16)
    xt, bt, abt, rt = dev(xh), dev(bh), dev(abh), dev(rh)
    kw = dict(pads=(1, 1, 1, 1), eps=1e-5, gamma=abt, beta=abt, scale_offset=0, bias_offset=cout, relu=True)
    ctx.set_tile(tile)
    try:
        nchw = ctx.conv2d_instnorm(xt, wt, bt, residual=rt if residual else None, **kw)
        xn = xt.permute(0, 2, 3, 1).contiguous()
        rn = rt.permute(0, 2, 3, 1).contiguous()
        for _ in range(2):
            got = ctx.conv2d_instnorm(xn, wt, bt, residual=rn if residual else None, nhwc=True, **kw)
            assert torch.equal(got.permute(0, 3, 1, 2), nchw)
    finally:
        ctx.set_tile(0)
    conv = O.half_bits_to_f32(O.conv_half(xh, wh, bh, pads=(1, 1, 1, 1))).astype(np.float64)
    g64 = O.half_bits_to_f32(abh).astype(np.float64)
    rnd = lambda v: O.half_bits_to_f32(O.f32_to_half_bits(v.astype(np.float32))).astype(np.float64)  # noqa: E731
    mean = conv.mean(axis=(2, 3), keepdims=True)
    var = ((conv - mean) ** 2).mean(axis=(2, 3), keepdims=True)
    want = rnd(rnd(rnd((conv - mean) / np.sqrt(var + 1e-5)) * g64[:, :cout, None, None]) + g64[:, cout:, None, None])
    want = np.maximum(want, 0.0)
    if residual:
        want = want + O.half_bits_to_f32(rh).astype(np.float64)
    got = O.half_bits_to_f32(nchw.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
    assert _rel_err(got, want) <= HALF_TOL


# ------------------------------------------------------------------ integer GEMM
@pytest.mark.parametrize("mkn", [(1, 16, 16), (4, 768, 96), (37, 100, 53), (128, 768, 3072), (300, 256, 200)],
                         ids=str)
@pytest.mark.parametrize("a_u8", [True, False], ids=["u8", "i8"])
def test_qlinear_matmul_bit_exact(torch, ctx, mkn, a_u8):
    from oxionnx_amd import _lib as L
    m, k, n = mkn
    rng = np.random.default_rng(m * 3 + n)
    if a_u8:
        a = rng.integers(0, 256, (m, k)).astype(np.uint8)
        azp = 128
    else:
        a = rng.integers(-128, 128, (m, k)).astype(np.int8)
        azp = -3
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    a_s, b_s, y_s = np.float32(0.02), np.float32(0.0041), np.float32(0.05)
    y_zp = 128 if a_u8 else 0
    lo, hi = (0, 255) if a_u8 else (-128, 127)
    w = ctx.weight_qgemm(b, zp=0, scale=b_s)
    y = ctx.qgemm(_dev(torch, a), w, a_zp=azp, out_kind=L.QOUT_U8 if a_u8 else L.QOUT_I8, a_scale=float(a_s),
                  y_scale=float(y_s), y_zp=y_zp, lo=lo, hi=hi).cpu().numpy()
    want = O.qlinear_matmul(a, a_s, azp, b, b_s, 0, y_s, y_zp, sat_range=(lo, hi))
    np.testing.assert_array_equal(y.astype(np.float32), want)


@pytest.mark.parametrize("mkn", [(37, 100, 53), (300, 768, 600), (513, 1024, 200)], ids=str)
@pytest.mark.parametrize("out", ["u8", "i32"])
def test_qgemm_192x256_tile_bit_exact(torch, ctx, mkn, out):
    """The 192x256 tile (18; one block per CU for short-K grids of more
    than two rounds of 128x128 tiles), u8 outputs staged through LDS (12
    16-byte chunks a staged row) and raw int32, ragged edges on both axes."""
    from oxionnx_amd import _lib as L
    m, k, n = mkn
    rng = np.random.default_rng(m + 2 * n)
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    bs = rng.uniform(0.001, 0.01, n).astype(np.float32)
    ctx.set_tile(18)
    try:
        if out == "u8":
            w = ctx.weight_qgemm(b, zp=0, scale=np.float32(0.0041))
            y = ctx.qgemm(_dev(torch, a), w, a_zp=128, out_kind=L.QOUT_U8, a_scale=0.02, y_scale=0.05,
                          y_zp=128, lo=0, hi=255).cpu().numpy()
            want = O.qlinear_matmul(a, np.float32(0.02), 128, b, np.float32(0.0041), 0, np.float32(0.05), 128,
                                    sat_range=(0, 255))
            np.testing.assert_array_equal(y.astype(np.float32), want)
        else:
            w = ctx.weight_qgemm(b, zp=0)
            y = ctx.qgemm(_dev(torch, a), w, a_zp=128, out_kind=L.QOUT_I32).cpu().numpy()
            np.testing.assert_array_equal(y, O.matmul_integer(a, b, 128, 0))
    finally:
        ctx.set_tile(0)


@pytest.mark.parametrize("tile", [6, 16, 8, 12])
@pytest.mark.parametrize("mkn", [(300, 1664, 520), (257, 1000, 300)], ids=str)
def test_qgemm_large_tiles_bit_exact(torch, ctx, mkn, tile):
    """The 256x256 tiles (16: unrolled three-deep X ring) and the int8
    128x128 ones: K of 13 whole stages (the whole-stage loader; two six-stage
    trips and a one-stage tail on tile 16) and K with a tail (the loader with
    the per-load select), ragged edges, u8 outputs."""
    from oxionnx_amd import _lib as L
    m, k, n = mkn
    rng = np.random.default_rng(m + k + n)
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    ctx.set_tile(tile)
    try:
        w = ctx.weight_qgemm(b, zp=0, scale=np.float32(0.0041))
        y = ctx.qgemm(_dev(torch, a), w, a_zp=128, out_kind=L.QOUT_U8, a_scale=0.02, y_scale=0.05,
                      y_zp=128, lo=0, hi=255).cpu().numpy()
    finally:
        ctx.set_tile(0)
    want = O.qlinear_matmul(a, np.float32(0.02), 128, b, np.float32(0.0041), 0, np.float32(0.05), 128,
                            sat_range=(0, 255))
    np.testing.assert_array_equal(y.astype(np.float32), want)


def test_matmul_integer_per_row_zero_point(torch, ctx):
    from oxionnx_amd import _lib as L
    rng = np.random.default_rng(9)
    m, k, n = 45, 200, 70
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(0, 256, (k, n)).astype(np.uint8)
    azp = rng.integers(0, 256, m).astype(np.int32)
    bzp = rng.integers(100, 156, n).astype(np.int32)
    w = ctx.weight_qgemm(b, zp=bzp)
    y = ctx.qgemm(_dev(torch, a), w, a_zp=azp, out_kind=L.QOUT_I32).cpu().numpy()
    np.testing.assert_array_equal(y, O.matmul_integer(a, b, azp, bzp))


def test_qlinear_matmul_per_column_scale(torch, ctx):
    """Spec per-column b_scale (the reference itself reads only b_scale[0])."""
    from oxionnx_amd import _lib as L
    rng = np.random.default_rng(10)
    m, k, n = 64, 768, 96
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    bs = rng.uniform(0.001, 0.01, n).astype(np.float32)
    w = ctx.weight_qgemm(b, zp=0, scale=bs)
    y = ctx.qgemm(_dev(torch, a), w, a_zp=128, a_scale=0.02, y_scale=0.05, y_zp=128).cpu().numpy()
    acc, _ = O.integer_matmul(a, b, 128, 0)
    acc = acc.reshape(m, n)
    comb = (np.float32(0.02) * bs) / np.float32(0.05)
    want = np.clip(np.rint(acc * comb.astype(np.float64) + 128.0), 0, 255)
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("c", G.cases("MatMulInteger") + G.cases("QLinearMatMul"), ids=lambda c: c["name"])
def test_integer_matmul_golden_vectors(torch, ctx, c):
    from oxionnx_amd import _lib as L
    dts = c["dtypes"]
    npdt = {"u8": np.uint8, "i8": np.int8}
    a = G.arr(c, "a").astype(npdt[dts["a"]])
    b = G.arr(c, "b").astype(npdt[dts["b"]])
    g = lambda nm, d=0: (G.arr(c, nm) if G.arr(c, nm) is not None else np.array([d]))
    azp = g("a_zp").astype(np.int32)
    bzp = g("b_zp").astype(np.int32)
    if c["op"] == "MatMulInteger":
        w = ctx.weight_qgemm(b, zp=bzp)
        y = ctx.qgemm(_dev(torch, a), w, a_zp=azp, out_kind=L.QOUT_I32).cpu().numpy()
        assert y.ravel().tolist() == c["expected"]
        return
    lo, hi = O.satrange_infer(g("y_zp"), azp)
    w = ctx.weight_qgemm(b, zp=bzp, scale=g("b_scale")[:1])
    # the union range [-128, 255] has no 8-bit type: f32 lanes, like the reference Tensor
    kind = L.QOUT_F32 if (lo, hi) == (-128, 255) else (L.QOUT_U8 if lo == 0 else L.QOUT_I8)
    y = ctx.qgemm(_dev(torch, a), w, a_zp=azp, out_kind=kind, a_scale=float(g("a_scale")[0]),
                  y_scale=float(g("y_scale")[0]), y_zp=int(g("y_zp")[0]), lo=lo, hi=hi).cpu().numpy()
    assert y.astype(np.float32).ravel().tolist() == c["expected"]


# ------------------------------------------------------------------ integer Conv
QCONV_CASES = [
    ((1, 3, 40, 40), (16, 3, 3, 3), (2, 2), (1, 1, 1, 1), (1, 1)),
    ((1, 16, 20, 20), (32, 16, 3, 3), (1, 1), (1, 1, 1, 1), (1, 1)),
    ((2, 32, 11, 9), (24, 32, 1, 1), (1, 1), (0, 0, 0, 0), (1, 1)),
    ((1, 20, 12, 12), (8, 20, 3, 3), (1, 1), (2, 1, 0, 2), (2, 2)),
    ((1, 64, 10, 10), (64, 64, 5, 5), (1, 1), (2, 2, 2, 2), (1, 1)),
    # row-tiled staging: 3 channels padded to 16, a partial channel tile
    ((1, 3, 32, 32), (16, 3, 3, 3), (2, 2), (1, 1, 1, 1), (1, 1)),
    ((2, 80, 16, 16), (16, 80, 1, 1), (1, 1), (0, 0, 0, 0), (1, 1)),
    # few taps x channels (the tiled stem kernel): 40 outputs, one channel
    # with 25 taps over two images (odd rows: the thread-per-output kernel),
    # dilation with asymmetric pads
    ((1, 2, 17, 24), (40, 2, 3, 3), (1, 2), (1, 0, 2, 1), (1, 1)),
    ((2, 1, 19, 15), (16, 1, 5, 5), (2, 1), (2, 2, 2, 2), (1, 1)),
    ((1, 3, 30, 32), (24, 3, 3, 3), (1, 1), (2, 1, 2, 0), (2, 2)),
    ((1, 3, 30, 30), (16, 3, 3, 3), (2, 2), (1, 1, 1, 1), (1, 1)),   # rows not 4-byte multiples
]


@pytest.mark.parametrize("case", QCONV_CASES, ids=lambda c: f"{c[0]}x{c[1]}")
@pytest.mark.parametrize("x_u8", [True, False], ids=["u8", "i8"])
@pytest.mark.parametrize("out_layout", ["nchw", "nhwc"])
def test_qlinear_conv_bit_exact(torch, ctx, case, x_u8, out_layout):
    from oxionnx_amd import _lib as L
    xs, ws, s, p, d = case
    rng = np.random.default_rng(sum(xs) * 5 + sum(ws))
    if x_u8:
        x = rng.integers(0, 256, xs).astype(np.uint8)
        xzp = 7
    else:
        x = rng.integers(-128, 128, xs).astype(np.int8)
        xzp = -5
    w = rng.integers(-127, 127, ws).astype(np.int8)
    wzp = rng.integers(-1, 2, ws[0]).astype(np.int32)
    wsc = rng.uniform(0.002, 0.02, ws[0]).astype(np.float32)
    bias = rng.integers(-2000, 2000, ws[0]).astype(np.int32)
    xs_, ys_ = np.float32(1 / 255), np.float32(0.05)
    yzp, lo, hi = (128, 0, 255) if x_u8 else (-2, -128, 127)
    wt = ctx.weight_qconv(w, zp=wzp, scale=wsc)
    layout = L.NCHW if out_layout == "nchw" else L.NHWC
    y = ctx.qconv2d(_dev(torch, x), wt, _dev(torch, bias), x_zp=xzp,
                    out_kind=L.QOUT_U8 if x_u8 else L.QOUT_I8, x_scale=float(xs_), y_scale=float(ys_), y_zp=yzp,
                    lo=lo, hi=hi, strides=s, pads=p, dilations=d, out_layout=layout)
    if layout == L.NHWC:
        y = y[..., :ws[0]].permute(0, 3, 1, 2)
    want = O.qlinear_conv(x, xs_, xzp, w, wsc, wzp, ys_, yzp, bias=bias, sat_range=(lo, hi), strides=s,
                          pads=p, dilations=d)
    np.testing.assert_array_equal(y.cpu().numpy().astype(np.float32), want)


@pytest.mark.parametrize("case", QCONV_CASES[:3], ids=lambda c: f"{c[0]}x{c[1]}")
def test_conv_integer_bit_exact(torch, ctx, case):
    from oxionnx_amd import _lib as L
    xs, ws, s, p, d = case
    rng = np.random.default_rng(17)
    x = rng.integers(0, 256, xs).astype(np.uint8)
    w = rng.integers(-127, 128, ws).astype(np.int8)
    wt = ctx.weight_qconv(w, zp=3)
    y = ctx.qconv2d(_dev(torch, x), wt, x_zp=100, out_kind=L.QOUT_I32, strides=s, pads=p, dilations=d)
    want = O.conv_integer(x, w, 100, 3, strides=s, pads=p, dilations=d)
    np.testing.assert_array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("wzp", [3, -128], ids=["split_rows", "flipped_channels"])
@pytest.mark.parametrize("out_kind", ["i32", "u8"])
def test_stem_integer_conv_split_and_flipped_rows(torch, ctx, wzp, out_kind):
    """The stem kernel's filter staging: rows split in two int8 halves
    (w_zp 3) and negated channels (w_zp -128)."""
    from oxionnx_amd import _lib as L
    rng = np.random.default_rng(41 + abs(wzp))
    x = rng.integers(0, 256, (1, 3, 33, 36)).astype(np.uint8)
    w = rng.integers(-127, 128, (16, 3, 3, 3)).astype(np.int8)
    if out_kind == "i32":
        wt = ctx.weight_qconv(w, zp=wzp)
        y = ctx.qconv2d(_dev(torch, x), wt, x_zp=9, out_kind=L.QOUT_I32, strides=(2, 2), pads=(1, 1, 1, 1))
        want = O.conv_integer(x, w, 9, wzp, strides=(2, 2), pads=[1, 1, 1, 1])
        np.testing.assert_array_equal(y.cpu().numpy(), want)
    else:
        wsc = rng.uniform(0.0005, 0.002, 16).astype(np.float32)
        wt = ctx.weight_qconv(w, zp=wzp, scale=wsc)
        y = ctx.qconv2d(_dev(torch, x), wt, x_zp=9, out_kind=L.QOUT_U8, x_scale=1 / 255, y_scale=0.05, y_zp=128,
                        lo=0, hi=255, strides=(2, 2), pads=(1, 1, 1, 1), out_layout=L.NHWC)
        got = y[..., :16].permute(0, 3, 1, 2).cpu().numpy()
        want = O.qlinear_conv(x, np.float32(1 / 255), 9, w, wsc, np.full(16, wzp), np.float32(0.05), 128,
                              strides=(2, 2), pads=[1, 1, 1, 1])
        np.testing.assert_array_equal(got.astype(np.float32), want)


@pytest.mark.parametrize("case", GROUP_CASES, ids=lambda c: f"{c[0]}x{c[1]}g{c[2]}")
@pytest.mark.parametrize("wzp", [3, -128], ids=["split_rows", "flipped_channels"])
def test_grouped_integer_conv_bit_exact(torch, ctx, case, wzp):
    """Grouped / depthwise ConvInteger and QLinearConv against integer_conv.
    w_zp 3 pushes w - w_zp past int8 (the packed rows split in two halves);
    w_zp -128 pushes it past 254 (the channel is stored negated)."""
    from oxionnx_amd import _lib as L
    xs, ws, grp, s, p, d = case
    rng = np.random.default_rng(sum(xs) + sum(ws) + grp + abs(wzp))
    x = rng.integers(0, 256, xs).astype(np.uint8)
    w = rng.integers(-127, 128, ws).astype(np.int8)
    w.flat[0] = 127
    wt = ctx.weight_qconv(w, zp=wzp, scale=rng.uniform(0.001, 0.01, ws[0]).astype(np.float32))
    y = ctx.qconv2d(_dev(torch, x), wt, x_zp=100, out_kind=L.QOUT_I32, strides=s, pads=p, dilations=d,
                    group=grp)
    want = O.conv_integer(x, w, 100, wzp, strides=s, pads=p, dilations=d, group=grp)
    np.testing.assert_array_equal(y.cpu().numpy(), want)
    bias = rng.integers(-5000, 5000, ws[0]).astype(np.int32)
    ws_ = rng.uniform(0.001, 0.01, ws[0]).astype(np.float32)
    wt = ctx.weight_qconv(w, zp=wzp, scale=ws_)
    y = ctx.qconv2d(_dev(torch, x), wt, _dev(torch, bias), x_zp=100, out_kind=L.QOUT_U8, x_scale=0.02,
                    y_scale=0.05, y_zp=128, lo=0, hi=255, strides=s, pads=p, dilations=d, group=grp)
    want = O.qlinear_conv(x, 0.02, 100, w, ws_, wzp, 0.05, 128, bias, strides=s, pads=p, dilations=d,
                          group=grp)
    np.testing.assert_array_equal(y.cpu().numpy().astype(np.float32), want)


@pytest.mark.parametrize("c", G.cases("ConvInteger") + G.cases("QLinearConv"), ids=lambda c: c["name"])
def test_integer_conv_golden_vectors(torch, ctx, c):
    from oxionnx_amd import _lib as L
    dts = c["dtypes"]
    npdt = {"u8": np.uint8, "i8": np.int8}
    x = G.arr(c, "x").astype(npdt[dts["x"]])
    w = G.arr(c, "w").astype(npdt[dts["w"]])
    attrs = G.conv_attrs(c)
    grp = c["attrs"].get("group", 1)
    s, p, d, _ = O.conv_geometry(x.shape, w.shape, attrs.get("strides"), attrs.get("pads"),
                                 attrs.get("dilations"), grp, attrs.get("auto_pad", "NOTSET"))
    g = lambda nm: G.arr(c, nm)
    xzp = int(g("x_zp")[0]) if g("x_zp") is not None else 0
    wzp = g("w_zp").astype(np.int32) if g("w_zp") is not None else np.array([0], np.int32)
    if c["op"] == "ConvInteger":
        wt = ctx.weight_qconv(w, zp=wzp)
        y = ctx.qconv2d(_dev(torch, x), wt, x_zp=xzp, out_kind=L.QOUT_I32, strides=s, pads=p, dilations=d,
                        group=grp)
        assert y.cpu().numpy().ravel().tolist() == c["expected"]
        return
    lo, hi = O.satrange_infer(g("y_zp"), [xzp])
    kind = L.QOUT_F32 if (lo, hi) == (-128, 255) else (L.QOUT_U8 if lo == 0 else L.QOUT_I8)
    wt = ctx.weight_qconv(w, zp=wzp, scale=g("w_scale"))
    bias = None if g("b") is None else _dev(torch, g("b").astype(np.int32))
    y = ctx.qconv2d(_dev(torch, x), wt, bias, x_zp=xzp, out_kind=kind,
                    x_scale=float(g("x_scale")[0]), y_scale=float(g("y_scale")[0]), y_zp=int(g("y_zp")[0]),
                    lo=lo, hi=hi, strides=s, pads=p, dilations=d, group=grp)
    assert y.cpu().numpy().astype(np.float32).ravel().tolist() == c["expected"]


def test_weight_cache_counters(torch, ctx):
    rng = np.random.default_rng(1)
    b = rng.normal(size=(64, 32)).astype(np.float32)
    ctx.reset_counters()
    w1 = ctx.weight_gemm(b, name="W", label="Gemm.B")
    w2 = ctx.weight_gemm(b, name="W", label="Gemm.B")
    c = ctx.counters()
    assert c["weight_misses"] == 1 and c["weight_hits"] == 1
    assert w1.handle.value == w2.handle.value
    ctx.weight_gemm(b, trans_b=True, name="W", label="Gemm.B")   # different form -> own entry
    assert ctx.counters()["weight_misses"] == 2


@pytest.mark.parametrize("wide", ["split", "flip"])
def test_wide_integer_weights_stay_exact(torch, ctx, wide):
    """w - w_zp outside int8: the packer splits rows into two int8 halves and,
    for a channel reaching +255, stores it negated; results stay bit-exact."""
    from oxionnx_amd import _lib as L
    rng = np.random.default_rng(21)
    m, k, n = 70, 96, 40
    a = rng.integers(0, 256, (m, k)).astype(np.uint8)
    if wide == "split":
        b = rng.integers(0, 256, (k, n)).astype(np.uint8)
        bzp = rng.integers(60, 200, n).astype(np.int32)
    else:
        b = rng.integers(0, 256, (k, n)).astype(np.uint8)
        b[0, :] = 255
        bzp = np.zeros(n, np.int32)
    w = ctx.weight_qgemm(b, zp=bzp)
    y = ctx.qgemm(_dev(torch, a), w, a_zp=3, out_kind=L.QOUT_I32).cpu().numpy()
    np.testing.assert_array_equal(y, O.matmul_integer(a, b, 3, bzp))
    x = rng.integers(0, 256, (1, 8, 9, 9)).astype(np.uint8)
    wc = rng.integers(0, 256, (6, 8, 3, 3)).astype(np.uint8)
    if wide == "flip":
        wc[:, 0, 0, 0] = 255
    wzp = np.array([0, 3, 200, 255, 128, 7], np.int32) if wide == "split" else np.zeros(6, np.int32)
    wt = ctx.weight_qconv(wc, zp=wzp)
    yc = ctx.qconv2d(_dev(torch, x), wt, x_zp=9, out_kind=L.QOUT_I32, pads=(1, 1, 1, 1)).cpu().numpy()
    np.testing.assert_array_equal(yc, O.conv_integer(x, wc, 9, wzp, pads=[1, 1, 1, 1]))
