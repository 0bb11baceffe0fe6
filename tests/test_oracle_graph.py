"""Pins the node functions of the CPU graph executor (oracle/graph_ref.py)
that the end-to-end workloads use besides the contractions: nearest Resize,
MaxPool, Pad, QuantizeLinear / DequantizeLinear, the unary activations and
OxiInstanceNorm.

Each is checked against the reference's own known answers
(tests/golden/reference_vectors.json, transcribed with file:line) and against
an independent formulation that a plausible mistake would break: exact
rational arithmetic for the nearest index rules, torch's float64 pooling and
padding, float64 closed forms for the activations and the normalisation, and
the saturation ranges of the reference's QuantizeLinear.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import graph_ref as GR
from oxionnx_amd import ep
from oxionnx_amd.session import Graph
from tests import _golden as G

A = ep.Attributes


def run_node(op, x, inits=(), attrs=None, extra=()):
    """One node through graph_ref: x is the graph input, `inits` are the
    other inputs (name, array) in order; '' leaves a slot empty."""
    names = ["x"] + [n for n, _ in inits]
    node = ep.Node(op, names, ["y"], attrs or A())
    g = Graph([node], {n: np.asarray(v, np.float32) for n, v in inits if n}, ["x"], ["y"])
    return GR.run_graph(g, {"x": np.asarray(x, np.float32)})["y"]


def _attrs(d):
    a = A()
    for k, v in d.items():
        if isinstance(v, list):
            a.int_lists[k] = v
        elif isinstance(v, str):
            a.strings[k] = v
        elif isinstance(v, float):
            a.floats[k] = v
        else:
            a.ints[k] = v
    return a


# ------------------------------------------------------------ golden vectors
@pytest.mark.parametrize("c", G.cases("Resize"), ids=lambda c: c["name"])
def test_resize_nearest_golden(c):
    y = run_node("Resize", G.arr(c, "x"), [("", None), ("sc", G.arr(c, "scales"))], _attrs(c["attrs"]))
    assert list(y.shape) == c["shape"]
    assert y.ravel().tolist() == c["expected"]


@pytest.mark.parametrize("c", G.cases("ResizeShape"), ids=lambda c: c["name"])
def test_resize_output_shape_is_floor_golden(c):
    y = run_node("Resize", G.arr(c, "x"), [("", None), ("sc", G.arr(c, "scales"))], _attrs(c["attrs"]))
    assert list(y.shape) == c["shape"]


@pytest.mark.parametrize("c", G.cases("MaxPool"), ids=lambda c: c["name"])
def test_maxpool_golden(c):
    y = run_node("MaxPool", G.arr(c, "x"), attrs=_attrs(c["attrs"]))
    assert list(y.shape) == c["shape"]
    assert y.ravel().tolist() == c["expected"]


@pytest.mark.parametrize("c", G.cases("Pad"), ids=lambda c: c["name"])
def test_pad_golden(c):
    y = run_node("Pad", G.arr(c, "x"), [("p", G.arr(c, "pads"))], _attrs(c["attrs"]))
    assert list(y.shape) == c["shape"]
    assert y.ravel().tolist() == c["expected"]


@pytest.mark.parametrize("c", G.cases("QuantizeLinear") + G.cases("DequantizeLinear"), ids=lambda c: c["name"])
def test_quantize_dequantize_golden(c):
    ins = [("s", G.arr(c, "scale"))] + ([("z", G.arr(c, "zp"))] if G.arr(c, "zp") is not None else [])
    y = run_node(c["op"], G.arr(c, "x"), ins)
    np.testing.assert_allclose(y.ravel(), c["expected"], atol=c.get("tol", 0.0), rtol=0)


@pytest.mark.parametrize("c", G.cases("Sigmoid") + G.cases("Tanh") + G.cases("Silu") + G.cases("LeakyRelu"),
                         ids=lambda c: c["name"])
def test_unary_golden(c):
    y = run_node(c["op"], G.arr(c, "x"), attrs=_attrs(c["attrs"]))
    np.testing.assert_allclose(y.ravel(), c["expected"], atol=c["tol"], rtol=0)


# ------------------------------------------------------------ nearest index rules, exactly
def _exact_src(j, in_len, out_len, scale, coord):
    x, s = Fraction(j), Fraction(scale)
    if coord == "asymmetric":
        return x / s
    if coord == "align_corners":
        return Fraction(0) if out_len <= 1 else x * (in_len - 1) / (out_len - 1)
    if coord == "pytorch_half_pixel":
        return (x + Fraction(1, 2)) / s - Fraction(1, 2) if out_len > 1 else Fraction(0)
    if coord == "tf_half_pixel_for_nn":
        return (x + Fraction(1, 2)) / s
    return (x + Fraction(1, 2)) / s - Fraction(1, 2)   # half_pixel


def _exact_pick(src, rule):
    if rule == "floor":
        return math.floor(src)
    if rule == "ceil":
        return math.ceil(src)
    fl = math.floor(src)
    if src - fl == Fraction(1, 2):
        return fl + 1 if rule == "round_prefer_ceil" else fl
    return math.floor(src + Fraction(1, 2))


@pytest.mark.parametrize("coord", ["half_pixel", "asymmetric", "align_corners", "pytorch_half_pixel",
                                   "tf_half_pixel_for_nn"])
@pytest.mark.parametrize("rule", ["round_prefer_floor", "round_prefer_ceil", "floor", "ceil"])
@pytest.mark.parametrize("in_len,scale", [(4, 2.0), (7, 1.5), (8, 0.75), (5, 3.0), (6, 2.5), (9, 0.5), (1, 4.0)])
def test_nearest_index_rule_matches_exact_arithmetic(coord, rule, in_len, scale):
    out_len = math.floor(in_len * scale)
    got = [GR._nearest_src(j, in_len, out_len, scale, coord, rule) for j in range(out_len)]
    want = [min(max(_exact_pick(_exact_src(j, in_len, out_len, scale, coord), rule), 0), in_len - 1)
            for j in range(out_len)]
    assert got == want


@pytest.mark.parametrize("scale", [2.0, 4.0, 0.5])
def test_nearest_resize_matches_torch(scale):
    """torch 'nearest' is asymmetric + floor; 'nearest-exact' is half_pixel +
    round_prefer_ceil (exact for power-of-two scales)."""
    x = np.random.default_rng(1).normal(size=(2, 3, 8, 12)).astype(np.float32)
    sc = np.asarray([1, 1, scale, scale], np.float32)
    for coord, rule, mode in (("asymmetric", "floor", "nearest"), ("half_pixel", "round_prefer_ceil", "nearest-exact")):
        y = run_node("Resize", x, [("", None), ("sc", sc)],
                     A(strings={"mode": "nearest", "coordinate_transformation_mode": coord, "nearest_mode": rule}))
        t = F.interpolate(torch.from_numpy(x), scale_factor=scale, mode=mode).numpy()
        np.testing.assert_array_equal(y, t)


# ------------------------------------------------------------ MaxPool
@pytest.mark.parametrize("ks,st,pads", [((5, 5), (1, 1), (2, 2, 2, 2)), ((3, 3), (2, 2), (1, 1, 1, 1)),
                                        ((2, 3), (2, 1), (0, 1, 1, 0)), ((3, 2), (1, 2), (0, 0, 0, 0))])
def test_maxpool_matches_torch(ks, st, pads):
    # all-negative inputs: a zero-filled border instead of -inf would show
    x = -np.abs(np.random.default_rng(2).normal(size=(1, 4, 11, 10))).astype(np.float32) - 0.5
    y = run_node("MaxPool", x, attrs=A(int_lists={"kernel_shape": list(ks), "strides": list(st), "pads": list(pads)}))
    xt = F.pad(torch.from_numpy(x).double(), (pads[1], pads[3], pads[0], pads[2]), value=-math.inf)
    t = F.max_pool2d(xt, ks, st).numpy()
    np.testing.assert_array_equal(y, t)


# ------------------------------------------------------------ Pad
@pytest.mark.parametrize("mode,tmode", [("reflect", "reflect"), ("edge", "replicate"), ("constant", "constant")])
def test_pad_matches_torch(mode, tmode):
    x = np.random.default_rng(3).normal(size=(1, 3, 6, 7)).astype(np.float32)
    p = [0, 0, 2, 1, 0, 0, 3, 2]  # [n, c, top, left, n, c, bottom, right]
    y = run_node("Pad", x, [("p", np.asarray(p, np.float32))], A(strings={"mode": mode}))
    t = F.pad(torch.from_numpy(x).double(), (p[3], p[7], p[2], p[6]), mode=tmode).numpy()
    np.testing.assert_array_equal(y, t)


def test_pad_reflect_index_formula():
    """Reflect excludes the edge element: index i in [-p, n+p) maps to
    |i| for i < 0 and 2(n-1) - i for i >= n."""
    n, p = 5, 3
    x = np.arange(1, n + 1, dtype=np.float32)
    y = run_node("Pad", x, [("p", np.asarray([p, p], np.float32))], A(strings={"mode": "reflect"}))
    idx = [abs(i) if i < 0 else (2 * (n - 1) - i if i >= n else i) for i in range(-p, n + p)]
    assert y.tolist() == [float(x[i]) for i in idx]


# ------------------------------------------------------------ Quantize / Dequantize
def test_quantize_rounds_ties_to_even_and_saturates():
    x = np.asarray([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 1e6, -1e6, 0.49999997], np.float32)
    s = np.asarray([1.0], np.float32)
    # zero point above 127: uint8 range
    y = run_node("QuantizeLinear", x, [("s", s), ("z", np.asarray([200.0], np.float32))])
    assert y.tolist() == [200, 202, 202, 200, 198, 198, 255, 0, 200]
    # zero point <= 127 (declared or not): the int8 range, as saturation_range decides
    y = run_node("QuantizeLinear", x, [("s", s), ("z", np.asarray([-5.0], np.float32))])
    assert y.tolist() == [-5, -3, -3, -5, -7, -7, 127, -128, -5]
    # no zero point: uint8 with zero point 0
    y = run_node("QuantizeLinear", x, [("s", s)])
    assert y.tolist() == [0, 2, 2, 0, 0, 0, 255, 0, 0]


def test_quantize_divides_in_f32_then_rounds():
    rng = np.random.default_rng(4)
    x = rng.normal(0, 3, 4000).astype(np.float32)
    s = np.float32(0.0371)
    y = run_node("QuantizeLinear", x, [("s", np.asarray([s])), ("z", np.asarray([128.0], np.float32))])
    want = [min(max(round(float(np.float32(v) / s)) + 128, 0), 255) for v in x]   # Python round: ties to even
    assert y.astype(np.int64).tolist() == want


def test_dequantize_closed_form():
    q = np.arange(-128, 128, dtype=np.float32)
    y = run_node("DequantizeLinear", q, [("s", np.asarray([0.0173], np.float32)), ("z", np.asarray([-7.0], np.float32))])
    np.testing.assert_array_equal(y, ((q.astype(np.float32) + np.float32(7)) * np.float32(0.0173)))


# ------------------------------------------------------------ unary activations
GRID = np.concatenate([np.linspace(-30, 30, 6001), [-100.0, -88.0, 88.0, 100.0, 0.0, -0.0, 1e-30]]).astype(np.float32)


@pytest.mark.parametrize("op,f", [
    ("Sigmoid", lambda v: 1 / (1 + np.exp(-v))),
    ("Tanh", np.tanh),
    ("Silu", lambda v: v / (1 + np.exp(-v))),
    ("LeakyRelu", lambda v: np.where(v >= 0, v, 0.2 * v)),
    ("Relu", lambda v: np.maximum(v, 0)),
])
def test_unary_matches_float64(op, f):
    y = run_node(op, GRID, attrs=A(floats={"alpha": 0.2}) if op == "LeakyRelu" else None)
    want = f(GRID.astype(np.float64))
    assert np.all(np.isfinite(y))
    # a few f32 ulps of the result, absolute near zero
    np.testing.assert_allclose(y, want, rtol=4e-7, atol=1e-37 if op in ("Relu", "LeakyRelu") else 1e-7)


# ------------------------------------------------------------ OxiInstanceNorm
def _ramp(shape, scale, offset):
    """The input generator of registry/oxi_instance_norm.rs:266-272."""
    i = np.arange(int(np.prod(shape)))
    return (offset + scale * ((i % 17) - 8.0) + 0.25 * np.sin(i)).astype(np.float32).reshape(shape)


def _unfused_chain(x, eps):
    """ReduceMean -> Sub -> Mul -> ReduceMean -> Add(eps) -> Sqrt -> Div(1, .) -> Mul,
    in float64 (registry/oxi_instance_norm.rs:243-264)."""
    sp = int(np.prod(x.shape[2:]))
    p = x.astype(np.float64).reshape(-1, sp)
    d = p - p.mean(axis=1, keepdims=True)
    var = (d * d).mean(axis=1, keepdims=True)
    return (d * (1.0 / np.sqrt(var + eps))).reshape(x.shape)


def _instnorm(x, eps):
    return run_node("OxiInstanceNorm", x, attrs=A(floats={"epsilon": eps}))


@pytest.mark.parametrize("shape,scale,offset,eps", [((2, 3, 4, 5), 1.5, 3.0, 1e-8), ((4, 16, 16, 16), 0.7, 2.0, 1e-5),
                                                    ((1, 1, 4, 4), 1.0, 0.0, 100.0), ((1, 8, 32, 32), 2.0, -7.0, 1e-5)])
def test_instance_norm_matches_unfused_chain(shape, scale, offset, eps):
    x = _ramp(shape, scale, offset)
    y = _instnorm(x, eps)
    want = _unfused_chain(x, eps)
    assert np.all(np.abs(y - want) <= 1e-6 + 1e-5 * np.abs(want))
    # and torch's float64 instance norm (population variance, eps inside the root)
    t = F.instance_norm(torch.from_numpy(x).double(), eps=eps).numpy()
    assert np.all(np.abs(y - t) <= 1e-6 + 1e-5 * np.abs(t))


def test_instance_norm_planes_are_independent():
    x = _ramp((2, 3, 4, 4), 2.0, -7.0)
    x[1, 2] += 1000.0   # one plane far off: the others must not move
    y = _instnorm(x, 1e-12).reshape(6, 16)
    np.testing.assert_allclose(y.mean(axis=1), 0, atol=1e-4)
    np.testing.assert_allclose(y.var(axis=1), 1, atol=1e-3)


def test_instance_norm_constant_plane_and_rank3():
    y = _instnorm(np.full((1, 2, 2, 2), 5.0, np.float32), 1e-8)
    assert np.all(np.isfinite(y)) and np.all(np.abs(y) < 1e-6)
    y = _instnorm(np.asarray([[[1.0, 2.0, 3.0], [10.0, 20.0, 30.0]]], np.float32), 0.0)
    r = math.sqrt(1.5)   # (x - mean) / sqrt(2/3) = ±sqrt(3/2)
    np.testing.assert_allclose(y.ravel(), [-r, 0, r, -r, 0, r], atol=1e-5)
