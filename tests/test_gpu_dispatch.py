"""Node-level parity through the drop-in boundary (ohip_try_dispatch), written
like the reference's session tests (tests/w2_quantized_ops_e2e.rs,
tests/conformance_conv.rs): one node, graph inputs as host tensors, quantized
outputs compared exactly, float outputs within the reference tolerance."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests import _golden as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    assert torch.cuda.is_available()
    from oxionnx_amd import _lib as L
    from oxionnx_amd import ep
    c = ep.HipContext(0)
    t = L.Tuning()
    L.lib().ohip_tuning_for_class(L.CLASS_PARITY, ctypes.byref(t))
    c.set_tuning(t)   # GpuTuning::PARITY: numerics tests run at hand-checkable sizes
    yield c
    c.close()


def _attrs(c):
    from oxionnx_amd.ep import Attributes
    a = Attributes()
    for k, v in c["attrs"].items():
        if isinstance(v, list):
            a.int_lists[k] = v
        elif isinstance(v, str):
            a.strings[k] = v
        elif isinstance(v, float):
            a.floats[k] = v
        else:
            a.ints[k] = v
    return a


def _node(c, order, weights_names):
    from oxionnx_amd.ep import Node
    return Node(op=c["op"].replace("Conv1D", "Conv").replace("GemmF16", "Gemm"), inputs=order,
                attrs=_attrs(c))


INPUT_ORDER = {
    "MatMulInteger": ["a", "b", "a_zp", "b_zp"],
    "QLinearMatMul": ["a", "a_scale", "a_zp", "b", "b_scale", "b_zp", "y_scale", "y_zp"],
    "ConvInteger": ["x", "w", "x_zp", "w_zp"],
    "QLinearConv": ["x", "x_scale", "x_zp", "w", "w_scale", "w_zp", "y_scale", "y_zp", "b"],
    "Conv": ["x", "w", "b"], "Conv1D": ["x", "w", "b"], "Gemm": ["a", "b"], "MatMul": ["a", "b"],
}
GRAPH_INPUTS = {"a", "x"}


def _run(ctx, c):
    from oxionnx_amd import ep
    order = [n if n in c["inputs"] else "" for n in INPUT_ORDER[c["op"]]]
    while order and order[-1] == "":
        order.pop()
    feeds, weights = {}, {}
    for n in order:
        if not n:
            continue
        v = np.asarray(c["inputs"][n]["data"], np.float64).reshape(c["inputs"][n]["shape"]).astype(np.float32)
        (feeds if n in GRAPH_INPUTS else weights)[n] = v
    return ep.try_hip_dispatch(_node(c, order, weights), weights, feeds, ctx)


QUANT = G.cases("MatMulInteger") + G.cases("QLinearMatMul") + G.cases("ConvInteger") + G.cases("QLinearConv")


@pytest.mark.parametrize("c", QUANT, ids=lambda c: c["name"])
def test_quantized_golden_through_the_boundary(ctx, c):
    out = _run(ctx, c)   # grouped (depthwise) convolutions included
    assert out is not None, ctx.last_decline()
    assert list(out[0].shape) == c["shape"]
    assert out[0].dtype == np.float32
    assert out[0].ravel().tolist() == [float(v) for v in c["expected"]]


FLOAT = G.cases("Conv") + G.cases("Conv1D") + G.cases("Gemm") + G.cases("MatMul")


@pytest.mark.parametrize("c", FLOAT, ids=lambda c: c["name"])
def test_float_golden_through_the_boundary(ctx, c):
    out = _run(ctx, c)   # grouped convolutions included (group > 1 runs on the device)
    assert out is not None, ctx.last_decline()
    assert list(out[0].shape) == c["shape"]
    np.testing.assert_allclose(out[0].ravel(), c["expected"], atol=c["tol"])


def test_zero_scale_is_declined_to_the_cpu_operator(ctx):
    """tests/w2_quantized_ops_e2e.rs:485-530: the CPU operator owns the error."""
    from oxionnx_amd import ep
    node = ep.Node("QLinearConv", ["x", "xs", "xzp", "w", "ws", "wzp", "ys", "yzp"])
    w = {k: np.array([v], np.float32) for k, v in
         dict(xs=0.1, xzp=0.0, ws=0.1, wzp=0.0, ys=0.0, yzp=0.0).items()}
    w["w"] = np.ones((1, 1, 1, 1), np.float32)
    assert ep.try_hip_dispatch(node, w, {"x": np.arange(4, dtype=np.float32).reshape(1, 1, 2, 2)}, ctx) is None
    assert "scale" in ctx.last_decline()


def test_typed_y_zero_point_pins_the_range(ctx):
    """SatRange::for_dtype (quant_ops/mod.rs:215-221): the union-range case
    resolves to int8 when y_zero_point is declared int8."""
    from oxionnx_amd import ep
    c = G.cases("QLinearMatMul")[-1]   # the union-range vector
    assert c["name"] == "qlinear_matmul_ambiguous_zero_points_use_the_union_range"
    g = lambda n: np.asarray(c["inputs"][n]["data"], np.float32).reshape(c["inputs"][n]["shape"])
    weights = {n: g(n) for n in ["a_scale", "a_zp", "b", "b_scale", "b_zp", "y_scale"]}
    weights["y_zp"] = ep.Typed(np.array([100], np.int8), declared="i8")
    node = ep.Node("QLinearMatMul", INPUT_ORDER["QLinearMatMul"])
    out = ep.try_hip_dispatch(node, weights, {"a": g("a")}, ctx)
    acc, _ = O.integer_matmul(g("a"), g("b"), 0, 0)
    want = O.qlinear_matmul(g("a"), 1.0, 0, g("b"), 1.0, 0, 1.0, 100, sat_range=(-128, 127))
    assert out[0].ravel().tolist() == want.ravel().tolist() == [127.0, -50.0, 100.0, 100.0]


def test_default_gate_declines_toy_shapes():
    import torch
    from oxionnx_amd import ep
    c = ep.HipContext(0)
    try:
        node = ep.Node("Gemm", ["a", "b"])
        out = ep.try_hip_dispatch(node, {"b": np.ones((4, 4), np.float32)}, {"a": np.ones((4, 4), np.float32)}, c)
        assert out is None and "gate" in c.last_decline()
        assert c.counters()["declined"] == 1
    finally:
        c.close()


def test_resident_chain_keeps_activations_on_the_device(ctx):
    """Conv -> Conv with the intermediate resident: the second node binds the
    first one's device output (accepts_resident_slot(Conv, 0)), nothing is
    read back in between, and the result equals the host round-trip path."""
    from oxionnx_amd import ep
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, (1, 16, 24, 24)).astype(np.float32)
    w1 = rng.normal(0, 0.1, (32, 16, 3, 3)).astype(np.float32)
    w2 = rng.normal(0, 0.1, (8, 32, 3, 3)).astype(np.float32)
    weights = {"w1": w1, "w2": w2}
    relu = ep.Attributes(strings={"activation": "relu"}, int_lists={"pads": [1, 1, 1, 1]})
    n1 = ep.Node("Conv", ["x", "w1"], ["h"], relu)
    n2 = ep.Node("Conv", ["h", "w2"], ["y"], ep.Attributes(int_lists={"pads": [1, 1, 1, 1]}))
    host_h = ep.try_hip_dispatch(n1, weights, {"x": x}, ctx)[0]
    host_y = ep.try_hip_dispatch(n2, weights, {"h": host_h}, ctx)[0]
    ctx.reset_counters()
    dx = ep.DeviceTensor.from_host(ctx, x)
    dh = ep.try_hip_dispatch_resident(n1, weights, {"x": dx}, ctx)[0]
    dy = ep.try_hip_dispatch_resident(n2, weights, {"h": dh}, ctx)[0]
    c = ctx.counters()
    assert c["d2h_bytes"] == 0 and c["h2d_bytes"] == x.nbytes
    assert c["weight_hits"] == 2 and c["weight_misses"] == 0
    np.testing.assert_array_equal(dy.to_host(ctx), host_y)
    want = O.conv(O.conv(x, w1, activation="relu", pads=[1, 1, 1, 1]), w2, pads=[1, 1, 1, 1])
    assert np.max(np.abs(host_y - want)) <= 1e-4 * np.max(np.abs(want))


@pytest.mark.parametrize("attrs", [
    dict(strides=[2, 2]),
    dict(strides=[2, 2], output_shape=[1, 3, 10, 10]),
    dict(strides=[2, 2], auto_pad="SAME_UPPER"),
    dict(strides=[2, 2], auto_pad="SAME_LOWER", output_padding=[1, 0]),
    dict(strides=[1, 2], pads=[1, 0, 0, 1], dilations=[2, 1], group=2, kernel_shape=[3, 3]),
], ids=["natural", "output_shape", "same_upper", "same_lower_outpad", "group_dilated"])
def test_conv_transpose_node_through_the_boundary(ctx, attrs):
    """ConvTranspose (registry/conv_ops/conv.rs:556-710): the node's output_shape /
    auto_pad / output_padding resolve to the extent and pads the reference
    derives (conv.rs:412-470), and the values equal the scatter's."""
    from oxionnx_amd import ep
    from oxionnx_amd.ep import Attributes
    rng = np.random.default_rng(23)
    g = attrs.get("group", 1)
    x = rng.uniform(-1, 1, (1, 4, 5, 5)).astype(np.float32)
    w = rng.normal(0, 0.3, (4, 6 // g if g > 1 else 3, 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.1, w.shape[1] * g).astype(np.float32)
    a = Attributes()
    for k, v in attrs.items():
        if isinstance(v, list):
            a.int_lists[k] = v
        elif isinstance(v, str):
            a.strings[k] = v
        else:
            a.ints[k] = v
    node = ep.Node("ConvTranspose", ["x", "w", "b"], attrs=a)
    out = ep.try_hip_dispatch(node, {"w": w, "b": b}, {"x": x}, ctx)
    assert out is not None, ctx.last_decline()
    want = O.conv_transpose(x, w, b, **attrs)
    assert out[0].shape == want.shape
    assert np.max(np.abs(out[0].astype(np.float64) - want)) <= 1e-4 * max(1.0, float(np.abs(want).max()))


def test_batched_matmul_node_through_the_boundary(ctx):
    """MatMulOp with a batched B (matmul_gemm.rs:9-126): the batch prefixes
    broadcast and slice s pairs A slice s % a_batches with B slice s % b_batches
    (math_typed.rs:352-369)."""
    from oxionnx_amd import ep
    rng = np.random.default_rng(31)
    for ash, bsh in [((2, 3, 40, 24), (3, 24, 36)), ((5, 17, 64), (5, 64, 9))]:
        a = rng.uniform(-1, 1, ash).astype(np.float32)
        b = rng.normal(0, 0.2, bsh).astype(np.float32)
        out = ep.try_hip_dispatch(ep.Node("MatMul", ["a", "b"]), {"b": b}, {"a": a}, ctx)
        assert out is not None, ctx.last_decline()
        want = O.matmul_batched(a, b)
        assert out[0].shape == want.shape
        assert np.max(np.abs(out[0] - want)) <= 1e-4 * max(1.0, float(np.abs(want).max()))
