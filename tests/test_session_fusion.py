"""Graph rewrites of the session's fusion pass, checked on the CPU: the
rewritten graph, run through the oracle's graph runner, gives the original
graph's outputs (merging sibling Gemms only regroups columns, so the f32
results agree to the oracle's own summation differences)."""
import numpy as np
import pytest

from oracle import graph_ref as G
from oxionnx_amd import ep
from oxionnx_amd.ep import Attributes as A
from oxionnx_amd.session import Graph, fuse


def _f32(v):
    return np.asarray(v, np.float32)


@pytest.mark.parametrize("trans_b", [0, 1])
def test_sibling_gemms_merge_into_one(trans_b):
    rng = np.random.default_rng(trans_b)
    widths = [6, 10, 4]
    inits, nodes = {}, []
    for i, n in enumerate(widths):
        w = rng.normal(0, 0.3, (n, 8) if trans_b else (8, n)).astype(np.float32)
        inits[f"W{i}"], inits[f"C{i}"] = w, rng.normal(0, 0.1, n).astype(np.float32)
        nodes.append(ep.Node("Gemm", ["lat", f"W{i}", f"C{i}"], [f"s{i}"], A(ints={"transB": trans_b}), name=f"g{i}"))
    # s0: two column slices; s1: a graph output and a Relu; s2: a slice with an end past the width
    inits.update({"a0": _f32([0]), "b0": _f32([3]), "a1": _f32([3]), "b1": _f32([6]), "ax": _f32([1]),
                  "a2": _f32([1]), "b2": _f32([99])})
    nodes += [ep.Node("Slice", ["s0", "a0", "b0", "ax"], ["p0"], name="sl0"),
              ep.Node("Slice", ["s0", "a1", "b1", "ax"], ["p1"], name="sl1"),
              ep.Node("Relu", ["s1"], ["r1"], name="relu"),
              ep.Node("Slice", ["s2", "a2", "b2", "ax"], ["p2"], name="sl2")]
    g = Graph(nodes, inits, ["lat"], ["p0", "p1", "s1", "r1", "p2"])
    f = fuse(g)
    assert [n.op for n in f.nodes].count("Gemm") == 1
    feeds = {"lat": rng.normal(0, 1, (2, 8)).astype(np.float32)}
    want, got = G.run_graph(g, feeds), G.run_graph(f, feeds)
    for k in g.outputs:
        assert got[k].shape == want[k].shape, k
        np.testing.assert_allclose(got[k], want[k], rtol=1e-6, atol=1e-6, err_msg=k)


def test_gemms_with_different_a_or_attributes_stay_apart():
    rng = np.random.default_rng(2)
    inits = {f"W{i}": rng.normal(0, 1, (4, 3)).astype(np.float32) for i in range(3)}
    inits.update({f"C{i}": np.zeros(3, np.float32) for i in range(3)})
    nodes = [ep.Node("Gemm", ["x", "W0", "C0"], ["y0"]),
             ep.Node("Gemm", ["z", "W1", "C1"], ["y1"]),
             ep.Node("Gemm", ["x", "W2", "C2"], ["y2"], A(floats={"alpha": 0.5}))]
    g = Graph(nodes, inits, ["x", "z"], ["y0", "y1", "y2"])
    assert [n.op for n in fuse(g).nodes] == ["Gemm", "Gemm", "Gemm"]


def test_face_swap_style_gemms_merge():
    from oxionnx_amd import workloads
    g, _ = workloads.face_swap_generator(dtype="f32", n_blocks=2)
    ops = [n.op for n in fuse(g).nodes]
    # each residual conv and its AdaIN norm become one fused node
    assert ops.count("Gemm") == 1 and ops.count("OhipConvInstanceNorm") == 4
    assert ops.count("OxiInstanceNorm") == 0 and ops.count("Conv") == 6


def test_conv_instnorm_fusion_attributes():
    """Conv (reflect Pad folded in) -> AdaIN norm -> Relu becomes one node
    carrying both halves' attributes; a grouped conv, or a conv with a second
    consumer, is left alone."""
    from oxionnx_amd import workloads
    g, _ = workloads.face_swap_generator(dtype="f32", n_blocks=1)
    nodes = fuse(g).nodes
    fused = [n for n in nodes if n.op == "OhipConvInstanceNorm"]
    assert len(fused) == 2
    first, second = fused
    assert first.attrs.strings.get("pad_mode") == "reflect"
    assert first.attrs.strings.get("norm_activation") == "relu" and "norm_activation" not in second.attrs.strings
    assert len(first.inputs) == 5 and first.inputs[3] == first.inputs[4]
    assert first.attrs.floats["epsilon"] == 1e-5
    assert first.attrs.ints["bias_offset"] - first.attrs.ints["scale_offset"] == 512
    assert "activation" not in first.attrs.strings
    # the block's skip Add folds into the second node as its residual (input 5)
    assert len(second.inputs) == 6 and second.outputs[0].startswith("skip")
    assert not any(n.op == "Add" for n in nodes)


@pytest.mark.parametrize("dt", ["f16", "f32"])
def test_nhwc_plan_hints_conv_and_resize_chains(dt):
    """The layout plan marks a conv output NHWC when every consumer reads it
    in place (a zero-padded ungrouped conv, a hinted nearest Resize, the
    reflect-padded RGB head in f16, whose few-output MFMA kernel pads in its
    loader), never a graph output, and not the f32 head's input (its
    few-output kernel reads NCHW)."""
    from oxionnx_amd import workloads
    g, _ = workloads.face_swap_generator(dtype=dt, n_blocks=1)
    nodes = fuse(g).nodes
    hinted = {n.outputs[0] for n in nodes if n.attrs.ints.get("out_nhwc")}
    by_out = {n.outputs[0]: n for n in nodes}
    assert not hinted & set(g.outputs)
    resizes = [n for n in nodes if n.op == "Resize"]
    assert resizes and all(n.attrs.ints.get("out_nhwc") for n in resizes)
    head = [n for n in nodes if n.op == "Conv" and n.attrs.strings.get("pad_mode") == "reflect"
            and n.attrs.int_lists.get("kernel_shape") == [7, 7] and n.inputs[0] != "x"]
    assert len(head) == 1
    assert (head[0].inputs[0] in hinted) == (dt == "f16")
    assert any(by_out[t].op in ("Conv", "OhipConvInstanceNorm") for t in hinted)


def test_nhwc_plan_skips_a_broadcast_residual():
    """A fused conv -> norm node whose residual is a [1, C, 1, 1]
    initializer (added by the NCHW broadcast kernel after the pair) gets no
    NHWC hint, although its consumer, a zero-padded conv, reads NHWC; the
    same chain with a full-shape residual is hinted."""
    rng = np.random.default_rng(5)
    conv = {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}

    def graph(residual_init):
        inits = {"W": rng.normal(0, 0.05, (16, 16, 3, 3)).astype(np.float32), "B": _f32(np.zeros(16)),
                 "W2": rng.normal(0, 0.05, (8, 16, 3, 3)).astype(np.float32)}
        other = "x"
        if residual_init:
            inits["rb"] = rng.normal(0, 1, (1, 16, 1, 1)).astype(np.float32)
            other = "rb"
        nodes = [ep.Node("Conv", ["x", "W", "B"], ["h"], A(int_lists=dict(conv)), name="c1"),
                 ep.Node("OxiInstanceNorm", ["h"], ["n"], A(floats={"epsilon": 1e-5}), name="nm"),
                 ep.Node("Add", ["n", other], ["r"], name="add"),
                 ep.Node("Conv", ["r", "W2"], ["y"], A(int_lists=dict(conv)), name="c2")]
        return Graph(nodes, inits, ["x"], ["y"])

    for residual_init, hinted in ((True, False), (False, True)):
        nodes = fuse(graph(residual_init)).nodes
        fused = [n for n in nodes if n.op == "OhipConvInstanceNorm"]
        assert len(fused) == 1 and len(fused[0].inputs) == 6
        assert bool(fused[0].attrs.ints.get("out_nhwc")) == hinted


def test_reference_chains_of_fused_nodes_reproduce_the_unfused_graph():
    """The node-by-node f16 parity test evaluates each node of the fused
    graph as the chain of reference operators it replaces; fed the unfused
    graph's own values, every chain gives that graph's values bit for bit
    (the merged style Gemm, which has no counterpart value, evaluated as it
    is)."""
    from oxionnx_amd import workloads
    from tests.test_gpu_f16_nodes import _reference_chain, _ulps
    g, feeds = workloads.face_swap_generator(dtype="f16", n_blocks=1)
    fused = fuse(g)
    names = {n.outputs[0] for n in g.nodes}
    outs = [n.outputs[0] for n in fused.nodes if n.outputs[0] in names]
    full = G.run_graph(Graph(g.nodes, g.initializers, g.inputs, outs), feeds, half=True)
    vals = {**{k: np.asarray(v) for k, v in feeds.items()}, **{k: v.astype(np.float16) for k, v in full.items()}}
    for n in fused.nodes:
        if n.outputs[0] not in names:
            vals[n.outputs[0]] = G.run_graph(Graph([n], fused.initializers, ["latent"], n.outputs), feeds,
                                             half=True)[n.outputs[0]].astype(np.float16)
    shapes = {k: np.shape(v) for k, v in vals.items()}
    shapes.update({k: np.shape(np.asarray(getattr(v, "data", v))) for k, v in fused.initializers.items()})
    ops = set()
    for n in fused.nodes:
        chain, extra = _reference_chain(n, shapes)
        ins = [t for t in n.inputs if t and t not in fused.initializers]
        ref = G.run_graph(Graph(chain, {**fused.initializers, **extra}, ins, [n.outputs[0]]),
                          {t: vals[t] for t in ins}, half=True)[n.outputs[0]]
        assert _ulps(vals[n.outputs[0]], ref).max() == 0, n.outputs[0]
        ops.add((n.op, n.attrs.strings.get("activation"), len(n.inputs)))
    assert ("OhipConvInstanceNorm", None, 6) in ops and ("Conv", "leaky_relu", 3) in ops
