"""Config 4's f16 generator checked node by node: every node of the forward
the device runs (after the provider's fusions) is compared with the oracle
evaluated on the device's own inputs for that node, so a rounding point the
device places differently from the reference shows at the node that places
it, not only as drift at the graph output.

The oracle for a fused node is the chain of reference operators it replaces,
each rounding its output to f16 as the reference's f16 nodes do
(conv_typed.rs:54-109 for Conv, registry/oxi_instance_norm.rs:56-65 for the
norm, the same storage rule for Mul / Add / Relu / LeakyRelu / Tanh):
  Conv [pad_mode] [activation]   Pad -> Conv -> LeakyRelu / Relu
  OhipConvInstanceNorm           Pad -> Conv -> OxiInstanceNorm -> Mul(gamma)
                                 -> Add(beta) [-> Relu] [-> Add(residual)]
The merged style Gemm, Resize and Tanh are reference operators as they are.
"""
import numpy as np
import pytest

from oracle import graph_ref as G
from oxionnx_amd import ep, workloads
from oxionnx_amd.session import Graph, Session, fuse

pytestmark = pytest.mark.gpu

A = ep.Attributes


@pytest.fixture(scope="module")
def ctx():
    import ctypes

    import torch  # noqa: F401  (HIP runtime initialisation on the test process)
    from oxionnx_amd import _lib as L
    c = ep.HipContext(0)
    t = L.Tuning()
    L.lib().ohip_tuning_for_class(L.CLASS_PARITY, ctypes.byref(t))
    L.lib().ohip_set_tuning(c.h, ctypes.byref(t))
    yield c
    c.close()


def _reference_chain(node, shapes):
    """(nodes, extra initializers) of the reference operators one node of the
    fused graph stands for; `shapes` maps tensor names to their shapes."""
    a = node.attrs
    f = lambda v: np.asarray(v, np.float32)
    extra, nodes = {}, []
    tag = node.outputs[0]
    if node.op not in ("Conv", "OhipConvInstanceNorm"):
        return [node], extra
    x = node.inputs[0]
    conv_lists = dict(a.int_lists)
    mode = a.strings.get("pad_mode")
    if mode and mode != "constant":
        pt, pl, pb, pr = conv_lists.pop("pads")
        extra[tag + ".pads"] = f([0, 0, pt, pl, 0, 0, pb, pr])
        nodes.append(ep.Node("Pad", [x, tag + ".pads"], [tag + ".xp"], A(strings={"mode": mode})))
        x = tag + ".xp"
    conv_ints = {k: v for k, v in a.ints.items() if k == "group"}
    last = tag + ".conv"
    nodes.append(ep.Node("Conv", [x] + list(node.inputs[1:3]), [last], A(ints=conv_ints, int_lists=conv_lists)))
    if node.op == "Conv":
        act = a.strings.get("activation")
        if act == "leaky_relu":
            nodes.append(ep.Node("LeakyRelu", [last], [tag + ".act"],
                                 A(floats={"alpha": a.floats.get("activation_alpha", 0.01)})))
            last = tag + ".act"
        elif act == "relu":
            nodes.append(ep.Node("Relu", [last], [tag + ".act"]))
            last = tag + ".act"
        elif act:
            raise NotImplementedError(act)
    else:
        nodes.append(ep.Node("OxiInstanceNorm", [last], [tag + ".norm"],
                             A(floats={"epsilon": a.floats.get("epsilon", 1e-5)})))
        last = tag + ".norm"
        if len(node.inputs) > 4 and node.inputs[3]:
            n_img, s = shapes[node.inputs[3]]
            c = shapes[node.inputs[1]][0]
            for part, key, src in (("g", "scale_offset", node.inputs[3]), ("b", "bias_offset", node.inputs[4])):
                o = a.ints.get(key, 0)
                extra[tag + part + ".st"], extra[tag + part + ".en"] = f([o]), f([o + c])
                extra[tag + part + ".ax"], extra[tag + part + ".sh"] = f([1]), f([n_img, c, 1, 1])
                nodes.append(ep.Node("Slice", [src, tag + part + ".st", tag + part + ".en", tag + part + ".ax"],
                                     [tag + part + ".sl"]))
                nodes.append(ep.Node("Reshape", [tag + part + ".sl", tag + part + ".sh"], [tag + part + ".4d"]))
            nodes.append(ep.Node("Mul", [last, tag + "g.4d"], [tag + ".mul"]))
            nodes.append(ep.Node("Add", [tag + ".mul", tag + "b.4d"], [tag + ".aff"]))
            last = tag + ".aff"
        if a.strings.get("norm_activation") == "relu":
            nodes.append(ep.Node("Relu", [last], [tag + ".relu"]))
            last = tag + ".relu"
        if len(node.inputs) > 5 and node.inputs[5]:
            nodes.append(ep.Node("Add", [last, node.inputs[5]], [tag + ".res"]))
            last = tag + ".res"
    nodes[-1].outputs = [node.outputs[0]]
    return nodes, extra


def _ulps(got, ref):
    """f16 distance in units in the last place (ordered bit patterns)."""
    def key(v):
        b = np.asarray(v, np.float16).view(np.int16).astype(np.int32)
        return np.where(b < 0, -(b & 0x7FFF), b)
    return np.abs(key(got) - key(ref))


def _node_by_node(ctx, g, feeds):
    """Runs the fused f16 graph on the device with every node's output kept,
    then each node through the oracle on the device's inputs; returns
    (fused graph, device values, per-node stats)."""
    fused = fuse(g)
    outs = [o for n in fused.nodes for o in n.outputs]
    probe = Graph(fused.nodes, fused.initializers, fused.inputs, outs)
    dev = Session(probe, ctx, optimize=False).run(feeds)
    vals = {**{k: np.asarray(v) for k, v in feeds.items()}, **dev}
    shapes = {k: np.shape(v) for k, v in vals.items()}
    shapes.update({k: np.shape(np.asarray(getattr(v, "data", v))) for k, v in fused.initializers.items()})
    stats = []
    for n in fused.nodes:
        chain, extra = _reference_chain(n, shapes)
        ins = [t for t in n.inputs if t and t not in fused.initializers]
        mini = Graph(chain, {**fused.initializers, **extra}, ins, [n.outputs[0]])
        ref = G.run_graph(mini, {t: vals[t] for t in ins}, half=True)[n.outputs[0]]
        got = np.asarray(vals[n.outputs[0]], np.float32)
        assert got.shape == ref.shape, (n.op, n.outputs[0], got.shape, ref.shape)
        u = _ulps(got, ref)
        scale = float(np.abs(ref).max())
        stats.append({"node": n.outputs[0], "op": n.op, "rel": float(np.abs(got - ref).max()) / scale,
                      "max_ulp": int(u.max()), "exact": float(np.mean(u == 0)), "within1": float(np.mean(u <= 1))})
    return fused, vals, stats


def test_face_swap_f16_node_by_node(ctx):
    """Every node of the device's f16 forward, given the device's inputs for
    it, is within 1e-2 of its output magnitude of the oracle, at least 99.5 %
    of its elements are bit-identical to the oracle's and 99.9 % within one
    f16 ulp.  What differs is a sum that lands near an f16 rounding boundary
    and rounds the other way (the f32 sums of the conv and the norm's
    statistics run in another order); a rounding point placed differently
    (a fused activation applied before the conversion where the reference
    converts first) would show as a large share of one-ulp differences."""
    g, feeds = workloads.face_swap_generator(dtype="f16")
    _, _, stats = _node_by_node(ctx, g, feeds)
    for s in stats:
        print(f"{s['op']:22s} {s['node']:16s} rel {s['rel']:.2e} max_ulp {s['max_ulp']:3d} "
              f"exact {s['exact']:.5f} <=1ulp {s['within1']:.5f}")
    for s in stats:
        assert s["rel"] <= 1e-2, s
        assert s["exact"] >= 0.995, s
        assert s["within1"] >= 0.999, s


def _torch_order_conv_half(x_bits, w_bits, b_bits=None, bf16=False, activation=None, act_min=float("-inf"),
                           act_max=float("inf"), strides=None, pads=None, dilations=None, group=1, nthreads=None):
    """conv_half with the f32 convolution summed by torch (CPU float32) in
    place of the oracle's sgemm: the same arithmetic (f16 operands, f32
    accumulation, one rounding to f16), another summation order."""
    import torch
    from oracle import oracle as O
    assert activation is None
    t = lambda v: torch.from_numpy(O.half_bits_to_f32(v, bf16))
    pt, pl, pb, pr = pads or (0, 0, 0, 0)
    x = torch.nn.functional.pad(t(x_bits), (pl, pr, pt, pb))
    y = torch.nn.functional.conv2d(x, t(w_bits), None if b_bits is None else t(b_bits),
                                   stride=tuple(strides or (1, 1)), dilation=tuple(dilations or (1, 1)), groups=group)
    return O.f32_to_half_bits(y.numpy(), bf16)


def test_face_swap_f16_graph_output_error(ctx, monkeypatch):
    """The logits against the oracle's f16 forward are within 1e-2 of
    max |logits|.  The graph output y = Tanh(logits) is held to what a
    second correct CPU forward reaches: the oracle with its convolutions'
    f32 sums taken in torch's order instead of its sgemm's.  Summation order
    alone moves y by about 2e-2 of max |y| (the six residual blocks'
    instance norms amplify one-ulp flips), so no implementation that does
    not reproduce the reference's sgemm order bit for bit -- the oracle
    included -- is within 1e-2 of max |y| of the reference; the device is
    required to be no further from the oracle than that second forward."""
    from oracle import oracle as O
    g, feeds = workloads.face_swap_generator(dtype="f16")
    out = Session(g, ctx).run(feeds)
    ref = G.run_graph(g, feeds, half=True)
    monkeypatch.setattr(O, "conv_half", _torch_order_conv_half)
    alt = G.run_graph(g, feeds, half=True)
    rel = lambda a, b: float(np.abs(np.asarray(a, np.float32) - b).max()) / float(np.abs(b).max())
    dev = {k: rel(out[k], ref[k]) for k in ("logits", "y")}
    order = {k: rel(alt[k], ref[k]) for k in ("logits", "y")}
    print("f16 graph outputs, error as a fraction of max |oracle|: device", dev, "summation order only", order)
    assert dev["logits"] <= 1e-2, dev
    assert order["y"] > 1e-2, order    # the premise: the bar on y is out of reach of any other order
    assert dev["y"] <= order["y"], (dev, order)
