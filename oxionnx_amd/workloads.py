"""Synthetic graphs of the two end-to-end workloads (random-init weights,
seeded), built from the reference's node vocabulary (oxionnx_core::Node with
ONNX op types; OxiInstanceNorm is the reference optimizer's fused spatial
normalisation, registry/oxi_instance_norm.rs).

face_swap_generator: an InSwapper-128-style conv encoder-decoder.
    x [1,3,128,128] ~U(0,1), latent [1,512] ~N(0,1).
    stem      Pad(reflect 3) -> Conv 7x7 3->128 -> LeakyRelu(0.2)          @128^2
    down 1/2  Conv 3x3 s2 p1 128->256->512, LeakyRelu(0.2)                  @64^2, @32^2
    6 blocks  2 x [Pad(reflect 1) -> Conv 3x3 512->512 -> OxiInstanceNorm ->
              Mul(gamma) -> Add(beta)] with Relu after the first, + skip Add;
              gamma / beta = Slice + Reshape of Gemm(latent, [512,1024]) (AdaIN)
    up 1/2    Resize(nearest x2) -> Conv 3x3 p1 512->256->128 -> LeakyRelu(0.2)
    final     Pad(reflect 3) -> Conv 7x7 128->3 ("logits") -> Tanh ("y")     @128^2
    Weights ~N(0, 0.02).  41.69 GMAC of convolution.

yolo_backbone_int8: a YOLOv8n-style CSP/C2f backbone in QOperator form.
    x uint8 [1,3,640,640] ~U{0..255}, scale 1/255, zero point 0.
    Conv unit = QLinearConv (per-channel int8 weights ~U{-127..127}, scales
    ~U(0.002, 0.02)) -> DequantizeLinear -> Silu -> QuantizeLinear.
    widths 16-32-64-128-256, 3x3 stride-2 downsamples, C2f blocks
    (1x1 conv, Slice halves, bottlenecks of two 3x3 convs with a
    dequantised residual Add, Concat, 1x1 conv), SPPF (1x1, three 5x5
    MaxPools, Concat, 1x1).  Outputs P3 (80^2), P4 (40^2), P5 (20^2).
    Activation scales are calibrated on a shadow float run of the same
    weights at a reduced input size, so the quantised activations use their
    range.
"""
import math

import numpy as np

from . import ep
from .session import Graph

A = ep.Attributes


def _f32(v):
    return np.asarray(v, np.float32)


# ---------------------------------------------------------------- config 4
def face_swap_generator(seed=4, dtype="f32", n_blocks=6):
    rng = np.random.default_rng(seed)
    inits = {}
    nodes = []
    cnt = [0]

    def name(p):
        cnt[0] += 1
        return f"{p}{cnt[0]}"

    def conv(x, cin, cout, k, stride=1, pad=0, act=None):
        w, b, y = name("W"), name("B"), name("conv")
        inits[w] = rng.normal(0, 0.02, (cout, cin, k, k)).astype(np.float32)
        inits[b] = rng.normal(0, 0.02, cout).astype(np.float32)
        nodes.append(ep.Node("Conv", [x, w, b], [y], A(int_lists={"strides": [stride, stride],
                                                                  "pads": [pad] * 4,
                                                                  "kernel_shape": [k, k]}), name=y))
        if act == "leaky":
            z = name("lrelu")
            nodes.append(ep.Node("LeakyRelu", [y], [z], A(floats={"alpha": 0.2}), name=z))
            return z
        if act == "relu":
            z = name("relu")
            nodes.append(ep.Node("Relu", [y], [z], name=z))
            return z
        if act == "tanh":
            z = name("tanh")
            nodes.append(ep.Node("Tanh", [y], [z], name=z))
            return z
        return y

    def pad(x, p):
        pv, y = name("pads"), name("pad")
        inits[pv] = _f32([0, 0, p, p, 0, 0, p, p])
        nodes.append(ep.Node("Pad", [x, pv], [y], A(strings={"mode": "reflect"}), name=y))
        return y

    def adain(h, c):
        # style = latent @ W + b -> gamma = style[:, :c], beta = style[:, c:]
        w, b, s = name("Wstyle"), name("Bstyle"), name("style")
        inits[w] = rng.normal(0, 0.02, (512, 2 * c)).astype(np.float32)
        inits[b] = (rng.normal(0, 0.02, 2 * c) + np.r_[np.ones(c), np.zeros(c)]).astype(np.float32)
        nodes.append(ep.Node("Gemm", ["latent", w, b], [s], name=s))
        out = []
        for part, (lo, hi) in (("gamma", (0, c)), ("beta", (c, 2 * c))):
            st, en, ax, sl, sh, r = name("st"), name("en"), name("ax"), name(part), name("shape"), name(part + "4d")
            inits[st], inits[en], inits[ax] = _f32([lo]), _f32([hi]), _f32([1])
            inits[sh] = _f32([1, c, 1, 1])
            nodes.append(ep.Node("Slice", [s, st, en, ax], [sl], name=sl))
            nodes.append(ep.Node("Reshape", [sl, sh], [r], name=r))
            out.append(r)
        nrm, mul, add = name("norm"), name("mul"), name("add")
        nodes.append(ep.Node("OxiInstanceNorm", [h], [nrm], A(floats={"epsilon": 1e-5}), name=nrm))
        nodes.append(ep.Node("Mul", [nrm, out[0]], [mul], name=mul))
        nodes.append(ep.Node("Add", [mul, out[1]], [add], name=add))
        return add

    def upsample(x):
        sc, y = name("scales"), name("up")
        inits[sc] = _f32([1, 1, 2, 2])
        nodes.append(ep.Node("Resize", [x, "", sc], [y], A(strings={"mode": "nearest"}), name=y))
        return y

    h = conv(pad("x", 3), 3, 128, 7, act="leaky")
    h = conv(h, 128, 256, 3, stride=2, pad=1, act="leaky")
    h = conv(h, 256, 512, 3, stride=2, pad=1, act="leaky")
    for _ in range(n_blocks):
        r = conv(pad(h, 1), 512, 512, 3)
        r = adain(r, 512)
        rr = name("relu")
        nodes.append(ep.Node("Relu", [r], [rr], name=rr))
        r = conv(pad(rr, 1), 512, 512, 3)
        r = adain(r, 512)
        s = name("skip")
        nodes.append(ep.Node("Add", [h, r], [s], name=s))
        h = s
    h = conv(upsample(h), 512, 256, 3, pad=1, act="leaky")
    h = conv(upsample(h), 256, 128, 3, pad=1, act="leaky")
    y = conv(pad(h, 3), 128, 3, 7, act="tanh")
    nodes[-2].outputs = ["logits"]
    nodes[-1].inputs = ["logits"]
    nodes[-1].outputs = ["y"]
    nodes[-1].name = "y"
    feeds = {"x": rng.uniform(0, 1, (1, 3, 128, 128)).astype(np.float32),
             "latent": rng.normal(0, 1, (1, 512)).astype(np.float32)}
    if dtype == "f16":
        for k, v in list(inits.items()):
            if v.ndim == 4 or k.startswith(("B", "Wstyle", "Bstyle")):
                inits[k] = v.astype(np.float16)
        feeds = {k: v.astype(np.float16) for k, v in feeds.items()}
    g = Graph(nodes, inits, ["x", "latent"], ["y", "logits"], name=f"face_swap_generator_{dtype}")
    g.notes["conv_gmac"] = conv_macs(g, {"x": (1, 3, 128, 128)}) / 1e9
    return g, feeds


def conv_macs(graph, shapes):
    """Multiply-accumulates of the Conv / QLinearConv nodes, by shape
    propagation through the node list."""
    shp = dict(shapes)
    total = 0
    for n in graph.nodes:
        x = shp.get(n.inputs[0])
        if x is None:
            continue
        if n.op in ("Conv", "QLinearConv"):
            w = graph.initializers[n.inputs[1 if n.op == "Conv" else 3]]
            w = np.asarray(w.data if isinstance(w, ep.Typed) else w)
            s = n.attrs.int_lists.get("strides", [1, 1])
            p = n.attrs.int_lists.get("pads", [0, 0, 0, 0])
            oh = (x[2] + p[0] + p[2] - w.shape[2]) // s[0] + 1
            ow = (x[3] + p[1] + p[3] - w.shape[3]) // s[1] + 1
            shp[n.outputs[0]] = (x[0], w.shape[0], oh, ow)
            total += x[0] * w.shape[0] * oh * ow * w.shape[1] * w.shape[2] * w.shape[3]
        elif n.op == "Pad":
            p = np.asarray(graph.initializers[n.inputs[1]]).astype(int)
            shp[n.outputs[0]] = tuple(int(x[i] + p[i] + p[i + 4]) for i in range(4))
        elif n.op == "Resize":
            sc = np.asarray(graph.initializers[n.inputs[2]])
            shp[n.outputs[0]] = tuple(int(math.floor(x[i] * sc[i])) for i in range(4))
        elif n.op == "MaxPool":
            shp[n.outputs[0]] = x
        else:
            shp[n.outputs[0]] = x
    return total


# ---------------------------------------------------------------- config 5
def _conv_f32(x, w, stride, pad):
    """Plain float conv (NCHW, im2col + matmul) for scale calibration."""
    n, c, h, wd = x.shape
    co, ci, kh, kw = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    oh = (h + 2 * pad - kh) // stride + 1
    ow = (wd + 2 * pad - kw) // stride + 1
    cols = np.empty((n, c, kh, kw, oh, ow), np.float32)
    for ky in range(kh):
        for kx in range(kw):
            cols[:, :, ky, kx] = xp[:, :, ky:ky + stride * (oh - 1) + 1:stride, kx:kx + stride * (ow - 1) + 1:stride]
    cols = cols.reshape(n, c * kh * kw, oh * ow)
    return np.einsum("ok,nkp->nop", w.reshape(co, -1), cols).reshape(n, co, oh, ow)


def _quant(v, s, z, lo, hi):
    return np.clip(np.rint(v / np.float32(s)) + z, lo, hi)


def yolo_backbone_int8(seed=5, size=640, calib_size=128):
    """Scales are calibrated on a shadow float run at calib_size: each conv's
    pre-activation scale covers +-3 standard deviations around zero point 128
    (u8), each Silu output (i8, zero point -100) covers [-28, 227] steps up
    to its 99.9th percentile."""
    rng = np.random.default_rng(seed)
    inits = {}
    nodes = []
    cnt = [0]

    def name(p):
        cnt[0] += 1
        return f"{p}{cnt[0]}"

    def qparam(scale, zp, zp_dtype):
        s, z = name("s"), name("zp")
        inits[s] = _f32([scale])
        inits[z] = np.asarray([zp], zp_dtype)
        return s, z

    class Q:
        """A quantised activation: tensor name, parameter names and values,
        and its dequantised shadow at the calibration size."""
        def __init__(self, t, s, z, sv, zv, shadow):
            self.t, self.s, self.z, self.sv, self.zv, self.shadow = t, s, z, sv, zv, shadow

    def conv_unit(x: Q, cout, k, stride=1, out_params=None):
        cin = x.shadow.shape[1]
        w = rng.integers(-127, 128, (cout, cin, k, k)).astype(np.int8)
        ws = rng.uniform(0.002, 0.02, cout).astype(np.float32)
        wn, wsn, wzn = name("W"), name("ws"), name("wzp")
        inits[wn], inits[wsn], inits[wzn] = w, ws, np.zeros(cout, np.int8)
        pre = _conv_f32(x.shadow, w.astype(np.float32) * ws[:, None, None, None], stride, k // 2)
        sigma = float(pre.std()) or 1e-3
        pre_scale = 6.0 * sigma / 255.0
        ps, pz = qparam(pre_scale, 128, np.uint8)
        y = name("qconv")
        nodes.append(ep.Node("QLinearConv", [x.t, x.s, x.z, wn, wsn, wzn, ps, pz], [y],
                             A(int_lists={"strides": [stride, stride], "pads": [k // 2] * 4,
                                          "kernel_shape": [k, k]}), name=y))
        d, si, q = name("dq"), name("silu"), name("q")
        nodes.append(ep.Node("DequantizeLinear", [y, ps, pz], [d], name=d))
        nodes.append(ep.Node("Silu", [d], [si], name=si))
        deq = (_quant(pre, pre_scale, 128, 0, 255) - 128) * np.float32(pre_scale)
        with np.errstate(over="ignore"):
            act = deq / (1 + np.exp(-deq))
        if out_params is None:
            top = float(np.percentile(act, 99.9)) or 1e-3
            sv = top / 227.0
            s, z = qparam(sv, -100, np.int8)
            out_params = (s, z, sv, -100)
        s, z, sv, zv = out_params
        nodes.append(ep.Node("QuantizeLinear", [si, s, z], [q], name=q))
        shadow = (_quant(act, sv, zv, -128, 127) - zv) * np.float32(sv)
        return Q(q, s, z, sv, zv, shadow.astype(np.float32))

    def slice_c(x: Q, lo, hi):
        st, en, ax, y = name("st"), name("en"), name("ax"), name("half")
        inits[st], inits[en], inits[ax] = _f32([lo]), _f32([hi]), _f32([1])
        nodes.append(ep.Node("Slice", [x.t, st, en, ax], [y], name=y))
        return Q(y, x.s, x.z, x.sv, x.zv, x.shadow[:, lo:hi])

    def concat(xs):
        y = name("cat")
        nodes.append(ep.Node("Concat", [v.t for v in xs], [y], A(ints={"axis": 1}), name=y))
        return Q(y, xs[0].s, xs[0].z, xs[0].sv, xs[0].zv, np.concatenate([v.shadow for v in xs], 1))

    def qadd(a: Q, b: Q):
        # the dequantised residual: DequantizeLinear x2 -> Add -> QuantizeLinear
        da, db, s, q = name("dqa"), name("dqb"), name("sum"), name("qsum")
        nodes.append(ep.Node("DequantizeLinear", [a.t, a.s, a.z], [da], name=da))
        nodes.append(ep.Node("DequantizeLinear", [b.t, b.s, b.z], [db], name=db))
        nodes.append(ep.Node("Add", [da, db], [s], name=s))
        nodes.append(ep.Node("QuantizeLinear", [s, a.s, a.z], [q], name=q))
        sh = (_quant(a.shadow + b.shadow, a.sv, a.zv, -128, 127) - a.zv) * np.float32(a.sv)
        return Q(q, a.s, a.z, a.sv, a.zv, sh.astype(np.float32))

    def c2f(x: Q, cout, n, shortcut=True):
        c = cout // 2
        y = conv_unit(x, 2 * c, 1)
        common = (y.s, y.z, y.sv, y.zv)
        parts = [slice_c(y, 0, c), slice_c(y, c, 2 * c)]
        for _ in range(n):
            last = parts[-1]
            h = conv_unit(last, c, 3, out_params=common)
            h = conv_unit(h, c, 3, out_params=common)
            parts.append(qadd(last, h) if shortcut else h)
        return conv_unit(concat(parts), cout, 1)

    def maxpool5(x: Q):
        m = name("pool")
        nodes.append(ep.Node("MaxPool", [x.t], [m], A(int_lists={"kernel_shape": [5, 5], "strides": [1, 1],
                                                                "pads": [2, 2, 2, 2]}), name=m))
        xp = np.pad(x.shadow, ((0, 0), (0, 0), (2, 2), (2, 2)), constant_values=-np.inf)
        h, w = x.shadow.shape[2:]
        sh = np.max(np.stack([xp[:, :, i:i + h, j:j + w] for i in range(5) for j in range(5)]), 0)
        return Q(m, x.s, x.z, x.sv, x.zv, sh)

    def sppf(x: Q, cout):
        y = conv_unit(x, x.shadow.shape[1] // 2, 1)
        outs = [y]
        for _ in range(3):
            outs.append(maxpool5(outs[-1]))
        return conv_unit(concat(outs), cout, 1)

    xs, xz = qparam(1.0 / 255.0, 0, np.uint8)
    xcal = rng.integers(0, 256, (1, 3, calib_size, calib_size)).astype(np.float32) / np.float32(255.0)
    x = Q("x", xs, xz, 1.0 / 255.0, 0, xcal)
    h = conv_unit(x, 16, 3, stride=2)
    h = conv_unit(h, 32, 3, stride=2)
    h = c2f(h, 32, 1)
    h = conv_unit(h, 64, 3, stride=2)
    p3 = c2f(h, 64, 2)
    h = conv_unit(p3, 128, 3, stride=2)
    p4 = c2f(h, 128, 2)
    h = conv_unit(p4, 256, 3, stride=2)
    h = c2f(h, 256, 1)
    p5 = sppf(h, 256)
    rename = {p3.t: "p3", p4.t: "p4", p5.t: "p5"}
    for n in nodes:
        n.outputs = [rename.get(t, t) for t in n.outputs]
        n.inputs = [rename.get(t, t) for t in n.inputs]
    feeds = {"x": rng.integers(0, 256, (1, 3, size, size)).astype(np.uint8)}
    g = Graph(nodes, inits, ["x"], ["p3", "p4", "p5"], name="yolo_backbone_int8")
    g.notes["conv_gmac"] = conv_macs(g, {"x": (1, 3, size, size)}) / 1e9
    return g, feeds
