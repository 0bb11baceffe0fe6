"""A sequential run loop over the provider, in the shape of the reference
session's ``run_sequential_inner`` (src/session/run/sequential.rs:614-665)
with every node offered to ``try_hip_dispatch_resident`` and activations kept
resident between nodes (``RunActivations``, src/session/gpu_activations.rs:102-431:
an activation is released after its last consumer).

A node the provider cannot claim (no device arm, or a decline at dispatch
time) runs on the caller's CPU operators, ``cpu_ops(node, inputs)``, the way
the reference session falls back to its own operators
(src/session/run/sequential.rs:886-932, ``materialize_resident_cuda_inputs``):
a resident operand is read back once per run and the host copy memoized for
every later CPU consumer, and a host value is uploaded once for its device
consumers.  This package has no CPU operators of its own; with no
``cpu_ops`` such a node raises ``NodeDeclined`` naming it and the provider's
reason.

``optimize`` applies node fusions before the run, in the manner of the
reference's optimizer passes (src/optimizer/fusion/mod.rs):
  * Conv followed by its only consumer Relu / LeakyRelu becomes one Conv with
    the ``activation`` attribute (the reference's Conv+Relu fusion contract,
    registry/conv_ops/conv.rs:124-156; LeakyRelu is this provider's addition);
  * QLinearConv -> DequantizeLinear -> Silu -> QuantizeLinear, each the only
    consumer of the previous, becomes one QLinearConv whose requantised bytes
    pass through a 256-entry table that reproduces the three nodes exactly;
  * a reflect / edge Pad consumed only by an unpadded Conv becomes the Conv's
    pads with ``pad_mode`` (applied while the input is staged);
  * OxiInstanceNorm -> Mul(gamma) -> Add(beta) [-> Relu], where gamma and beta
    are Reshape(Slice(style)) column ranges of one style tensor (AdaIN),
    becomes one OxiInstanceNorm that reads the modulation from the style rows.
  * DequantizeLinear(A), DequantizeLinear(B) -> Add -> QuantizeLinear, each
    the only consumer of the previous (the dequantised residual sum of a
    quantised network), becomes one QLinearAdd node (the ONNX contrib
    operator's inputs) that the provider runs as the same steps in one pass.
Nodes left without consumers are dropped.
"""
import ctypes
from dataclasses import dataclass, field, replace
from typing import Dict, List

import numpy as np

from . import _lib as L
from . import ep


class NodeDeclined(RuntimeError):
    """The provider declined a node that this run loop cannot run elsewhere."""


@dataclass
class Graph:
    nodes: List[ep.Node]
    initializers: Dict[str, object]
    inputs: List[str]
    outputs: List[str]
    name: str = "graph"
    notes: Dict[str, object] = field(default_factory=dict)


def _consumers(nodes):
    cons = {}
    for i, n in enumerate(nodes):
        for t in n.inputs:
            if t:
                cons.setdefault(t, []).append(i)
    return cons


def _scalar(inits, name):
    v = inits.get(name)
    if v is None:
        return None
    a = np.asarray(v.data if isinstance(v, ep.Typed) else v).reshape(-1)
    return float(a[0]) if a.size == 1 else None


def fuse(graph: Graph, level: str = "all", nhwc: bool = True) -> Graph:
    """level "all": every fusion below; level "reference": only the fusion the
    reference's own optimizer produces for these graphs, Conv followed by its
    only consumer Relu (registry/conv_ops/conv.rs:124-156)."""
    ref_only = level == "reference"
    if ref_only:
        nodes, inits = list(graph.nodes), dict(graph.initializers)
    else:
        nodes, inits = _merge_sibling_gemms(list(graph.nodes), dict(graph.initializers), set(graph.outputs))
    keep_out = set(graph.outputs)
    changed = True
    while changed:
        changed = False
        cons = _consumers(nodes)

        def sole(tensor):
            c = cons.get(tensor, [])
            return c[0] if len(c) == 1 and tensor not in keep_out else None

        for i, n in enumerate(nodes):
            if n is None:
                continue
            if n.op == "Conv" and "activation" not in n.attrs.strings:
                j = sole(n.outputs[0])
                if j is not None and nodes[j].op in (("Relu",) if ref_only else ("Relu", "LeakyRelu")):
                    a = replace(n.attrs, strings=dict(n.attrs.strings), floats=dict(n.attrs.floats))
                    if nodes[j].op == "Relu":
                        a.strings["activation"] = "relu"
                    else:
                        a.strings["activation"] = "leaky_relu"
                        a.floats["activation_alpha"] = nodes[j].attrs.floats.get("alpha", 0.01)
                    nodes[i] = replace(n, attrs=a, outputs=list(nodes[j].outputs))
                    nodes[j] = None
                    changed = True
                    break
            if ref_only:
                continue
            if n.op == "QLinearConv" and "activation" not in n.attrs.strings:
                j = sole(n.outputs[0])
                if j is None or nodes[j].op != "DequantizeLinear":
                    continue
                dq = nodes[j]
                if (_scalar(inits, dq.inputs[1]) != _scalar(inits, n.inputs[6]) or
                        _scalar(inits, dq.inputs[2] if len(dq.inputs) > 2 else "") !=
                        _scalar(inits, n.inputs[7] if len(n.inputs) > 7 else "")):
                    continue
                k = sole(dq.outputs[0])
                if k is None or nodes[k].op != "Silu":
                    continue
                q = sole(nodes[k].outputs[0])
                if q is None or nodes[q].op != "QuantizeLinear":
                    continue
                qn = nodes[q]
                ys = _scalar(inits, qn.inputs[1])
                yz = _scalar(inits, qn.inputs[2]) if len(qn.inputs) > 2 and qn.inputs[2] else 0.0
                if ys is None or yz is None:
                    continue
                a = replace(n.attrs, strings=dict(n.attrs.strings), floats=dict(n.attrs.floats),
                            ints=dict(n.attrs.ints))
                a.strings["activation"] = "silu"
                a.floats["activation_y_scale"] = ys
                if len(qn.inputs) > 2 and qn.inputs[2]:
                    a.ints["activation_y_zero_point"] = int(yz)
                nodes[i] = replace(n, attrs=a, outputs=list(qn.outputs))
                nodes[j] = nodes[k] = nodes[q] = None
                changed = True
                break
            if n.op == "Pad" and n.attrs.strings.get("mode", "constant") in ("reflect", "edge"):
                if _fuse_pad_into_conv(nodes, i, sole, inits):
                    changed = True
                    break
            if n.op == "Add" and _fuse_qadd(nodes, i, sole, cons):
                changed = True
                break
            if n.op == "OxiInstanceNorm" and len([t for t in n.inputs if t]) == 1:
                if _fuse_adain(nodes, i, sole, inits):
                    changed = True
                    break
        nodes = [n for n in nodes if n is not None] if changed else nodes
    if not ref_only:
        nodes = _fuse_conv_instnorm(nodes, keep_out, inits)
        if nhwc:
            nodes = _plan_nhwc(_drop_dead(nodes, keep_out), keep_out, inits)
    return replace(graph, nodes=_drop_dead(nodes, keep_out), initializers=inits)


def _nhwc_reader(node, inits):
    """A conv the device runs on a resident NHWC input in place: ungrouped,
    an f32 / f16 filter, and either zero padding (the engine's implicit
    im2col reads NHWC as it is) or a fused reflect / edge Pad that a loader
    applies: the halo-patch geometry (3x3, stride and dilation 1) or the
    few-output MFMA kernel (f16, at most 4 output channels, square 5x5 /
    7x7).  The dispatcher checks dtypes, extents and sizes and converts
    otherwise."""
    if node.op not in ("Conv", "OhipConvInstanceNorm"):
        return False
    a = node.attrs
    if a.ints.get("group", 1) != 1:
        return False
    w = inits.get(node.inputs[1]) if len(node.inputs) > 1 else None
    if w is None:
        return False
    wd = np.asarray(w.data if isinstance(w, ep.Typed) else w)
    if wd.ndim != 4 or wd.dtype not in (np.float16, np.float32):
        return False
    if a.strings.get("pad_mode", "constant") in ("constant", ""):
        return True
    unit = (all(v == 1 for v in a.int_lists.get("strides", [1, 1]))
            and all(v == 1 for v in a.int_lists.get("dilations", [1, 1])))
    # the halo-patch path (3x3), or the few-output kernel (an RGB head)
    return unit and (wd.shape[2:] == (3, 3) or (wd.dtype == np.float16 and wd.shape[0] <= 4
                                                and wd.shape[2] == wd.shape[3] and wd.shape[2] in (5, 7)))


def _plan_nhwc(nodes, keep_out, inits):
    """Layout hints for float activations: a Conv / OhipConvInstanceNorm
    output whose every consumer reads it in place as NHWC (the input of an
    ungrouped conv with zero padding or on the halo path, the residual of a
    fused node that has the same shape, or a nearest Resize that is itself
    hinted) is produced NHWC ("out_nhwc"), which removes the consumers' NCHW
    -> NHWC staging; a nearest Resize (4-D, scales on H and W only) is
    hinted when every consumer of its output reads NHWC, and then resizes
    NHWC -> NHWC.  Nodes are visited from the end, so a consumer's hint is
    known when its producer is decided.  The dispatcher treats the hints as
    preferences and converts for any consumer that cannot take the layout."""
    cons = _consumers(nodes)
    out = list(nodes)

    def reads_nhwc(un, t):
        if un.inputs and un.inputs[0] == t and _nhwc_reader(un, inits) and t not in un.inputs[1:5]:
            return True
        if un.op == "OhipConvInstanceNorm" and len(un.inputs) > 5 and un.inputs[5] == t and un.inputs[0] != t:
            return True
        return un.op == "Resize" and un.inputs and un.inputs[0] == t and un.attrs.ints.get("out_nhwc") == 1

    for i in range(len(out) - 1, -1, -1):
        n = out[i]
        if n.op == "Resize":
            if n.attrs.strings.get("mode") != "nearest" or "axes" in n.attrs.int_lists:
                continue
        elif n.op not in ("Conv", "OhipConvInstanceNorm") or n.attrs.ints.get("group", 1) != 1:
            continue
        elif n.op == "OhipConvInstanceNorm" and len(n.inputs) > 5 and n.inputs[5] in inits:
            # an initializer residual broadcasts (a [1, C, 1, 1] shift); the
            # binary kernel that adds it after the fused pair reads NCHW
            continue
        t = n.outputs[0]
        users = cons.get(t, [])
        if t in keep_out or not users:
            continue
        if all(reads_nhwc(out[u], t) for u in users):
            a = replace(n.attrs, ints=dict(n.attrs.ints))
            a.ints["out_nhwc"] = 1
            out[i] = replace(n, attrs=a)
    return out


def _fuse_conv_instnorm(nodes, keep_out, inits):
    """Conv (ungrouped, no activation) whose only consumer is an
    OxiInstanceNorm (plain, or the fused AdaIN form above): one
    OhipConvInstanceNorm node, inputs [x, W, B or '', gamma rows, beta rows
    (or '', ''), residual], the Conv's attributes plus the norm's epsilon,
    modulation offsets and activation (as "norm_activation"); a two-input
    Add that is the norm's only consumer becomes the residual.  Runs after
    the other fusions so the AdaIN tail is already folded into the norm."""
    cons = _consumers(nodes)
    out = list(nodes)
    for i, n in enumerate(out):
        if n is None or n.op != "Conv" or "activation" in n.attrs.strings or n.attrs.ints.get("group", 1) != 1:
            continue
        c = cons.get(n.outputs[0], [])
        if len(c) != 1 or n.outputs[0] in keep_out:
            continue
        norm = out[c[0]]
        if norm is None or norm.op != "OxiInstanceNorm":
            continue
        w = inits.get(n.inputs[1]) if len(n.inputs) > 1 else None
        if w is None or np.asarray(w.data if isinstance(w, ep.Typed) else w).dtype not in (np.float32, np.float16):
            continue   # the fused kernels cover f32 / f16
        extra = [t for t in norm.inputs[1:] if t]
        if extra and len(extra) != 2:
            continue
        a = replace(n.attrs, strings=dict(n.attrs.strings), floats=dict(n.attrs.floats), ints=dict(n.attrs.ints))
        a.floats["epsilon"] = norm.attrs.floats.get("epsilon", 1e-5)
        for key in ("scale_offset", "bias_offset"):
            if key in norm.attrs.ints:
                a.ints[key] = norm.attrs.ints[key]
        if "activation" in norm.attrs.strings:
            a.strings["norm_activation"] = norm.attrs.strings["activation"]
        ins = list(n.inputs) + [""] * (3 - len(n.inputs))
        ins += extra if extra else ["", ""]
        outs, pos = list(norm.outputs), c[0]
        # a residual Add as the norm's only consumer folds in as input 5
        r = cons.get(norm.outputs[0], [])
        if len(r) == 1 and norm.outputs[0] not in keep_out and out[r[0]] is not None and out[r[0]].op == "Add":
            add = out[r[0]]
            if len(add.inputs) == 2 and add.inputs.count(norm.outputs[0]) == 1:
                ins.append(add.inputs[1] if add.inputs[0] == norm.outputs[0] else add.inputs[0])
                outs, pos = list(add.outputs), r[0]
                out[r[0]] = None
        if len(ins) == 5 and not extra:
            ins = ins[:3]
        # at the last folded node's position: the modulation rows and the
        # residual may be produced after the conv
        out[pos] = replace(n, op="OhipConvInstanceNorm", inputs=ins, outputs=outs, attrs=a)
        if pos != c[0]:
            out[c[0]] = None
        out[i] = None
    return [n for n in out if n is not None]


def _init_array(inits, name):
    v = inits.get(name) if name else None
    if v is None or isinstance(v, ep.Typed):
        return None
    return np.asarray(v)


def _merge_sibling_gemms(nodes, inits, keep_out):
    """Gemm nodes that read the same A with initializer B / C (same transB,
    alpha, beta, K and dtype, no fused attribute) become one Gemm over the
    concatenated weights; each former output is a column range of the merged
    one.  Column Slices of a former output are re-pointed at the merged
    output with shifted bounds (on a single-row output the provider serves
    them as views, so the merge costs no copy); any other use gets a Slice
    node.  One launch replaces several skinny ones (the per-block style Gemms
    of a style-modulated generator all read one latent row)."""
    groups = {}
    for i, n in enumerate(nodes):
        if n.op != "Gemm" or len(n.inputs) != 3 or n.attrs.strings or n.attrs.ints.get("transA", 0):
            continue
        b, c = _init_array(inits, n.inputs[1]), _init_array(inits, n.inputs[2])
        if b is None or c is None or b.ndim != 2 or c.ndim != 1 or b.dtype != c.dtype:
            continue
        tb = n.attrs.ints.get("transB", 0)
        k, nn = (b.shape[1], b.shape[0]) if tb else b.shape
        if c.shape[0] != nn:
            continue
        key = (n.inputs[0], tb, n.attrs.floats.get("alpha", 1.0), n.attrs.floats.get("beta", 1.0), str(b.dtype), k)
        groups.setdefault(key, []).append(i)
    cons = _consumers(nodes)
    inserted = {}
    for key, members in groups.items():
        if len(members) < 2:
            continue
        tb = key[1]
        first = nodes[members[0]]
        bs = [_init_array(inits, nodes[m].inputs[1]) for m in members]
        cs = [_init_array(inits, nodes[m].inputs[2]) for m in members]
        wname, bname, out = first.name + "_mB", first.name + "_mC", first.outputs[0] + "_merged"
        inits[wname] = np.concatenate(bs, axis=0 if tb else 1)
        inits[bname] = np.concatenate(cs)
        merged = ep.Node("Gemm", [first.inputs[0], wname, bname], [out], replace(first.attrs), name=first.name + "_merged")
        extra = []
        off = 0
        for m, c in zip(members, cs):
            o, width = nodes[m].outputs[0], c.shape[0]
            users = cons.get(o, [])
            movable = o not in keep_out and all(_column_slice(nodes[u], o, inits) is not None for u in users)
            if movable:
                for u in users:
                    lo, hi = _column_slice(nodes[u], o, inits)
                    lo, hi = max(0, min(lo, width)), max(0, min(hi, width))
                    sn, en = nodes[u].name + "_ms", nodes[u].name + "_me"
                    inits[sn], inits[en] = np.asarray([off + lo], np.float32), np.asarray([off + max(lo, hi)], np.float32)
                    nodes[u] = replace(nodes[u], inputs=[out, sn, en] + list(nodes[u].inputs[3:]))
            else:
                sn, en, ax = o + "_ms", o + "_me", o + "_max"
                inits[sn], inits[en], inits[ax] = (np.asarray([off], np.float32), np.asarray([off + width], np.float32),
                                                   np.asarray([1], np.float32))
                extra.append(ep.Node("Slice", [out, sn, en, ax], [o], name=o + "_view"))
            off += width
        nodes[members[0]] = merged
        inserted[members[0]] = extra
        for m in members[1:]:
            nodes[m] = None
    result = []
    for i, n in enumerate(nodes):
        if n is not None:
            result.append(n)
            result.extend(inserted.get(i, []))
    return result, inits


def _column_slice(node, tensor, inits):
    """(start, end) of a unit-step Slice of `tensor` along axis 1 (or -1) of
    a matrix, normalised against nothing yet (negative bounds excluded)."""
    if node.op != "Slice" or len(node.inputs) < 4 or node.inputs[0] != tensor:
        return None
    st, en, ax = _ints(inits, node.inputs[1]), _ints(inits, node.inputs[2]), _ints(inits, node.inputs[3])
    if not st or not en or ax not in ([1], [-1]) or len(st) != 1 or len(en) != 1 or st[0] < 0 or en[0] < 0:
        return None
    if node.inputs[4:] and node.inputs[4] and _ints(inits, node.inputs[4]) != [1]:
        return None
    return st[0], en[0]


def _fuse_qadd(nodes, i, sole, cons):
    """Add(DequantizeLinear(a), DequantizeLinear(b)) -> QuantizeLinear as one
    QLinearAdd [a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp]."""
    add = nodes[i]
    if len(add.inputs) != 2:
        return False
    producers = {}
    for j, m in enumerate(nodes):
        if m is not None:
            for o in m.outputs:
                producers[o] = j
    deqs = []
    for t in add.inputs:
        j = producers.get(t)
        if j is None or nodes[j].op != "DequantizeLinear" or sole(t) != i or len(nodes[j].inputs) < 2:
            return False
        deqs.append(j)
    if deqs[0] == deqs[1]:
        return False
    q = sole(add.outputs[0])
    if q is None or nodes[q].op != "QuantizeLinear" or len(nodes[q].inputs) < 2:
        return False

    def three(m):
        ins = list(m.inputs) + [""] * (3 - len(m.inputs))
        return ins[:3]

    inputs = three(nodes[deqs[0]]) + three(nodes[deqs[1]]) + three(nodes[q])[1:]
    nodes[i] = ep.Node("QLinearAdd", inputs, list(nodes[q].outputs), name=add.name)
    nodes[deqs[0]] = nodes[deqs[1]] = nodes[q] = None
    return True


def _drop_dead(nodes, keep):
    """Removes nodes none of whose outputs is consumed or a graph output."""
    while True:
        used = {t for n in nodes for t in n.inputs if t}
        live = [n for n in nodes if any(o in used or o in keep for o in n.outputs)]
        if len(live) == len(nodes):
            return nodes
        nodes = live


def _ints(inits, name):
    v = inits.get(name)
    if v is None:
        return None
    return [int(x) for x in np.asarray(v.data if isinstance(v, ep.Typed) else v).reshape(-1)]


def _fuse_pad_into_conv(nodes, i, sole, inits):
    """Pad(reflect | edge) on H / W only, consumed only by an unpadded Conv:
    the Conv takes the pads with pad_mode, and its input staging applies them."""
    pad = nodes[i]
    j = sole(pad.outputs[0])
    if j is None or nodes[j].op != "Conv" or nodes[j].inputs[0] != pad.outputs[0]:
        return False
    conv = nodes[j]
    p = _ints(inits, pad.inputs[1]) if len(pad.inputs) > 1 and pad.inputs[1] else pad.attrs.int_lists.get("pads")
    if p is None or len(p) != 8 or p[0] or p[1] or p[4] or p[5] or min(p) < 0:
        return False
    if any(conv.attrs.int_lists.get("pads", [0, 0, 0, 0])) or conv.attrs.strings.get("auto_pad", "NOTSET") not in ("NOTSET", ""):
        return False
    if conv.attrs.ints.get("group", 1) != 1 or "pad_mode" in conv.attrs.strings:
        return False
    a = replace(conv.attrs, strings=dict(conv.attrs.strings), int_lists=dict(conv.attrs.int_lists))
    a.int_lists["pads"] = [p[2], p[3], p[6], p[7]]
    a.strings["pad_mode"] = pad.attrs.strings.get("mode")
    nodes[j] = replace(conv, inputs=[pad.inputs[0]] + list(conv.inputs[1:]), attrs=a)
    nodes[i] = None
    return True


def _modulation(nodes, producer, inits, tensor):
    """tensor = Reshape(Slice(S, [a], [b], [1]), [N, b - a, 1, 1]) -> (S, a), else None."""
    r = producer.get(tensor)
    if r is None or nodes[r] is None or nodes[r].op != "Reshape":
        return None
    sl = producer.get(nodes[r].inputs[0])
    if sl is None or nodes[sl] is None or nodes[sl].op != "Slice" or len(nodes[sl].inputs) < 4:
        return None
    s = nodes[sl]
    st, en, ax = _ints(inits, s.inputs[1]), _ints(inits, s.inputs[2]), _ints(inits, s.inputs[3])
    shp = _ints(inits, nodes[r].inputs[1])
    if not st or not en or ax != [1] or len(st) != 1 or len(en) != 1 or st[0] < 0 or en[0] <= st[0]:
        return None
    if s.inputs[4:] and s.inputs[4] and _ints(inits, s.inputs[4]) != [1]:
        return None
    if shp is None or len(shp) != 4 or shp[1] != en[0] - st[0] or shp[2] != 1 or shp[3] != 1:
        return None
    return s.inputs[0], st[0]


def _fuse_adain(nodes, i, sole, inits):
    """OxiInstanceNorm -> Mul(gamma) -> Add(beta) [-> Relu], gamma / beta being
    Reshape(Slice(style)) column ranges of one style tensor: one
    OxiInstanceNorm reading the modulation straight from the style rows."""
    producer = {o: k for k, nd in enumerate(nodes) if nd is not None for o in nd.outputs}
    norm = nodes[i]
    j = sole(norm.outputs[0])
    if j is None or nodes[j].op != "Mul":
        return False
    mul = nodes[j]
    g = mul.inputs[1] if mul.inputs[0] == norm.outputs[0] else mul.inputs[0]
    k = sole(mul.outputs[0])
    if k is None or nodes[k].op != "Add":
        return False
    add = nodes[k]
    b = add.inputs[1] if add.inputs[0] == mul.outputs[0] else add.inputs[0]
    gm, bm = _modulation(nodes, producer, inits, g), _modulation(nodes, producer, inits, b)
    if gm is None or bm is None or gm[0] != bm[0]:
        return False
    last, act = k, None
    r = sole(add.outputs[0])
    if r is not None and nodes[r].op == "Relu":
        last, act = r, "relu"
    a = replace(norm.attrs, strings=dict(norm.attrs.strings), ints=dict(norm.attrs.ints))
    a.ints["scale_offset"], a.ints["bias_offset"] = gm[1], bm[1]
    if act:
        a.strings["activation"] = act
    nodes[i] = replace(norm, inputs=[norm.inputs[0], gm[0], bm[0]], outputs=list(nodes[last].outputs), attrs=a)
    for idx in {j, k, last}:
        nodes[idx] = None
    return True


class Session:
    """Runs a Graph on one HipContext with resident activations."""

    def __init__(self, graph: Graph, ctx: ep.HipContext, optimize=True, cpu_ops=None, nhwc=True):
        """optimize: True (every fusion), "reference" (only the reference
        optimizer's Conv + Relu) or False; nhwc: with every fusion, the NHWC
        layout hints for float activations (False keeps them NCHW).  cpu_ops(node, inputs) -> list of
        host arrays: the host's operators for nodes the provider does not
        claim (inputs are host arrays, initializers included; '' slots are
        None)."""
        self.cpu_ops = cpu_ops
        if optimize == "reference":
            self.graph = fuse(graph, level="reference")
        else:
            self.graph = fuse(graph, nhwc=nhwc) if optimize else graph
        self.ctx = ctx
        outs = set(self.graph.outputs)
        self.last_use = {}
        for i, n in enumerate(self.graph.nodes):
            for t in n.inputs:
                if t and t not in self.graph.initializers:
                    self.last_use[t] = i
        for o in outs:
            self.last_use[o] = len(self.graph.nodes)
        self.prepared = [ep.PreparedNode(n, self.graph.initializers) for n in self.graph.nodes]
        # planned CPU islands: ops with no device arm (is_supported_op, lib.rs:217)
        self.cpu_planned = [not ep.is_supported_op(n.op) for n in self.graph.nodes]
        # per node: the activations whose last consumer it is
        self.release = [[t for t in dict.fromkeys(n.inputs) if t and self.last_use.get(t) == i]
                        for i, n in enumerate(self.graph.nodes)]

    def _host_value(self, acts, host, name):
        """The host copy of a run value: read back once and memoized."""
        if name in host:
            return host[name]
        v = acts[name]
        if isinstance(v, ep.DeviceTensor):
            v = v.to_host(self.ctx)
        host[name] = v
        return v

    def _run_on_cpu(self, i, acts, host, reason):
        n = self.graph.nodes[i]
        if self.cpu_ops is None:
            raise NodeDeclined(f"{n.op} node '{n.name}': {reason}")
        inits = self.graph.initializers
        ins = []
        for t in n.inputs:
            if not t:
                ins.append(None)
            elif t in inits:
                v = inits[t]
                ins.append(np.asarray(v.data if isinstance(v, ep.Typed) else v))
            else:
                ins.append(self._host_value(acts, host, t))
        outs = self.cpu_ops(n, ins)
        for name, v in zip(n.outputs, outs):
            acts[name] = np.ascontiguousarray(v)
            host[name] = acts[name]

    def _forward(self, acts, keep, capturing=False):
        """Dispatches every node; frees each activation after its last
        consumer unless it is in `keep`.  Values produced on the host (CPU
        islands) are uploaded once for their device consumers."""
        host = {}
        for i, pn in enumerate(self.prepared):
            n = pn.node
            if self.cpu_planned[i]:
                if capturing:
                    raise NodeDeclined(f"{n.op} node '{n.name}': a CPU island cannot be captured")
                self._run_on_cpu(i, acts, host, "no device arm for this op")
            else:
                for _, t in pn.dynamic:
                    if not isinstance(acts[t], ep.DeviceTensor):
                        acts[t] = ep.DeviceTensor.from_host(self.ctx, acts[t])
                res = pn.dispatch_resident(acts, self.ctx)
                if res is None:
                    reason = self.ctx.last_decline()
                    if capturing:
                        raise NodeDeclined(f"{n.op} node '{n.name}': {reason}")
                    self._run_on_cpu(i, acts, host, reason)
                else:
                    acts[n.outputs[0]] = res
            for t in self.release[i]:
                if t in acts and t not in keep:
                    v = acts.pop(t)
                    host.pop(t, None)
                    if isinstance(v, ep.DeviceTensor):
                        v.free()
        # graph outputs leave in the ONNX layout (resident convolution
        # outputs are NHWC inside the forward)
        for o in self.graph.outputs:
            t = acts.get(o)
            if isinstance(t, ep.DeviceTensor) and t not in keep:
                c = t.to_nchw(self.ctx)
                if c is not t:
                    t.free()
                    acts[o] = c

    def run(self, feeds: Dict[str, np.ndarray], keep_device: bool = False):
        acts = {}
        try:
            # graph inputs stay host values until a device node consumes them
            for name in self.graph.inputs:
                acts[name] = np.ascontiguousarray(feeds[name])
            self._forward(acts, ())
            if keep_device:
                out = {}
                for o in self.graph.outputs:
                    v = acts.pop(o)
                    out[o] = v if isinstance(v, ep.DeviceTensor) else ep.DeviceTensor.from_host(self.ctx, v)
            else:
                out = {o: (acts[o].to_host(self.ctx) if isinstance(acts[o], ep.DeviceTensor) else acts[o])
                       for o in self.graph.outputs}
            return out
        finally:
            for t in acts.values():
                if isinstance(t, ep.DeviceTensor):
                    t.free()

    def capture(self, feeds: Dict[str, np.ndarray]) -> "CapturedForward":
        """Records one forward into a HIP graph (the reference's CUDA-graph
        cache, oxionnx-cuda/src/graph_cache.rs).  Two eager forwards warm the
        caches; a dry run with parked buffers leaves every buffer the forward
        needs in the pool; the captured forward then owns its buffers."""
        lib = L.lib()
        self.run(feeds)
        self.run(feeds)
        L.check(lib.ohip_pool_parking(self.ctx.h, 1))
        try:
            self.run(feeds)
        finally:
            L.check(lib.ohip_pool_parking(self.ctx.h, 0))
        inputs = {n: ep.DeviceTensor.from_host(self.ctx, np.ascontiguousarray(feeds[n])) for n in self.graph.inputs}
        L.check(lib.ohip_sync(self.ctx.h))
        acts = dict(inputs)
        L.check(lib.ohip_graph_begin(self.ctx.h))
        try:
            self._forward(acts, set(inputs), capturing=True)
        except BaseException:
            g = ctypes.c_void_p()
            if lib.ohip_graph_end(self.ctx.h, ctypes.byref(g)) == L.OK:
                lib.ohip_graph_destroy(g)
            raise
        g = ctypes.c_void_p()
        L.check(lib.ohip_graph_end(self.ctx.h, ctypes.byref(g)))
        outputs = {o: acts.pop(o) for o in self.graph.outputs}
        for t in acts.values():
            if t not in inputs.values():
                t.free()
        return CapturedForward(self.ctx, g, inputs, outputs)


class CapturedForward:
    """A replayable forward: refill the captured inputs, launch, read the
    captured outputs."""

    def __init__(self, ctx, graph, inputs, outputs):
        self.ctx, self.g, self.inputs, self.outputs = ctx, graph, inputs, outputs

    def replay(self, feeds, download: bool = True):
        """feeds None: the captured inputs keep their device contents."""
        lib = L.lib()
        for name, t in (self.inputs.items() if feeds is not None else ()):
            arr = np.ascontiguousarray(feeds[name])
            L.check(lib.ohip_dtensor_upload(self.ctx.h, t.h, arr.ctypes.data_as(ctypes.c_void_p)))
        L.check(lib.ohip_graph_launch(self.g))
        if not download:
            return None
        return {o: t.to_host(self.ctx) for o, t in self.outputs.items()}

    def close(self):
        if self.g:
            L.lib().ohip_graph_destroy(self.g)
            self.g = None
        for t in list(self.inputs.values()) + list(self.outputs.values()):
            t.free()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
