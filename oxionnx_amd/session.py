"""A sequential run loop over the provider, in the shape of the reference
session's ``run_sequential_inner`` (src/session/run/sequential.rs:614-665)
with every node offered to ``try_hip_dispatch_resident`` and activations kept
resident between nodes (``RunActivations``, src/session/gpu_activations.rs:102-431:
an activation is released after its last consumer).

The reference session runs a declined node on its CPU operator; this package
has no CPU operators, so a decline here raises ``NodeDeclined`` naming the
node and the provider's reason.

``optimize`` applies two node fusions before the run, in the manner of the
reference's optimizer passes (src/optimizer/fusion/mod.rs):
  * Conv followed by its only consumer Relu / LeakyRelu becomes one Conv with
    the ``activation`` attribute (the reference's Conv+Relu fusion contract,
    registry/conv_ops/conv.rs:124-156; LeakyRelu is this provider's addition);
  * QLinearConv -> DequantizeLinear -> Silu -> QuantizeLinear, each the only
    consumer of the previous, becomes one QLinearConv whose requantised bytes
    pass through a 256-entry table that reproduces the three nodes exactly.
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


def fuse(graph: Graph) -> Graph:
    nodes = list(graph.nodes)
    inits = graph.initializers
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
                if j is not None and nodes[j].op in ("Relu", "LeakyRelu"):
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
        nodes = [n for n in nodes if n is not None] if changed else nodes
    return replace(graph, nodes=nodes)


class Session:
    """Runs a Graph on one HipContext with resident activations."""

    def __init__(self, graph: Graph, ctx: ep.HipContext, optimize: bool = True):
        self.graph = fuse(graph) if optimize else graph
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
        # per node: the activations whose last consumer it is
        self.release = [[t for t in dict.fromkeys(n.inputs) if t and self.last_use.get(t) == i]
                        for i, n in enumerate(self.graph.nodes)]

    def _forward(self, acts, keep):
        """Dispatches every node; frees each activation after its last
        consumer unless it is in `keep`."""
        for i, pn in enumerate(self.prepared):
            res = pn.dispatch_resident(acts, self.ctx)
            if res is None:
                n = pn.node
                raise NodeDeclined(f"{n.op} node '{n.name}': {self.ctx.last_decline()}")
            acts[pn.node.outputs[0]] = res
            for t in self.release[i]:
                if t in acts and t not in keep:
                    acts.pop(t).free()

    def run(self, feeds: Dict[str, np.ndarray], keep_device: bool = False):
        acts = {}
        try:
            for name in self.graph.inputs:
                acts[name] = ep.DeviceTensor.from_host(self.ctx, np.ascontiguousarray(feeds[name]))
            self._forward(acts, ())
            if keep_device:
                out = {o: acts.pop(o) for o in self.graph.outputs}
            else:
                out = {o: acts[o].to_host(self.ctx) for o in self.graph.outputs}
            return out
        finally:
            for t in acts.values():
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
            self._forward(acts, set(inputs))
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

    def replay(self, feeds: Dict[str, np.ndarray], download: bool = True):
        lib = L.lib()
        for name, t in self.inputs.items():
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
