"""Activation residency through the session run loop, as exact transfer
counts (tests/cuda_activation_residency.rs:22-40 of the reference, its four
claims):

1. an all-claimed chain costs one upload, one download and one fence;
2. a CPU island in the middle costs exactly one extra round trip;
3. a node that declines at dispatch time reads its resident operand back
   exactly once, memoized for a second CPU consumer;
4. steady-state frames allocate no device memory and hand every activation
   back to the pool.

The host's CPU operators (the reference's own, in a real session) are
stood in for by numpy here; every run is also compared element for element
with the same graph run entirely on them.
"""
import math

import numpy as np
import pytest

from oxionnx_amd import ep
from oxionnx_amd.session import Graph, Session

pytestmark = pytest.mark.gpu

N = 65536
B = N * 4


@pytest.fixture(scope="module")
def ctx():
    import torch  # noqa: F401  (HIP runtime initialisation on the test process)
    c = ep.HipContext(0)
    yield c
    c.close()


_erf = np.vectorize(lambda v: np.float32(math.erf(float(v))), otypes=[np.float32])


def cpu_ops(node, ins):
    x = ins[0]
    if node.op == "Relu":
        return [np.maximum(x, np.float32(0))]
    if node.op == "Erf":
        return [_erf(x)]
    if node.op == "Add":
        return [(x + ins[1]).astype(np.float32)]
    if node.op == "Resize":   # the linear mode at unit scales is the identity
        assert node.attrs.strings["mode"] == "linear" and np.all(ins[2] == 1)
        return [x.copy()]
    raise NotImplementedError(node.op)


def all_on_cpu(graph, feeds):
    env = dict(feeds)
    for n in graph.nodes:
        ins = [None if not t else (env[t] if t in env else np.asarray(graph.initializers[t])) for t in n.inputs]
        env[n.outputs[0]] = cpu_ops(n, ins)[0]
    return {o: env[o] for o in graph.outputs}


def node(op, name, ins, outs, **strings):
    return ep.Node(op, ins, outs, ep.Attributes(strings=strings), name=name)


def counted_run(sess, ctx, feeds):
    sess.run(feeds)                 # warm: pool buffers, kernels loaded
    ctx.reset_counters()
    out = sess.run(feeds)
    return out, ctx.counters()


def x_input():
    return np.random.default_rng(5).normal(size=(4, 16, 32, 32)).astype(np.float32)


def test_claimed_chain_costs_one_upload_one_download_one_fence(ctx):
    g = Graph([node("Relu", f"n{i}", [f"h{i - 1}" if i else "x"], [f"h{i}" if i < 4 else "y"]) for i in range(5)],
              {}, ["x"], ["y"])
    sess = Session(g, ctx, optimize=False)
    out, c = counted_run(sess, ctx, {"x": x_input()})
    assert (c["h2d_bytes"], c["d2h_bytes"], c["stream_syncs"]) == (B, B, 1)
    np.testing.assert_array_equal(out["y"], all_on_cpu(g, {"x": x_input()})["y"])


def test_cpu_island_costs_one_extra_round_trip(ctx):
    g = Graph([node("Relu", "n0", ["x"], ["h0"]), node("Relu", "n1", ["h0"], ["h1"]),
               node("Erf", "island", ["h1"], ["h2"]), node("Relu", "n3", ["h2"], ["h3"]),
               node("Relu", "n4", ["h3"], ["y"])], {}, ["x"], ["y"])
    assert not ep.is_supported_op("Erf")
    sess = Session(g, ctx, optimize=False, cpu_ops=cpu_ops)
    out, c = counted_run(sess, ctx, {"x": x_input()})
    # up: the graph input and the island's result; down: h1 for the island and y
    assert (c["h2d_bytes"], c["d2h_bytes"], c["stream_syncs"]) == (2 * B, 2 * B, 2)
    np.testing.assert_array_equal(out["y"], all_on_cpu(g, {"x": x_input()})["y"])
    with pytest.raises(Exception):
        Session(g, ctx, optimize=False).run({"x": x_input()})   # no CPU operators: NodeDeclined


def test_runtime_decline_reads_its_resident_operand_back_once(ctx):
    """Resize in linear mode has a device arm for nearest only, so it declines
    at dispatch with h1 resident; the CPU Erf reading h1 next finds the
    memoized host copy."""
    g = Graph([node("Relu", "n0", ["x"], ["h0"]), node("Relu", "n1", ["h0"], ["h1"]),
               node("Resize", "wide", ["h1", "", "sc"], ["h2"], mode="linear"),
               node("Erf", "island", ["h1"], ["h3"]), node("Add", "join", ["h2", "h3"], ["y"])],
              {"sc": np.ones(4, np.float32)}, ["x"], ["y"])
    assert ep.is_supported_op("Resize")
    sess = Session(g, ctx, optimize=False, cpu_ops=cpu_ops)
    out, c = counted_run(sess, ctx, {"x": x_input()})
    # up: x, h2 and h3 re-entering for the Add; down: h1 once (memoized), y
    assert (c["h2d_bytes"], c["d2h_bytes"], c["stream_syncs"]) == (3 * B, 2 * B, 2)
    assert "nearest" in ctx.last_decline()
    np.testing.assert_array_equal(out["y"], all_on_cpu(g, {"x": x_input()})["y"])


def test_steady_state_frames_allocate_nothing_and_return_every_activation(ctx):
    g = Graph([node("Relu", "n0", ["x"], ["h0"]), node("Relu", "n1", ["h0"], ["h1"]),
               node("Relu", "n2", ["h1"], ["y"])], {}, ["x"], ["y"])
    sess = Session(g, ctx, optimize=False)
    feeds = {"x": x_input()}
    for _ in range(2):
        sess.run(feeds)
    ctx.reset_counters()
    live = ctx.counters()["pool_live"]
    for _ in range(8):
        sess.run(feeds)
        assert ctx.counters()["pool_live"] == live
    c = ctx.counters()
    assert c["device_allocs"] == 0
    assert c["stream_syncs"] == 8
    assert c["h2d_bytes"] == 8 * B and c["d2h_bytes"] == 8 * B
