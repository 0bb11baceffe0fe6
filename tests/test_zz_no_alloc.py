"""ohip_conv2d_noalloc (no device allocation, static per-GPU scratch) against
ohip_conv2d through the C ABI: identical results on two calls in a row, the
second with a smaller input, and no device allocation by either noalloc
call.  The cases use the scratch: an NCHW input (the staging copy) and a
split-K contraction (partial sums)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a GPU"
    return t


@pytest.fixture(scope="module")
def ctx(torch):
    from oxionnx_amd.device import HipContext
    c = HipContext(0)
    yield c
    c.close()


def _case(torch, ctx, dt, xs, ws, pads, seed):
    from oxionnx_amd import _lib as L
    rng = np.random.default_rng(seed)
    tdt = {"f32": torch.float32, "f16": torch.float16}[dt]
    x = torch.from_numpy(rng.uniform(-1, 1, xs).astype(np.float32)).cuda().to(tdt)
    w = rng.normal(0, 0.05, ws).astype(np.float32)
    b = torch.from_numpy(rng.normal(0, 0.01, ws[0]).astype(np.float32)).cuda().to(tdt)
    wt = ctx.weight_conv(w, dtype=L.F32 if dt == "f32" else L.F16)
    return x, wt, b


# (dtype, x shape, w shape, pads, strides).  Every call uses the scratch:
# the f16 calls stage their NCHW input as NHWC (the first also splits K on
# the halo-patch path, a 512 -> 512 3x3 conv at 32x32, 4.8 GFLOP); the f32
# 512 -> 512 conv takes the halo-patch path too (staging + split-K partial
# sums: the f32 NCHW kernel that reads its input in place is used only
# below the halo path's 3 GFLOP), and the second f32 call has stride 2,
# which that in-place kernel does not take, so it stages its input for the
# engine
CALLS = [("f16", (1, 512, 32, 32), (512, 512, 3, 3), (1, 1, 1, 1), (1, 1)),
         ("f16", (1, 64, 20, 24), (96, 64, 3, 3), (1, 1, 1, 1), (1, 1)),
         ("f32", (1, 512, 32, 32), (512, 512, 3, 3), (1, 1, 1, 1), (1, 1)),
         ("f32", (2, 16, 9, 11), (24, 16, 3, 3), (0, 1, 2, 1), (2, 2))]


@pytest.mark.parametrize("pair", [(0, 1), (2, 3)], ids=["f16", "f32"])
def test_noalloc_matches_conv2d_twice(torch, ctx, pair):
    from oxionnx_amd import _lib as L
    for i in pair:
        dt, xs, ws, pads, strides = CALLS[i]
        x, wt, b = _case(torch, ctx, dt, xs, ws, pads, seed=i)
        want = ctx.conv2d(x, wt, b, strides=strides, pads=pads, act=L.ACT_RELU)
        got = torch.full_like(want, float("nan"))
        torch.cuda.synchronize()
        ctx.reset_counters()
        ctx.conv2d(x, wt, b, strides=strides, pads=pads, act=L.ACT_RELU, out=got, noalloc=True)
        torch.cuda.synchronize()
        assert ctx.counters()["device_allocs"] == 0
        assert torch.equal(got, want), (i, float((got.float() - want.float()).abs().max()))


def test_noalloc_rejects_more_scratch_than_the_static_array(torch, ctx):
    from oxionnx_amd import _lib as L
    # an NCHW f16 input of 40 MiB needs an NHWC staging copy larger than
    # 32 MiB (f32 NCHW 1x1 / 3x3 convs read their input in place)
    x = torch.zeros((1, 320, 256, 256), dtype=torch.float16, device="cuda")
    wt = ctx.weight_conv(np.zeros((16, 320, 1, 1), np.float32), dtype=L.F16)
    out = torch.zeros((1, 16, 256, 256), dtype=torch.float16, device="cuda")
    with pytest.raises(L.OhipError) as e:
        ctx.conv2d(x, wt, None, out=out, noalloc=True)
    assert e.value.code == L.E_NOMEM and "static" in str(e.value)
