"""Device-free tests of the dispatch gate (GpuTuning, oxionnx-gpu/src/context/tuning.rs:271-611)
and of the op-support predicates, the pattern of tuning.rs:622-868."""
import ctypes

import pytest

from oxionnx_amd import _lib as L
from oxionnx_amd import ep
from oracle import oracle as O


def tuning(cls):
    t = L.Tuning()
    assert L.lib().ohip_tuning_for_class(cls, ctypes.byref(t)) == 0
    return t


def admits(t, m, k, n, cached):
    return bool(L.lib().ohip_gemm_admits(ctypes.byref(t), m, k, n, int(cached)))


def conv_admits(t, m, k, n):
    return bool(L.lib().ohip_conv_admits(ctypes.byref(t), m, k, n))


def test_legacy_class_reproduces_the_reference_measured_table():
    """tuning.rs:698-748: with the reference's discrete-class numbers the gate
    must reach exactly the reference's measured admit/decline decisions."""
    t = tuning(L.CLASS_LEGACY)
    losses = [(1, 25088, 512), (2, 25088, 512), (8, 25088, 512), (16, 25088, 512), (24, 25088, 512),
              (12, 1024, 1024), (16, 1024, 1024), (24, 1024, 1024), (2, 4096, 4096), (4, 4096, 4096),
              (8, 4096, 4096), (48, 512, 512), (64, 512, 512), (32, 512, 1024), (32, 1024, 512)]
    wins = [(32, 1024, 1024), (32, 2048, 2048), (32, 4096, 4096), (32, 25088, 512), (48, 512, 1024),
            (96, 512, 512), (256, 1024, 1024), (384, 256, 256)]
    for s in losses:
        assert not admits(t, *s, cached=False), s
    for s in wins:
        assert admits(t, *s, cached=False), s


def test_cached_weight_skips_the_intensity_gate():
    """tuning.rs:757-766: ArcFace's head declines uploading, dispatches cached."""
    t = tuning(L.CLASS_LEGACY)
    assert not admits(t, 1, 25088, 512, False)
    assert admits(t, 1, 25088, 512, True)
    assert not admits(t, 1, 512, 2048, True)


def test_intensity_closed_forms():
    """tuning.rs:676-693."""
    gi = L.lib().ohip_gemm_intensity
    assert gi(1, 1 << 20, 1 << 20) == 1
    assert gi(16, 1 << 20, 1 << 20) == 31
    assert gi(1 << 20, 1 << 20, 1) == gi(1, 1 << 20, 1 << 20)
    assert gi(1 << 20, 1, 1 << 20) == gi(1, 1 << 20, 1 << 20)
    assert gi(0, 0, 0) == 0


def test_conv_threshold_and_overflow():
    t = tuning(L.CLASS_LEGACY)
    assert conv_admits(t, 10_000_000, 1, 1)
    assert not conv_admits(t, 9_999_999, 1, 1)
    huge = 1 << 40
    assert not admits(t, huge, huge, huge, True)
    assert not admits(t, huge, huge, huge, False)
    assert not conv_admits(t, huge, huge, huge)
    assert not admits(t, 0, 4096, 4096, False)
    assert not admits(t, 4096, 0, 4096, True)


def test_parity_and_never_presets():
    p = tuning(L.CLASS_PARITY)
    assert admits(p, 1, 1, 1, False) and admits(p, 1, 1, 1, True) and conv_admits(p, 1, 1, 1)
    assert not admits(p, 0, 8, 8, False)
    nv = tuning(L.CLASS_NEVER)
    assert not admits(nv, 4096, 4096, 4096, True)
    assert not admits(nv, 4096, 4096, 4096, False)
    assert not conv_admits(nv, 4096, 4096, 4096)


# The MI355X crossover table (bench.py --only gate on an MI355X box; the
# GPU / CPU ratios are recorded in the measured-table summary of profiles/).
# (m, k, n, upload ratio, cached ratio): > 1 means the GPU lost.
MI355X_GEMM = [
    (1, 128, 128, 5.659, 4.006), (16, 128, 128, 3.987, 2.825), (64, 128, 128, 1.972, 1.269),
    (96, 128, 128, 1.479, 0.966), (128, 128, 128, 1.159, 0.748), (256, 128, 128, 0.664, 0.459),
    (1, 256, 256, 2.906, 1.817), (16, 256, 256, 1.625, 1.057), (24, 256, 256, 1.552, 0.920),
    (32, 256, 256, 1.113, 0.663), (48, 256, 256, 0.883, 0.531), (64, 256, 256, 0.677, 0.411),
    (1, 512, 512, 1.334, 0.488), (4, 512, 512, 1.318, 0.499), (8, 512, 512, 0.862, 0.354),
    (12, 512, 512, 1.056, 0.436), (16, 512, 512, 0.783, 0.326), (64, 512, 512, 0.259, 0.128),
    (1, 1024, 1024, 0.622, 0.123), (16, 1024, 1024, 0.325, 0.089), (1, 4096, 4096, 0.225, 0.004),
    (256, 4096, 4096, 0.025, 0.005), (1, 25088, 512, 0.262, 0.007), (32, 25088, 512, 0.124, 0.012),
]
# (channels, H = W, ratio) of a 3x3 pad-1 conv, implied m*k*n = c*c*9*hw*hw
MI355X_CONV = [(8, 8, 1.489), (8, 16, 1.233), (16, 8, 1.447), (16, 16, 1.012), (8, 32, 0.723),
               (32, 8, 0.223), (16, 32, 0.416), (64, 8, 0.176), (128, 64, 0.069)]


def test_mi355x_class_reproduces_the_measured_table():
    """Every measured loss is declined; every admitted shape measured a win
    (the floors err towards the CPU: some small wins are declined too)."""
    t = tuning(L.CLASS_MI355X)
    for m, k, n, up, cached in MI355X_GEMM:
        if up >= 1:
            assert not admits(t, m, k, n, False), (m, k, n, up)
        if cached >= 1:
            assert not admits(t, m, k, n, True), (m, k, n, cached)
        if admits(t, m, k, n, False):
            assert up < 1, (m, k, n, up)
        if admits(t, m, k, n, True):
            assert cached < 1, (m, k, n, cached)
    for c, hw, r in MI355X_CONV:
        mk = (c, c * 9, hw * hw)
        if r >= 1:
            assert not conv_admits(t, *mk), (c, hw, r)
        if conv_admits(t, *mk):
            assert r < 1, (c, hw, r)
    # the skinny shapes the reference's discrete-GPU gate declines by
    # intensity win on this box, uploading B or not
    assert admits(t, 1, 4096, 4096, False) and admits(t, 1, 25088, 512, False)


def test_mi355x_class_admits_every_configured_workload():
    """The recalibrated MI355X floors claim every configured dense
    contraction and still decline toy shapes."""
    t = tuning(L.CLASS_MI355X)
    assert admits(t, 1, 25088, 512, True)            # config 2a, resident B
    for m, k, n in [(128, 768, 3072), (2048, 4096, 4096), (4096, 4096, 11008)]:
        assert admits(t, m, k, n, True) and admits(t, m, k, n, False)
    assert admits(t, 4096, 768, 3072, True)         # config 3
    assert conv_admits(t, 64, 64 * 9, 128 * 128)    # config 1
    assert conv_admits(t, 16, 3 * 9, 320 * 320)     # config 5 stem
    assert not admits(t, 4, 8, 8, False)
    assert not admits(t, 1, 256, 256, True)
    assert not conv_admits(t, 1, 9, 16)


def test_op_support_predicates():
    # the contraction arms plus the memory-bound arms of the reference CUDA
    # provider's claim list (oxionnx-cuda/src/lib.rs:101-119) that conv
    # networks need between their contractions
    for op in ["Conv", "ConvTranspose", "Gemm", "MatMul", "QLinearMatMul", "MatMulInteger", "QLinearConv",
               "ConvInteger", "Relu", "LeakyRelu", "Tanh", "Sigmoid", "Silu", "Add", "Sub", "Mul", "Div", "OxiInstanceNorm",
               "InstanceNormalization", "Resize", "Pad", "MaxPool", "Concat", "Slice", "Reshape", "Flatten",
               "Squeeze", "Unsqueeze", "QuantizeLinear", "DequantizeLinear", "QLinearAdd"]:
        assert ep.is_supported_op(op), op
    for op in ["Transpose", "Softmax", "LSTM", ""]:
        assert not ep.is_supported_op(op)
    assert ep.accepts_resident_slot("Conv", 0) and not ep.accepts_resident_slot("Conv", 1)
    assert ep.accepts_resident_slot("ConvTranspose", 0) and not ep.accepts_resident_slot("ConvTranspose", 1)
    assert ep.accepts_resident_slot("Gemm", 0) and not ep.accepts_resident_slot("Gemm", 1)
    assert ep.accepts_resident_slot("QLinearConv", 0) and not ep.accepts_resident_slot("QLinearConv", 3)
    assert ep.accepts_resident_slot("QLinearAdd", 0) and ep.accepts_resident_slot("QLinearAdd", 3)
    assert not ep.accepts_resident_slot("QLinearAdd", 1) and not ep.accepts_resident_slot("QLinearAdd", 6)
    assert ep.accepts_resident_slot("Add", 1) and not ep.accepts_resident_slot("Add", 2)
    assert ep.accepts_resident_slot("Concat", 3)
    assert not ep.accepts_resident_slot("QLinearMatMul", 0)
    assert not ep.accepts_resident_slot("Reshape", 1)


def test_try_new_is_gated_by_the_env_flag(monkeypatch):
    monkeypatch.delenv("OXIONNX_HIP", raising=False)
    assert ep.HipContext.try_new() is None
    monkeypatch.setenv("OXIONNX_HIP", "off")
    assert ep.HipContext.try_new() is None
    h = ctypes.c_void_p()
    assert L.lib().ohip_ctx_try_new(ctypes.byref(h)) == L.DECLINED


def test_conv_transpose_extent_matches_the_oracle_geometry():
    """ohip_conv_transpose_out_dim (device-free) against the oracle's
    conv_transpose_geometry, including invalid crops."""
    from oxionnx_amd import _lib as L
    for (i, s, op, k, d, pb, pe) in [(5, 2, 1, 3, 1, 1, 1), (7, 3, 0, 4, 2, 0, 2), (1, 1, 0, 1, 1, 0, 0),
                                     (3, 2, 0, 3, 1, 4, 4)]:
        got = L.lib().ohip_conv_transpose_out_dim(i, s, op, k, d, pb, pe)
        try:
            want = O.conv_transpose_geometry((1, 1, i, i), (1, 1, k, k), [s, s], [pb, pb, pe, pe], [d, d], 1,
                                             [op, op])[3][2]
        except ValueError:
            want = -1
        assert got == want, (i, s, op, k, d, pb, pe)
