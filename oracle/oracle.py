"""CPU oracle for the OxiONNX dense-contraction hot path (ctypes wrapper).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker or as the CPU baseline -- never as a product path.

The functions mirror the reference CPU operators (cool-japan/oxionnx v0.1.7):

* ``matmul_integer`` / ``qlinear_matmul`` --
  oxionnx-ops/src/registry/quant_ops/qlinear_matmul.rs:174-254
* ``conv_integer`` / ``qlinear_conv`` --
  oxionnx-ops/src/registry/quant_ops/qlinear_conv.rs:34-203 and
  conv_kernel.rs:134-254
* ``conv`` -- oxionnx-ops/src/registry/conv_ops/conv.rs:26-227 over
  conv/conv2d.rs:246-547
* ``conv_half`` -- oxionnx-ops/src/conv_typed.rs:54-153
* ``gemm`` (f32) -- math_typed.rs:759-788 + math/matmul.rs:138-190
* ``gemm_half`` -- math_typed.rs:589-686
* ``matmul`` (f32) -- math_typed.rs:334-423

Parity status of each function is recorded in tests/test_oracle.py, which
pins them against the reference's golden vectors and closed forms.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

I64 = ctypes.c_int64
I32P = ctypes.POINTER(ctypes.c_int32)


def build():
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        L = _lib
        L.orc_round_ties_even_f64.restype = ctypes.c_double
        L.orc_round_ties_even_f64.argtypes = [ctypes.c_double]
        L.orc_requantize.restype = ctypes.c_float
        L.orc_requantize.argtypes = [I64, ctypes.c_float, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.orc_conv_out_dim.restype = I64
        L.orc_conv_out_dim.argtypes = [I64] * 6
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_hardware_threads.restype = ctypes.c_int
        L.orc_conv_transpose2d_f32.argtypes = [ctypes.c_void_p, I64, I64, I64, I64, ctypes.c_void_p, I64, I64, I64,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p, I64, I64, I64, ctypes.c_void_p]
        L.orc_gemm_half.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, I64, I64, I64,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                    ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, I64, I64]
        L.orc_gemm_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, I64, I64, I64, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_void_p,
                                   I64, I64, ctypes.c_void_p, ctypes.c_int]
        L.orc_conv2d_f32.restype = ctypes.c_int
        L.orc_conv2d_f32.argtypes = [ctypes.c_void_p, I64, I64, I64, I64, ctypes.c_void_p, I64, I64,
                                     I64, I64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, I64, I64, I64, ctypes.c_void_p, ctypes.c_int]
        L.orc_apply_activation.argtypes = [ctypes.c_void_p, I64, ctypes.c_int, ctypes.c_float,
                                           ctypes.c_float]
        L.orc_integer_matmul.restype = ctypes.c_int
        L.orc_integer_matmul.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int, ctypes.c_void_p, ctypes.c_int, I64,
                                         ctypes.c_int, ctypes.c_int, I64, I64, I64, ctypes.c_void_p]
        L.orc_qlinear_requant.argtypes = [ctypes.c_void_p, I64, ctypes.c_float, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
        L.orc_integer_conv2d.restype = ctypes.c_int
        L.orc_integer_conv2d.argtypes = [ctypes.c_void_p, I64, I64, I64, I64, ctypes.c_void_p, I64,
                                         I64, I64, I64, ctypes.c_int32, ctypes.c_void_p,
                                         ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p, I64, I64, I64,
                                         ctypes.c_void_p]
        L.orc_qlinear_conv_requant.argtypes = [ctypes.c_void_p, I64, I64, I64, ctypes.c_float,
                                               ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
                                               ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                               ctypes.c_void_p]
        L.orc_satrange_infer.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_resolve_pads2d.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 6
        L.orc_unary_f32.argtypes = [ctypes.c_void_p, I64, ctypes.c_int, ctypes.c_float]
        L.orc_instance_norm_f32.argtypes = [ctypes.c_void_p, I64, I64, ctypes.c_float]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _i64(v):
    return np.ascontiguousarray(np.asarray(v, dtype=np.int64))


def hardware_threads():
    return lib().orc_hardware_threads()


def round_ties_even(v):
    return lib().orc_round_ties_even_f64(float(v))


# ---------------------------------------------------------------- quant ops
def _lanes(v):
    """zero_point_lanes (quant_ops/mod.rs:121-127): absent/empty -> [0]."""
    if v is None:
        return np.zeros(1, np.int32)
    a = np.asarray(v).reshape(-1)
    if a.size == 0:
        return np.zeros(1, np.int32)
    return np.ascontiguousarray(np.rint(a.astype(np.float64)).astype(np.int32))


def satrange_infer(y_zp, x_zp):
    y, x = _lanes(y_zp), _lanes(x_zp)
    lo, hi = np.zeros(1, np.int32), np.zeros(1, np.int32)
    lib().orc_satrange_infer(_p(y), y.size, _p(x), x.size, _p(lo), _p(hi))
    return int(lo[0]), int(hi[0])


def range_for_dtype(dtype):
    """SatRange::for_dtype (quant_ops/mod.rs:215-221)."""
    dt = np.dtype(dtype)
    if dt == np.uint8:
        return (0, 255)
    if dt == np.int8:
        return (-128, 127)
    return None


def _mm_shapes(a_shape, b_shape):
    """resolve_shapes (qlinear_matmul.rs:30-90)."""
    a1, b1 = len(a_shape) == 1, len(b_shape) == 1
    ad = [1, a_shape[0]] if a1 else list(a_shape)
    bd = [b_shape[0], 1] if b1 else list(b_shape)
    m, k, kb, n = ad[-2], ad[-1], bd[-2], bd[-1]
    if k != kb:
        raise ValueError(f"inner dimensions disagree: {k} vs {kb}")
    ba = int(np.prod(ad[:-2])) if len(ad) > 2 else 1
    bb = int(np.prod(bd[:-2])) if len(bd) > 2 else 1
    if ba == bb:
        batch = ba
    elif ba == 1:
        batch = bb
    elif bb == 1:
        batch = ba
    else:
        raise ValueError("batch dimensions disagree")
    prefix = ad[:-2] if ba >= bb else bd[:-2]
    out = list(prefix) + ([] if a1 else [m]) + ([] if b1 else [n])
    return batch, m, k, n, out, (ba == 1 and batch != 1), (bb == 1 and batch != 1)


def integer_matmul(a, b, a_zp=None, b_zp=None):
    a = np.asarray(a)
    b = np.asarray(b)
    batch, m, k, n, out_shape, abc, bbc = _mm_shapes(a.shape, b.shape)
    az, bz = _lanes(a_zp), _lanes(b_zp)
    if az.size not in (1, m):
        raise ValueError(f"a_zero_point has {az.size} entries, expected 1 (per tensor) or {m}")
    if bz.size not in (1, n):
        raise ValueError(f"b_zero_point has {bz.size} entries, expected 1 (per tensor) or {n}")
    ai = np.ascontiguousarray(a.astype(np.int32))
    bi = np.ascontiguousarray(b.astype(np.int32))
    acc = np.zeros(batch * m * n, np.int64)
    lib().orc_integer_matmul(_p(ai), _p(bi), _p(az), az.size, _p(bz), bz.size, batch, int(abc),
                             int(bbc), m, k, n, _p(acc))
    return acc, out_shape


def matmul_integer(a, b, a_zp=None, b_zp=None):
    """MatMulIntegerOp::execute (qlinear_matmul.rs:174-199) -> int32 values."""
    acc, shape = integer_matmul(a, b, a_zp, b_zp)
    return np.clip(acc, -2**31, 2**31 - 1).astype(np.int32).reshape(shape)


def _scale(v):
    """scale_input (quant_ops/mod.rs:100-118): first element, finite, non-zero."""
    s = float(np.asarray(v, dtype=np.float32).reshape(-1)[0])
    if not np.isfinite(s):
        raise ValueError("scale must be finite")
    if s == 0.0:
        raise ValueError("scale is zero")
    return np.float32(s)


def qlinear_matmul(a, a_scale, a_zp, b, b_scale, b_zp, y_scale, y_zp, sat_range=None):
    """QLinearMatMulOp::run (qlinear_matmul.rs:220-254).  Only b_scale[0] is
    read, exactly like the reference's scale_input."""
    acc, shape = integer_matmul(a, b, a_zp, b_zp)
    ylanes = _lanes(y_zp)
    lo, hi = sat_range if sat_range is not None else satrange_infer(ylanes, _lanes(a_zp))
    combined = np.float32(np.float32(_scale(a_scale) * _scale(b_scale)) / _scale(y_scale))
    out = np.zeros(acc.size, np.float32)
    lib().orc_qlinear_requant(_p(acc), acc.size, float(combined), int(ylanes[0]), lo, hi, _p(out))
    return out.reshape(shape)


def conv_geometry(x_shape, w_shape, strides=None, pads=None, dilations=None, group=1,
                  auto_pad="NOTSET"):
    """ConvGeometry::from_attrs (registry/conv_ops/conv.rs:38-121), rank 2."""
    strides = list(strides) if strides else [1, 1]
    dilations = list(dilations) if dilations else [1, 1]
    pads = list(pads) if pads else [0, 0, 0, 0]
    if w_shape[1] * group != x_shape[1]:
        raise ValueError("input channels != weight input channels * group")
    if w_shape[0] % group:
        raise ValueError("output channels not divisible by group")
    mode = {"NOTSET": 0, "VALID": 1, "SAME_UPPER": 2, "SAME_LOWER": 3}[auto_pad]
    out_p = np.zeros(4, np.int64)
    lib().orc_resolve_pads2d(mode, _p(_i64(x_shape[2:])), _p(_i64(w_shape[2:])), _p(_i64(strides)),
                             _p(_i64(dilations)), _p(_i64(pads)), _p(out_p))
    pads = [int(v) for v in out_p]
    oh = lib().orc_conv_out_dim(x_shape[2], pads[0], pads[2], w_shape[2], dilations[0], strides[0])
    ow = lib().orc_conv_out_dim(x_shape[3], pads[1], pads[3], w_shape[3], dilations[1], strides[1])
    if oh < 0 or ow < 0:
        raise ValueError("padded input extent is smaller than the dilated kernel extent")
    return strides, pads, dilations, [x_shape[0], w_shape[0], oh, ow]


def _convt_natural(in_dim, stride, out_pad, k, d):
    """conv_transpose_natural_dim (conv/spatial.rs:370-407)."""
    return stride * (in_dim - 1) + out_pad + (k - 1) * d + 1


def conv_transpose_geometry(x_shape, w_shape, strides=None, pads=None, dilations=None, group=1,
                            output_padding=None, output_shape=None, auto_pad="NOTSET"):
    """ConvTransposeGeometry::from_attrs (registry/conv_ops/conv.rs:349-470) with
    derive_transpose_pads (:519-554) and read_output_shape_attr (:490-515),
    rank 2.  W is [C_in, C_out/group, kH, kW]."""
    strides = list(strides) if strides else [1, 1]
    dilations = list(dilations) if dilations else [1, 1]
    out_pad = list(output_padding) if output_padding else [0, 0]
    if x_shape[1] != w_shape[0]:
        raise ValueError("ConvTranspose: input channels != weight input channels")
    if x_shape[1] % group:
        raise ValueError("ConvTranspose: input channels not divisible by group")
    target = None
    if output_shape:
        target = list(output_shape[-2:]) if len(output_shape) in (2, 4) else None
        if target is None or min(target) < 1:
            raise ValueError("ConvTranspose: output_shape")
    elif auto_pad in ("SAME_UPPER", "SAME_LOWER"):
        target = [x_shape[2 + a] * strides[a] for a in range(2)]
    if target is None:
        pads = [0, 0, 0, 0] if auto_pad == "VALID" else (list(pads) if pads else [0, 0, 0, 0])
    else:
        pads = [0, 0, 0, 0]
        for a in range(2):
            nat = _convt_natural(x_shape[2 + a], strides[a], out_pad[a], w_shape[2 + a], dilations[a])
            total = nat - target[a]
            if total < 0:
                raise ValueError("ConvTranspose: output_shape exceeds the un-cropped extent")
            half = total // 2
            begin, end = (half, total - half) if auto_pad == "SAME_UPPER" else (total - half, half)
            pads[a], pads[a + 2] = begin, end
    out = [x_shape[0], w_shape[1] * group]
    for a in range(2):
        nat = _convt_natural(x_shape[2 + a], strides[a], out_pad[a], w_shape[2 + a], dilations[a])
        if nat - pads[a] - pads[a + 2] < 0:
            raise ValueError("ConvTranspose: pads exceed the un-cropped output extent")
        out.append(nat - pads[a] - pads[a + 2])
    return strides, pads, dilations, out


def conv_transpose(x, w, b=None, **attrs):
    """ConvTransposeOp::execute for rank 2, f32 (registry/conv_ops/conv.rs:561-582,
    conv/transpose.rs:78-309)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    group = attrs.get("group", 1)
    s, p, d, out_shape = conv_transpose_geometry(x.shape, w.shape, attrs.get("strides"), attrs.get("pads"),
                                                 attrs.get("dilations"), group, attrs.get("output_padding"),
                                                 attrs.get("output_shape"), attrs.get("auto_pad", "NOTSET"))
    out = np.zeros(out_shape, np.float32)
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    rc = lib().orc_conv_transpose2d_f32(_p(x), *x.shape, _p(w), w.shape[1], w.shape[2], w.shape[3],
                                        None if bb is None else _p(bb), _p(_i64(s)), _p(_i64(p)),
                                        _p(_i64(d)), group, out_shape[2], out_shape[3], _p(out))
    if rc:
        raise ValueError("ConvTranspose: bad arguments")
    return out


def conv_transpose_half(x_bits, w_bits, b_bits=None, bf16=False, **attrs):
    """conv_transpose_f16 / _bf16 (conv_typed.rs:159-222): promote, f32 scatter,
    round the result back (RNE)."""
    xf = half_bits_to_f32(x_bits, bf16)
    wf = half_bits_to_f32(w_bits, bf16)
    bf = None if b_bits is None else half_bits_to_f32(b_bits, bf16)
    return f32_to_half_bits(conv_transpose(xf, wf, bf, **attrs), bf16)


def integer_conv(x, w, x_zp=0, w_zp=None, bias=None, **attrs):
    x = np.asarray(x)
    w = np.asarray(w)
    group = attrs.get("group", 1)
    s, p, d, out_shape = conv_geometry(x.shape, w.shape, attrs.get("strides"), attrs.get("pads"),
                                       attrs.get("dilations"), group,
                                       attrs.get("auto_pad", "NOTSET"))
    wz = _lanes(w_zp)
    xi = np.ascontiguousarray(x.astype(np.int32))
    wi = np.ascontiguousarray(w.astype(np.int32))
    bi = None if bias is None else np.ascontiguousarray(np.asarray(bias).astype(np.int32))
    acc = np.zeros(int(np.prod(out_shape)), np.int64)
    rc = lib().orc_integer_conv2d(_p(xi), *x.shape, _p(wi), w.shape[0], w.shape[1], w.shape[2],
                                  w.shape[3], int(x_zp), _p(wz), wz.size, _p(bi), _p(_i64(s)),
                                  _p(_i64(p)), _p(_i64(d)), group, out_shape[2], out_shape[3],
                                  _p(acc))
    if rc:
        raise ValueError("w_zero_point has the wrong length")
    return acc, out_shape


def conv_integer(x, w, x_zp=None, w_zp=None, **attrs):
    """ConvIntegerOp::execute (qlinear_conv.rs:173-203)."""
    acc, shape = integer_conv(x, w, int(_lanes(x_zp)[0]), w_zp, None, **attrs)
    return np.clip(acc, -2**31, 2**31 - 1).astype(np.int32).reshape(shape)


def qlinear_conv(x, x_scale, x_zp, w, w_scale, w_zp, y_scale, y_zp, bias=None, sat_range=None,
                 **attrs):
    """QLinearConvOp::run (qlinear_conv.rs:34-103)."""
    xz = int(_lanes(x_zp)[0])
    ylanes = _lanes(y_zp)
    acc, shape = integer_conv(x, w, xz, w_zp, bias, **attrs)
    ws = np.ascontiguousarray(np.asarray(w_scale, np.float32).reshape(-1))
    if ws.size > 1 and ws.size != shape[1]:
        raise ValueError("w_scale has the wrong length")
    lo, hi = sat_range if sat_range is not None else satrange_infer(ylanes, [xz])
    out = np.zeros(acc.size, np.float32)
    lib().orc_qlinear_conv_requant(_p(acc), shape[0], shape[1], shape[2] * shape[3],
                                   float(_scale(x_scale)), _p(ws), ws.size,
                                   float(_scale(y_scale)), int(ylanes[0]), lo, hi, _p(out))
    return out.reshape(shape)


# ---------------------------------------------------------------- float ops
ACT = {None: 0, "": 0, "relu": 1, "clip": 2}


def apply_activation(y, activation=None, lo=float("-inf"), hi=float("inf")):
    y = np.ascontiguousarray(y, np.float32)
    lib().orc_apply_activation(_p(y), y.size, ACT[activation], lo, hi)
    return y


def conv(x, w, b=None, activation=None, act_min=float("-inf"), act_max=float("inf"),
         nthreads=None, **attrs):
    """ConvOp::execute (registry/conv_ops/conv.rs:163-189) for rank 2, f32."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    group = attrs.get("group", 1)
    s, p, d, out_shape = conv_geometry(x.shape, w.shape, attrs.get("strides"), attrs.get("pads"),
                                       attrs.get("dilations"), group,
                                       attrs.get("auto_pad", "NOTSET"))
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    out = np.zeros(out_shape, np.float32)
    nt = nthreads or hardware_threads()
    lib().orc_conv2d_f32(_p(x), *x.shape, _p(w), *w.shape, _p(bb), _p(_i64(s)), _p(_i64(p)),
                         _p(_i64(d)), group, out_shape[2], out_shape[3], _p(out), nt)
    return apply_activation(out, activation, act_min, act_max).reshape(out_shape)


def f32_to_half_bits(x, bf16=False):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.shape, np.uint16)
    fn = lib().orc_f32_to_bf16_n if bf16 else lib().orc_f32_to_f16_n
    fn(_p(x), _p(out), ctypes.c_int64(x.size))
    return out


def half_bits_to_f32(h, bf16=False):
    h = np.ascontiguousarray(h, np.uint16)
    out = np.zeros(h.shape, np.float32)
    fn = lib().orc_bf16_to_f32_n if bf16 else lib().orc_f16_to_f32_n
    fn(_p(h), _p(out), ctypes.c_int64(h.size))
    return out


def conv_half(x_bits, w_bits, b_bits=None, bf16=False, activation=None,
              act_min=float("-inf"), act_max=float("inf"), **attrs):
    """conv_f16 / conv_bf16 (conv_typed.rs:54-153): promote, f32 conv,
    activation, round back."""
    xf = half_bits_to_f32(x_bits, bf16)
    wf = half_bits_to_f32(w_bits, bf16)
    bf = None if b_bits is None else half_bits_to_f32(b_bits, bf16)
    y = conv(xf, wf, bf, activation, act_min, act_max, **attrs)
    return f32_to_half_bits(y, bf16)


def _c_kind(c, m, n):
    if c is None:
        return 0
    c = np.asarray(c)
    if c.ndim == 0:
        return 1
    if c.shape == (n,):
        return 2
    if c.shape == (m, n):
        return 3
    raise ValueError("unsupported bias shape")


def gemm_half(a_bits, b_bits, c_bits=None, alpha=1.0, beta=1.0, trans_a=0, trans_b=0,
              bf16=False, rows=None):
    """gemm_f16 / gemm_bf16 (math_typed.rs:589-686); rows=(r0, r1) evaluates a
    row band only (used to bound the CPU baseline)."""
    a = np.ascontiguousarray(a_bits, np.uint16)
    b = np.ascontiguousarray(b_bits, np.uint16)
    m, k = (a.shape[1], a.shape[0]) if trans_a else a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    ck = _c_kind(c_bits, m, n)
    c = None if c_bits is None else np.ascontiguousarray(np.asarray(c_bits, np.uint16).reshape(-1))
    out = np.zeros((m, n), np.uint16)
    r0, r1 = rows if rows else (0, m)
    lib().orc_gemm_half(int(bf16), _p(a), _p(b), m, k, n, int(trans_a), int(trans_b),
                        float(alpha), float(beta), _p(c), ck, _p(out), r0, r1)
    return out


def typed_matmul_batch_info(a_shape, b_shape):
    """typed_matmul_batch_info (math_typed.rs:85-115): the output batch is the
    numpy broadcast of the batch prefixes; a_batches / b_batches are the
    products of each operand's own prefix."""
    if len(a_shape) < 2 or len(b_shape) < 2 or a_shape[-1] != b_shape[-2]:
        raise ValueError("typed matmul: shapes")
    out_batch = list(np.broadcast_shapes(tuple(a_shape[:-2]), tuple(b_shape[:-2])))
    batch = int(np.prod(out_batch)) if out_batch else 1
    a_batches = int(np.prod(a_shape[:-2])) if len(a_shape) > 2 else 1
    b_batches = int(np.prod(b_shape[:-2])) if len(b_shape) > 2 else 1
    return batch, a_batches, b_batches, out_batch + [a_shape[-2], b_shape[-1]]


def matmul_batched(a, b):
    """matmul_f32_into (math_typed.rs:334-423): slice s is A slice s % a_batches
    times B slice s % b_batches; each slice in float64 (the reference's sgemm
    is pinned at tolerance)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    batch, na, nb, shape = typed_matmul_batch_info(a.shape, b.shape)
    a3 = a.reshape(na, a.shape[-2], a.shape[-1]).astype(np.float64)
    b3 = b.reshape(nb, b.shape[-2], b.shape[-1]).astype(np.float64)
    out = np.stack([a3[s % na] @ b3[s % nb] for s in range(batch)])
    return out.reshape(shape)


def matmul_batched_half(a_bits, b_bits, bf16=False):
    """matmul_f16 / matmul_bf16 (math_typed.rs:147-189, 258-317): the same slice
    rule, each slice the per-element ascending-p f32 loop rounded once (RNE),
    which is gemm_half with alpha 1 and no C."""
    a = np.asarray(a_bits, np.uint16)
    b = np.asarray(b_bits, np.uint16)
    batch, na, nb, shape = typed_matmul_batch_info(a.shape, b.shape)
    a3 = a.reshape(na, a.shape[-2], a.shape[-1])
    b3 = b.reshape(nb, b.shape[-2], b.shape[-1])
    out = np.stack([gemm_half(a3[s % na], b3[s % nb], None, bf16=bf16) for s in range(batch)])
    return out.reshape(shape)


def gemm(a, b, c=None, alpha=1.0, beta=1.0, trans_a=0, trans_b=0, nthreads=1):
    """gemm_f32 (math_typed.rs:759-788); single-threaded like the reference's
    2-D sgemm (matrixmultiply threading off, Cargo.toml:43)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = (a.shape[1], a.shape[0]) if trans_a else a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    out = np.zeros((m, n), np.float32)
    cc, cr, ccol = None, 0, 0
    if c is not None:
        cc = np.asarray(c, np.float32)
        shp = list(cc.shape)
        while len(shp) < 2:
            shp = [1] + shp
        cr, ccol = shp[-2], shp[-1]
        cc = np.ascontiguousarray(np.broadcast_to(cc.reshape(cr, ccol), (cr, ccol)))
    lib().orc_gemm_f32(_p(a), _p(b), m, k, n, int(trans_a), int(trans_b), float(alpha),
                       float(beta), _p(cc), cr, ccol, _p(out), nthreads)
    return out


def matmul(a, b, nthreads=1):
    """2-D matmul_f32_into (math_typed.rs:334-423)."""
    return gemm(a, b, nthreads=nthreads)
