"""TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's
cpu_baseline leg): a CPU executor that runs a graph node by node with the
restated reference operators, the way the reference session runs a graph
with no accelerator (src/session/run/sequential.rs).

Every tensor is held as the reference holds it: f32 lanes (quantised
tensors as integer-valued f32 lanes).  ``half=True`` models an f16 graph:
every float node reads f16-rounded inputs, computes in f32 and rounds its
output to f16 (conv_typed.rs:54-153 for Conv; the same storage rule for the
other float nodes).

Operators and the reference code each one restates:
  Conv              oracle.conv / conv_half (conv2d.rs im2col + sgemm, conv.rs:26-227)
  Gemm              oracle.gemm / gemm_half (matmul_gemm.rs:135-170, math_typed.rs)
  QLinearConv       oracle.qlinear_conv (qlinear_conv.rs:34-103, conv_kernel.rs)
  LeakyRelu / Tanh / Sigmoid / Silu / Relu   orc_unary_f32 (nn/activations.rs,
                    registry/nn_ops/activations.rs:477)
  OxiInstanceNorm   orc_instance_norm_f32 (registry/oxi_instance_norm.rs:56-65)
  Add / Sub / Mul / Div   numpy broadcasting in f32 (one IEEE operation per element)
  Resize (nearest)  resize.rs:578-622, 712-722 restated below (f32 coordinate maths)
  Pad               ONNX Pad constant / reflect / edge (numpy.pad has the same semantics)
  MaxPool           conv/pooling.rs:166-240 (strictly greater update from -inf)
  Concat / Slice / Reshape   plain numpy indexing
  QuantizeLinear / DequantizeLinear   indexing/quantize.rs:96-190
"""
import math

import numpy as np

from . import oracle as O

_UNARY = {"LeakyRelu": 0, "Tanh": 1, "Sigmoid": 2, "Silu": 3, "Relu": 4}


def _arr(v):
    data = getattr(v, "data", v)
    return np.asarray(data)


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def _nearest_src(j, in_len, out_len, scale, coord, rule):
    x = np.float32(j)
    scale = np.float32(scale)
    if coord == "asymmetric":
        src = x / scale
    elif coord == "align_corners":
        src = np.float32(0) if out_len <= 1 else x * (np.float32(in_len) - 1) / (np.float32(out_len) - 1)
    elif coord == "pytorch_half_pixel":
        src = (x + np.float32(0.5)) / scale - np.float32(0.5) if out_len > 1 else np.float32(0)
    elif coord == "tf_half_pixel_for_nn":
        src = (x + np.float32(0.5)) / scale
    else:
        src = (x + np.float32(0.5)) / scale - np.float32(0.5)
    guard = np.float32(6.0)
    src = np.float32(min(max(src, -guard), np.float32(in_len - 1) + guard))
    if rule == "round_prefer_ceil":
        p = math.floor(np.float32(src + np.float32(0.5)))
    elif rule == "floor":
        p = math.floor(src)
    elif rule == "ceil":
        p = math.ceil(src)
    else:
        p = math.ceil(np.float32(src - np.float32(0.5)))
    return int(min(max(p, 0), in_len - 1))


def _maxpool(x, ks, strides, pads):
    n, c, h, w = x.shape
    oh = (h + pads[0] + pads[2] - ks[0]) // strides[0] + 1
    ow = (w + pads[1] + pads[3] - ks[1]) // strides[1] + 1
    xp = np.full((n, c, h + pads[0] + pads[2], w + pads[1] + pads[3]), -np.inf, np.float32)
    xp[:, :, pads[0]:pads[0] + h, pads[1]:pads[1] + w] = x
    out = np.full((n, c, oh, ow), -np.inf, np.float32)
    for ky in range(ks[0]):
        for kx in range(ks[1]):
            win = xp[:, :, ky:ky + strides[0] * (oh - 1) + 1:strides[0], kx:kx + strides[1] * (ow - 1) + 1:strides[1]]
            out = np.where(win > out, win, out)
    return out


def _quantize(x, scale, zp_arr):
    scale = np.float32(scale)
    if zp_arr is None:
        zp, lo, hi = np.float32(0), 0.0, 255.0
    else:
        zp = np.float32(zp_arr.reshape(-1)[0])
        lo, hi = (0.0, 255.0) if np.any(zp_arr > 127) else (-128.0, 127.0)
    v = np.asarray(x, np.float32) / scale
    r = np.where(np.isfinite(v), np.rint(v), v).astype(np.float32)
    return np.clip(r + zp, lo, hi).astype(np.float32)


def run_graph(graph, feeds, half=False, nthreads=None):
    """Runs every node in order; returns {output name: f32 lanes array}."""
    inits = graph.initializers
    env = {k: np.asarray(v, np.float32) if not half else _f16(v) for k, v in feeds.items()}
    if any(_arr(v).dtype in (np.uint8, np.int8) for v in feeds.values()):
        env = {k: np.asarray(v).astype(np.float32) for k, v in feeds.items()}

    def get(name):
        if name in env:
            return env[name]
        return _arr(inits[name]).astype(np.float32)

    for n in graph.nodes:
        a = n.attrs
        x = get(n.inputs[0]) if n.inputs and n.inputs[0] else None
        op = n.op
        if op == "Conv":
            w = get(n.inputs[1])
            b = get(n.inputs[2]) if len(n.inputs) > 2 and n.inputs[2] else None
            kw = dict(strides=a.int_lists.get("strides"), pads=a.int_lists.get("pads"),
                      dilations=a.int_lists.get("dilations"), group=a.ints.get("group", 1))
            if half:
                yb = O.conv_half(O.f32_to_half_bits(x), O.f32_to_half_bits(w),
                                 None if b is None else O.f32_to_half_bits(b), nthreads=nthreads, **kw)
                y = O.half_bits_to_f32(yb)
            else:
                y = O.conv(x, w, b, nthreads=nthreads, **kw)
        elif op == "Gemm":
            w = get(n.inputs[1])
            c = get(n.inputs[2]) if len(n.inputs) > 2 and n.inputs[2] else None
            if half:
                y = O.half_bits_to_f32(O.gemm_half(O.f32_to_half_bits(x), O.f32_to_half_bits(w),
                                                   None if c is None else O.f32_to_half_bits(c),
                                                   a.floats.get("alpha", 1.0), a.floats.get("beta", 1.0),
                                                   a.ints.get("transA", 0), a.ints.get("transB", 0)))
            else:
                y = O.gemm(x, w, c, a.floats.get("alpha", 1.0), a.floats.get("beta", 1.0),
                           a.ints.get("transA", 0), a.ints.get("transB", 0))
        elif op == "QLinearConv":
            i = n.inputs
            y = O.qlinear_conv(x, _arr(inits[i[1]]), _arr(inits[i[2]]), _arr(inits[i[3]]), _arr(inits[i[4]]),
                               _arr(inits[i[5]]), _arr(inits[i[6]]), _arr(inits[i[7]]),
                               _arr(inits[i[8]]) if len(i) > 8 and i[8] else None,
                               strides=a.int_lists.get("strides"), pads=a.int_lists.get("pads"),
                               dilations=a.int_lists.get("dilations"))
        elif op in _UNARY:
            y = np.array(x, np.float32, copy=True)
            O.lib().orc_unary_f32(y.ctypes.data, y.size, _UNARY[op], float(a.floats.get("alpha", 0.01)))
            if half:
                y = _f16(y)
        elif op == "OxiInstanceNorm":
            y = np.array(x, np.float32, copy=True)
            spatial = int(np.prod(y.shape[2:]))
            O.lib().orc_instance_norm_f32(y.ctypes.data, y.size // spatial, spatial,
                                          float(a.floats.get("epsilon", 1e-5)))
            if half:
                y = _f16(y)
        elif op in ("Add", "Sub", "Mul", "Div"):
            b = get(n.inputs[1])
            y = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide}[op](
                x.astype(np.float32), b.astype(np.float32))
            if half:
                y = _f16(y)
        elif op == "Resize":
            sc = _arr(inits[n.inputs[2]]).astype(np.float32)
            cm = a.strings.get("coordinate_transformation_mode", "half_pixel")
            nm = a.strings.get("nearest_mode", "round_prefer_floor")
            oh = int(math.floor(np.float32(x.shape[2]) * sc[2]))
            ow = int(math.floor(np.float32(x.shape[3]) * sc[3]))
            iy = [_nearest_src(j, x.shape[2], oh, sc[2], cm, nm) for j in range(oh)]
            ix = [_nearest_src(j, x.shape[3], ow, sc[3], cm, nm) for j in range(ow)]
            y = x[:, :, iy][:, :, :, ix]
        elif op == "Pad":
            p = _arr(inits[n.inputs[1]]).astype(np.int64)
            r = x.ndim
            mode = a.strings.get("mode", "constant")
            width = [(int(p[i]), int(p[i + r])) for i in range(r)]
            if mode == "constant":
                cv = float(_arr(inits[n.inputs[2]]).reshape(-1)[0]) if len(n.inputs) > 2 and n.inputs[2] else 0.0
                y = np.pad(x, width, mode="constant", constant_values=cv)
            else:
                y = np.pad(x, width, mode={"reflect": "reflect", "edge": "edge", "wrap": "wrap"}[mode])
        elif op == "MaxPool":
            y = _maxpool(x, a.int_lists["kernel_shape"], a.int_lists.get("strides", [1, 1]),
                         a.int_lists.get("pads", [0, 0, 0, 0]))
        elif op == "Concat":
            y = np.concatenate([get(t) for t in n.inputs], axis=a.ints.get("axis", 0))
        elif op == "Slice":
            st = _arr(inits[n.inputs[1]]).astype(np.int64)
            en = _arr(inits[n.inputs[2]]).astype(np.int64)
            ax = _arr(inits[n.inputs[3]]).astype(np.int64) if len(n.inputs) > 3 else np.arange(len(st))
            sl = [slice(None)] * x.ndim
            for s_, e_, x_ in zip(st, en, ax):
                sl[int(x_)] = slice(int(s_), int(e_))
            y = x[tuple(sl)]
        elif op == "Reshape":
            y = x.reshape([int(v) for v in _arr(inits[n.inputs[1]])])
        elif op == "QuantizeLinear":
            zp = _arr(inits[n.inputs[2]]) if len(n.inputs) > 2 and n.inputs[2] else None
            y = _quantize(x, _arr(inits[n.inputs[1]]).reshape(-1)[0], zp)
        elif op == "DequantizeLinear":
            s = np.float32(_arr(inits[n.inputs[1]]).reshape(-1)[0])
            z = np.float32(_arr(inits[n.inputs[2]]).reshape(-1)[0]) if len(n.inputs) > 2 and n.inputs[2] else 0
            y = (x.astype(np.float32) - np.float32(z)) * s
        else:
            raise NotImplementedError(op)
        env[n.outputs[0]] = np.asarray(y, np.float32)
    return {o: env[o] for o in graph.outputs}
