"""Device-level Python handle over the C ABI, with torch tensors as device memory.

PyTorch only provides allocation and the stream here; every contraction runs
in libohip.so.  The context adopts torch's current stream so library work and
torch work are ordered without extra synchronisation.
"""
import ctypes

import numpy as np

from . import _lib as L

_TORCH_DT = None


def _torch():
    import torch
    return torch


def torch_dtype(dt):
    torch = _torch()
    return {L.F32: torch.float32, L.F16: torch.float16, L.BF16: torch.bfloat16, L.U8: torch.uint8,
            L.I8: torch.int8, L.I32: torch.int32}[dt]


def ohip_dtype(tdt):
    torch = _torch()
    return {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16, torch.uint8: L.U8,
            torch.int8: L.I8, torch.int32: L.I32}[tdt]


def _np_ohip_dtype(a):
    return {np.dtype(np.float32): L.F32, np.dtype(np.float16): L.F16, np.dtype(np.uint8): L.U8,
            np.dtype(np.int8): L.I8}[a.dtype]


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _key(name, label):
    if name is None:
        return None
    return ctypes.byref(L.WeightKey(name.encode(), (label or "").encode()))


class Weight:
    """A packed, device-resident operand (cached in the context when keyed)."""

    def __init__(self, ctx, handle, kind, dtype, shape, cached):
        self.ctx, self.handle, self.kind, self.dtype, self.shape, self.cached = ctx, handle, kind, dtype, shape, cached
        ctx._weights.add(self)

    @property
    def nbytes(self):
        return L.lib().ohip_weight_bytes(self.handle)

    def release(self):
        if self.handle is not None and not self.cached:
            L.lib().ohip_weight_release(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class HipContext:
    """Owns one ohip_ctx on one GPU (oxionnx-cuda's CudaContext counterpart)."""

    def __init__(self, device=0, adopt_torch_stream=True):
        import weakref
        torch = _torch()
        self.device = device
        self._weights = weakref.WeakSet()
        self._dtensors = weakref.WeakSet()
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_ctx_create(device, ctypes.byref(h)))
        self.h = h
        if adopt_torch_stream:
            # torch's default stream is the legacy null stream (handle 0); the
            # context's own stream is a blocking stream, which the null stream
            # already orders against, so only a non-default torch stream is
            # adopted explicitly.
            with torch.cuda.device(device):
                s = torch.cuda.current_stream(device).cuda_stream
            if s:
                L.check(L.lib().ohip_ctx_set_stream(self.h, ctypes.c_void_p(s)))

    def close(self):
        if self.h:
            for w in list(self._weights):
                w.handle = None       # the context frees every weight it owns
            for t in list(self._dtensors):
                t.free()              # device tensors return their buffers to the context's pool
            L.lib().ohip_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # --------------------------------------------------------------- admin
    def sync(self):
        L.check(L.lib().ohip_sync(self.h))

    def set_tile(self, tile_id):
        """Force the MFMA block tile by id (include/ohip.h); 0 = automatic."""
        L.check(L.lib().ohip_set_tile_override(self.h, tile_id))

    def tuning(self):
        t = L.Tuning()
        L.check(L.lib().ohip_get_tuning(self.h, ctypes.byref(t)))
        return t

    def set_tuning(self, t):
        L.check(L.lib().ohip_set_tuning(self.h, ctypes.byref(t)))

    def counters(self):
        c = L.Counters()
        L.check(L.lib().ohip_get_counters(self.h, ctypes.byref(c)))
        return {f: getattr(c, f) for f, _ in L.Counters._fields_}

    def reset_counters(self):
        L.check(L.lib().ohip_reset_counters(self.h))

    def stream(self):
        return L.lib().ohip_ctx_stream(self.h)

    # --------------------------------------------------------------- weights
    def weight_gemm(self, b, trans_b=False, dtype=L.F32, name=None, label="Gemm.B"):
        b = np.ascontiguousarray(b)
        if b.dtype == np.float64:
            b = b.astype(np.float32)
        k, n = (b.shape[1], b.shape[0]) if trans_b else b.shape
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_weight_gemm(self.h, _key(name, label), _np_ohip_dtype(b),
                                         b.ctypes.data_as(ctypes.c_void_p), k, n, int(trans_b), dtype,
                                         ctypes.byref(h)))
        return Weight(self, h, "gemm", dtype, (k, n), name is not None)

    def weight_conv(self, w, dtype=L.F32, name=None, label="Conv.W"):
        w = np.ascontiguousarray(w)
        if w.dtype == np.float64:
            w = w.astype(np.float32)
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_weight_conv(self.h, _key(name, label), _np_ohip_dtype(w),
                                         w.ctypes.data_as(ctypes.c_void_p), *w.shape, dtype, ctypes.byref(h)))
        return Weight(self, h, "conv", dtype, w.shape, name is not None)

    def weight_conv_transpose(self, w, dtype=L.F32, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1),
                              group=1, name=None, label="ConvTranspose.W"):
        """ConvTranspose filter [Cin, Cout/group, KH, KW], packed for the node's
        strides / top-left pads / dilations / group."""
        w = np.ascontiguousarray(w)
        if w.dtype == np.float64:
            w = w.astype(np.float32)
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_weight_conv_transpose(self.h, _key(name, label), _np_ohip_dtype(w),
                                                   w.ctypes.data_as(ctypes.c_void_p), *w.shape, strides[0],
                                                   strides[1], pads[0], pads[1], dilations[0], dilations[1],
                                                   group, dtype, ctypes.byref(h)))
        return Weight(self, h, "convt", dtype, w.shape, name is not None)

    def weight_qgemm(self, b, zp=None, scale=None, trans_b=False, name=None, label="QLinearMatMul.B"):
        b = np.ascontiguousarray(b)
        k, n = (b.shape[1], b.shape[0]) if trans_b else b.shape
        zp_a = None if zp is None else np.ascontiguousarray(np.atleast_1d(np.asarray(zp, np.int32)))
        sc = None if scale is None else np.ascontiguousarray(np.atleast_1d(np.asarray(scale, np.float32)))
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_weight_qgemm(
            self.h, _key(name, label), _np_ohip_dtype(b), b.ctypes.data_as(ctypes.c_void_p), k, n, int(trans_b),
            None if zp_a is None else zp_a.ctypes.data_as(ctypes.c_void_p), 0 if zp_a is None else zp_a.size,
            None if sc is None else sc.ctypes.data_as(ctypes.c_void_p), 0 if sc is None else sc.size,
            ctypes.byref(h)))
        return Weight(self, h, "qgemm", L.I8, (k, n), name is not None)

    def weight_qconv(self, w, zp=None, scale=None, name=None, label="QLinearConv.W"):
        w = np.ascontiguousarray(w)
        zp_a = None if zp is None else np.ascontiguousarray(np.atleast_1d(np.asarray(zp, np.int32)))
        sc = None if scale is None else np.ascontiguousarray(np.atleast_1d(np.asarray(scale, np.float32)))
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_weight_qconv(
            self.h, _key(name, label), _np_ohip_dtype(w), w.ctypes.data_as(ctypes.c_void_p), *w.shape,
            None if zp_a is None else zp_a.ctypes.data_as(ctypes.c_void_p), 0 if zp_a is None else zp_a.size,
            None if sc is None else sc.ctypes.data_as(ctypes.c_void_p), 0 if sc is None else sc.size,
            ctypes.byref(h)))
        return Weight(self, h, "qconv", L.I8, w.shape, name is not None)

    # --------------------------------------------------------------- ops
    def gemm(self, a, w, c=None, alpha=1.0, beta=1.0, trans_a=False, act=L.ACT_NONE, act_lo=0.0, act_hi=0.0,
             out=None):
        torch = _torch()
        dt = ohip_dtype(a.dtype)
        m = a.shape[1] if trans_a else a.shape[0]
        k, n = w.shape
        if out is None:
            out = torch.empty((m, n), dtype=a.dtype, device=a.device)
        c_kind = L.C_NONE
        if c is not None:
            c_kind = L.C_SCALAR if c.numel() == 1 else (L.C_ROW if c.dim() == 1 else L.C_FULL)
        d = L.GemmDesc(m, k, n, dt, int(trans_a), alpha, beta, c_kind, act, act_lo, act_hi,
                       a.stride(0), out.stride(0))
        L.check(L.lib().ohip_gemm(self.h, ctypes.byref(d), _ptr(a), w.handle, _ptr(c), _ptr(out)))
        return out

    def conv2d(self, x, w, bias=None, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1), act=L.ACT_NONE,
               act_lo=0.0, act_hi=0.0, in_layout=L.NCHW, out_layout=L.NCHW, out=None, group=1, noalloc=False):
        """pads = [top, left, bottom, right]; x NCHW (or NHWC channel-padded);
        w holds Cin / group input channels per filter (ONNX Conv's group).
        noalloc=True calls ohip_conv2d_noalloc (static scratch, no device
        allocation; `out` should then be given)."""
        torch = _torch()
        dt = ohip_dtype(x.dtype)
        cout, cin, kh, kw = w.shape
        if in_layout == L.NCHW:
            n, c, h, wd = x.shape
        else:
            n, h, wd = x.shape[:3]
            c = cin * group
        oh = L.lib().ohip_conv_out_dim(h, pads[0], pads[2], kh, dilations[0], strides[0])
        ow = L.lib().ohip_conv_out_dim(wd, pads[1], pads[3], kw, dilations[1], strides[1])
        if oh < 0 or ow < 0:
            raise L.OhipError(L.E_SHAPE, "bad conv geometry")
        if out is None:
            if out_layout == L.NCHW:
                out = torch.empty((n, cout, oh, ow), dtype=x.dtype, device=x.device)
            else:
                ce = 16 // L.ELEM_BYTES[dt]
                out = torch.zeros((n, oh, ow, (cout + ce - 1) // ce * ce), dtype=x.dtype, device=x.device)
        d = L.ConvDesc(n, c, h, wd, cout, kh, kw, group, strides[0], strides[1], dilations[0], dilations[1],
                       pads[0], pads[1], pads[2], pads[3], dt, in_layout, out_layout, act, act_lo, act_hi)
        fn = L.lib().ohip_conv2d_noalloc if noalloc else L.lib().ohip_conv2d
        L.check(fn(self.h, ctypes.byref(d), _ptr(x), w.handle, _ptr(bias), _ptr(out)))
        return out

    def conv2d_instnorm(self, x, w, bias=None, pads=(0, 0, 0, 0), strides=(1, 1), dilations=(1, 1), eps=1e-5,
                        gamma=None, beta=None, scale_offset=0, bias_offset=0, relu=False, out=None,
                        residual=None, nhwc=False):
        """Conv (ungrouped, no activation) followed by instance
        normalisation in one call (ohip_conv2d_instnorm); gamma / beta are
        optional [N, S] device rows of the tensor's dtype (the AdaIN form:
        channel c of sample n reads element n * S + offset + c); residual is
        added last.  nhwc: x, the output and the residual are NHWC (channels
        a whole number of 16-byte chunks), else NCHW."""
        torch = _torch()
        dt = ohip_dtype(x.dtype)
        cout, cin, kh, kw = w.shape
        if nhwc:
            n, h, wd, c = x.shape
        else:
            n, c, h, wd = x.shape
        oh = L.lib().ohip_conv_out_dim(h, pads[0], pads[2], kh, dilations[0], strides[0])
        ow = L.lib().ohip_conv_out_dim(wd, pads[1], pads[3], kw, dilations[1], strides[1])
        if out is None:
            shape = (n, oh, ow, cout) if nhwc else (n, cout, oh, ow)
            out = torch.empty(shape, dtype=x.dtype, device=x.device)
        lay = L.NHWC if nhwc else L.NCHW
        d = L.ConvDesc(n, c, h, wd, cout, kh, kw, 1, strides[0], strides[1], dilations[0], dilations[1],
                       pads[0], pads[1], pads[2], pads[3], dt, lay, lay, L.ACT_NONE, 0.0, 0.0, 0)
        nd = L.NormDesc(eps, None, None, 0, 0, 0, L.ACT_RELU if relu else L.ACT_NONE, 0.0,
                        None if residual is None else residual.data_ptr(), lay)
        if gamma is not None:
            eb = L.ELEM_BYTES[dt]
            nd.scale = gamma.data_ptr() + scale_offset * eb
            nd.bias = beta.data_ptr() + bias_offset * eb
            nd.per_sample, nd.stride, nd.same_type = 1, gamma.shape[1], 1
        L.check(L.lib().ohip_conv2d_instnorm(self.h, ctypes.byref(d), _ptr(x), w.handle, _ptr(bias),
                                             ctypes.byref(nd), _ptr(out)))
        return out

    def matmul(self, a, b, out=None):
        """Batched MatMul of two device tensors, [..., M, K] x [..., K, N], with the
        reference's slice rule (slice s: A slice s % a_batches, B slice s % b_batches)."""
        torch = _torch()
        dt = ohip_dtype(a.dtype)
        batch_shape = list(np.broadcast_shapes(tuple(a.shape[:-2]), tuple(b.shape[:-2])))
        batch = int(np.prod(batch_shape)) if batch_shape else 1
        na = int(np.prod(a.shape[:-2])) if a.dim() > 2 else 1
        nb = int(np.prod(b.shape[:-2])) if b.dim() > 2 else 1
        m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
        if out is None:
            out = torch.empty(batch_shape + [m, n], dtype=a.dtype, device=a.device)
        d = L.MatMulDesc(m, k, n, batch, na, nb, dt)
        L.check(L.lib().ohip_matmul(self.h, ctypes.byref(d), _ptr(a.contiguous()), _ptr(b.contiguous()), _ptr(out)))
        return out

    def conv_transpose2d(self, x, w, bias=None, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1),
                         output_padding=(0, 0), group=1, out=None):
        """ConvTranspose, NCHW; pads = [top, left, bottom, right] (already resolved)."""
        torch = _torch()
        dt = ohip_dtype(x.dtype)
        cin, coutg, kh, kw = w.shape
        n, c, h, wd = x.shape
        oh = L.lib().ohip_conv_transpose_out_dim(h, strides[0], output_padding[0], kh, dilations[0], pads[0], pads[2])
        ow = L.lib().ohip_conv_transpose_out_dim(wd, strides[1], output_padding[1], kw, dilations[1], pads[1], pads[3])
        if oh < 0 or ow < 0:
            raise L.OhipError(L.E_SHAPE, "bad ConvTranspose geometry")
        if out is None:
            out = torch.empty((n, coutg * group, oh, ow), dtype=x.dtype, device=x.device)
        d = L.ConvTDesc(n, c, h, wd, coutg * group, kh, kw, group, strides[0], strides[1], dilations[0],
                        dilations[1], pads[0], pads[1], pads[2], pads[3], output_padding[0], output_padding[1], dt)
        L.check(L.lib().ohip_conv_transpose2d(self.h, ctypes.byref(d), _ptr(x), w.handle, _ptr(bias), _ptr(out)))
        return out

    def qgemm(self, a, w, a_zp=0, out_kind=L.QOUT_U8, a_scale=1.0, y_scale=1.0, y_zp=0, lo=0, hi=255, out=None):
        torch = _torch()
        m, k = a.shape
        n = w.shape[1]
        azp = np.ascontiguousarray(np.atleast_1d(np.asarray(a_zp, np.int32)))
        if out is None:
            odt = {L.QOUT_U8: torch.uint8, L.QOUT_I8: torch.int8, L.QOUT_I32: torch.int32,
                   L.QOUT_F32: torch.float32}[out_kind]
            out = torch.empty((m, n), dtype=odt, device=a.device)
        d = L.QGemmDesc(m, k, n, ohip_dtype(a.dtype), azp.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                        azp.size, out_kind, a_scale, y_scale, y_zp, lo, hi, a.stride(0), out.stride(0))
        L.check(L.lib().ohip_qgemm(self.h, ctypes.byref(d), _ptr(a), w.handle, _ptr(out)))
        return out

    def qconv2d(self, x, w, bias=None, x_zp=0, out_kind=L.QOUT_U8, x_scale=1.0, y_scale=1.0, y_zp=0, lo=0,
                hi=255, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1), in_layout=L.NCHW,
                out_layout=L.NCHW, out=None, group=1):
        torch = _torch()
        cout, cin, kh, kw = w.shape
        if in_layout == L.NCHW:
            n, c, h, wd = x.shape
        else:
            n, h, wd = x.shape[:3]
            c = cin * group
        oh = L.lib().ohip_conv_out_dim(h, pads[0], pads[2], kh, dilations[0], strides[0])
        ow = L.lib().ohip_conv_out_dim(wd, pads[1], pads[3], kw, dilations[1], strides[1])
        if oh < 0 or ow < 0:
            raise L.OhipError(L.E_SHAPE, "bad conv geometry")
        odt = {L.QOUT_U8: torch.uint8, L.QOUT_I8: torch.int8, L.QOUT_I32: torch.int32,
                   L.QOUT_F32: torch.float32}[out_kind]
        if out is None:
            if out_layout == L.NCHW:
                out = torch.empty((n, cout, oh, ow), dtype=odt, device=x.device)
            else:
                ld = (cout + 15) // 16 * 16 if out_kind in (L.QOUT_U8, L.QOUT_I8) else (cout + 3) // 4 * 4
                out = torch.zeros((n, oh, ow, ld), dtype=odt, device=x.device)
        d = L.QConvDesc(n, c, h, wd, cout, kh, kw, group, strides[0], strides[1], dilations[0], dilations[1],
                        pads[0], pads[1], pads[2], pads[3], ohip_dtype(x.dtype), int(x_zp), out_kind, x_scale,
                        y_scale, y_zp, lo, hi, in_layout, out_layout)
        L.check(L.lib().ohip_qconv2d(self.h, ctypes.byref(d), _ptr(x), w.handle, _ptr(bias), _ptr(out)))
        return out
