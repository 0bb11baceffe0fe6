"""The provider's surface in the reference's own vocabulary (oxionnx-cuda/src/lib.rs).

``is_supported_op``, ``accepts_resident_slot``, ``HipContext.try_new`` and
``try_hip_dispatch`` / ``try_hip_dispatch_resident`` mirror
``is_supported_op`` (lib.rs:217), ``accepts_resident_slot`` (:419),
``CudaContext::try_new`` (context.rs:467-481), ``try_cuda_dispatch`` (:354) and
``try_cuda_dispatch_resident`` (:561): a node is offered with its weights (graph
initializers) and intermediates (run-time activations); the result is
``None`` when the provider declines (the caller runs its CPU operator) or the
list of output tensors.  Errors raise ``OhipError`` (the caller logs and falls
back, src/session/run/sequential.rs:1019-1031).  All work happens in
libohip.so's ``ohip_try_dispatch``; this module only marshals operands.
"""
import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from . import _lib as L
from .device import HipContext as _DeviceContext

_NP2OHIP = {np.dtype(np.float32): L.F32, np.dtype(np.float16): L.F16, np.dtype(np.uint8): L.U8,
            np.dtype(np.int8): L.I8, np.dtype(np.int32): L.I32}
_OHIP2NP = {L.F32: np.float32, L.F16: np.float16, L.U8: np.uint8, L.I8: np.int8, L.I32: np.int32,
            L.BF16: np.uint16}


@dataclass
class Attributes:
    """oxionnx_core::Attributes (oxionnx-core/src/graph.rs:696-705), the fields this provider reads."""
    ints: Dict[str, int] = field(default_factory=dict)
    floats: Dict[str, float] = field(default_factory=dict)
    strings: Dict[str, str] = field(default_factory=dict)
    int_lists: Dict[str, List[int]] = field(default_factory=dict)


@dataclass
class Node:
    """oxionnx_core::Node: op type, name, input / output tensor names, attributes."""
    op: str
    inputs: List[str]
    outputs: List[str] = field(default_factory=lambda: ["y"])
    attrs: Attributes = field(default_factory=Attributes)
    name: str = "node"


@dataclass
class Typed:
    """A typed operand (TypedTensor): bf16 travels as uint16 bits; for
    integer operands ``declared`` names the ONNX element type ('u8'/'i8')."""
    data: np.ndarray
    declared: Optional[str] = None
    bf16: bool = False


def is_supported_op(op: str) -> bool:
    return bool(L.lib().ohip_is_supported_op(op.encode()))


def accepts_resident_slot(op: str, index: int) -> bool:
    return bool(L.lib().ohip_accepts_resident_slot(op.encode(), index))


class HipContext(_DeviceContext):
    """CudaContext's counterpart: one device, one stream, the weight cache."""

    @classmethod
    def try_new(cls) -> Optional["HipContext"]:
        """None unless OXIONNX_HIP is truthy and a gfx950 device exists."""
        if not L.lib().ohip_env_flag(b"OXIONNX_HIP"):
            return None
        try:
            return cls(0)
        except L.OhipError:
            return None

    def last_decline(self) -> str:
        return L.lib().ohip_last_decline(self.h).decode(errors="replace")


class _Marshal:
    def __init__(self):
        self.keep = []

    def tensor(self, name, value, is_init):
        t = L.TensorRef()
        t.name = name.encode()
        t.is_initializer = int(is_init)
        if value is None:
            return t
        declared = 0
        if isinstance(value, Typed):
            declared = {"u8": L.U8, "i8": L.I8, None: 0}[value.declared]
            bf16 = value.bf16
            value = value.data
        else:
            bf16 = False
        if isinstance(value, DeviceTensor):
            t.device = value.h
            t.dtype = value.dtype
            shape = value.shape
        else:
            arr = np.ascontiguousarray(value)
            if arr.dtype == np.float64:
                arr = arr.astype(np.float32)
            t.dtype = L.BF16 if bf16 else _NP2OHIP[arr.dtype]
            t.data = arr.ctypes.data_as(ctypes.c_void_p)
            self.keep.append(arr)
            shape = arr.shape
        t.declared_dtype = declared
        sh = (L.I64 * max(1, len(shape)))(*shape)
        self.keep.append(sh)
        t.shape = sh
        t.rank = len(shape)
        return t

    def attrs(self, a: Attributes):
        out = []
        for k, v in a.ints.items():
            out.append(L.Attr(k.encode(), L.ATTR_INT, int(v), 0.0, None, 0, None))
        for k, v in a.floats.items():
            out.append(L.Attr(k.encode(), L.ATTR_FLOAT, 0, float(v), None, 0, None))
        for k, v in a.strings.items():
            out.append(L.Attr(k.encode(), L.ATTR_STRING, 0, 0.0, None, 0, v.encode()))
        for k, v in a.int_lists.items():
            arr = (L.I64 * max(1, len(v)))(*v)
            self.keep.append(arr)
            out.append(L.Attr(k.encode(), L.ATTR_INTS, 0, 0.0, arr, len(v), None))
        return out


class DeviceTensor:
    """HipDeviceTensor: a run-scoped device activation (implements the
    DeviceActivation contract of src/session/gpu_activations.rs:117-189)."""

    def __init__(self, handle, ctx=None):
        self.h = handle
        if ctx is not None:
            ctx._dtensors.add(self)   # freed by the context's close() if still alive
        dt, rank = ctypes.c_int(), ctypes.c_int()
        shape = (L.I64 * 8)()
        nbytes = ctypes.c_size_t()
        L.check(L.lib().ohip_dtensor_info(handle, ctypes.byref(dt), ctypes.byref(rank), shape, ctypes.byref(nbytes)))
        self.dtype, self.shape, self.nbytes = dt.value, tuple(shape[:rank.value]), nbytes.value
        self.c_shape = shape

    @classmethod
    def from_host(cls, ctx, arr):
        arr = np.ascontiguousarray(arr)
        shape = (L.I64 * max(1, arr.ndim))(*arr.shape)
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_dtensor_alloc(ctx.h, _NP2OHIP[arr.dtype], arr.ndim, shape, L.NCHW, ctypes.byref(h)))
        L.check(L.lib().ohip_dtensor_upload(ctx.h, h, arr.ctypes.data_as(ctypes.c_void_p)))
        return cls(h, ctx)

    def to_nchw(self, ctx):
        """This tensor in NCHW layout: itself, or a converted copy (the
        conversion is enqueued on the context's stream)."""
        if L.lib().ohip_dtensor_layout(self.h) == L.NCHW:
            return self
        h = ctypes.c_void_p()
        L.check(L.lib().ohip_dtensor_to_nchw(ctx.h, self.h, ctypes.byref(h)))
        return DeviceTensor(h, ctx)

    def to_host(self, ctx):
        out = np.empty(self.shape, _OHIP2NP[self.dtype])
        L.check(L.lib().ohip_dtensor_download(ctx.h, self.h, out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def free(self):
        if self.h:
            L.lib().ohip_dtensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _dispatch(node, weights, intermediates, ctx, placement):
    m = _Marshal()
    refs = []
    for name in node.inputs:
        if not name:
            refs.append(m.tensor("", None, False))
        elif name in weights:
            refs.append(m.tensor(name, weights[name], True))
        elif name in intermediates:
            refs.append(m.tensor(name, intermediates[name], False))
        else:
            raise KeyError(f"input '{name}' of node '{node.name}' is not available")
    attrs = m.attrs(node.attrs)
    arr_in = (L.TensorRef * max(1, len(refs)))(*refs)
    arr_at = (L.Attr * max(1, len(attrs)))(*attrs)
    nd = L.Node(node.op.encode(), node.name.encode(), len(refs), arr_in, len(attrs), arr_at)
    out = L.Output()
    rc = L.lib().ohip_try_dispatch(ctx.h, ctypes.byref(nd), placement, ctypes.byref(out))
    if rc == L.DECLINED:
        return None
    L.check(rc)
    shape = tuple(out.shape[:out.rank])
    if placement == L.PLACE_DEVICE:
        return [DeviceTensor(out.device, ctx)]
    dt = _OHIP2NP[out.dtype]
    n = int(np.prod(shape)) if shape else 1
    buf = (ctypes.c_char * (n * np.dtype(dt).itemsize)).from_address(out.data)
    res = np.frombuffer(buf, dtype=dt).copy().reshape(shape)
    L.lib().ohip_output_free(ctypes.byref(out))
    if out.dtype == L.I32:
        # MatMulInteger / ConvInteger: saturate_i32 as f32 lanes (quant_ops/mod.rs:243)
        res = res.astype(np.float32)
    return [res]


class PreparedNode:
    """A node marshalled once for repeated resident dispatch: initializer
    operands and attributes are fixed C structures; only the resident
    activation slots are refreshed per call (the run loop's hot path)."""

    def __init__(self, node: Node, weights: dict):
        self.node = node
        self.m = _Marshal()
        n = len(node.inputs)
        self.refs = (L.TensorRef * max(1, n))()
        self.dynamic = []
        for i, name in enumerate(node.inputs):
            if not name:
                self.refs[i] = self.m.tensor("", None, False)
            elif name in weights:
                self.refs[i] = self.m.tensor(name, weights[name], True)
            else:
                self.refs[i] = self.m.tensor(name, None, False)
                self.dynamic.append((i, name))
        attrs = self.m.attrs(node.attrs)
        self.attrs = (L.Attr * max(1, len(attrs)))(*attrs)
        self.op_b, self.name_b = node.op.encode(), node.name.encode()
        self.nd = L.Node(self.op_b, self.name_b, n, self.refs, len(attrs), self.attrs)
        self._fn = L.lib().ohip_try_dispatch

    def dispatch_resident(self, acts: dict, ctx: HipContext):
        for i, name in self.dynamic:
            t = acts[name]
            r = self.refs[i]
            r.device = t.h
            r.dtype = t.dtype
            r.shape = t.c_shape
            r.rank = len(t.shape)
        out = L.Output()
        rc = self._fn(ctx.h, ctypes.byref(self.nd), L.PLACE_DEVICE, ctypes.byref(out))
        if rc == L.DECLINED:
            return None
        L.check(rc)
        return DeviceTensor(out.device, ctx)


def try_hip_dispatch(node: Node, weights: dict, intermediates: dict, ctx: HipContext):
    """Host tensors in, host tensors out (try_cuda_dispatch, lib.rs:354)."""
    return _dispatch(node, weights, intermediates, ctx, L.PLACE_HOST)


def try_hip_dispatch_resident(node: Node, weights: dict, activations: dict, ctx: HipContext):
    """Operands may be resident DeviceTensors; the output stays on the device
    (try_cuda_dispatch_resident with CudaOutputPlacement::Device, lib.rs:561)."""
    return _dispatch(node, weights, activations, ctx, L.PLACE_DEVICE)
