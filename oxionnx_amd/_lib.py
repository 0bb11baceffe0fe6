"""ctypes binding of libohip.so (include/ohip.h).

The library is loaded from this package directory only.  If it is missing the
import does not fall back to anything: every call raises ``OhipUnavailable``.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libohip.so")

OK, DECLINED = 0, 1
E_INVALID, E_HIP, E_SHAPE, E_NOMEM, E_NODEVICE = -1, -2, -3, -4, -5

F32, U8, I8, I32, F16, BF16 = 1, 2, 3, 6, 10, 16
ACT_NONE, ACT_RELU, ACT_CLIP, ACT_LEAKY_RELU = 0, 1, 2, 3
C_NONE, C_SCALAR, C_ROW, C_FULL = 0, 1, 2, 3
NCHW, NHWC = 0, 1
PAD_ZEROS, PAD_REFLECT, PAD_EDGE = 0, 1, 2
QOUT_U8, QOUT_I8, QOUT_I32, QOUT_F32 = 0, 1, 2, 3
CLASS_MI355X, CLASS_PARITY, CLASS_NEVER, CLASS_LEGACY = 0, 1, 2, 3

ELEM_BYTES = {F32: 4, U8: 1, I8: 1, I32: 4, F16: 2, BF16: 2}

I64 = ctypes.c_int64
VP = ctypes.c_void_p


class OhipUnavailable(RuntimeError):
    """libohip.so is not built or cannot be loaded."""


class OhipDeclined(RuntimeError):
    """The provider declined the configuration (the caller runs its CPU kernel)."""


class OhipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"ohip error {code}: {msg}")
        self.code = code


class Tuning(ctypes.Structure):
    _fields_ = [("perf_class", ctypes.c_int), ("gemm_min_mac", ctypes.c_uint64),
                ("gemm_min_mac_cached", ctypes.c_uint64), ("gemm_min_intensity", ctypes.c_uint64),
                ("conv_min_mac", ctypes.c_uint64)]


class WeightKey(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("label", ctypes.c_char_p)]


class GemmDesc(ctypes.Structure):
    _fields_ = [("m", I64), ("k", I64), ("n", I64), ("dtype", ctypes.c_int), ("trans_a", ctypes.c_int),
                ("alpha", ctypes.c_float), ("beta", ctypes.c_float), ("c_kind", ctypes.c_int),
                ("act", ctypes.c_int), ("act_lo", ctypes.c_float), ("act_hi", ctypes.c_float),
                ("lda", I64), ("ldy", I64)]


class ConvDesc(ctypes.Structure):
    _fields_ = [(f, I64) for f in ("n", "c", "h", "w", "cout", "kh", "kw", "group", "stride_h", "stride_w",
                                    "dil_h", "dil_w", "pad_t", "pad_l", "pad_b", "pad_r")] + \
               [("dtype", ctypes.c_int), ("in_layout", ctypes.c_int), ("out_layout", ctypes.c_int),
                ("act", ctypes.c_int), ("act_lo", ctypes.c_float), ("act_hi", ctypes.c_float),
                ("pad_mode", ctypes.c_int)]


class NormDesc(ctypes.Structure):
    _fields_ = [("epsilon", ctypes.c_float), ("scale", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("per_sample", ctypes.c_int), ("stride", I64), ("same_type", ctypes.c_int), ("act", ctypes.c_int),
                ("alpha", ctypes.c_float), ("residual", ctypes.c_void_p), ("residual_layout", ctypes.c_int)]


class ConvTDesc(ctypes.Structure):
    _fields_ = [(f, I64) for f in ("n", "c", "h", "w", "cout", "kh", "kw", "group", "stride_h", "stride_w",
                                    "dil_h", "dil_w", "pad_t", "pad_l", "pad_b", "pad_r", "out_pad_h",
                                    "out_pad_w")] + [("dtype", ctypes.c_int)]


class MatMulDesc(ctypes.Structure):
    _fields_ = [(f, I64) for f in ("m", "k", "n", "batch", "a_batches", "b_batches")] + [("dtype", ctypes.c_int)]


class QGemmDesc(ctypes.Structure):
    _fields_ = [("m", I64), ("k", I64), ("n", I64), ("a_dtype", ctypes.c_int),
                ("a_zp", ctypes.POINTER(ctypes.c_int32)), ("n_azp", ctypes.c_int), ("out_kind", ctypes.c_int),
                ("a_scale", ctypes.c_float), ("y_scale", ctypes.c_float), ("y_zp", ctypes.c_int32),
                ("lo", ctypes.c_int32), ("hi", ctypes.c_int32), ("lda", I64), ("ldy", I64)]


class QConvDesc(ctypes.Structure):
    _fields_ = [(f, I64) for f in ("n", "c", "h", "w", "cout", "kh", "kw", "group", "stride_h", "stride_w",
                                    "dil_h", "dil_w", "pad_t", "pad_l", "pad_b", "pad_r")] + \
               [("x_dtype", ctypes.c_int), ("x_zp", ctypes.c_int32), ("out_kind", ctypes.c_int),
                ("x_scale", ctypes.c_float), ("y_scale", ctypes.c_float), ("y_zp", ctypes.c_int32),
                ("lo", ctypes.c_int32), ("hi", ctypes.c_int32), ("in_layout", ctypes.c_int),
                ("out_layout", ctypes.c_int), ("out_table", VP), ("in_pitch", I64)]


class Attr(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("kind", ctypes.c_int), ("i", I64), ("f", ctypes.c_float),
                ("ints", ctypes.POINTER(I64)), ("n_ints", ctypes.c_int), ("s", ctypes.c_char_p)]


class TensorRef(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("declared_dtype", ctypes.c_int),
                ("rank", ctypes.c_int), ("shape", ctypes.POINTER(I64)), ("data", VP), ("device", VP),
                ("is_initializer", ctypes.c_int)]


class Node(ctypes.Structure):
    _fields_ = [("op_type", ctypes.c_char_p), ("name", ctypes.c_char_p), ("n_inputs", ctypes.c_int),
                ("inputs", ctypes.POINTER(TensorRef)), ("n_attrs", ctypes.c_int), ("attrs", ctypes.POINTER(Attr))]


class Output(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("rank", ctypes.c_int), ("shape", I64 * 8), ("data", VP), ("device", VP)]


ATTR_INT, ATTR_FLOAT, ATTR_INTS, ATTR_STRING = 0, 1, 2, 3
PLACE_HOST, PLACE_DEVICE = 0, 1


class Counters(ctypes.Structure):
    _fields_ = [(f, ctypes.c_uint64) for f in (
        "weight_hits", "weight_misses", "weight_transient", "weight_uploaded_bytes", "weight_resident_bytes",
        "h2d_bytes", "d2h_bytes", "dispatches", "declined", "device_allocs", "stream_syncs",
        "pool_live", "contraction_launches")]


# name -> (restype, argtypes); the list is the C ABI of include/ohip.h.
SIGNATURES = {
    "ohip_ctx_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(VP)]),
    "ohip_ctx_destroy": (None, [VP]),
    "ohip_ctx_set_stream": (ctypes.c_int, [VP, VP]),
    "ohip_ctx_stream": (VP, [VP]),
    "ohip_sync": (ctypes.c_int, [VP]),
    "ohip_pool_parking": (ctypes.c_int, [VP, ctypes.c_int]),
    "ohip_graph_begin": (ctypes.c_int, [VP]),
    "ohip_graph_end": (ctypes.c_int, [VP, ctypes.POINTER(VP)]),
    "ohip_graph_launch": (ctypes.c_int, [VP]),
    "ohip_graph_destroy": (None, [VP]),
    "ohip_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "ohip_last_error": (ctypes.c_char_p, []),
    "ohip_version": (ctypes.c_char_p, []),
    "ohip_env_flag": (ctypes.c_int, [ctypes.c_char_p]),
    "ohip_malloc": (ctypes.c_int, [VP, ctypes.c_size_t, ctypes.POINTER(VP)]),
    "ohip_free": (ctypes.c_int, [VP, VP]),
    "ohip_memcpy_h2d": (ctypes.c_int, [VP, VP, VP, ctypes.c_size_t]),
    "ohip_memcpy_d2h": (ctypes.c_int, [VP, VP, VP, ctypes.c_size_t]),
    "ohip_memcpy_d2d": (ctypes.c_int, [VP, VP, VP, ctypes.c_size_t]),
    "ohip_tuning_for_class": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(Tuning)]),
    "ohip_set_tuning": (ctypes.c_int, [VP, ctypes.POINTER(Tuning)]),
    "ohip_get_tuning": (ctypes.c_int, [VP, ctypes.POINTER(Tuning)]),
    "ohip_gemm_mac": (ctypes.c_uint64, [I64, I64, I64]),
    "ohip_gemm_intensity": (ctypes.c_uint64, [I64, I64, I64]),
    "ohip_gemm_admits": (ctypes.c_int, [ctypes.POINTER(Tuning), I64, I64, I64, ctypes.c_int]),
    "ohip_conv_admits": (ctypes.c_int, [ctypes.POINTER(Tuning), I64, I64, I64]),
    "ohip_weight_gemm": (ctypes.c_int, [VP, ctypes.POINTER(WeightKey), ctypes.c_int, VP, I64, I64, ctypes.c_int,
                                        ctypes.c_int, ctypes.POINTER(VP)]),
    "ohip_weight_conv": (ctypes.c_int, [VP, ctypes.POINTER(WeightKey), ctypes.c_int, VP, I64, I64, I64, I64,
                                        ctypes.c_int, ctypes.POINTER(VP)]),
    "ohip_weight_qgemm": (ctypes.c_int, [VP, ctypes.POINTER(WeightKey), ctypes.c_int, VP, I64, I64, ctypes.c_int,
                                         VP, ctypes.c_int, VP, ctypes.c_int, ctypes.POINTER(VP)]),
    "ohip_weight_qconv": (ctypes.c_int, [VP, ctypes.POINTER(WeightKey), ctypes.c_int, VP, I64, I64, I64, I64,
                                         VP, ctypes.c_int, VP, ctypes.c_int, ctypes.POINTER(VP)]),
    "ohip_weight_release": (None, [VP]),
    "ohip_weight_bytes": (ctypes.c_size_t, [VP]),
    "ohip_gemm": (ctypes.c_int, [VP, ctypes.POINTER(GemmDesc), VP, VP, VP, VP]),
    "ohip_conv2d": (ctypes.c_int, [VP, ctypes.POINTER(ConvDesc), VP, VP, VP, VP]),
    "ohip_conv2d_noalloc": (ctypes.c_int, [VP, ctypes.POINTER(ConvDesc), VP, VP, VP, VP]),
    "ohip_conv2d_instnorm": (ctypes.c_int, [VP, ctypes.POINTER(ConvDesc), VP, VP, VP, ctypes.POINTER(NormDesc), VP]),
    "ohip_matmul": (ctypes.c_int, [VP, ctypes.POINTER(MatMulDesc), VP, VP, VP]),
    "ohip_conv_out_dim": (I64, [I64, I64, I64, I64, I64, I64]),
    "ohip_weight_conv_transpose": (ctypes.c_int, [VP, ctypes.POINTER(WeightKey), ctypes.c_int, VP, I64, I64, I64,
                                                  I64, I64, I64, I64, I64, I64, I64, I64, ctypes.c_int,
                                                  ctypes.POINTER(VP)]),
    "ohip_conv_transpose2d": (ctypes.c_int, [VP, ctypes.POINTER(ConvTDesc), VP, VP, VP, VP]),
    "ohip_conv_transpose_out_dim": (I64, [I64, I64, I64, I64, I64, I64, I64]),
    "ohip_qgemm": (ctypes.c_int, [VP, ctypes.POINTER(QGemmDesc), VP, VP, VP]),
    "ohip_qconv2d": (ctypes.c_int, [VP, ctypes.POINTER(QConvDesc), VP, VP, VP, VP]),
    "ohip_get_counters": (ctypes.c_int, [VP, ctypes.POINTER(Counters)]),
    "ohip_reset_counters": (ctypes.c_int, [VP]),
    "ohip_set_tile_override": (ctypes.c_int, [VP, ctypes.c_int]),
    "ohip_dtensor_alloc": (ctypes.c_int, [VP, ctypes.c_int, ctypes.c_int, ctypes.POINTER(I64), ctypes.c_int,
                                          ctypes.POINTER(VP)]),
    "ohip_dtensor_wrap": (ctypes.c_int, [VP, VP, ctypes.c_int, ctypes.c_int, ctypes.POINTER(I64), ctypes.POINTER(VP)]),
    "ohip_dtensor_upload": (ctypes.c_int, [VP, VP, VP]),
    "ohip_dtensor_download": (ctypes.c_int, [VP, VP, VP]),
    "ohip_dtensor_ptr": (VP, [VP]),
    "ohip_dtensor_layout": (ctypes.c_int, [VP]),
    "ohip_dtensor_to_nchw": (ctypes.c_int, [VP, VP, ctypes.POINTER(VP)]),
    "ohip_dtensor_info": (ctypes.c_int, [VP, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                         ctypes.POINTER(I64), ctypes.POINTER(ctypes.c_size_t)]),
    "ohip_dtensor_free": (None, [VP]),
    "ohip_is_supported_op": (ctypes.c_int, [ctypes.c_char_p]),
    "ohip_accepts_resident_slot": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int]),
    "ohip_try_dispatch": (ctypes.c_int, [VP, ctypes.POINTER(Node), ctypes.c_int, ctypes.POINTER(Output)]),
    "ohip_output_free": (None, [ctypes.POINTER(Output)]),
    "ohip_ctx_try_new": (ctypes.c_int, [ctypes.POINTER(VP)]),
    "ohip_note_declined": (None, [VP, ctypes.c_char_p]),
    "ohip_last_decline": (ctypes.c_char_p, [VP]),
}

_lib = None


def lib():
    """Load libohip.so (once).  Raises OhipUnavailable if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OhipUnavailable(f"{LIB_PATH} is not built; run `python -m oxionnx_amd.build`")
        try:
            L = ctypes.CDLL(LIB_PATH)
        except OSError as e:
            raise OhipUnavailable(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().ohip_last_error().decode(errors="replace")


def check(rc):
    """Map a status code: 0 -> None, 1 -> OhipDeclined, <0 -> OhipError."""
    if rc == OK:
        return
    msg = last_error()
    if rc == DECLINED:
        raise OhipDeclined(msg)
    raise OhipError(rc, msg)
