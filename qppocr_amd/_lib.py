"""ctypes binding of libqppocr_hip.so (the C ABI declared in include/qppocr_hip.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in this package.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# QPPOCR_HIP_LIB names another build of the same library (the host-code
# sanitizer build, for CPU runs of the host-side checks)
LIB_PATH = os.environ.get("QPPOCR_HIP_LIB") or os.path.join(HERE, "libqppocr_hip.so")

QPH_OK = 0
ACT_NONE, ACT_GELU, ACT_RELU, ACT_HARDSWISH, ACT_SIGMOID = 0, 1, 2, 3, 4
OP_CONV, OP_CONVT_PAIR_SIG, OP_LINEAR, OP_LAYERNORM, OP_ATTENTION = 1, 2, 3, 4, 5
OP_SOFTMAX_ARGMAX, OP_CONVT, OP_ACT = 6, 7, 8
OP_GAP, OP_MUL_ADD_SCALE, OP_POOL, OP_RESIZE, OP_TRANSPOSE, OP_COPY_SLOT = 9, 10, 11, 12, 13, 14
ACT_HARDSIGMOID = 5
ACT_CLIP, ACT_HARDSWISH_CLIP = 6, 7
OP_BINARY = 15
BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV = 0, 1, 2, 3
RUN_UPLOAD, RUN_DOWNLOAD = 1, 2
NET_SEPARATE_LAUNCHES = 1
NET_FUSED_HEAD = 2
NOALLOC_WK_FLOATS = 1 << 20

I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float
P = ctypes.c_void_p


class ConvParams(ctypes.Structure):
    """qph_conv_params == ConvParams (qppocr-kernels/src/conv.rs:124-143)."""
    _fields_ = [("sh", I64), ("sw", I64), ("ph", I64), ("pw", I64), ("peh", I64),
                ("pew", I64), ("dh", I64), ("dw", I64), ("group", I64)]


class Act(ctypes.Structure):
    _fields_ = [("kind", I32), ("c1", F32), ("c2", F32), ("c3", F32)]


class ConvEpilogue(ctypes.Structure):
    _fields_ = [("residual", P), ("res_up", I32), ("y_ctotal", I64), ("y_coff", I64),
                ("y_up", I64), ("trans_out", I32)]


class Node(ctypes.Structure):
    _fields_ = [("op", I32), ("in_", I32), ("in2", I32), ("out", I32), ("out2", I32),
                ("w", I32), ("bias", I32), ("w2", I32), ("ws", I64 * 4), ("w2s", I64 * 4),
                ("cp", ConvParams), ("act", Act), ("res_up", I32), ("trans_out", I32),
                ("y_ctotal", I64), ("y_coff", I64), ("y_up", I64), ("heads", I64),
                ("dh", I64), ("eps", F32), ("scale", F32), ("in3", I32)]


class NetSpec(ctypes.Structure):
    _fields_ = [("n_tensors", I32), ("shapes", ctypes.POINTER(I64)),
                ("alias", ctypes.POINTER(I32)), ("n_nodes", I32), ("nodes", ctypes.POINTER(Node)),
                ("n_weights", I32), ("weight_sizes", ctypes.POINTER(I64)), ("n_outputs", I32),
                ("outputs", ctypes.POINTER(I32)), ("flags", I32)]


class PlanUpload(ctypes.Structure):
    _fields_ = [("off", ctypes.c_uint32), ("n_words", ctypes.c_uint32), ("words", P)]


class PlanDispatch(ctypes.Structure):
    _fields_ = [("kernel", I32), ("p_off", ctypes.c_uint32), ("groups", ctypes.c_uint32 * 3)]


class PlanSpec(ctypes.Structure):
    _fields_ = [("total_words", ctypes.c_uint32), ("n_uploads", I32),
                ("uploads", ctypes.POINTER(PlanUpload)), ("n_dispatches", I32),
                ("dispatches", ctypes.POINTER(PlanDispatch)), ("in_f32_off", ctypes.c_uint32),
                ("in_numel", I64), ("n_outputs", I32), ("out_offs", ctypes.POINTER(ctypes.c_uint32)),
                ("out_numel", ctypes.POINTER(I64))]


# exported symbol -> (argtypes, restype); every symbol include/qppocr_hip.h declares
SIGNATURES = {
    "qph_ctx_create": ([ctypes.c_int, ctypes.POINTER(P)], ctypes.c_int),
    "qph_ctx_destroy": ([P], ctypes.c_int),
    "qph_ctx_set_stream": ([P, P], ctypes.c_int),
    "qph_ctx_stream": ([P], P),
    "qph_sync": ([P], ctypes.c_int),
    "qph_last_error": ([], ctypes.c_char_p),
    "qph_version": ([], ctypes.c_char_p),
    "qph_malloc": ([P, ctypes.POINTER(P), ctypes.c_size_t], ctypes.c_int),
    "qph_free": ([P, P], ctypes.c_int),
    "qph_memcpy_h2d": ([P, P, P, ctypes.c_size_t], ctypes.c_int),
    "qph_memcpy_d2h": ([P, P, P, ctypes.c_size_t], ctypes.c_int),
    "qph_memset": ([P, P, ctypes.c_int, ctypes.c_size_t], ctypes.c_int),
    "qph_ctx_scratch_bytes": ([P, ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "qph_conv2d_out_shape": ([P, P, ctypes.POINTER(ConvParams), P], ctypes.c_int),
    "qph_conv2d": ([P, P, P, P, P, P, ctypes.POINTER(ConvParams), ctypes.POINTER(Act), P, P, P],
                   ctypes.c_int),
    "qph_linear_softmax_argmax": ([P, P, P, P, I64, I64, I64, P], ctypes.c_int),
    "qph_global_avg_pool": ([P, P, I64, I64, I64, P], ctypes.c_int),
    "qph_mul_add_scale": ([P, P, P, P, I64, I64, I64, P], ctypes.c_int),
    "qph_pool2d": ([P, P, P] + [I64] * 8 + [I32, P, P], ctypes.c_int),
    "qph_resize_bilinear": ([P, P, I64, I64, I64, I64, I64, I32, P], ctypes.c_int),
    "qph_transpose": ([P, P, P, P, P], ctypes.c_int),
    "qph_det_normalize_u8": ([P, P, I64, I64, P], ctypes.c_int),
    "qph_resize_bilinear_rgb_u8": ([P, P, I64, I64, P, I64, I64], ctypes.c_int),
    "qph_pack_crop": ([P, P, I64, I64, I64, I64, I32, P], ctypes.c_int),
    "qph_pack_crops": ([P, I32, P, P, P, P, I64, I64, P], ctypes.c_int),
    "qph_db_mask": ([P, P, I64, I64, F32, I32, P], ctypes.c_int),
    "qph_conv2d_noalloc": ([P, P, P, P, P, P, ctypes.POINTER(ConvParams), ctypes.POINTER(Act), P,
                            P, P], ctypes.c_int),
    "qph_conv2d_ex": ([P, P, P, P, P, P, ctypes.POINTER(ConvParams), ctypes.POINTER(Act),
                       ctypes.POINTER(ConvEpilogue), P], ctypes.c_int),
    "qph_convtranspose2d": ([P, P, P, P, P, I64, I64, I64, I64, P, P], ctypes.c_int),
    "qph_convt2x2_pair_sigmoid": ([P, P, P, P, P, P, P, P], ctypes.c_int),
    "qph_sgemm": ([P, P, P, P, I64, I64, I64, I64, P, ctypes.POINTER(Act), P, I32], ctypes.c_int),
    "qph_matmul": ([P, P, P, P, I64, I64, I64, I64, I32], ctypes.c_int),
    "qph_linear": ([P, P, P, P, I64, I64, I64, ctypes.POINTER(Act), P, P], ctypes.c_int),
    "qph_layernorm": ([P, P, P, P, F32, I64, I64, P], ctypes.c_int),
    "qph_softmax_last_dim": ([P, P, I64, I64], ctypes.c_int),
    "qph_softmax_argmax": ([P, P, I64, I64, P, P], ctypes.c_int),
    "qph_ctc_argmax": ([P, P, I64, I64, I64, P, P], ctypes.c_int),
    "qph_attention": ([P, P, I64, I64, I64, I64, F32, P], ctypes.c_int),
    "qph_activation": ([P, P, P, I64, ctypes.POINTER(Act)], ctypes.c_int),
    "qph_hardsigmoid": ([P, P, P, I64, F32, F32], ctypes.c_int),
    "qph_resize_nearest": ([P, P, I64, I64, I64, I64, I64, P], ctypes.c_int),
    "qph_binary_inplace": ([P, P, P, I64, I64, I32, I32], ctypes.c_int),
    "qph_reduce_mean_last": ([P, P, I64, I64, P], ctypes.c_int),
    "qph_net_create": ([P, ctypes.POINTER(NetSpec), ctypes.POINTER(P), ctypes.POINTER(P)],
                       ctypes.c_int),
    "qph_net_destroy": ([P], ctypes.c_int),
    "qph_net_run": ([P, P, I32, ctypes.POINTER(P)], ctypes.c_int),
    "qph_net_tensor": ([P, I32, ctypes.POINTER(P), ctypes.POINTER(I64)], ctypes.c_int),
    "qph_net_set_real_n": ([P, I32], ctypes.c_int),
    "qph_net_real_n": ([P, ctypes.POINTER(I32), ctypes.POINTER(I32)], ctypes.c_int),
    "qph_net_staging": ([P, I32, ctypes.POINTER(P), ctypes.POINTER(I64)], ctypes.c_int),
    "qph_net_run_async": ([P, I32], ctypes.c_int),
    "qph_net_complete": ([P], ctypes.c_int),
    "qph_net_set_profiling": ([P, I32], ctypes.c_int),
    "qph_net_node_times": ([P, ctypes.POINTER(ctypes.c_double), I32], ctypes.c_int),
    "qph_net_plan": ([P, P, P, P, I32, P], ctypes.c_int),
    "qph_plan_kernel_id": ([ctypes.c_char_p], ctypes.c_int),
    "qph_plan_create": ([P, ctypes.POINTER(PlanSpec), ctypes.POINTER(P)], ctypes.c_int),
    "qph_plan_validate": ([ctypes.POINTER(PlanSpec)], ctypes.c_int),
    "qph_plan_destroy": ([P], ctypes.c_int),
    "qph_plan_set_real_n": ([P, ctypes.c_uint32], ctypes.c_int),
    "qph_plan_run": ([P, P, I32, P], ctypes.c_int),
    "qph_plan_arena": ([P, ctypes.POINTER(P), ctypes.POINTER(I64)], ctypes.c_int),
    "qph_plan_launches": ([P, ctypes.POINTER(I32)], ctypes.c_int),
}

_lib = None


class QphError(RuntimeError):
    """A failed C-ABI call: status code + the library's message (Error::Device / Graph)."""

    def __init__(self, code, msg):
        super().__init__(f"qph error {code}: {msg}")
        self.code = code


def load():
    """Load the built library; raise if it is missing (no fallback path exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -c 'import __graft_entry__; __graft_entry__.build()')")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def check(rc):
    if rc != QPH_OK:
        raise QphError(rc, load().qph_last_error().decode(errors="replace"))
    return rc


def i64arr(seq):
    a = (I64 * len(seq))(*[int(v) for v in seq])
    return a
