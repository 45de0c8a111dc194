"""ctypes binding of include/smoe.h (libsmoe.so).

Loading fails loudly when the library has not been built: there is no
fallback path. Build with ``python streamoe_amd/build.py``.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# SMOE_LIB names another build of the same library (e.g. one compiled with
# different kernel tunables); the default is the in-tree build.
LIB_PATH = os.environ.get("SMOE_LIB") or os.path.join(HERE, "libsmoe.so")

SMOE_MAX_K = 16
SMOE_ABI_VERSION = 2  # the struct layouts below (include/smoe.h SMOE_ABI_VERSION)

STATUS = {
    0: "SMOE_OK",
    1: "SMOE_ERR_INVALID_ARG",
    2: "SMOE_ERR_BAD_K",
    3: "SMOE_ERR_IN_DIM_NOT_MULTIPLE",
    4: "SMOE_ERR_UNSUPPORTED_BITS",
    5: "SMOE_ERR_UNSUPPORTED_GROUP",
    6: "SMOE_ERR_UNSUPPORTED_SHAPE",
    7: "SMOE_ERR_MISALIGNED",
    8: "SMOE_ERR_SCRATCH_TOO_SMALL",
    9: "SMOE_ERR_WORKSPACE_TOO_SMALL",
    10: "SMOE_ERR_HIP",
    11: "SMOE_ERR_NO_DEVICE",
    12: "SMOE_ERR_DEVICE_TIMEOUT",
    13: "SMOE_ERR_IO",
}
SMOE_OPT_DECODE_PATH = 1
SMOE_OPT_TRACE_BUFFER = 2
SMOE_OPT_PREFILL_GEMM = 3
CODES = {v: k for k, v in STATUS.items()}


class SmoeError(RuntimeError):
    """A non-zero status from libsmoe."""

    def __init__(self, status, where):
        self.status = status
        self.name = STATUS.get(status, f"status {status}")
        super().__init__(f"{where}: {self.name}")


class QWeights(C.Structure):
    _fields_ = [
        ("base", C.c_void_p),
        ("packed_offset", C.c_uint64),
        ("scales_offset", C.c_uint64),
        ("biases_offset", C.c_uint64),
        ("group_size", C.c_uint32),
        ("bits", C.c_uint32),
    ]


class ExpertShape(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32),
        ("inter", C.c_uint32),
        ("group", C.c_uint32),
        ("bits", C.c_uint32),
    ]


class Binding(C.Structure):
    _fields_ = [("base", C.c_void_p), ("offset", C.c_uint64)]


class Layer(C.Structure):
    _fields_ = [
        ("shape", ExpertShape),
        ("experts", C.c_void_p),
        ("stride", C.c_uint64),
        ("n_experts", C.c_uint32),
        ("k", C.c_uint32),
        ("normalize", C.c_int32),
        ("router_w", C.c_void_p),
        ("shared_expert", C.c_void_p),
        ("shared_gate", C.c_void_p),
        ("router_q", C.c_void_p),        # const smoe_qweights* (8-bit router) or NULL
        ("shared_gate_q", C.c_void_p),   # const smoe_qweights* (8-bit shared gate) or NULL
    ]


class FileLayout(C.Structure):
    _fields_ = [
        ("bits", C.c_uint32),
        ("reserved", C.c_uint32),
        ("expert_size", C.c_uint64),
        ("stride", C.c_uint64),
    ]


_P = C.c_void_p
_U32 = C.c_uint32
_U64 = C.c_uint64
_I = C.c_int

# name -> (restype, argtypes); the order follows include/smoe.h.
PROTOTYPES = {
    "smoe_strerror": (C.c_char_p, [_I]),
    "smoe_abi_version": (_U32, []),
    "smoe_create": (_I, [_I, _P, C.POINTER(_P)]),
    "smoe_destroy": (_I, [_P]),
    "smoe_set_stream": (_I, [_P, _P]),
    "smoe_reserve": (_I, [_P, _U32, _U32, _U32]),
    "smoe_sync": (_I, [_P]),
    "smoe_set_option": (_I, [_P, _I, C.c_int64]),
    "smoe_qmv": (_I, [_P, C.POINTER(QWeights), _P, _P, _U32, _U32]),
    "smoe_qmv_argmax": (_I, [_P, C.POINTER(QWeights), _P, _P, _U32, _U32, _P]),
    "smoe_qmm_workspace_size": (_U64, [_U32, _U32, _U32]),
    "smoe_qmm": (_I, [_P, C.POINTER(QWeights), _P, _P, _U32, _U32, _U32, _P, _U64]),
    "smoe_argmax": (_I, [_P, _P, _U32, _P]),
    "smoe_dequant": (_I, [_P, C.POINTER(QWeights), _U32, _U32, _U32, _P]),
    "smoe_router": (_I, [_P, _P, _P, _U32, _U32, _U32, _U32, _I, _P, _P, _P]),
    "smoe_softmax_topk": (_I, [_P, _P, _U32, _U32, _U32, _I, _P, _P]),
    "smoe_softmax": (_I, [_P, _P, _U32, _U32, _P]),
    "smoe_expf": (_I, [_P, _P, _P, _U64]),
    "smoe_topk": (_I, [_P, _P, _U32, _U32, _U32, _P, _P]),
    "smoe_noaux_tc_topk": (_I, [_P, _P, _P, _U32, _U32, _U32, _U32, _U32, C.c_float, _P, _P, _P]),
    "smoe_expert_bytes": (_U64, [C.POINTER(ExpertShape)]),
    "smoe_experts_decode": (_I, [_P, C.POINTER(ExpertShape), C.POINTER(Binding), _U32, C.POINTER(C.c_float),
                                 _P, _P, _P, C.c_float, _P]),
    "smoe_moe_decode_layer": (_I, [_P, C.POINTER(Layer), _P, _P, _P, _P, _P]),
    "smoe_moe_decode_layers": (_I, [_P, C.POINTER(Layer), _U32, C.POINTER(_P), C.c_float, _P, _P, _P]),
    "smoe_moe_decode_layers_noalloc": (_I, [_P, C.POINTER(Layer), _U32, C.POINTER(_P), C.c_float, _P, _P]),
    "smoe_moe_decode_tokens": (_I, [_P, C.POINTER(Layer), _U32, C.POINTER(_P), C.c_float, _U32, _P, _P, _P, _P,
                                    _P]),
    "smoe_moe_prefill_workspace_size": (_U64, [C.POINTER(ExpertShape), _U32, _U32, _U32]),
    "smoe_moe_prefill": (_I, [_P, C.POINTER(ExpertShape), _P, _U64, _U32, _P, _P, _P, _I, _U32, _U32, _P, _P,
                              _U64]),
    "smoe_moe_prefill_block_workspace_size": (_U64, [C.POINTER(ExpertShape), _U32, _U32, _U32, _I]),
    "smoe_moe_prefill_block": (_I, [_P, C.POINTER(ExpertShape), _P, _U64, _U32, _P, _P, _P, _I, _U32, _U32, _P,
                                    _P, _P, _P, _P, _U64]),
    "smoe_layer_file_layout": (_I, [_U64, _U32, _U32, _U32, _U32, _U64, _U64, C.POINTER(FileLayout)]),
    "smoe_load_file": (_I, [_P, C.c_char_p, _U64, _U64, _P, _U64, C.POINTER(_U64)]),
    "smoe_stream_read": (_I, [_P, _P, C.c_uint64, _P]),
    "smoe_synth_experts": (_I, [_P, _P, _U32, _U64, C.POINTER(ExpertShape), _U64, C.c_float, C.c_float]),
    "smoe_synth_normal_f32": (_I, [_P, _P, _U64, _U64, C.c_float]),
    "smoe_synth_normal_bf16": (_I, [_P, _P, _U64, _U64, C.c_float]),
}

_lib = None


def load():
    """Load libsmoe.so once; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python streamoe_amd/build.py` (no CPU fallback exists)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.smoe_abi_version() != SMOE_ABI_VERSION:
        raise ImportError(f"{LIB_PATH} has ABI version {lib.smoe_abi_version()}, these bindings "
                          f"{SMOE_ABI_VERSION}; rebuild it (python streamoe_amd/build.py)")
    _lib = lib
    return lib


def check(status, where):
    if status != 0:
        raise SmoeError(status, where)
    return status
