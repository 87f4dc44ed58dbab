"""ctypes binding of libkvq.so (include/kvq.h).

Loading the library needs the ROCm runtime (libamdhip64) but no GPU; every argument
check in the library runs before any HIP call. There is deliberately no fallback: if the
library is missing the import of the op fails loudly.
"""
import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libkvq.so")

# kvq_status (include/kvq.h)
KVQ_OK = 0
KVQ_ERR_NULL_POINTER = -1
KVQ_ERR_SHAPE = -2
KVQ_ERR_UNSUPPORTED = -3
KVQ_ERR_ALIGNMENT = -4
KVQ_ERR_SPLITS = -5
KVQ_ERR_FORMAT = -6
KVQ_ERR_HIP = -7
KVQ_ERR_SCRATCH = -8

# KVQ_STATIC_SCRATCH_BYTES: the static device buffer of kvq_paged_decode_static
STATIC_SCRATCH_BYTES = 16 * 1024 * 1024

# kvq_kv_format
KV_FORMATS = {"fp16": 0, "int8": 1, "fp8_e4m3": 2, "int4": 3}

# Every symbol include/kvq.h declares; tests check the library exports all of them.
EXPORTED_SYMBOLS = (
    "kvq_version",
    "kvq_cache_format_version",
    "kvq_head_blocks",
    "kvq_status_string",
    "kvq_choose_num_splits",
    "kvq_plan_decode",
    "kvq_normalize_splits",
    "kvq_decode_split",
    "kvq_decode_merge",
    "kvq_decode_single",
    "kvq_paged_decode",
    "kvq_decode_units",
    "kvq_decode_units_split",
    "kvq_decode_units_merge",
    "kvq_plan_units",
    "kvq_quantize_cache",
    "kvq_quantize_append",
    "kvq_append_kv",
    "kvq_reshape_and_cache",
    "kvq_paged_decode_static",
)

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)


class DecodeArgs(ctypes.Structure):
    """Mirror of struct kvq_decode_args."""
    _fields_ = [
        ("q", _vp), ("q_stride_b", _i64), ("q_stride_h", _i64),
        ("k_cache", _vp), ("k_stride_blk", _i64), ("k_stride_tok", _i64), ("k_stride_head", _i64),
        ("v_cache", _vp), ("v_stride_blk", _i64), ("v_stride_tok", _i64), ("v_stride_head", _i64),
        ("block_table", _vp), ("bt_stride_b", _i64),
        ("seq_lens", _vp),
        ("out", _vp), ("o_stride_b", _i64), ("o_stride_h", _i64),
        ("batch", _i32), ("q_heads", _i32), ("kv_heads", _i32), ("head_dim", _i32),
        ("block_size", _i32), ("max_blocks", _i32), ("num_blocks", _i32),
        ("scale", ctypes.c_float),
        ("kv_format", _i32),
        ("k_group", _i32),
        ("k_scale", _vp), ("k_zero", _vp), ("v_scale", _vp), ("v_zero", _vp),
        ("waves_per_group", _i32),
        ("pipeline", _i32),
    ]


class KvqError(RuntimeError):
    """A libkvq call returned a negative kvq_status."""

    def __init__(self, func, status, text):
        super().__init__(f"{func} failed: {text} (status {status})")
        self.status = status


_lib = None


def lib():
    """The loaded library (loaded on first use)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m kvq_decode_amd.build` "
                "(there is no CPU fallback for this op)")
        L = ctypes.CDLL(LIB_PATH)
        L.kvq_version.restype = ctypes.c_char_p
        L.kvq_version.argtypes = []
        L.kvq_cache_format_version.restype = ctypes.c_int
        L.kvq_cache_format_version.argtypes = []
        L.kvq_head_blocks.restype = ctypes.c_int
        L.kvq_head_blocks.argtypes = [_i32, _i32]
        L.kvq_status_string.restype = ctypes.c_char_p
        L.kvq_status_string.argtypes = [ctypes.c_int]
        L.kvq_choose_num_splits.restype = ctypes.c_int
        L.kvq_choose_num_splits.argtypes = [_i32] * 7
        L.kvq_plan_decode.restype = ctypes.c_int
        L.kvq_plan_decode.argtypes = [_i32] * 8 + [ctypes.POINTER(_i32)] * 2
        L.kvq_plan_units.restype = ctypes.c_int
        L.kvq_plan_units.argtypes = [_i32] * 8 + [ctypes.POINTER(_i32)] * 2
        L.kvq_normalize_splits.restype = ctypes.c_int
        L.kvq_normalize_splits.argtypes = [_i32, _i32, ctypes.POINTER(_i32), ctypes.POINTER(_i32)]
        args_p = ctypes.POINTER(DecodeArgs)
        L.kvq_decode_split.restype = ctypes.c_int
        L.kvq_decode_split.argtypes = [args_p, _i32, _i32, _vp, _vp, _vp]
        L.kvq_decode_merge.restype = ctypes.c_int
        L.kvq_decode_merge.argtypes = [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp]
        L.kvq_decode_single.restype = ctypes.c_int
        L.kvq_decode_single.argtypes = [args_p, _vp]
        L.kvq_paged_decode.restype = ctypes.c_int
        L.kvq_paged_decode.argtypes = [args_p, _i32, _vp, _vp, _vp]
        L.kvq_decode_units.restype = ctypes.c_int
        L.kvq_decode_units.argtypes = [args_p, _i32, _vp, _vp, _vp]
        L.kvq_decode_units_split.restype = ctypes.c_int
        L.kvq_decode_units_split.argtypes = [args_p, _i32, _vp, _vp, _vp]
        L.kvq_decode_units_merge.restype = ctypes.c_int
        L.kvq_decode_units_merge.argtypes = [args_p, _i32, _vp, _vp, _vp]
        L.kvq_quantize_cache.restype = ctypes.c_int
        L.kvq_quantize_cache.argtypes = [args_p, _vp, _vp, _i64, _i64, _i64, _vp]
        L.kvq_quantize_append.restype = ctypes.c_int
        L.kvq_quantize_append.argtypes = [args_p, _vp, _vp, _vp, _vp]
        L.kvq_append_kv.restype = ctypes.c_int
        L.kvq_append_kv.argtypes = [args_p, _vp, _vp, _vp]
        L.kvq_reshape_and_cache.restype = ctypes.c_int
        L.kvq_reshape_and_cache.argtypes = [args_p, _vp, _vp, _i64, _i64, _vp, _i32, _vp]
        L.kvq_paged_decode_static.restype = ctypes.c_int
        L.kvq_paged_decode_static.argtypes = [args_p, _i32, _i32, _vp]
        _lib = L
    return _lib


def check(func, status):
    """Raise KvqError for a negative status; return the status otherwise."""
    if status < 0:
        text = lib().kvq_status_string(status).decode()
        raise KvqError(func, status, text)
    return status


def version():
    return lib().kvq_version().decode()
