"""ctypes binding of libq6moe.so, the C ABI declared in include/q6moe.h.

The library is built in-tree (``data-synth-tpu_amd/build.py``). There is no
fallback: if the shared object is missing or a call fails, the wrappers raise.
"""

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libq6moe.so"

F32 = 0
BF16 = 1
Q5_1 = 7
Q8_0 = 8
Q4_K = 12
Q5_K = 13
Q6_K = 14
# expert-table formats of the routed FFN
QTYPE_CODES = {"Q5_1": Q5_1, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}
# every GGUF tensor type q6moe_gguf_decode takes (GGMLQuantizationType values)
GGUF_TYPE_CODES = dict(QTYPE_CODES, F32=0, F16=1, Q4_0=2, Q4_1=3, Q5_0=6, IQ4_NL=20, BF16=30)

ERRORS = {-1: "invalid argument", -2: "HIP error", -3: "unsupported"}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_size = ctypes.c_size_t


class Table(ctypes.Structure):
    _fields_ = [
        ("qtype", _int),
        ("data", _vp),
        ("data_stride", _i64),
        ("scales", _vp),
        ("scale_stride", _i64),
    ]


class MoeArgs(ctypes.Structure):
    _fields_ = [
        ("gate", Table),
        ("up", Table),
        ("down", Table),
        ("experts", _i64),
        ("hidden", _i64),
        ("intermediate", _i64),
        ("x", _vp),
        ("ids", _vp),
        ("weights", _vp),
        ("tokens", _i64),
        ("top_k", _i64),
        ("shared_gate", Table),
        ("shared_up", Table),
        ("shared_down", Table),
        ("shared_intermediate", _i64),
        ("shared_scale", _vp),
        ("out", _vp),
        ("workspace", _vp),
        ("workspace_bytes", _size),
        ("mode", _int),
        ("events", ctypes.POINTER(_vp)),
        ("shared_router", _vp),
        ("compute", _int),
    ]


class KvArgs(ctypes.Structure):
    _fields_ = [
        ("codes", _vp),
        ("scales", _vp),
        ("scale_dtype", _int),
        ("scale_layout", _int),
        ("page_table", _vp),
        ("pool_pages", _i64),
        ("pages_per_seq", _i64),
        ("page_size", _i64),
        ("indices", _vp),
        ("batch", _i64),
        ("selected", _i64),
        ("capacity", _i64),
        ("kv_heads", _i64),
        ("head_dim", _i64),
        ("group", _i64),
        ("out", _vp),
        ("out_dtype", _int),
    ]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp),
        ("k_codes", _vp),
        ("v_codes", _vp),
        ("k_scales", _vp),
        ("v_scales", _vp),
        ("page_table", _vp),
        ("lengths", _vp),
        ("batch", _i64),
        ("query_heads", _i64),
        ("kv_heads", _i64),
        ("head_dim", _i64),
        ("pool_pages", _i64),
        ("pages_per_seq", _i64),
        ("page_size", _i64),
        ("out", _vp),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class KvWriteArgs(ctypes.Structure):
    _fields_ = [
        ("x", _vp),
        ("x_dtype", _int),
        ("codes", _vp),
        ("scales", _vp),
        ("scale_dtype", _int),
        ("scale_layout", _int),
        ("page_table", _vp),
        ("pool_pages", _i64),
        ("pages_per_seq", _i64),
        ("page_size", _i64),
        ("indices", _vp),
        ("active", _vp),
        ("batch", _i64),
        ("capacity", _i64),
        ("kv_heads", _i64),
        ("head_dim", _i64),
        ("group", _i64),
    ]


# name -> (restype, argtypes); exactly the entry points of include/q6moe.h
SIGNATURES = {
    "q6moe_version": (_int, []),
    "q6moe_last_error": (ctypes.c_char_p, []),
    "q6moe_q6_matmul": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _int, _i64, _vp]),
    "q6moe_q6_decode": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp]),
    "q6moe_q6_pack": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "q6moe_gguf_decode": (_int, [_vp, _int, _i64, _i64, _vp, _int, _vp]),
    "q6moe_moe_table_bytes": (_size, [_int, _i64, _i64]),
    "q6moe_moe_pack": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp]),
    "q6moe_moe_unpack": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _int, _vp, _vp]),
    "q6moe_sigmoid_probe": (_int, [_vp, _i64, _vp, _vp, _vp]),
    "q6moe_moe_workspace_size": (_size, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "q6moe_moe_forward": (_int, [ctypes.POINTER(MoeArgs), _vp]),
    "q6moe_moe_forward_noalloc": (_int, [ctypes.POINTER(MoeArgs), _vp]),
    "q6moe_q8_matmul_workspace_size": (_size, [_i64, _i64]),
    "q6moe_q8_matmul": (_int, [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _size, _vp]),
    "q6moe_kv_read": (_int, [ctypes.POINTER(KvArgs), _vp]),
    "q6moe_kv_gather_scales": (_int, [_vp, _int, _vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "q6moe_kv_quantize": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _int, _vp]),
    "q6moe_kv_write": (_int, [ctypes.POINTER(KvWriteArgs), _vp]),
    "q6moe_attn_workspace_size": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64]),
    "q6moe_route_topk": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "q6moe_kv_decode_attention": (_int, [ctypes.POINTER(AttnArgs), _vp]),
}

_lib = None


class Q6MoeError(RuntimeError):
    pass


def load(path=None):
    """Load (once) and return the shared library with typed entry points."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    target = Path(path) if path else Path(os.environ.get("Q6MOE_LIB", LIB_PATH))
    if not target.exists():
        raise Q6MoeError(
            f"{target} is missing: build it with `python data-synth-tpu_amd/build.py` "
            "(there is no CPU fallback)"
        )
    lib = ctypes.CDLL(str(target))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(rc, what):
    if rc != 0:
        msg = load().q6moe_last_error().decode(errors="replace")
        raise Q6MoeError(f"{what} failed ({ERRORS.get(rc, rc)}): {msg}")


def ptr(tensor):
    """Device pointer of a torch tensor (None -> NULL)."""
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def stream_handle(device=None):
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
