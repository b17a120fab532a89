"""ctypes binding of libdrofell_w4a16.so (C ABI: include/drofell_w4a16.h).

The library is built in-tree by ``drofell-for-revision_amd/csrc/Makefile``
(``__graft_entry__.build()`` runs it).  There is no fallback: if the shared
object is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

LIB_NAME = "libdrofell_w4a16.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

DW4_OK = 0
DW4_ERR_INVALID_ARG = 1
DW4_ERR_UNSUPPORTED = 2
DW4_ERR_MISALIGNED = 3
DW4_ERR_BAD_GIDX = 4
DW4_ERR_WORKSPACE = 5
DW4_ERR_LAUNCH = 6
DW4_ERR_DEVICE = 7
DW4_ERR_SCRATCH = 8
NOALLOC_SCRATCH_BYTES = 64 << 20

DW4_PATH_AUTO = 0
DW4_PATH_DECODE = 1
DW4_PATH_PREFILL = 2

_c = ctypes
_P = _c.c_void_p
_SZ = _c.POINTER(_c.c_size_t)


class Item(ctypes.Structure):
    """``dw4_item``: one quantized matrix (packed buffers) and its output."""

    _fields_ = [("k", _c.c_int), ("n", _c.c_int), ("group_size", _c.c_int),
                ("packed_qweight", _P), ("packed_zeros", _P), ("packed_scales", _P),
                ("perm", _P), ("bias", _P), ("y", _P), ("ldy", _c.c_int64)]


_IP = _c.POINTER(Item)


class ChainLink(ctypes.Structure):
    """``dw4_chain_link``: one projection of a decode chain."""

    _fields_ = [("k", _c.c_int), ("n", _c.c_int), ("group_size", _c.c_int),
                ("packed_qweight", _P), ("packed_zeros", _P), ("packed_scales", _P),
                ("perm", _P), ("x", _P), ("ldx", _c.c_int64), ("bias", _P),
                ("residual", _P), ("ldres", _c.c_int64), ("y", _P), ("ldy", _c.c_int64),
                ("after", _c.c_int)]


class ChainPlan(ctypes.Structure):
    """``dw4_chain_plan``: filled by dw4_chain_prepare, read by dw4_gemm_chain."""

    _fields_ = [("count", _c.c_int), ("m", _c.c_int), ("workgroups", _c.c_int),
                ("waves", _c.c_int), ("ring", _c.c_int), ("max_k", _c.c_int),
                ("max_strips", _c.c_int), ("max_groups", _c.c_int),
                ("smem_bytes", _c.c_size_t)]


_CLP = _c.POINTER(ChainLink)
_CPP = _c.POINTER(ChainPlan)

# Every symbol the public header declares, with its ctypes signature.
SIGNATURES = {
    "dw4_abi_version": (_c.c_int, []),
    "dw4_strerror": (_c.c_char_p, [_c.c_int]),
    "dw4_query_sizes": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                   _SZ, _SZ, _SZ, _SZ, _SZ]),
    "dw4_workspace_size": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _SZ]),
    "dw4_make_perm": (_c.c_int, [_c.c_int, _c.c_int, _P, _P]),
    "dw4_repack": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _P, _P, _P, _P, _P, _P, _P, _P]),
    "dw4_gemm": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int64,
                            _P, _P, _P, _P, _P, _P, _c.c_int64, _P, _c.c_size_t, _P]),
    "dw4_gemm_bf16": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int64,
                                 _P, _P, _P, _P, _P, _P, _c.c_int64, _P, _c.c_size_t, _P]),
    "dw4_gemm_path": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                 _P, _c.c_int64, _P, _P, _P, _P, _P, _P, _c.c_int64,
                                 _P, _c.c_size_t, _P]),
    "dw4_dequant": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _P, _P, _P, _P, _P,
                               _c.c_int64, _P]),
    "dw4_gemm_noalloc": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int64,
                                    _P, _P, _P, _P, _P, _P, _c.c_int64, _P]),
    "dw4_dequant_bf16": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _P, _P, _P, _P, _P,
                                    _c.c_int64, _P]),
    "dw4_stream_read": (_c.c_int, [_P, _c.c_size_t, _c.c_int, _c.c_int, _c.c_uint32, _P, _P]),
    "dw4_gemm_t": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int64, _P, _P, _P,
                              _P, _P, _c.c_int64, _P, _c.c_size_t, _P]),
    "dw4_gemm_t_workspace_size": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                             _c.POINTER(_c.c_size_t)]),
    "dw4_reshape_and_cache": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int64,
                                         _P, _c.c_int64, _P, _P, _c.c_int, _P, _P]),
    "dw4_restore_from_cache": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int64,
                                          _P, _c.c_int64, _P, _P, _c.c_int, _P, _P]),
    "dw4_paged_attention": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _P,
                                       _c.c_int64, _P, _c.c_int64, _P, _P, _c.c_int, _c.c_float,
                                       _P, _c.c_int, _P, _c.c_int, _P, _P, _c.c_size_t, _P]),
    "dw4_paged_attention_workspace_size": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                                      _c.c_int, _c.c_int,
                                                      _c.POINTER(_c.c_size_t)]),
    "dw4_rope": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _P, _P, _P, _c.c_int,
                            _c.c_int, _P, _P]),
    "dw4_rope_and_cache": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _P,
                                      _c.c_int64, _P, _c.c_int64, _P, _c.c_int64, _P, _P,
                                      _c.c_int, _P, _P, _c.c_int, _P, _P, _c.c_int, _P, _P]),
    "dw4_gemm_group": (_c.c_int, [_c.c_int, _IP, _c.c_int, _P, _c.c_int64, _P, _c.c_size_t, _P]),
    "dw4_gemm_silu_mul": (_c.c_int, [_c.c_int, _P, _c.c_int64, _IP, _IP, _P, _c.c_int64,
                                     _P, _c.c_size_t, _P]),
    "dw4_rms_norm": (_c.c_int, [_c.c_int, _c.c_int, _P, _c.c_int64, _P, _c.c_float, _P,
                                _c.c_int64, _P]),
    "dw4_attention_qkv_stage": (_c.c_int, [_c.c_int, _P, _c.c_int64, _P, _c.c_float, _P,
                                           _c.c_int64, _IP, _IP, _IP, _P, _c.c_size_t, _P]),
    "dw4_mlp_forward": (_c.c_int, [_c.c_int, _P, _c.c_int64, _P, _c.c_float, _P, _c.c_int64,
                                   _IP, _IP, _IP, _P, _c.c_size_t, _P]),
    "dw4_decoder_after_stage": (_c.c_int, [_c.c_int, _P, _c.c_int64, _P, _c.c_int64, _IP, _P,
                                           _c.c_float, _P, _c.c_int64, _IP, _IP, _IP, _P,
                                           _c.c_size_t, _P]),
    "dw4_chain_buffer_size": (_c.c_int, [_c.c_int, _SZ]),
    "dw4_chain_prepare": (_c.c_int, [_c.c_int, _CLP, _c.c_int, _P, _c.c_size_t, _CPP]),
    "dw4_gemm_chain": (_c.c_int, [_CPP, _P, _P]),
    "dw4_chain_timed_out": (_c.c_int, [_P, _c.POINTER(_c.c_int)]),
}
ABI_VERSION = 11
BF16_MAX_M = 64  # DW4_BF16_MAX_M

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


class W4A16Error(RuntimeError):
    """A non-zero status returned by the native library."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the native library; raises if it is absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"{LIB_NAME} is not built ({path} missing); run "
                "`make -C drofell-for-revision_amd/csrc` or __graft_entry__.build()")
        # torch first: its wheel carries its own HIP runtime, and the library's
        # libamdhip64.so.7 dependency binds to the one already loaded.  Loaded
        # before torch, the library would bring in the system runtime and the
        # process would hold two (kernel launches then fail, and pointers and
        # streams from torch would belong to the other runtime).
        import torch  # noqa: F401
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.dw4_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def strerror(status: int) -> str:
    return load().dw4_strerror(status).decode()


def check(fn: str, status: int) -> None:
    if status != DW4_OK:
        raise W4A16Error(fn, status, strerror(status))


def call(fn: str, *args) -> None:
    lib = load()
    check(fn, getattr(lib, fn)(*args))


def query_sizes(k: int, n: int, group_size: int, act_order: bool, max_m: int) -> dict:
    lib = load()
    out = [ctypes.c_size_t(0) for _ in range(5)]
    check("dw4_query_sizes", lib.dw4_query_sizes(
        k, n, group_size, int(act_order), max_m, *[ctypes.byref(o) for o in out]))
    keys = ("packed_qweight", "packed_scales", "packed_zeros", "perm", "workspace")
    return {key: o.value for key, o in zip(keys, out)}


def workspace_size(m: int, k: int, n: int, group_size: int, act_order: bool) -> int:
    lib = load()
    out = ctypes.c_size_t(0)
    check("dw4_workspace_size", lib.dw4_workspace_size(m, k, n, group_size, int(act_order),
                                                       ctypes.byref(out)))
    return out.value


def gemm_t_workspace_size(m: int, k: int, n: int, group_size: int) -> int:
    lib = load()
    out = ctypes.c_size_t(0)
    check("dw4_gemm_t_workspace_size",
          lib.dw4_gemm_t_workspace_size(m, k, n, group_size, ctypes.byref(out)))
    return out.value


def paged_attention_workspace_size(num_seqs: int, num_heads: int, num_kv_heads: int,
                                   head_size: int, block_size: int, max_context_len: int) -> int:
    lib = load()
    out = ctypes.c_size_t(0)
    check("dw4_paged_attention_workspace_size", lib.dw4_paged_attention_workspace_size(
        num_seqs, num_heads, num_kv_heads, head_size, block_size, max_context_len,
        ctypes.byref(out)))
    return out.value
