"""ctypes binding of libnva_attn.so (the C ABI in include/nva_attention.h).

The library is built in-tree by nano-vllm_amd/build.py.  There is no fallback:
if it is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libnva_attn.so"

NVA_OK = 0
NVA_ERR_INVALID_ARGUMENT = 1
NVA_ERR_UNSUPPORTED = 2
NVA_ERR_HIP = 3
NVA_ERR_WORKSPACE = 4

NVA_DTYPE_BF16 = 0
NVA_DTYPE_FP8_E4M3 = 1

NVA_PREFILL_ERR_SPLIT_WAIT = 1
# byte offset of the prefill workspace's poll-limit word (a test hook: 0 = default bound)
NVA_PREFILL_SPLIT_WAIT_LIMIT_OFFSET = 132

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# name -> (restype, argtypes); the order follows include/nva_attention.h.
SIGNATURES = {
    "nva_version": (_i32, []),
    "nva_last_error": (ctypes.c_char_p, []),
    "nva_store_kvcache": (_i32, [
        _c_void_p, _i64, _c_void_p, _i64,  # key, key_row_stride, value, value_row_stride
        _c_void_p, _c_void_p, _i64,        # k_cache, v_cache, num_slots
        _c_void_p, _i64,                   # slot_mapping, num_tokens
        _i32, _i32, _i32,                  # num_kv_heads, head_dim, cache_dtype
        _c_void_p, _c_void_p, _c_void_p,   # k_scale, v_scale, stream
    ]),
    "nva_prefill": (_i32, [
        _c_void_p, _i64,                   # q, q_row_stride
        _c_void_p, _i64, _c_void_p, _i64,  # k, k_row_stride, v, v_row_stride
        _c_void_p, _i64, _i32, _i32, _i64,  # block_table, bt_row_stride, max_blocks, block_size, num_blocks
        _c_void_p, _c_void_p, _i32, _i32, _i32,  # cu_q, cu_k, num_seqs, max_seqlen_q, max_seqlen_k
        _i32, _i32, _i32, _f32,            # num_heads, num_kv_heads, head_dim, softmax_scale
        _c_void_p, _i64,                   # out, out_row_stride
        _c_void_p, _i64, _c_void_p,        # workspace, workspace_bytes, stream
    ]),
    "nva_prefill_workspace_bytes": (_i64, []),
    "nva_prefill_workspace_errors": (_i32, [
        _c_void_p, _i64, ctypes.POINTER(ctypes.c_uint32), _c_void_p,  # workspace, bytes, errors, stream
    ]),
    "nva_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "nva_store_decode": (_i32, [
        _c_void_p, _i64, _c_void_p, _i64,  # key, key_row_stride, value, value_row_stride
        _c_void_p,                         # slot_mapping
        _c_void_p, _i64,                   # q, q_row_stride
        _c_void_p, _c_void_p, _i32,        # k_cache, v_cache, kv_dtype
        _c_void_p, _c_void_p, _i64,        # k_scale, v_scale, num_blocks
        _c_void_p, _c_void_p, _i64, _i32, _i32,  # seqlens, block_table, bt_row_stride, max_blocks, block_size
        _i32, _i32, _i32, _i32, _f32, _i32,  # batch, nh, nkv, head_dim, scale, num_splits
        _c_void_p, _i64,                   # out, out_row_stride
        _c_void_p, _i64, _c_void_p,        # workspace, workspace_bytes, stream
    ]),
    "nva_decode": (_i32, [
        _c_void_p, _i64,                   # q, q_row_stride
        _c_void_p, _c_void_p, _i32,        # k_cache, v_cache, kv_dtype
        _c_void_p, _c_void_p, _i64,        # k_scale, v_scale, num_blocks
        _c_void_p, _c_void_p, _i64, _i32, _i32,  # seqlens, block_table, bt_row_stride, max_blocks, block_size
        _i32, _i32, _i32, _i32, _f32, _i32,  # batch, nh, nkv, head_dim, scale, num_splits
        _c_void_p, _i64,                   # out, out_row_stride
        _c_void_p, _i64, _c_void_p,        # workspace, workspace_bytes, stream
    ]),
    "nva_decode_noalloc": (_i32, [
        _c_void_p, _i64,                   # q, q_row_stride
        _c_void_p, _c_void_p, _i32,        # k_cache, v_cache, kv_dtype
        _c_void_p, _c_void_p, _i64,        # k_scale, v_scale, num_blocks
        _c_void_p, _c_void_p, _i64, _i32, _i32,  # seqlens, block_table, bt_row_stride, max_blocks, block_size
        _i32, _i32, _i32, _i32, _f32, _i32,  # batch, nh, nkv, head_dim, scale, num_splits
        _c_void_p, _i64, _c_void_p,        # out, out_row_stride, stream
    ]),
    "nva_decode_noalloc_max_workspace_bytes": (_i64, []),
    "nva_gather_kv": (_i32, [
        _c_void_p, _c_void_p, _i32,        # k_cache, v_cache, kv_dtype
        _c_void_p, _c_void_p, _i64,        # k_scale, v_scale, num_blocks
        _c_void_p, _i64, _i32, _i32,       # block_table, bt_row_stride, max_blocks, block_size
        _c_void_p, _i32, _i32,             # cu_seqlens_k, num_seqs, max_seqlen_k
        _i32, _i32,                        # num_kv_heads, head_dim
        _c_void_p, _c_void_p, _i64, _i64,  # k_out, v_out, out_rows, out_row_stride
        _c_void_p,                         # stream
    ]),
    "nva_qk_norm_rope": (_i32, [
        _c_void_p, _i64, _c_void_p, _i64,  # q, q_row_stride, k, k_row_stride
        _c_void_p, _i64, _c_void_p, _i64,  # q_out, q_out_row_stride, k_out, k_out_row_stride
        _c_void_p, _c_void_p, _f32,        # q_norm_weight, k_norm_weight, eps
        _c_void_p, _i64, _c_void_p, _i64,  # cos_sin_cache, max_position, positions, num_tokens
        _i32, _i32, _i32, _c_void_p,       # num_heads, num_kv_heads, head_dim, stream
    ]),
}


class NvaError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[nva error {code}] {message}")
        self.code = code


_lib = None
_lock = threading.Lock()


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with argument types set."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"{p} is not built: run `python nano-vllm_amd/build.py` (hipcc, gfx950); "
                "there is no non-HIP fallback")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def check(status: int) -> None:
    if status != NVA_OK:
        msg = load().nva_last_error()
        raise NvaError(status, msg.decode() if msg else "")
