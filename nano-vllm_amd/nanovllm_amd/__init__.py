"""nano-vllm's attention hot path, MI355X-native (gfx950 HIP kernels behind a C ABI).

Public surface, mirroring the reference package layout:
  nanovllm_amd.layers.attention   Attention, store_kvcache, flash_attn_varlen_func,
                                  flash_attn_with_kvcache, store_and_decode
  nanovllm_amd.utils.context      Context, get_context, set_context, reset_context
  nanovllm_amd.engine.kv_cache    allocate_kv_cache (model_runner.py:110-149, + fp8 scales)
  nanovllm_amd.engine.decode_graphs  DecodeGraphs (model_runner.py:260-336)
"""
from . import _capi
from .layers.attention import (Attention, flash_attn_varlen_func, flash_attn_with_kvcache,
                               store_and_decode, store_kvcache)
from .utils.context import Context, get_context, reset_context, set_context

__all__ = [
    "Attention", "store_kvcache", "flash_attn_varlen_func", "flash_attn_with_kvcache", "store_and_decode",
    "Context", "get_context", "set_context", "reset_context", "library_path",
]


def library_path() -> str:
    return str(_capi.LIB_PATH)
