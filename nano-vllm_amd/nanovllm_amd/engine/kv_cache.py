"""Paged KV-cache allocation, mirroring ModelRunner.allocate_kv_cache
(nanovllm/engine/model_runner.py:110-149), with the fp8 e4m3fn extension.

The reference sizes the cache from the memory budget (:113-134): one block holds
block_size tokens of every layer's K and V, so

    block_bytes = 2 * num_layers * block_size * num_kv_heads * head_dim * itemsize
    num_blocks  = (total * gpu_memory_utilization - used - peak + current) // block_bytes

then allocates one (2, L, num_blocks, block_size, nkv, d) tensor (:136-143) and
binds k_cache = kv[0, l], v_cache = kv[1, l] on the l-th module that has both
attributes, in module order (:144-149).  That layout is the contract of every
kernel here (a slot is nkv * d contiguous elements, a page block_size slots).

fp8 extension: with kv_dtype=torch.float8_e4m3fn the cache holds one byte per
element (twice the blocks for the same budget) and this allocator also owns the
scales: one float32 per (K/V, layer, kv head) in kv_scale (2, L, nkv), bound as
module.k_scale = kv_scale[0, l] and module.v_scale = kv_scale[1, l] (store_kvcache
stores e4m3fn(x / scale), decode and prefill read x = e4m3 * scale).  They start
at 1 and are set by the caller before the first store, e.g. from calibration
amax values with set_scales_from_amax (scale = amax / 448, the e4m3fn maximum).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable

import torch

FP8_E4M3_MAX = 448.0
_DTYPES = (torch.bfloat16, torch.float8_e4m3fn)


@dataclass
class KVCache:
    kv_cache: torch.Tensor           # (2, L, num_blocks, block_size, nkv, d)
    kv_scale: torch.Tensor | None    # (2, L, nkv) float32 for fp8, else None
    num_blocks: int
    block_size: int

    @property
    def num_layers(self) -> int:
        return self.kv_cache.shape[1]

    def set_scales_from_amax(self, layer: int, k_amax: torch.Tensor, v_amax: torch.Tensor) -> None:
        """Per-kv-head scales amax / 448 of one layer (fp8 only).  Set them before the
        layer's first store: stored codes are not rescaled."""
        if self.kv_scale is None:
            raise RuntimeError("a bf16 cache has no scales")
        self.kv_scale[0, layer].copy_(k_amax.float() / FP8_E4M3_MAX)
        self.kv_scale[1, layer].copy_(v_amax.float() / FP8_E4M3_MAX)


def kv_block_bytes(num_layers: int, block_size: int, num_kv_heads: int, head_dim: int,
                   kv_dtype: torch.dtype = torch.bfloat16) -> int:
    """Bytes of one block across all layers, K and V (model_runner.py:123-130)."""
    itemsize = torch.empty((), dtype=kv_dtype).element_size()
    return 2 * num_layers * block_size * num_kv_heads * head_dim * itemsize


def budget_num_blocks(block_bytes: int, gpu_memory_utilization: float, device=None) -> int:
    """Blocks that fit the memory budget, as model_runner.py:113-134 computes it."""
    free, total = torch.cuda.mem_get_info(device)
    used = total - free
    stats = torch.cuda.memory_stats(device)
    peak = stats.get("allocated_bytes.all.peak", 0)
    current = stats.get("allocated_bytes.all.current", 0)
    return int(total * gpu_memory_utilization - used - peak + current) // block_bytes


def allocate_kv_cache(modules: Iterable[torch.nn.Module], num_layers: int, block_size: int, num_kv_heads: int,
                      head_dim: int, *, kv_dtype: torch.dtype = torch.bfloat16, num_blocks: int | None = None,
                      gpu_memory_utilization: float = 0.9, device=None) -> KVCache:
    """Allocate the paged cache and bind it (and, for fp8, its scales) on every module
    that has k_cache and v_cache attributes, in order.  num_blocks=None sizes the
    cache from the memory budget like the reference."""
    if kv_dtype not in _DTYPES:
        raise ValueError(f"kv_dtype must be one of {_DTYPES}")
    targets = [m for m in modules if hasattr(m, "k_cache") and hasattr(m, "v_cache")]
    if len(targets) != num_layers:
        raise ValueError(f"{len(targets)} modules with k_cache/v_cache for {num_layers} layers")
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if num_blocks is None:
        num_blocks = budget_num_blocks(kv_block_bytes(num_layers, block_size, num_kv_heads, head_dim, kv_dtype),
                                       gpu_memory_utilization, device)
    assert num_blocks > 0, "no KV-cache block fits the memory budget"
    shape = (2, num_layers, num_blocks, block_size, num_kv_heads, head_dim)
    if kv_dtype == torch.float8_e4m3fn:
        kv = torch.zeros(shape, dtype=torch.uint8, device=device).view(torch.float8_e4m3fn)
        kv_scale = torch.ones(2, num_layers, num_kv_heads, dtype=torch.float32, device=device)
    else:
        kv = torch.zeros(shape, dtype=kv_dtype, device=device)
        kv_scale = None
    for layer_id, m in enumerate(targets):
        m.k_cache = kv[0, layer_id]
        m.v_cache = kv[1, layer_id]
        if kv_scale is not None:
            m.k_scale = kv_scale[0, layer_id]
            m.v_scale = kv_scale[1, layer_id]
        elif hasattr(m, "k_scale"):
            m.k_scale = m.v_scale = None
    return KVCache(kv, kv_scale, num_blocks, block_size)
