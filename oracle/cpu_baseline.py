"""PyTorch CPU restatement of the reference's attention path -- the timed CPU
baseline of bench.py (TEST / MEASUREMENT INFRASTRUCTURE ONLY; never the product).

The reference has no CPU attention path (nanovllm/layers/attention.py:6 imports
flash-attn unconditionally), so this restates attention.py:58-79 with torch CPU
operators, as the benchmark plan prescribes:
  * store: k_cache.view(-1, D).index_copy_(0, slot_mapping, key.reshape(T, D))
    (attention.py:32-39);
  * attention: per sequence, gather its pages through block_table
    (model_runner.py:151-159), then
    torch.nn.functional.scaled_dot_product_attention(..., enable_gqa=True) with a
    bottom-right causal mask (SDPA's is_causal is top-left aligned, so an explicit
    mask is passed whenever Lq != Lk);
  * fp8 caches are dequantised (code value * per-kv-head scale) per sequence.
Inputs stay bf16; the thread count is whatever torch.set_num_threads set.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    T, nkv, d = key.shape
    D = nkv * d
    idx = slot_mapping.long()
    k_cache.view(-1, D).index_copy_(0, idx, key.reshape(T, D))
    v_cache.view(-1, D).index_copy_(0, idx, value.reshape(T, D))


def store_kvcache_fp8(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale):
    """The fp8 cache's store: e4m3fn(x / scale[h]) by torch's float8_e4m3fn cast, then
    the byte rows copied as store_kvcache does (caches: float8_e4m3fn tensors)."""
    k8 = (key.float() / k_scale.view(1, -1, 1)).to(torch.float8_e4m3fn).view(torch.uint8)
    v8 = (value.float() / v_scale.view(1, -1, 1)).to(torch.float8_e4m3fn).view(torch.uint8)
    store_kvcache(k8, v8, k_cache.view(torch.uint8), v_cache.view(torch.uint8), slot_mapping)


def _gather(cache, table_row, L, bs):
    pages = table_row[: math.ceil(L / bs)].long()
    return cache.index_select(0, pages).reshape(-1, cache.shape[2], cache.shape[3])[:L]


def decode(q, k_cache, v_cache, context_lens, block_tables, scale, k_scale=None, v_scale=None):
    """q (B, nh, d) -> (B, nh, d)."""
    B, nh, d = q.shape
    bs = k_cache.shape[1]
    out = torch.zeros_like(q)
    lens = context_lens.tolist()
    for b in range(B):
        L = lens[b]
        if L <= 0:
            continue
        K = _gather(k_cache, block_tables[b], L, bs)
        V = _gather(v_cache, block_tables[b], L, bs)
        if k_scale is not None:
            K = (K.float() * k_scale.view(1, -1, 1)).to(q.dtype)
            V = (V.float() * v_scale.view(1, -1, 1)).to(q.dtype)
        o = F.scaled_dot_product_attention(q[b].view(1, nh, 1, d), K.permute(1, 0, 2)[None],
                                           V.permute(1, 0, 2)[None], scale=scale, enable_gqa=True)
        out[b] = o[0, :, 0]
    return out


def prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, block_table=None):
    """Varlen causal prefill over packed k/v, or over the paged caches."""
    total, nh, d = q.shape
    out = torch.zeros_like(q)
    cu_q = cu_seqlens_q.tolist()
    cu_k = cu_seqlens_k.tolist()
    for s in range(len(cu_q) - 1):
        Lq, Lk = cu_q[s + 1] - cu_q[s], cu_k[s + 1] - cu_k[s]
        if Lq == 0:
            continue
        if block_table is None:
            K, V = k[cu_k[s]:cu_k[s + 1]], v[cu_k[s]:cu_k[s + 1]]
        else:
            bs = k.shape[1]
            K, V = _gather(k, block_table[s], Lk, bs), _gather(v, block_table[s], Lk, bs)
        qs = q[cu_q[s]:cu_q[s + 1]].permute(1, 0, 2)[None]
        if Lq == Lk:
            o = F.scaled_dot_product_attention(qs, K.permute(1, 0, 2)[None], V.permute(1, 0, 2)[None],
                                               is_causal=True, scale=scale, enable_gqa=True)
        else:
            mask = torch.ones(Lq, Lk, dtype=torch.bool).tril(diagonal=Lk - Lq)
            o = F.scaled_dot_product_attention(qs, K.permute(1, 0, 2)[None], V.permute(1, 0, 2)[None],
                                               attn_mask=mask, scale=scale, enable_gqa=True)
        out[cu_q[s]:cu_q[s + 1]] = o[0].permute(1, 0, 2)
    return out
