"""Argument checks of the Python mirror (layers/attention.py) that must fire
before any launch: tensors on the wrong device, block tables with the wrong
number of rows, head dims that differ between q and the cache, packed k/v of
different shapes.  Everything here runs on the CPU, where every tensor is a
host tensor, so a check that did not fire would reach the C ABI with a host
pointer."""
from __future__ import annotations

import pytest
import torch

from nanovllm_amd.layers.attention import flash_attn_varlen_func, flash_attn_with_kvcache, store_kvcache

BF16 = torch.bfloat16


def _prefill_inputs(nseq=3, lq=5, nh=4, nkv=2, d=64):
    q = torch.zeros(nseq * lq, nh, d, dtype=BF16)
    cu = torch.arange(0, nseq * lq + 1, lq, dtype=torch.int32)
    return q, cu


def test_store_rejects_host_tensors():
    key = torch.zeros(4, 2, 64, dtype=BF16)
    cache = torch.zeros(8, 16, 2, 64, dtype=BF16)
    with pytest.raises(RuntimeError, match="CUDA"):
        store_kvcache(key, key.clone(), cache, cache.clone(), torch.zeros(4, dtype=torch.int32))


def test_prefill_paged_block_table_rows_must_match_sequences():
    q, cu = _prefill_inputs()
    cache = torch.zeros(8, 64, 2, 64, dtype=BF16)
    bt = torch.zeros(2, 4, dtype=torch.int32)  # 2 rows for 3 sequences
    with pytest.raises(RuntimeError, match="rows"):
        flash_attn_varlen_func(q, cache, cache.clone(), 5, cu, 5, cu, None, True, bt)


def test_prefill_paged_head_dim_must_match():
    q, cu = _prefill_inputs(d=64)
    cache = torch.zeros(8, 64, 2, 128, dtype=BF16)
    bt = torch.zeros(3, 4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="head_dim"):
        flash_attn_varlen_func(q, cache, cache.clone(), 5, cu, 5, cu, None, True, bt)


def test_prefill_packed_k_v_shapes_must_match():
    q, cu = _prefill_inputs()
    k = torch.zeros(15, 2, 64, dtype=BF16)
    v = torch.zeros(14, 2, 64, dtype=BF16)
    with pytest.raises(RuntimeError, match="packed k/v"):
        flash_attn_varlen_func(q, k, v, 5, cu, 5, cu)


@pytest.mark.parametrize("paged", [False, True])
def test_prefill_rejects_host_tensors(paged):
    q, cu = _prefill_inputs()
    if paged:
        k = torch.zeros(8, 64, 2, 64, dtype=BF16)
        bt = torch.zeros(3, 4, dtype=torch.int32)
    else:
        k = torch.zeros(15, 2, 64, dtype=BF16)
        bt = None
    with pytest.raises(RuntimeError, match="CUDA"):
        flash_attn_varlen_func(q, k, k.clone(), 5, cu, 5, cu, None, True, bt)


def test_decode_head_dim_must_match():
    q = torch.zeros(2, 1, 4, 64, dtype=BF16)
    cache = torch.zeros(8, 64, 2, 128, dtype=BF16)
    with pytest.raises(RuntimeError, match="head_dim"):
        flash_attn_with_kvcache(q, cache, cache.clone(), torch.ones(2, dtype=torch.int32),
                                torch.zeros(2, 4, dtype=torch.int32))


def test_decode_rejects_host_tensors():
    q = torch.zeros(2, 1, 4, 64, dtype=BF16)
    cache = torch.zeros(8, 64, 2, 64, dtype=BF16)
    with pytest.raises(RuntimeError, match="CUDA"):
        flash_attn_with_kvcache(q, cache, cache.clone(), torch.ones(2, dtype=torch.int32),
                                torch.zeros(2, 4, dtype=torch.int32))
