"""The largest sizes the reference's configuration admits, against the oracle.

- Prefill of one sequence of max_num_batched_tokens = 16384 tokens (config.py:8, the
  default; a single sequence that long needs max_model_len raised to match), packed, and
  as a prefix-cached call: 8192 new tokens after 8192 cached ones.  Rows sampled at the
  start, around the middle and at the end of the sequence (the last ones see all 16384
  keys).  The oracle computes rows [a, b) of a causal sequence as the bottom-right causal
  attention of q[a:b] over keys [0, b).
- Decode at Qwen3's max_position_embeddings (40960 keys; config.py:25 caps max_model_len
  there): two sequences of 40960 and 23000 keys and one empty row, bf16 and fp8 caches,
  the default plan and the balanced plan forced, every sequence against the oracle.

Bars: bf16 within 2e-2 max-abs / 2e-3 mean-abs, fp8 within 5e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import FP8_MAX_ABS, assert_attn_close, decode_reference, f32
from oracle import attention_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def _keys(case, s, n):
    """The first n keys/values of sequence s, float32 (n, nkv, d): from the packed
    rows, or gathered from the cache pages after the store."""
    cu_k = case.cu_seqlens_k.cpu().tolist()
    if case.block_tables is None:
        return f32(case.k[cu_k[s]:cu_k[s] + n]), f32(case.v[cu_k[s]:cu_k[s] + n])
    bs = case.block_size
    pages = case.block_tables[s, : (n + bs - 1) // bs].long()
    k = f32(case.k_cache.index_select(0, pages)).reshape(-1, case.num_kv_heads, case.head_dim)[:n]
    v = f32(case.v_cache.index_select(0, pages)).reshape(-1, case.num_kv_heads, case.head_dim)[:n]
    return k, v


@pytest.mark.parametrize("prefix", [0, 8192])
def test_prefill_longest_sequence(dev, prefix):
    import nanovllm_amd as nva
    from nanovllm_amd import workloads as W
    L = 16384 - prefix
    print(f"long prefill: {L} new tokens after {prefix} cached", flush=True)
    case = W.make_prefill_case([L], 32, 8, (prefix + L) // 256 + 4, prefix_len=prefix, seed=16384 + prefix,
                               bulk_device=dev)
    nva.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
    k, v = (case.k, case.v) if case.block_tables is None else (case.k_cache, case.v_cache)
    o = nva.flash_attn_varlen_func(case.q, k, v, case.max_seqlen_q, case.cu_seqlens_q, case.max_seqlen_k,
                                   case.cu_seqlens_k, case.scale, True, case.block_tables)
    torch.cuda.synchronize()
    got = f32(o)
    q = f32(case.q)
    Lk = prefix + L
    for a in (0, L // 2 - 32, L - 64):
        b = a + 64
        kk, vv = _keys(case, 0, prefix + b)
        ref = O.attention(q[a:b], kk, vv, case.scale, True)
        assert_attn_close(got[a:b], ref, what=f"long prefill rows {a}:{b} of {L} (keys {Lk}, prefix {prefix})")


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("num_splits", [0, -1])
def test_decode_longest_context(dev, fp8, num_splits):
    import nanovllm_amd as nva
    from nanovllm_amd import workloads as W
    lengths = [40960, 0, 23000]
    print(f"long decode: lengths {lengths} fp8={fp8} num_splits={num_splits}", flush=True)
    case = W.make_decode_case(3, 16, 8, 0, 0, sum(-(-x // 256) for x in lengths) + 2, fp8=fp8, seed=40960 + fp8,
                              bulk_device=dev, lengths=lengths)
    nva.store_kvcache(case.k_new, case.v_new, case.k_cache, case.v_cache, case.slot_mapping, case.k_scale,
                      case.v_scale)
    o = nva.flash_attn_with_kvcache(case.q.unsqueeze(1), case.k_cache, case.v_cache, case.context_lens,
                                    case.block_tables, case.scale, True, num_splits=num_splits,
                                    k_scale=case.k_scale, v_scale=case.v_scale)
    torch.cuda.synchronize()
    got = f32(o[:, 0])
    tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if fp8 else {}
    assert_attn_close(got, decode_reference(case), what=f"long decode fp8={fp8} splits={num_splits}", **tol)
    assert np.all(got[1] == 0)
