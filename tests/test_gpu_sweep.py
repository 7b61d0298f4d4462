"""Seeded random shapes through the Python mirror, each against the oracle.

Decode: spread, balanced and fixed-split plans (and the wide merge they lead to),
bf16 and fp8 caches, block sizes 32-256, GQA groups 1-16 over 1-8 kv heads,
ragged lengths including 0, through flash_attn_with_kvcache after store_kvcache or
through store_and_decode.  Prefill: the direct and the persistent grid, packed
and paged (mixed cached prefixes, block sizes 64-512), GQA groups 1-7, head_dim 64
and 128, ragged lengths including empty query segments.

Key halving: 24 launches of a few long sequences (the direct grid, whose longest
items then run as two key halves), packed and paged.

The shapes are drawn once from fixed seeds, so every run checks the same cases;
each is sized so the CPU oracle takes at most a few seconds.  Bars: bf16 within
2e-2 max-abs / 2e-3 mean-abs, fp8 within 5e-2 of the oracle on the dequantised
cache.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from _helpers import FP8_MAX_ABS, assert_attn_close, decode_reference, f32, prefill_reference

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def _decode_shapes(n=40, seed=2024):
    r = random.Random(seed)
    # (batch, longest context): at most ~400k keys per case for the oracle
    sizes = [(1, 9000), (2, 3000), (5, 9000), (17, 3000), (40, 3000), (64, 3000), (130, 700), (300, 700),
             (3, 40)]
    out = []
    for i in range(n):
        nkv = r.choice([1, 2, 4, 8])
        group = r.choice([1, 2, 3, 4, 7, 8, 16])
        fp8 = r.random() < 0.35
        B, ctx_hi = r.choice(sizes)
        out.append(dict(i=i, nkv=nkv, nh=group * nkv, fp8=fp8, d=128 if fp8 else r.choice([64, 128]),
                        bs=r.choice([32, 64, 128, 256]), B=B, ctx_hi=ctx_hi,
                        splits=r.choice([0, 0, 0, -1, 1, 3, 9]), fused=r.random() < 0.5))
    return out


def _prefill_shapes(n=30, seed=4048):
    r = random.Random(seed)
    out = []
    while len(out) < n:
        nkv = r.choice([1, 2, 4, 8])
        group = r.choice([1, 2, 4, 7])
        S = r.choice([1, 3, 9, 24, 40])
        lq_max = r.choice([100, 400, 700])
        paged = r.random() < 0.6
        bs = r.choice([64, 128, 256, 512]) if paged else 256
        lens = [r.choice([0, r.randint(1, lq_max), r.randint(1, lq_max)]) for _ in range(S)]
        lens[r.randrange(S)] = lq_max  # the longest one always present
        pre = [r.choice([0, 0, bs, 2 * bs]) for _ in range(S)] if paged else [0] * S
        work = sum(q * (q + p) for q, p in zip(lens, pre)) * group * nkv
        if work > 1.2e8:  # keep the CPU oracle within seconds
            continue
        out.append(dict(i=len(out), nkv=nkv, nh=group * nkv, d=r.choice([64, 128]), S=S, lens=lens, pre=pre,
                        paged=paged, bs=bs, shared=r.random() < 0.5))
    return out


def _split_shapes(n=24, seed=6060):
    """Few long sequences (direct grid, at most two items per CU), so that the
    longest items run as key halves: packed or paged at block sizes 64-512 with
    mixed cached prefixes, GQA groups 1-16 over 1-8 kv heads."""
    r = random.Random(seed)
    out = []
    while len(out) < n:
        nkv = r.choice([1, 2, 4, 8])
        group = r.choice([1, 2, 4, 7, 8, 16])
        bp = 256 // group
        S = r.randint(1, 6)
        lens = [r.randint(1, 2000) for _ in range(S)]
        lens[r.randrange(S)] = r.randint(600, 2000)
        paged = r.random() < 0.5
        bs = r.choice([64, 128, 256, 512]) if paged else 256
        pre = [r.choice([0, bs, 2 * bs, 4 * bs]) for _ in range(S)] if paged else [0] * S
        if S * nkv * -(-max(lens) // bp) > 512:  # the persistent grid would serve it
            continue
        work = sum(q * (q + x) for q, x in zip(lens, pre)) * group * nkv
        if work > 1.5e8:  # keep the CPU oracle within seconds
            continue
        out.append(dict(i=len(out), nkv=nkv, nh=group * nkv, d=r.choice([64, 128]), lens=lens, pre=pre,
                        paged=paged, bs=bs))
    return out


@pytest.mark.parametrize("shape", _decode_shapes(), ids=lambda s: f"d{s['i']}")
def test_decode_sweep(dev, shape):
    import nanovllm_amd as nva
    from nanovllm_amd import workloads as W
    s = shape
    print(f"decode sweep {s}", flush=True)
    pages = s["B"] * -(-s["ctx_hi"] // s["bs"]) + 2
    case = W.make_decode_case(s["B"], s["nh"], s["nkv"], 0, s["ctx_hi"], pages, block_size=s["bs"],
                              head_dim=s["d"], fp8=s["fp8"], seed=100 + s["i"], bulk_device=dev)
    q = case.q.unsqueeze(1)
    if s["fused"]:
        o = nva.store_and_decode(q, case.k_new, case.v_new, case.k_cache, case.v_cache, case.slot_mapping,
                                 case.context_lens, case.block_tables, case.scale, num_splits=s["splits"],
                                 k_scale=case.k_scale, v_scale=case.v_scale)
    else:
        nva.store_kvcache(case.k_new, case.v_new, case.k_cache, case.v_cache, case.slot_mapping, case.k_scale,
                          case.v_scale)
        o = nva.flash_attn_with_kvcache(q, case.k_cache, case.v_cache, case.context_lens, case.block_tables,
                                        case.scale, True, num_splits=s["splits"], k_scale=case.k_scale,
                                        v_scale=case.v_scale)
    torch.cuda.synchronize()
    got = f32(o[:, 0])
    tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if s["fp8"] else {}
    assert_attn_close(got, decode_reference(case), what=f"decode sweep {s}", **tol)
    # rows of empty sequences are zero
    lens = case.context_lens.cpu().numpy()
    assert np.all(got[lens == 0] == 0)


@pytest.mark.parametrize("shape", _prefill_shapes(), ids=lambda s: f"p{s['i']}")
def test_prefill_sweep(dev, shape):
    import nanovllm_amd as nva
    from nanovllm_amd import workloads as W
    s = shape
    print(f"prefill sweep {s}", flush=True)
    pages = sum(-(-(q + p) // s["bs"]) for q, p in zip(s["lens"], s["pre"])) + 4
    case = W.make_prefill_case(s["lens"], s["nh"], s["nkv"], pages, prefix_len=s["pre"], block_size=s["bs"],
                               head_dim=s["d"], seed=200 + s["i"], bulk_device=dev, shared_prefix=s["shared"])
    nva.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
    k, v = (case.k, case.v) if case.block_tables is None else (case.k_cache, case.v_cache)
    o = nva.flash_attn_varlen_func(case.q, k, v, case.max_seqlen_q, case.cu_seqlens_q, case.max_seqlen_k,
                                   case.cu_seqlens_k, case.scale, True, case.block_tables)
    torch.cuda.synchronize()
    assert_attn_close(f32(o), prefill_reference(case), what=f"prefill sweep {s}")


@pytest.mark.parametrize("shape", _split_shapes(), ids=lambda s: f"k{s['i']}")
def test_prefill_key_halves_sweep(dev, shape):
    import nanovllm_amd as nva
    from nanovllm_amd import workloads as W
    s = shape
    print(f"key halves sweep {s}", flush=True)
    pages = sum(-(-(q + p) // s["bs"]) for q, p in zip(s["lens"], s["pre"])) + 4
    case = W.make_prefill_case(s["lens"], s["nh"], s["nkv"], pages, prefix_len=s["pre"], block_size=s["bs"],
                               head_dim=s["d"], seed=300 + s["i"], bulk_device=dev, shared_prefix=False)
    nva.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
    k, v = (case.k, case.v) if case.block_tables is None else (case.k_cache, case.v_cache)
    o = nva.flash_attn_varlen_func(case.q, k, v, case.max_seqlen_q, case.cu_seqlens_q, case.max_seqlen_k,
                                   case.cu_seqlens_k, case.scale, True, case.block_tables)
    torch.cuda.synchronize()
    assert_attn_close(f32(o), prefill_reference(case), what=f"key halves sweep {s}")
