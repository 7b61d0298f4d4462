"""An fp8 e4m3fn KV cache end to end on the GPU: allocated and bound through
engine.kv_cache.allocate_kv_cache (the mirror of model_runner.py:110-149, which
also owns the per-(layer, kv head) scales), then Attention.forward over two
layers for a prefill (store), a prefix-cached prefill that reads cached pages
(gathered and dequantised) and a decode step, each against the CPU oracle.

Bars: the prefill without a cached prefix attends over the fresh bf16 k/v
(bf16 bar, 2e-2 / 2e-3); everything read back from the fp8 cache within 5e-2 of
the oracle on the dequantised cache; the stored codes bit-exact against the
oracle's e4m3fn quantisation.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _helpers import FP8_MAX_ABS, assert_attn_close, bits8, f32
from oracle import attention_oracle as O

pytestmark = pytest.mark.gpu

NH, NKV, D, BS, L, NB = 16, 8, 128, 256, 2, 40


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()
    return torch.device("cuda:0")


def _dequant_keys(layer, pages, n):
    """(n, nkv, d) float32 keys/values of a sequence from the fp8 cache: e4m3 * scale."""
    idx = torch.tensor(pages, dtype=torch.long, device=layer.k_cache.device)
    ks = f32(layer.k_scale)[None, None, :, None]
    vs = f32(layer.v_scale)[None, None, :, None]
    k = (O.e4m3fn_to_f32(bits8(layer.k_cache.index_select(0, idx))) * ks).reshape(-1, NKV, D)[:n]
    v = (O.e4m3fn_to_f32(bits8(layer.v_cache.index_select(0, idx))) * vs).reshape(-1, NKV, D)[:n]
    return k, v


def _slots(pages, lo, hi):
    return [pages[j // BS] * BS + j % BS for j in range(lo, hi)]


def test_fp8_cache_prefill_prefix_prefill_decode(dev):
    import nanovllm_amd as nva
    from nanovllm_amd.engine.kv_cache import FP8_E4M3_MAX, allocate_kv_cache
    g = torch.Generator(device=dev).manual_seed(7)
    layers = torch.nn.ModuleList([nva.Attention(NH, D, D ** -0.5, NKV) for _ in range(L)])
    kv = allocate_kv_cache(layers.modules(), L, BS, NKV, D, kv_dtype=torch.float8_e4m3fn, num_blocks=NB,
                           device=dev)
    assert kv.kv_cache.shape == (2, L, NB, BS, NKV, D) and kv.kv_scale.shape == (2, L, NKV)
    for i, a in enumerate(layers):
        assert a.k_cache.data_ptr() == kv.kv_cache[0, i].data_ptr() and a.k_scale.data_ptr() == kv.kv_scale[0, i].data_ptr()

    # every token of the three steps, drawn up front so the scales (amax / 448 per
    # kv head, set before the first store) cover them all
    lens1 = [300, 700, 513]            # step 1: prefill, no cached prefix
    pre2, new2 = [256, 512], [150, 90]  # step 2: sequences reusing pages of seqs 0 and 1
    T1, T2, B3 = sum(lens1), sum(new2), 2
    T = T1 + T2 + B3
    qs = [torch.randn(T, NH, D, generator=g, device=dev).bfloat16() for _ in range(L)]
    ks = [torch.randn(T, NKV, D, generator=g, device=dev).bfloat16() * (1 + i) for i in range(L)]
    vs = [torch.randn(T, NKV, D, generator=g, device=dev).bfloat16() * 0.5 for i in range(L)]
    for i in range(L):
        kv.set_scales_from_amax(i, ks[i].float().abs().amax(dim=(0, 2)), vs[i].float().abs().amax(dim=(0, 2)))
    assert torch.allclose(kv.kv_scale[0, 1] * FP8_E4M3_MAX, ks[1].float().abs().amax(dim=(0, 2)))

    # page assignment (distinct pages per sequence; step-2 sequences share the prefix pages)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(1)).tolist()
    pages1, at = [], 0
    for n in lens1:
        pages1.append(perm[at:at + math.ceil(n / BS)])
        at += math.ceil(n / BS)
    pages2 = []
    for s, (pre, new) in enumerate(zip(pre2, new2)):
        extra = math.ceil((pre + new) / BS) - pre // BS
        pages2.append(pages1[s][: pre // BS] + perm[at:at + extra])
        at += extra
    i32 = dict(dtype=torch.int32, device=dev)

    # ---- step 1: prefill (store + attention over the fresh bf16 k/v) ----------
    cu1 = torch.tensor(np.cumsum([0] + lens1), **i32)
    slots1 = torch.tensor(sum((_slots(p, 0, n) for p, n in zip(pages1, lens1)), []), **i32)
    nva.set_context(True, cu1, cu1, max(lens1), max(lens1), slots1, None, None)
    outs = [a(qs[i][:T1].reshape(T1, -1), ks[i][:T1].reshape(T1, -1), vs[i][:T1].reshape(T1, -1))
            for i, a in enumerate(layers)]
    torch.cuda.synchronize()
    nva.reset_context()
    for i, a in enumerate(layers):
        got = f32(outs[i]).reshape(T1, NH, D)
        c = cu1.tolist()
        for s in range(len(lens1)):
            ref = O.attention(f32(qs[i][c[s]:c[s + 1]]), f32(ks[i][c[s]:c[s + 1]]), f32(vs[i][c[s]:c[s + 1]]),
                              D ** -0.5, True)
            assert_attn_close(got[c[s]:c[s + 1]], ref, what=f"step 1 layer {i} seq {s}")
        # stored codes: e4m3fn(x / scale) at every slot
        sl = slots1.long().cpu().numpy()
        ek = O.quantize_e4m3fn(f32(ks[i][:T1]), f32(a.k_scale))
        ev = O.quantize_e4m3fn(f32(vs[i][:T1]), f32(a.v_scale))
        assert np.array_equal(bits8(a.k_cache).reshape(-1, NKV, D)[sl], ek)
        assert np.array_equal(bits8(a.v_cache).reshape(-1, NKV, D)[sl], ev)

    # ---- step 2: prefix-cached prefill (reads the fp8 pages) ------------------
    lens_k2 = [p + n for p, n in zip(pre2, new2)]
    cu_q2 = torch.tensor(np.cumsum([0] + new2), **i32)
    cu_k2 = torch.tensor(np.cumsum([0] + lens_k2), **i32)
    width = max(len(p) for p in pages2)
    bt2 = torch.tensor([p + [-1] * (width - len(p)) for p in pages2], **i32)
    slots2 = torch.tensor(sum((_slots(p, pre, pre + n) for p, pre, n in zip(pages2, pre2, new2)), []), **i32)
    nva.set_context(True, cu_q2, cu_k2, max(new2), max(lens_k2), slots2, None, bt2)
    outs = [a(qs[i][T1:T1 + T2].reshape(T2, -1), ks[i][T1:T1 + T2].reshape(T2, -1),
              vs[i][T1:T1 + T2].reshape(T2, -1)) for i, a in enumerate(layers)]
    torch.cuda.synchronize()
    nva.reset_context()
    for i, a in enumerate(layers):
        got = f32(outs[i]).reshape(T2, NH, D)
        c = cu_q2.tolist()
        for s in range(2):
            k, v = _dequant_keys(a, pages2[s], lens_k2[s])
            ref = O.attention(f32(qs[i][T1 + c[s]:T1 + c[s + 1]]), k, v, D ** -0.5, True)
            assert_attn_close(got[c[s]:c[s + 1]], ref, max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS,
                              what=f"step 2 (prefix, fp8 pages) layer {i} seq {s}")

    # ---- step 3: decode one token per step-2 sequence -------------------------
    ctx3 = [n + 1 for n in lens_k2]
    for s in range(2):
        if len(pages2[s]) * BS < ctx3[s]:
            pages2[s].append(perm[at])
            at += 1
    width = max(len(p) for p in pages2)
    bt3 = torch.tensor([p + [-1] * (width - len(p)) for p in pages2], **i32)
    slots3 = torch.tensor([pages2[s][(ctx3[s] - 1) // BS] * BS + (ctx3[s] - 1) % BS for s in range(2)], **i32)
    nva.set_context(False, slot_mapping=slots3, context_lens=torch.tensor(ctx3, **i32), block_tables=bt3)
    outs = [a(qs[i][T1 + T2:].reshape(B3, -1), ks[i][T1 + T2:].reshape(B3, -1), vs[i][T1 + T2:].reshape(B3, -1))
            for i, a in enumerate(layers)]
    torch.cuda.synchronize()
    nva.reset_context()
    for i, a in enumerate(layers):
        got = f32(outs[i]).reshape(B3, NH, D)
        for s in range(2):
            k, v = _dequant_keys(a, pages2[s], ctx3[s])
            ref = O.attention(f32(qs[i][T1 + T2 + s:T1 + T2 + s + 1]), k, v, D ** -0.5, True)
            assert_attn_close(got[s:s + 1], ref, max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS,
                              what=f"step 3 (decode) layer {i} seq {s}")


@pytest.mark.parametrize("fp8", [False, True])
def test_gather_kv_matches_oracle(dev, fp8):
    """nva_gather_kv alone: packed rows == the oracle's gather (and dequantisation,
    rounded to bf16 as the kernel does), zero rows for a page outside the pool."""
    import nanovllm_amd as nva
    from nanovllm_amd import _capi
    from nanovllm_amd import workloads as W
    case = W.make_decode_case(5, 16, 8, 0, 0, 40, fp8=fp8, seed=4, bulk_device=dev, lengths=[1, 300, 0, 513, 256],
                              table_width=4)
    bt = case.block_tables.clone()
    bt[3, 1] = -1  # a page outside the pool inside the visible range
    lens = case.lengths
    cu = torch.tensor(np.cumsum([0] + lens), dtype=torch.int32, device=dev)
    rows = sum(lens)
    kp = torch.full((rows, 8, 128), 3.0, dtype=torch.bfloat16, device=dev)
    vp = torch.full_like(kp, 3.0)
    code = _capi.NVA_DTYPE_FP8_E4M3 if fp8 else _capi.NVA_DTYPE_BF16
    lib = _capi.load()
    _capi.check(lib.nva_gather_kv(
        case.k_cache.data_ptr(), case.v_cache.data_ptr(), code,
        case.k_scale.data_ptr() if fp8 else None, case.v_scale.data_ptr() if fp8 else None,
        case.k_cache.shape[0], bt.data_ptr(), bt.stride(0), bt.shape[1], 256, cu.data_ptr(), len(lens), max(lens),
        8, 128, kp.data_ptr(), vp.data_ptr(), rows, 8 * 128, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    c = cu.tolist()
    for s, n in enumerate(lens):
        if n == 0:
            continue
        pages = bt[s, : -(-n // 256)].tolist()
        for name, cache, scale, packed in (("k", case.k_cache, case.k_scale, kp), ("v", case.v_cache, case.v_scale, vp)):
            ok = [p >= 0 for p in pages]
            safe = torch.tensor([p if p >= 0 else 0 for p in pages], dtype=torch.long, device=dev)
            if fp8:
                x = O.e4m3fn_to_f32(bits8(cache.index_select(0, safe))) * f32(scale)[None, None, :, None]
                x = torch.from_numpy(x).bfloat16().float().numpy()  # one rounding to bf16, as the kernel
            else:
                x = f32(cache.index_select(0, safe))
            for j, good in enumerate(ok):
                if not good:
                    x[j] = 0
            x = x.reshape(-1, 8, 128)[:n]
            assert np.array_equal(f32(packed[c[s]:c[s] + n]), x), f"{name} seq {s}"
