"""The timed CPU baseline (oracle/cpu_baseline.py, bench.py's cpu_baseline leg)
against the oracle, on the CPU: what bench.py times must be the reference's
computation, so a mask, gather, GQA or scale slip in it fails here.

  * store_kvcache (index_copy_) and the fp8 store (torch's e4m3fn cast) bit-exact
    against oracle.store_kvcache / quantize_e4m3fn on sentinel-filled pools;
  * decode over bf16 and fp8 caches (ragged lengths including 0 and 1, scattered
    pages) within the bf16 / fp8 bars of the oracle;
  * prefill packed (Lq == Lk, an empty sequence) and over the paged caches with
    cached prefixes (Lq < Lk: the bottom-right mask), after the baseline's own store.

Planted mistakes in copies of the baseline's source (top-left mask, wrong page,
dropped scale, dequantisation skipped, K/V swapped in the store) each fail a check.
"""
from __future__ import annotations

import inspect
import types

import numpy as np
import pytest
import torch

from _helpers import FP8_MAX_ABS, assert_attn_close, bits8, bits16, decode_reference, f32, prefill_reference
from oracle import attention_oracle as O
from oracle import cpu_baseline as CB


def _W():
    from nanovllm_amd import workloads as W
    return W


# a softmax scale other than SDPA's default 1/sqrt(d), so a dropped scale argument shows
SCALE = 0.05


def _decode_case(fp8):
    case = _W().make_decode_case(5, 16, 8, 0, 0, 40, fp8=fp8, seed=31 + fp8, lengths=[300, 0, 1, 513, 1000],
                                 table_width=5)
    case.scale = SCALE
    return case


def _prefill_cases():
    W = _W()
    packed = W.make_prefill_case([37, 0, 130, 300], 16, 8, 12, seed=41)
    paged = W.make_prefill_case([100, 1, 260, 0], 32, 8, 24, prefix_len=[256, 512, 0, 256], seed=42,
                                shared_prefix=False)
    packed.scale = paged.scale = SCALE
    return packed, paged


def _check_store(cb):
    g = torch.Generator().manual_seed(5)
    T, nkv, d, nb, bs = 70, 8, 128, 4, 32
    buf = torch.randn(T, 3 * nkv * d, generator=g).bfloat16()
    key = buf[:, :nkv * d].reshape(T, nkv, d)
    value = buf[:, 2 * nkv * d:].view(T, nkv, d)  # strided, as qwen3.py:89's v
    slots = torch.randperm(nb * bs, generator=g)[:T].int()
    kc = torch.full((nb, bs, nkv, d), 3.5, dtype=torch.bfloat16)
    vc = torch.full((nb, bs, nkv, d), -1.25, dtype=torch.bfloat16)
    ek, ev = bits16(kc), bits16(vc)
    O.store_kvcache(bits16(key), bits16(value), ek, ev, slots.numpy())
    cb.store_kvcache(key, value, kc, vc, slots)
    assert np.array_equal(bits16(kc), ek) and np.array_equal(bits16(vc), ev), "bf16 store"
    # fp8: codes of x / scale per kv head, bit-exact
    ks = torch.linspace(0.004, 0.02, nkv).float()
    vs = torch.linspace(0.03, 0.005, nkv).float()
    k8 = torch.zeros(nb, bs, nkv, d, dtype=torch.uint8).view(torch.float8_e4m3fn)
    v8 = torch.zeros_like(k8)
    ek8 = np.full((nb, bs, nkv, d), 0x11, np.uint8)
    ev8 = np.full((nb, bs, nkv, d), 0x22, np.uint8)
    k8.view(torch.uint8).fill_(0x11)
    v8.view(torch.uint8).fill_(0x22)
    O.store_kvcache(O.quantize_e4m3fn(f32(key), f32(ks)), O.quantize_e4m3fn(f32(value), f32(vs)), ek8, ev8,
                    slots.numpy())
    cb.store_kvcache_fp8(key, value, k8, v8, slots, ks, vs)
    assert np.array_equal(bits8(k8), ek8) and np.array_equal(bits8(v8), ev8), "fp8 store"


def _check_decode_bf16(cb):
    case = _decode_case(False)
    got = cb.decode(case.q, case.k_cache, case.v_cache, case.context_lens, case.block_tables, case.scale)
    assert_attn_close(f32(got), decode_reference(case), what="cpu baseline decode bf16")


def _check_decode_fp8(cb):
    case = _decode_case(True)
    got = cb.decode(case.q, case.k_cache, case.v_cache, case.context_lens, case.block_tables, case.scale,
                    k_scale=case.k_scale, v_scale=case.v_scale)
    assert_attn_close(f32(got), decode_reference(case), max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS,
                      what="cpu baseline decode fp8")


def _check_prefill_packed(cb):
    case, _ = _prefill_cases()
    assert case.block_tables is None
    got = cb.prefill(case.q, case.k, case.v, case.cu_seqlens_q, case.cu_seqlens_k, case.scale)
    assert_attn_close(f32(got), prefill_reference(case), what="cpu baseline packed prefill")


def _check_prefill_paged(cb):
    _, case = _prefill_cases()
    assert case.block_tables is not None
    assert any(lk > lq for lq, lk in zip(case.lens_q, case.lens_k))
    cb.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
    got = cb.prefill(case.q, case.k_cache, case.v_cache, case.cu_seqlens_q, case.cu_seqlens_k, case.scale,
                     case.block_tables)
    assert_attn_close(f32(got), prefill_reference(case), what="cpu baseline paged prefill (Lq < Lk)")


CHECKS = [_check_store, _check_decode_bf16, _check_decode_fp8, _check_prefill_packed, _check_prefill_paged]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__[7:])
def test_cpu_baseline_matches_oracle(check):
    check(CB)


MUTANTS = {
    "top_left_mask": ("tril(diagonal=Lk - Lq)", "tril(diagonal=0)"),
    "wrong_page": ("pages = table_row[: math.ceil(L / bs)].long()",
                   "pages = table_row[: math.ceil(L / bs)].long().flip(0)"),
    "dropped_scale": ("scale=scale, enable_gqa=True)\n        out[b]", "enable_gqa=True)\n        out[b]"),
    "no_dequantisation": ("K = (K.float() * k_scale.view(1, -1, 1)).to(q.dtype)", "K = K.to(q.dtype)"),
    "store_kv_swapped": ("v_cache.view(-1, D).index_copy_(0, idx, value.reshape(T, D))",
                         "v_cache.view(-1, D).index_copy_(0, idx, key.reshape(T, D))"),
    "fp8_store_unscaled": ("(key.float() / k_scale.view(1, -1, 1))", "(key.float())"),
}


def _mutant(old, new):
    src = inspect.getsource(CB)
    assert src.count(old) == 1, f"mutation anchor not found once: {old!r}"
    mod = types.ModuleType("cpu_baseline_mutant")
    exec(compile(src.replace(old, new), "cpu_baseline_mutant", "exec"), mod.__dict__)
    return mod


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_baseline_mistake_is_caught(name):
    mod = _mutant(*MUTANTS[name])
    caught = []
    for check in CHECKS:
        try:
            check(mod)
        except (AssertionError, RuntimeError, IndexError):
            caught.append(check.__name__)
    assert caught, f"mutant {name} passed every check"
