"""GPU parity of the HIP hot path against the CPU oracle (run on an MI355X).

Bars: store_kvcache cache contents bit-exact; bf16 attention within max-abs 2e-2
and mean-abs 2e-3 of the fp32 oracle; fp8-KV decode within 5e-2 of the oracle
on the dequantised cache.  Every call goes through the C ABI of libnva_attn.so
via the host mirror of the reference interface.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _helpers import (FP8_MAX_ABS, assert_attn_close, bits8, bits16, decode_reference, f32,
                      prefill_reference, rows_of)
from oracle import attention_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


def nva():
    import nanovllm_amd as m
    return m


# ----------------------------------------------------------------------------
# store_kvcache
# ----------------------------------------------------------------------------

def _sentinel_pool(case, dev, pattern=0x5A3C):
    kc = torch.full(case.k_cache.shape, pattern, dtype=torch.int16, device=dev).view(torch.bfloat16)
    vc = torch.full(case.v_cache.shape, pattern ^ 0x0F0F, dtype=torch.int16, device=dev).view(torch.bfloat16)
    return kc, vc


@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
def test_store_bitexact(dev, cfg):
    from nanovllm_amd import workloads as W
    case = W.CONFIGS[cfg](dev) if cfg == 3 else W.CONFIGS[cfg]("cpu").to(dev)
    if cfg in (1, 3):
        key, value, slots = case.k_new, case.v_new, case.slot_mapping
    else:
        key, value, slots = case.k, case.v, case.slot_mapping
    kc, vc = _sentinel_pool(case, dev)
    ekc, evc = bits16(kc), bits16(vc)
    O.store_kvcache(bits16(key), bits16(value), ekc, evc, slots.cpu().numpy())
    nva().store_kvcache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(kc), ekc)
    assert np.array_equal(bits16(vc), evc)


def test_store_skips_out_of_range_slots(dev):
    T, nkv, d, nb, bs = 40, 8, 128, 4, 16
    g = torch.Generator(device=dev).manual_seed(3)
    key = torch.randn(T, nkv, d, generator=g, device=dev).bfloat16()
    value = torch.randn(T, nkv, d, generator=g, device=dev).bfloat16()
    slots = torch.randperm(nb * bs, device=dev)[:T].int()
    slots[::5] = -1
    slots[3] = nb * bs  # one past the end
    slots[7] = 1 << 30
    kc = torch.zeros(nb, bs, nkv, d, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    ekc, evc = bits16(kc), bits16(vc)
    O.store_kvcache(bits16(key), bits16(value), ekc, evc, slots.cpu().numpy())
    nva().store_kvcache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(kc), ekc) and np.array_equal(bits16(vc), evc)


@pytest.mark.parametrize("row_pad", [0, 1, 4, 3000])
def test_store_unaligned_rows(dev, row_pad):
    """Row strides that are not 16-byte multiples take narrower vector paths."""
    T, nkv, d, nb, bs = 33, 2, 128, 3, 32
    g = torch.Generator(device=dev).manual_seed(row_pad)
    buf = torch.randn(T, nkv * d + row_pad, generator=g, device=dev).bfloat16()
    key = buf[:, :nkv * d].view(T, nkv, d)
    value = buf[:, row_pad:row_pad + nkv * d].view(T, nkv, d)
    slots = torch.randperm(nb * bs, device=dev)[:T].int()
    kc = torch.full((nb, bs, nkv, d), 7.0, dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, -3.0)
    ekc, evc = bits16(kc), bits16(vc)
    O.store_kvcache(bits16(key), bits16(value), ekc, evc, slots.cpu().numpy())
    nva().store_kvcache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(kc), ekc) and np.array_equal(bits16(vc), evc)


def test_store_fp8_bitexact(dev):
    """fp8 cache store == e4m3fn(x / scale) of the oracle and of torch's cast."""
    T, nkv, d, nb, bs = 300, 8, 128, 4, 256
    g = torch.Generator(device=dev).manual_seed(11)
    key = (torch.randn(T, nkv, d, generator=g, device=dev) * 3).bfloat16()
    value = (torch.randn(T, nkv, d, generator=g, device=dev) * 0.01).bfloat16()
    # exercise ties, subnormals, the 448/464 boundary and overflow to NaN
    key[0, 0, :8] = torch.tensor([464.0, 465.0, 480.0, -500.0, 448.0, 2 ** -10, 2 ** -9 * 1.5, 0.0])
    k_scale = torch.linspace(0.5, 2.0, nkv, device=dev).float()
    v_scale = (value.float().abs().amax(dim=(0, 2)) / 448).contiguous()
    slots = torch.randperm(nb * bs, device=dev)[:T].int()
    kc = torch.zeros(nb, bs, nkv, d, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    vc = torch.zeros_like(kc)
    nva().store_kvcache(key, value, kc, vc, slots, k_scale, v_scale)
    torch.cuda.synchronize()
    ek = np.zeros((nb, bs, nkv, d), np.uint8)
    ev = np.zeros_like(ek)
    O.store_kvcache(O.quantize_e4m3fn(f32(key), f32(k_scale)), O.quantize_e4m3fn(f32(value), f32(v_scale)),
                    ek, ev, slots.cpu().numpy())
    assert np.array_equal(bits8(kc), ek)
    assert np.array_equal(bits8(vc), ev)
    torch_k = (key.float().cpu() / k_scale.cpu().view(1, nkv, 1)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got_rows = bits8(kc).reshape(-1, nkv, d)[slots.cpu().numpy()]
    assert np.array_equal(got_rows, torch_k)


# ----------------------------------------------------------------------------
# decode
# ----------------------------------------------------------------------------

def _run_decode(case, num_splits=0, store=True):
    m = nva()
    if store:
        m.store_kvcache(case.k_new, case.v_new, case.k_cache, case.v_cache, case.slot_mapping,
                        case.k_scale, case.v_scale)
    o = m.flash_attn_with_kvcache(case.q.unsqueeze(1), case.k_cache, case.v_cache, case.context_lens,
                                  case.block_tables, case.scale, True, num_splits=num_splits,
                                  k_scale=case.k_scale, v_scale=case.v_scale)
    torch.cuda.synchronize()
    return f32(o[:, 0])


@pytest.mark.parametrize("shape", ["long_small_batch", "one_kv_head_fp8", "fixed_12_splits"])
def test_decode_wide_merge(dev, shape):
    """Plans with at least 8 partials per sequence on average take the wide merge (four
    waves per (sequence, head), states combined through LDS): 8 sequences of 15k-20k keys
    (balanced, 16 ranges each); 64 sequences over one kv head of an fp8 cache (the
    TP8 share of config 5: 32 ranges each); fixed 12-way splits with a length of 0 and
    one of 1.  Every sequence against the oracle."""
    from nanovllm_amd import workloads as W
    if shape == "long_small_batch":
        case = W.make_decode_case(8, 16, 8, 15000, 20000, 700, seed=91, bulk_device=dev)
        ns, tol = 0, {}
    elif shape == "one_kv_head_fp8":
        case = W.make_decode_case(64, 8, 1, 17000, 20000, 5100, fp8=True, seed=92, bulk_device=dev)
        ns, tol = 0, dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS)
    else:
        case = W.make_decode_case(5, 16, 8, 0, 0, 200, seed=93, bulk_device=dev, lengths=[3000, 0, 1, 2500, 7000])
        ns, tol = 12, {}
    got = _run_decode(case, ns)
    for b in range(case.batch):
        assert_attn_close(got[b:b + 1], decode_reference(case, [b]), what=f"{shape} seq {b}", **tol)


@pytest.mark.parametrize("num_splits", [0, -1, 1, 2, 3])
def test_decode_cfg1(dev, num_splits):
    from nanovllm_amd import workloads as W
    case = W.config1("cpu").to(dev)
    got = _run_decode(case, num_splits)
    assert_attn_close(got, decode_reference(case), what=f"cfg1 splits={num_splits}")


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("B,d,nh,nkv", [(1, 128, 16, 8), (3, 128, 16, 8), (7, 64, 16, 8), (32, 128, 16, 8),
                                        (64, 128, 16, 8), (64, 64, 16, 8), (256, 128, 16, 8), (160, 64, 14, 2)])
def test_store_decode_matches_two_calls(dev, fp8, B, d, nh, nkv):
    """nva_store_decode (Attention.forward's decode branch as one call) against
    store_kvcache + flash_attn_with_kvcache on copies of the same cache: identical
    output bits and identical cache bits, and the oracle over the stored cache.
    Batches up to 32 x 8 kv heads take the spread mode and larger ones the
    balanced mode (160 x 2 on one-wave workgroups); both store inside the decode
    launch, where the holder of key ctx-1 patches the new row into its registers
    (the balanced mode over an fp8 cache runs the store kernel first).  Lengths
    hit a step's first and last row, a page boundary, one key and none; a
    sequence with no context but a valid slot (row 2) is stored all the same."""
    if fp8 and d != 128:
        pytest.skip("fp8 decode supports head_dim 128 only (nva_decode refuses it)")
    from nanovllm_amd import workloads as W
    m = nva()
    base = [1, 33, 0, 256, 257, 700, 31, 32, 64, 1023]
    lengths = [base[i % len(base)] + (i // len(base)) * 5 for i in range(B)]
    case = W.make_decode_case(B, nh, nkv, 0, 0, 8 * B + 2, fp8=fp8, seed=B + 11 * d, head_dim=d, bulk_device=dev,
                              lengths=lengths, table_width=max(5, -(-max(lengths) // 256)))
    if B > 2 and lengths[2] == 0:
        # a page no sequence reads, for the empty sequence's new row
        used = {int(case.block_tables[b, j]) for b in range(B) for j in range(-(-lengths[b] // 256))}
        free = min(set(range(8 * B + 2)) - used)
        case.slot_mapping[2] = free * 256 + 7
    kc1, vc1 = case.k_cache.clone(), case.v_cache.clone()
    fused = m.store_and_decode(case.q.unsqueeze(1), case.k_new, case.v_new, kc1, vc1, case.slot_mapping,
                               case.context_lens, case.block_tables, softmax_scale=case.scale,
                               k_scale=case.k_scale, v_scale=case.v_scale)
    m.store_kvcache(case.k_new, case.v_new, case.k_cache, case.v_cache, case.slot_mapping, case.k_scale, case.v_scale)
    two = m.flash_attn_with_kvcache(case.q.unsqueeze(1), case.k_cache, case.v_cache, case.context_lens,
                                    case.block_tables, case.scale, True, k_scale=case.k_scale, v_scale=case.v_scale)
    torch.cuda.synchronize()
    view = bits8 if fp8 else bits16
    assert np.array_equal(view(kc1), view(case.k_cache)) and np.array_equal(view(vc1), view(case.v_cache))
    assert np.array_equal(bits16(fused), bits16(two)), f"B={B} fp8={fp8}: fused output differs from the two calls"
    tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if fp8 else {}
    assert_attn_close(f32(fused[:, 0]), decode_reference(case), what=f"store+decode B={B} fp8={fp8} d={d}", **tol)


def test_decode_cfg3_full(dev):
    from nanovllm_amd import workloads as W
    case = W.config3(dev)
    got = _run_decode(case)
    mx, mn = assert_attn_close(got, decode_reference(case), what="cfg3")
    print(f"cfg3 decode max-abs {mx:.3e} mean-abs {mn:.3e}")


def test_decode_cfg3_split_invariance(dev):
    from nanovllm_amd import workloads as W
    case = W.config3(dev)
    a = _run_decode(case, 0)
    b = _run_decode(case, 1, store=False)
    c = _run_decode(case, 8, store=False)
    assert np.abs(a - b).max() <= 1e-2 and np.abs(a - c).max() <= 1e-2


def test_decode_cfg5_fp8(dev):
    """All 64 sequences against the oracle on the dequantised cache, one at a time
    (each gathers ~24k keys)."""
    from nanovllm_amd import workloads as W
    case = W.config5(dev)
    got = _run_decode(case)
    worst = 0.0
    for b in range(case.batch):
        mx, _ = assert_attn_close(got[b:b + 1], decode_reference(case, [b]), max_abs=FP8_MAX_ABS,
                                  mean_abs=FP8_MAX_ABS, what=f"cfg5 fp8 seq {b}")
        worst = max(worst, mx)
    print(f"cfg5 fp8 decode max-abs {worst:.3e} over {case.batch} sequences")


@pytest.mark.parametrize("nh,nkv", [(8, 8), (16, 8), (32, 8), (64, 8), (16, 1), (128, 8)])
@pytest.mark.parametrize("fp8", [False, True])
def test_decode_group_sizes(dev, nh, nkv, fp8):
    from nanovllm_amd import workloads as W
    lengths = [1, 2, 31, 32, 33, 255, 256, 257, 700, 1025]
    case = W.make_decode_case(len(lengths), nh, nkv, 0, 0, 40, fp8=fp8, seed=nh * 10 + nkv, bulk_device=dev,
                              lengths=lengths, table_width=6)
    for ns in (0, 1, 4):
        got = _run_decode(case, ns, store=(ns == 0))
        tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if fp8 else {}
        assert_attn_close(got, decode_reference(case), what=f"nh={nh} nkv={nkv} fp8={fp8} splits={ns}", **tol)


@pytest.mark.parametrize("lengths,width", [
    ([5, 0, 3000, 1, 0, 64, 4097, 33], 17),   # zero-length rows mixed in, long rows spanning ranges
    ([1] * 9, 1),                              # more ranges than steps
    ([700] * 3 + [0] * 5, 3),
])
@pytest.mark.parametrize("fp8", [False, True])
def test_decode_balanced_partition(dev, lengths, width, fp8):
    """Balanced split-K (num_splits=-1 forces it at these small batches) against the
    oracle and against fixed splits and the size heuristic (0)."""
    from nanovllm_amd import workloads as W
    case = W.make_decode_case(len(lengths), 32, 8, 0, 0, 64, fp8=fp8, seed=len(lengths) + width,
                              bulk_device=dev, lengths=lengths, table_width=width)
    bal = _run_decode(case, -1, store=False)
    tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if fp8 else {}
    assert_attn_close(bal, decode_reference(case), what=f"balanced {lengths}", **tol)
    for ns in (0, 1, 3):
        fixed = _run_decode(case, ns, store=False)
        assert np.abs(fixed - bal).max() <= 1e-2
    for b, L in enumerate(lengths):
        if L == 0:
            assert np.all(bal[b] == 0)


@pytest.mark.parametrize("nh,nkv,d", [(16, 8, 128), (32, 8, 128), (128, 8, 128), (8, 1, 128), (14, 2, 64),
                                      (16, 8, 64)])
@pytest.mark.parametrize("fp8", [False, True])
def test_decode_spread(dev, nh, nkv, d, fp8):
    """The small-batch spread mode (one wave per share of a sequence's steps, the
    partials merged by decode_merge_kernel): ragged lengths incl. 0, 1 and a full
    16-page table, at batches of 1 to the largest it serves (batch * nkv = 256),
    against the oracle and the balanced mode; a second call gives the same bits."""
    if fp8 and d != 128:
        pytest.skip("fp8 decode supports head_dim 128 only (nva_decode refuses it)")
    from nanovllm_amd import workloads as W
    from nanovllm_amd import _capi
    for B in (1, 3, 256 // nkv):
        g = torch.Generator().manual_seed(B + nh)
        lengths = torch.randint(0, 4097, (B,), generator=g).tolist()
        lengths[0] = 4096 if B > 1 else 700
        if B > 2:
            lengths[1], lengths[2] = 0, 1
        case = W.make_decode_case(B, nh, nkv, 0, 0, 16 * B + 1, fp8=fp8, seed=B * 7 + nh, head_dim=d,
                                  bulk_device=dev, lengths=lengths, table_width=16)
        assert _capi.load().nva_decode_workspace_bytes(B, nh, nkv, d, 16, 256, int(fp8), 0) > 0
        got = _run_decode(case, 0, store=False)
        tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if fp8 else {}
        assert_attn_close(got, decode_reference(case), what=f"spread B={B} nh={nh} nkv={nkv} d={d}", **tol)
        assert np.array_equal(_run_decode(case, 0, store=False), got)
        bal = _run_decode(case, -1, store=False)
        assert np.abs(got - bal).max() <= 1e-2
        for b, L in enumerate(lengths):
            if L == 0:
                assert np.all(got[b] == 0)


def test_decode_balanced_many_sequences(dev):
    """Batch above one scan chunk (512 sequences) with short, uneven contexts."""
    from nanovllm_amd import workloads as W
    g = torch.Generator().manual_seed(5)
    lengths = torch.randint(0, 300, (1300,), generator=g).tolist()
    case = W.make_decode_case(1300, 16, 8, 0, 0, 1700, seed=8, bulk_device=dev, lengths=lengths, table_width=2)
    got = _run_decode(case, 0, store=False)
    seqs = list(range(0, 1300, 37))
    assert_attn_close(got[seqs], decode_reference(case, seqs), what="1300 sequences")
    assert np.all(got[[b for b, L in enumerate(lengths) if L == 0]] == 0)


def test_decode_zero_and_single_key(dev):
    from nanovllm_amd import workloads as W
    lengths = [0, 1, 5, 0]
    case = W.make_decode_case(4, 16, 8, 0, 0, 8, seed=5, bulk_device=dev, lengths=lengths, table_width=2)
    got = _run_decode(case, store=False)
    assert np.all(got[0] == 0) and np.all(got[3] == 0)
    # one key: o = v0 exactly (p = 1, l = 1)
    v0 = f32(case.v_cache[case.block_tables[1, 0].long(), 0])  # (nkv, d)
    assert np.array_equal(got[1], np.repeat(v0, 2, axis=0))


def test_decode_fp8_all_codes(dev):
    """ctx = 1 with v_scale = 1: the output is the e4m3fn value of each V code,
    exactly (every e4m3fn value is a bf16 value)."""
    nkv, d, bs = 2, 128, 32
    codes = torch.arange(256, dtype=torch.uint8, device=dev).view(1, 1, nkv, d)
    kc = torch.zeros(1, bs, nkv, d, dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    vc[:, 0] = codes[0]
    q = torch.randn(1, 1, 2 * nkv, d, device=dev).bfloat16()
    one = torch.ones(nkv, dtype=torch.float32, device=dev)
    o = nva().flash_attn_with_kvcache(q, kc.view(torch.float8_e4m3fn), vc.view(torch.float8_e4m3fn),
                                      torch.ones(1, dtype=torch.int32, device=dev),
                                      torch.zeros(1, 1, dtype=torch.int32, device=dev), 0.1,
                                      k_scale=one, v_scale=one)
    torch.cuda.synchronize()
    got = f32(o[0, 0]).reshape(nkv, 2, d)[:, 0].reshape(-1)  # head 2h reads kv head h
    expect = O.e4m3fn_table().astype(np.float32)
    nan = np.isnan(expect)
    assert np.array_equal(got[~nan], expect[~nan])
    assert np.isnan(got[nan]).all()


def test_decode_inconsistent_table_is_safe(dev):
    """-1 / out-of-range block ids inside the visible range are masked, not read."""
    from nanovllm_amd import workloads as W
    case = W.make_decode_case(2, 16, 8, 0, 0, 8, seed=9, bulk_device=dev, lengths=[600, 300], table_width=3)
    bt = case.block_tables.clone()
    bt[0, 1] = -1
    bt[1, 1] = 1 << 20
    o = nva().flash_attn_with_kvcache(case.q.unsqueeze(1), case.k_cache, case.v_cache, case.context_lens,
                                      bt, case.scale)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    # seq 1 keeps only its first page's 256 keys
    case.context_lens = torch.tensor([600, 256], dtype=torch.int32, device=dev)
    ref = decode_reference(case, [1])
    assert_attn_close(f32(o[1:, 0]), ref, what="masked page")


# ----------------------------------------------------------------------------
# prefill
# ----------------------------------------------------------------------------

def _run_prefill(case, store=True):
    m = nva()
    if store:
        m.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
    if case.block_tables is None:
        k, v = case.k, case.v
    else:
        k, v = case.k_cache, case.v_cache
    o = m.flash_attn_varlen_func(case.q, k, v, case.max_seqlen_q, case.cu_seqlens_q, case.max_seqlen_k,
                                 case.cu_seqlens_k, case.scale, True, case.block_tables)
    torch.cuda.synchronize()
    return f32(o)


def test_prefill_cfg2(dev):
    from nanovllm_amd import workloads as W
    case = W.config2("cpu").to(dev)
    got = _run_prefill(case)
    mx, mn = assert_attn_close(got, prefill_reference(case), what="cfg2")
    print(f"cfg2 prefill max-abs {mx:.3e} mean-abs {mn:.3e}")


def test_prefill_cfg4_prefix(dev):
    """Every row of all 16 sequences (the work-queue grid's full run), one sequence
    at a time."""
    from nanovllm_amd import workloads as W
    case = W.config4("cpu").to(dev)
    got = _run_prefill(case)
    worst = 0.0
    for s in range(len(case.lens_q)):
        mx, _ = assert_attn_close(got[rows_of(case, [s])], prefill_reference(case, [s]), what=f"cfg4 seq {s}")
        worst = max(worst, mx)
    print(f"cfg4 prefill max-abs {worst:.3e} over {len(case.lens_q)} sequences")


@pytest.mark.parametrize("nseq", [7, 40])
def test_prefill_mixed_prefix_lengths(dev, nseq):
    """Cached prefixes of 0, 256 and 1024 tokens in one paged call: with one cached
    prefix in the batch the reference sets block tables for every sequence
    (model_runner.py:189-190), so prefix-free ones (Lk == Lq) read their keys back
    from the pages the store just wrote.  7 sequences take the direct grid, 40 the
    persistent one."""
    from nanovllm_amd import workloads as W
    g = torch.Generator().manual_seed(nseq)
    lens = torch.randint(0, 400, (nseq,), generator=g).tolist()
    pre = [(0, 256, 1024)[i % 3] for i in range(nseq)]
    case = W.make_prefill_case(lens, 32, 8, 12 + 4 * nseq, prefix_len=pre, seed=nseq, bulk_device=dev)
    assert case.block_tables is not None
    got = _run_prefill(case)
    for s in range(nseq):
        assert_attn_close(got[rows_of(case, [s])], prefill_reference(case, [s]), what=f"mixed seq {s}")


def test_prefill_pages_outside_the_pool_are_safe(dev):
    """A block id outside [0, num_blocks) inside the visible range: the prefill
    redirects that tile to slot 0 (no access leaves the cache), so the call
    completes, every output is finite, and the other sequences' outputs still
    match the oracle.  (Unlike decode, prefill does not mask those keys: the
    affected sequences' values are unspecified.)  40 sequences take the
    persistent grid."""
    from nanovllm_amd import workloads as W
    g = torch.Generator().manual_seed(21)
    S = 40
    lens = torch.randint(30, 200, (S,), generator=g).tolist()
    case = W.make_prefill_case(lens, 32, 8, 4 * S + 4, prefix_len=512, seed=21, bulk_device=dev,
                               shared_prefix=False)
    m = nva()
    m.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
    bad = {3: (0, -1), 17: (1, 1 << 20), 30: (0, case.k_cache.shape[0]), 31: (2, -7)}
    bt = case.block_tables.clone()
    for s, (j, val) in bad.items():
        bt[s, j] = val
    o = m.flash_attn_varlen_func(case.q, case.k_cache, case.v_cache, case.max_seqlen_q, case.cu_seqlens_q,
                                 case.max_seqlen_k, case.cu_seqlens_k, case.scale, True, bt)
    torch.cuda.synchronize()
    got = f32(o)
    assert np.isfinite(got).all()
    good = [s for s in range(S) if s not in bad]
    for s in good:
        assert_attn_close(got[rows_of(case, [s])], prefill_reference(case, [s]), what=f"seq {s}")


@pytest.mark.parametrize("nh,nkv", [(16, 16), (16, 8), (32, 8), (64, 8), (14, 2), (64, 4)])
def test_prefill_shapes(dev, nh, nkv):
    from nanovllm_amd import workloads as W
    lens = [1, 63, 64, 65, 128, 129, 300, 0, 17]
    case = W.make_prefill_case(lens, nh, nkv, 16, seed=nh + nkv, bulk_device=dev, block_size=256)
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"prefill nh={nh} nkv={nkv}")


@pytest.mark.parametrize("prefix", [256, 512])
@pytest.mark.parametrize("shared", [True, False])
def test_prefill_prefix_shapes(dev, prefix, shared):
    from nanovllm_amd import workloads as W
    lens = [1, 100, 256, 0, 333]
    case = W.make_prefill_case(lens, 16, 8, 40, prefix_len=prefix, seed=prefix + shared, bulk_device=dev,
                               shared_prefix=shared)
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"prefix={prefix} shared={shared}")


@pytest.mark.parametrize("nh,nkv", [(16, 8), (64, 4)])
def test_prefill_one_new_token_after_long_prefix(dev, nh, nkv):
    """A prefix-cache hit that leaves a single token to compute (whole pages are cached,
    block_manager.py:60-82, so a prompt of 16 full pages plus one token prefills 1 query
    over 4097 keys), next to a fresh 300-token sequence and a 1-token suffix after one
    cached page; heads 16/8 and 64/4 (Qwen3-235B-A22B's GQA group 16: 16 positions per
    work item).  Every row against the oracle."""
    from nanovllm_amd import workloads as W
    lens, pre = [1, 300, 1], [4096, 0, 256]
    pages = sum(-(-(q + x) // 256) for q, x in zip(lens, pre)) + 4
    case = W.make_prefill_case(lens, nh, nkv, pages, prefix_len=pre, seed=4097 + nh, bulk_device=dev,
                               shared_prefix=False)
    assert case.block_tables is not None
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"one new token after a long prefix nh={nh} nkv={nkv}")


@pytest.mark.parametrize("prefix", [0, 256])
def test_prefill_group_16_prefix(dev, prefix):
    """GQA group 16 (heads 64/4) through the persistent grid, packed and prefix-cached:
    40 ragged sequences, every row against the oracle."""
    from nanovllm_amd import workloads as W
    gen = torch.Generator().manual_seed(1600 + prefix)
    lens = torch.randint(0, 200, (40,), generator=gen).tolist()
    lens[7] = 700
    pages = sum(-(-(prefix + x) // 256) for x in lens) + 4
    case = W.make_prefill_case(lens, 64, 4, pages, prefix_len=prefix, seed=1601 + prefix, bulk_device=dev,
                               shared_prefix=False)
    assert 40 * 4 * -(-700 // 16) > 2 * 256  # the persistent grid serves this call
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"group 16 prefix={prefix}")


@pytest.mark.parametrize("lens,prefix,nh,nkv,d,bs", [
    (None, 1024, 4, 1, 128, 256),  # config 4's lengths at heads 4/1 (one GPU's share at TP8)
    ([700, 300, 1000], [512, 0, 256], 16, 8, 128, 64),  # one tile per page, mixed prefixes
    ([900, 400], [1024, 512], 32, 8, 128, 512),  # eight tiles per page
    ([1500, 600], [256, 0], 14, 2, 64, 128),  # GQA 7, head_dim 64
])
def test_prefill_key_halves_paged(dev, monkeypatch, lens, prefix, nh, nkv, d, bs):
    """Prefix-cached (paged) direct-grid launches with key halving: a split
    item's halves meet at the page boundary nearest its middle, and the second
    half reads the block-table row from that page on.  Every row against the
    oracle and against whole items (no workspace); the control words consistent."""
    from nanovllm_amd import workloads as W
    from nanovllm_amd.layers import attention as A
    gen = None
    if lens is None:
        gen = torch.Generator().manual_seed(W.SEEDS[4])
        lens = torch.randint(256, 769, (16,), generator=gen).tolist()
    pre = prefix if isinstance(prefix, list) else [prefix] * len(lens)
    pages = sum(-(-(q + x) // bs) for q, x in zip(lens, pre)) + 4
    case = W.make_prefill_case(lens, nh, nkv, pages, prefix_len=pre, block_size=bs, head_dim=d,
                               seed=sum(lens) + bs, bulk_device=dev, shared_prefix=False, gen=gen)
    assert case.block_tables is not None
    bp = 256 // (nh // nkv)
    assert len(lens) * nkv * -(-max(lens) // bp) <= 2 * 256  # the direct grid serves this call
    print(f"paged key halves lens={lens} prefix={prefix} nh={nh} nkv={nkv} d={d} bs={bs}", flush=True)
    halved = _run_prefill(case)
    ws = A._PREFILL_WORKSPACES[(dev.index or 0, torch.cuda.current_stream(dev).cuda_stream)]
    _assert_ws_consistent(ws)
    ref = prefill_reference(case)
    assert_attn_close(halved, ref, what=f"paged key halves bs={bs}")
    monkeypatch.setattr(A, "_prefill_workspace", lambda device, stream: None)
    whole = _run_prefill(case, store=False)
    assert_attn_close(whole, ref, what=f"paged whole items bs={bs}")
    assert float(np.abs(halved - whole).max()) < 2e-2


SPIKE_POSITIONS = (5, 37, 70, 100, 131, 250)  # spread over both lane halves and several steps


@pytest.mark.parametrize("prefix", [0, 256])
def test_prefill_score_outliers(dev, prefix):
    """A few keys score ~160 log2 units above the rest.  A row maximum that
    misses any lane holding part of the row lets exp2 overflow to inf."""
    from nanovllm_amd import workloads as W
    lens = [200, 77, 300]
    case = W.make_prefill_case(lens, 16, 8, 24, prefix_len=prefix, seed=91 + prefix, bulk_device=dev,
                               shared_prefix=False)
    case.q.fill_(1.0)  # score of a key = scale * sum of its entries
    cu = case.cu_seqlens_q.cpu().tolist()
    for s, L in enumerate(lens):
        for p in SPIKE_POSITIONS:
            if p < L:
                case.k[cu[s] + p] = 10.0  # scale * 1280 = 113 nats
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"outliers prefix={prefix}")


def test_decode_score_outliers(dev):
    from nanovllm_amd import workloads as W
    case = W.make_decode_case(6, 16, 8, 300, 900, 24, seed=93, bulk_device=dev)
    case.q.fill_(1.0)
    bt = case.block_tables.cpu()
    for b in range(case.batch):
        for p in SPIKE_POSITIONS + (299,):
            page = int(bt[b, p // case.block_size])
            case.k_cache[page, p % case.block_size] = 10.0
    got = _run_decode(case)
    assert_attn_close(got, decode_reference(case), what="decode outliers")


def test_prefill_prefix_equals_full_tail(dev):
    """Prefix-cached prefill == the last Lq rows of a full prefill over prefix+suffix."""
    from nanovllm_amd import workloads as W
    m = nva()
    lens = [300, 129]
    case = W.make_prefill_case(lens, 16, 8, 16, prefix_len=256, seed=77, bulk_device=dev, shared_prefix=False)
    got = _run_prefill(case)
    bs = case.block_size
    for s, Lq in enumerate(lens):
        Lk = 256 + Lq
        bt = case.block_tables[s]
        pages = bt[: math.ceil(Lk / bs)].long()
        k_full = case.k_cache.index_select(0, pages).reshape(-1, 8, 128)[:Lk].contiguous()
        v_full = case.v_cache.index_select(0, pages).reshape(-1, 8, 128)[:Lk].contiguous()
        q_full = torch.cat([torch.randn(256, 16, 128, device=dev).bfloat16(),
                            case.q[case.cu_seqlens_q[s]:case.cu_seqlens_q[s + 1]]])
        cu = torch.tensor([0, Lk], dtype=torch.int32, device=dev)
        full = m.flash_attn_varlen_func(q_full, k_full, v_full, Lk, cu, Lk, cu, case.scale)
        torch.cuda.synchronize()
        rows = rows_of(case, [s])
        assert np.abs(f32(full[256:]) - got[rows]).max() <= 1e-2


# ----------------------------------------------------------------------------
# the Attention module behind the Context, and graph capture
# ----------------------------------------------------------------------------

def test_attention_module_prefill_then_decode(dev):
    from nanovllm_amd import workloads as W
    m = nva()
    nh, nkv, d, bs = 16, 8, 128, 256
    lens = [200, 513]
    case = W.make_prefill_case(lens, nh, nkv, 8, seed=21, bulk_device=dev)
    attn = m.Attention(nh, d, d ** -0.5, nkv)
    attn.k_cache, attn.v_cache = case.k_cache, case.v_cache
    m.set_context(True, case.cu_seqlens_q, case.cu_seqlens_k, case.max_seqlen_q, case.max_seqlen_k,
                  case.slot_mapping, None, None)
    o = attn(case.q.reshape(-1, nh * d), case.k.reshape(-1, nkv * d), case.v.reshape(case.v.shape[0], -1))
    torch.cuda.synchronize()
    assert o.shape == (sum(lens), nh * d)
    assert_attn_close(f32(o).reshape(-1, nh, d), prefill_reference(case), what="module prefill")
    # one decode step per sequence; the page table is read back from the prefill's
    # slot mapping (page i of sequence s holds its tokens i*bs .. i*bs+bs-1), and
    # the new token (position L, L % bs != 0 here) goes to the next slot of the last page
    bt = torch.full((2, 3), -1, dtype=torch.int32)
    slots = case.slot_mapping.cpu().tolist()
    cu = case.cu_seqlens_q.cpu().tolist()
    ctx, new_slots = [], []
    for s, L in enumerate(lens):
        seq_slots = slots[cu[s]:cu[s + 1]]
        pages = [seq_slots[i] // bs for i in range(0, L, bs)]
        bt[s, :len(pages)] = torch.tensor(pages, dtype=torch.int32)
        ctx.append(L + 1)
        assert L % bs
        new_slots.append(pages[-1] * bs + L % bs)
    g = torch.Generator(device=dev).manual_seed(4)
    q1 = torch.randn(2, nh * d, generator=g, device=dev).bfloat16()
    k1 = torch.randn(2, nkv * d, generator=g, device=dev).bfloat16()
    v1 = torch.randn(2, nkv * d, generator=g, device=dev).bfloat16()
    m.set_context(False, slot_mapping=torch.tensor(new_slots, dtype=torch.int32, device=dev),
                  context_lens=torch.tensor(ctx, dtype=torch.int32, device=dev), block_tables=bt.to(dev))
    o1 = attn(q1, k1, v1)
    torch.cuda.synchronize()
    m.reset_context()
    for s, L in enumerate(lens):
        k_all = torch.cat([case.k[cu[s]:cu[s + 1]], k1[s].view(1, nkv, d)])
        v_all = torch.cat([case.v[cu[s]:cu[s + 1]], v1[s].view(1, nkv, d)])
        ref = O.attention(f32(q1[s]).reshape(1, nh, d), f32(k_all), f32(v_all), d ** -0.5)[0]
        assert_attn_close(f32(o1[s]).reshape(nh, d), ref, what=f"module decode seq {s}")


def test_decode_graph_capture_replay(dev):
    """store + decode captured in one graph, replayed with new inputs copied into the
    static buffers (model_runner.py:266-282); every replay matches eager."""
    from nanovllm_amd import workloads as W
    m = nva()
    case = W.make_decode_case(16, 16, 8, 50, 900, 64, seed=31, bulk_device=dev, table_width=4)
    st = {k: getattr(case, k).clone() for k in ("q", "context_lens", "block_tables", "slot_mapping")}
    k_new, v_new = case.k_new.clone(), case.v_new.clone()

    def step(q, kn, vn, kc, vc, lens, bt, slots):
        m.store_kvcache(kn, vn, kc, vc, slots)
        return m.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, lens, bt, case.scale)

    step(st["q"], k_new, v_new, case.k_cache, case.v_cache, st["context_lens"], st["block_tables"],
         st["slot_mapping"])  # warmup
    torch.cuda.synchronize()
    kc_eager, vc_eager = case.k_cache.clone(), case.v_cache.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step(st["q"], k_new, v_new, case.k_cache, case.v_cache, st["context_lens"], st["block_tables"],
                   st["slot_mapping"])
    g = torch.Generator(device=dev).manual_seed(99)
    for rep in range(4):
        q = torch.randn(st["q"].shape, generator=g, device=dev).bfloat16()
        kn = torch.randn(k_new.shape, generator=g, device=dev).bfloat16()
        vn = torch.randn(v_new.shape, generator=g, device=dev).bfloat16()
        lens = torch.randint(1, 900, (16,), generator=g, device=dev).int()
        lens = torch.minimum(lens, case.context_lens)  # stay inside the allocated pages
        bt = case.block_tables
        slots = torch.tensor([int(bt[b, (int(L) - 1) // 256]) * 256 + (int(L) - 1) % 256
                              for b, L in enumerate(lens.cpu().tolist())], dtype=torch.int32, device=dev)
        st["q"].copy_(q)
        k_new.copy_(kn)
        v_new.copy_(vn)
        st["context_lens"].copy_(lens)
        st["slot_mapping"].copy_(slots)
        graph.replay()
        torch.cuda.synchronize()
        eager = step(q, kn, vn, kc_eager, vc_eager, lens, bt, slots)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from eager"
        assert torch.equal(case.k_cache, kc_eager) and torch.equal(case.v_cache, vc_eager)


# ----------------------------------------------------------------------------
# head_dim 64: Qwen2-0.5B heads 14/2 (GQA 7), qwen2_05b.txt:10,16,18
# ----------------------------------------------------------------------------

def test_store_head_dim_64_bitexact(dev):
    from nanovllm_amd import workloads as W
    case = W.make_prefill_case([37, 300, 1], 14, 2, 8, head_dim=64, seed=64, bulk_device=dev)
    kc, vc = _sentinel_pool(case, dev)
    ekc, evc = bits16(kc), bits16(vc)
    O.store_kvcache(bits16(case.k), bits16(case.v), ekc, evc, case.slot_mapping.cpu().numpy())
    nva().store_kvcache(case.k, case.v, kc, vc, case.slot_mapping)
    torch.cuda.synchronize()
    assert np.array_equal(bits16(kc), ekc) and np.array_equal(bits16(vc), evc)


@pytest.mark.parametrize("nh,nkv", [(16, 8), (16, 1), (64, 8)])
@pytest.mark.parametrize("fp8", [False, pytest.param(True, marks=pytest.mark.skip(
    reason="paged_decode_balanced_kernel<fp8, 8 waves, d=64> ended a run with a memory aperture violation at "
           "heads 16/8 (cause not found; a host replay of its indices stays in bounds); nva_decode refuses fp8 "
           "at head_dim 64"))])
def test_decode_head_dim_64(dev, nh, nkv, fp8):
    from nanovllm_amd import workloads as W
    lengths = [1, 2, 31, 33, 256, 257, 700, 1025, 0, 3000]
    case = W.make_decode_case(len(lengths), nh, nkv, 0, 0, 40, fp8=fp8, seed=640 + fp8 + nh + nkv,
                              bulk_device=dev, lengths=lengths, table_width=12, head_dim=64)
    for ns in (0, 1, 3):
        got = _run_decode(case, ns, store=(ns == 0))
        tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if fp8 else {}
        assert_attn_close(got, decode_reference(case), what=f"d=64 nh={nh} nkv={nkv} fp8={fp8} splits={ns}", **tol)


@pytest.mark.skip(reason="the two-wave workgroup shape of the balanced decode (used for two kv heads) returned an "
                         "illegal address once (cause not found); it is no longer launched -- 14/2 decode runs one "
                         "wave per workgroup or the spread mode (golden decode_d64_g7, "
                         "test_decode_spread) -- and this test stays skipped until that fault has a cause")
@pytest.mark.parametrize("head_dim", [64, 128])
def test_decode_two_kv_heads(dev, head_dim):
    """Qwen2-0.5B heads 14/2 (qwen2_05b.txt:10,16,18)."""
    from nanovllm_amd import workloads as W
    lengths = [1, 2, 31, 33, 256, 257, 700, 1025, 0, 3000]
    case = W.make_decode_case(len(lengths), 14, 2, 0, 0, 40, seed=642, bulk_device=dev, lengths=lengths,
                              table_width=12, head_dim=head_dim)
    for ns in (0, 1, 3):
        got = _run_decode(case, ns, store=(ns == 0))
        assert_attn_close(got, decode_reference(case), what=f"nkv=2 d={head_dim} splits={ns}")


@pytest.mark.parametrize("nh,nkv,d,prefix", [(14, 2, 64, 0), (14, 2, 64, 256), (32, 8, 128, 0), (32, 8, 128, 256)])
def test_prefill_persistent_many_sequences(dev, nh, nkv, d, prefix):
    """Enough (sequence, kv head, query tile) items for the persistent grid
    (more than twice the CU count): ragged lengths with empty query segments
    (a full prefix hit), one long sequence; every output row vs the oracle."""
    from nanovllm_amd import workloads as W
    gen = torch.Generator().manual_seed(900 + nh + d + prefix)
    S = 40 if d == 64 else 24
    lens = torch.randint(0, 301 if d == 64 else 401, (S,), generator=gen).tolist()
    lens[3] = 0
    lens[7] = 0
    lens[S - 2] = 1000
    bs = 256
    pages = sum(-(-(prefix + x) // bs) for x in lens) + 4
    case = W.make_prefill_case(lens, nh, nkv, pages, prefix_len=prefix, head_dim=d, seed=901 + nh,
                               bulk_device=dev, shared_prefix=False)
    G = nh // nkv
    bp = 256 // G
    assert S * nkv * -(-max(lens) // bp) > 2 * 256  # the persistent grid serves this call
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"persistent prefill nh={nh} nkv={nkv} d={d} prefix={prefix}")


def test_prefill_work_queue_matches_static_order(dev, monkeypatch):
    """The persistent grid hands items out from a work queue in the workspace
    the mirror caches per stream, or in a static order without one.  Each item
    is computed the same way wherever it runs, so the outputs are bit-identical;
    every call leaves the queue zero, so consecutive calls of different sizes
    (config 4, a smaller head_dim-64 GQA-7 call, config 4 again) reuse it."""
    from nanovllm_amd import workloads as W
    from nanovllm_amd.layers import attention as A
    gen = torch.Generator().manual_seed(4242)
    lens = torch.randint(0, 301, (40,), generator=gen).tolist()
    lens[-1] = 1000
    pages = sum(-(-(256 + x) // 256) for x in lens) + 4
    small = W.make_prefill_case(lens, 14, 2, pages, prefix_len=256, head_dim=64, seed=4243, bulk_device=dev,
                                shared_prefix=False)
    big = W.config4(dev)
    orig = A._prefill_workspace
    for case in (big, small, big):
        print(f"work queue vs static: {case.name if hasattr(case, 'name') else 'case'}", flush=True)
        queued = _run_prefill(case)
        ws = A._PREFILL_WORKSPACES[(dev.index or 0, torch.cuda.current_stream(dev).cuda_stream)]
        _assert_ws_consistent(ws)
        monkeypatch.setattr(A, "_prefill_workspace", lambda device, stream: None)
        static = _run_prefill(case, store=False)
        monkeypatch.setattr(A, "_prefill_workspace", orig)
        assert np.array_equal(queued, static)
        again = _run_prefill(case, store=False)
        assert np.array_equal(again, queued)
        _assert_ws_consistent(ws)


# The prefill workspace's control words fill its first 2048 bytes: the work queue
# (9 words from byte 0), the error word and the merge wait's poll-limit word (bytes
# 128 and 132), then three words per key-split slot from byte 256 (arrival count,
# ready word, epoch; 128 slots).  The rest holds the partial results and is
# overwritten by every split call.
_WS_CTL_BYTES = 2048
_WS_ERR, _WS_LIMIT, _WS_SLOTS, _WS_NSLOTS = 128, 132, 256, 128


def _ws_words(ws):
    return ws[:_WS_CTL_BYTES].cpu().numpy().view(np.uint32)


def _assert_ws_consistent(ws):
    """What every completed call leaves: the queue, error and limit words zero, and
    each slot's arrival count twice its epoch with the ready word at the epoch (the
    value a partial of the last completed use carries; the next use waits for
    epoch + 1)."""
    w = _ws_words(ws)
    assert not w[:_WS_SLOTS // 4].any(), "the queue, error and limit words must be left zero"
    end = _WS_SLOTS // 4 + 3 * _WS_NSLOTS
    assert not w[end:].any(), "the words past the last slot must stay zero"
    slots = w[_WS_SLOTS // 4:end].reshape(-1, 3)
    count, ready, epoch = slots[:, 0].astype(np.int64), slots[:, 1].astype(np.int64), slots[:, 2].astype(np.int64)
    assert np.array_equal(count, 2 * epoch), "arrival counts out of step with the epochs"
    assert np.array_equal(ready, epoch), "ready words out of step with the epochs"
    return epoch


@pytest.mark.parametrize("lens,nh,nkv,d", [
    ([512, 540, 147, 296, 319, 300, 927, 255], 16, 8, 128),  # config 2's lengths
    ([1000] * 8, 16, 8, 128),  # 512 items: no CU left free, so the compact grid runs every item whole
    ([1000] * 6, 8, 1, 128),  # 84 pairs of >= 10 key tiles, 64 of them split (the workspace's slots)
    ([900, 37, 0, 650], 14, 2, 64),  # GQA 7 (36 positions per tile), head_dim 64, an empty sequence
    ([2048], 32, 8, 128),  # one fresh prompt (Qwen3-8B heads): 256 items, the 4 heaviest levels split
])
def test_prefill_key_halves(dev, monkeypatch, lens, nh, nkv, d):
    """A direct-grid launch (at most two grid cells per CU) over packed k/v runs
    on the compact grid, heaviest items first, and its items of many key tiles
    as two workgroups, one per key half; the one that finishes second merges the
    other's float32 partial (O, row maximum and sum) from the mirror's
    workspace.  Without a workspace every item runs whole on the plain grid.
    Both against the oracle on every row (the early rows of an item see no key of
    its second half), the halves within the bf16 bar of the whole items, the
    control words consistent after each call, and a second call reusing the slots."""
    from nanovllm_amd import workloads as W
    from nanovllm_amd.layers import attention as A
    pages = sum(-(-x // 256) for x in lens) + 4
    case = W.make_prefill_case(lens, nh, nkv, pages, head_dim=d, seed=sum(lens) + d, bulk_device=dev)
    assert case.block_tables is None
    bp = 256 // (nh // nkv)
    assert len(lens) * nkv * -(-max(lens) // bp) <= 2 * 256  # the direct grid serves this call
    print(f"key halves lens={lens} nh={nh} nkv={nkv} d={d}", flush=True)
    halved = _run_prefill(case)
    ws = A._PREFILL_WORKSPACES[(dev.index or 0, torch.cuda.current_stream(dev).cuda_stream)]
    _assert_ws_consistent(ws)
    ref = prefill_reference(case)
    assert_attn_close(halved, ref, what=f"key halves {lens}")
    again = _run_prefill(case, store=False)
    _assert_ws_consistent(ws)
    assert_attn_close(again, ref, what=f"key halves, second call {lens}")
    monkeypatch.setattr(A, "_prefill_workspace", lambda device, stream: None)
    whole = _run_prefill(case, store=False)
    assert_attn_close(whole, ref, what=f"whole items {lens}")
    assert float(np.abs(halved - whole).max()) < 2e-2


def _cfg2_case(dev):
    from nanovllm_amd import workloads as W
    lens = [512, 540, 147, 296, 319, 300, 927, 255]  # config 2's lengths: key halving on the compact grid
    return W.make_prefill_case(lens, 16, 8, sum(-(-x // 256) for x in lens) + 4, seed=2202, bulk_device=dev)


def test_prefill_key_half_wait_gives_up_loudly(dev):
    """The key-half merge's bounded wait, forced to give up from the host: the
    workspace's poll-limit word set to allow no poll, so every split item's merging
    half gives up.  The call completes (every kernel exits), the split items' rows
    come back NaN -- whole (position, head) rows, never mixed with numbers -- while
    every other row matches the oracle, and the error word reports it (read and
    cleared by prefill_workspace_errors).  With the limit word back to 0 the next
    call is clean: every row against the oracle, no error, the words consistent."""
    from nanovllm_amd import _capi
    from nanovllm_amd.layers import attention as A
    case = _cfg2_case(dev)
    ref = prefill_reference(case)
    clean = _run_prefill(case)
    key = (dev.index or 0, torch.cuda.current_stream(dev).cuda_stream)
    ws = A._PREFILL_WORKSPACES[key]
    assert A.prefill_workspace_errors()[key] == 0
    epoch0 = _assert_ws_consistent(ws)
    assert_attn_close(clean, ref, what="key halves before the forced give-up")
    off = _capi.NVA_PREFILL_SPLIT_WAIT_LIMIT_OFFSET
    ws[off:off + 4] = torch.tensor([1, 0, 0, 0], dtype=torch.uint8, device=dev)  # n - 1 = 0 polls
    print("prefill with the merge wait limited to no poll", flush=True)
    forced = _run_prefill(case, store=False)
    ws[off:off + 4] = 0
    assert A.prefill_workspace_errors()[key] == _capi.NVA_PREFILL_ERR_SPLIT_WAIT
    assert A.prefill_workspace_errors()[key] == 0  # cleared by the read
    nan = np.isnan(forced)
    assert nan.any(), "no split item gave up"
    rows_nan = nan.all(axis=-1)
    assert np.array_equal(rows_nan, nan.any(axis=-1)), "NaN must fill whole rows"
    ok = ~rows_nan
    assert_attn_close(forced[ok], ref[ok], what="rows of items that were not split")
    epoch1 = _assert_ws_consistent(ws)
    assert (epoch1 >= epoch0).all() and (epoch1 > epoch0).any()
    again = _run_prefill(case, store=False)
    assert A.prefill_workspace_errors()[key] == 0
    assert_attn_close(again, ref, what="key halves after the forced give-up")
    # (which half merges depends on which finishes first: equal up to float32 rounding)
    assert float(np.abs(again - clean).max()) <= 1e-2
    _assert_ws_consistent(ws)


def test_prefill_key_halves_arrival_count_out_of_step(dev):
    """A slot whose arrival count is odd at the start of a call (words out of step:
    the first half to arrive takes the merging role and waits for the second) still
    merges the right partial, and the call leaves the slot consistent again."""
    from nanovllm_amd.layers import attention as A
    case = _cfg2_case(dev)
    ref = prefill_reference(case)
    clean = _run_prefill(case)
    key = (dev.index or 0, torch.cuda.current_stream(dev).cuda_stream)
    ws = A._PREFILL_WORKSPACES[key]
    epoch = _assert_ws_consistent(ws)
    used = np.nonzero(epoch)[0]
    assert used.size, "no split slot was used"
    for s in used[:4]:
        b = _WS_SLOTS + 12 * int(s)
        count = int(2 * epoch[s] + 1)
        ws[b:b + 4] = torch.tensor(list(count.to_bytes(4, "little")), dtype=torch.uint8, device=dev)
    print(f"prefill with slots {used[:4].tolist()} out of step", flush=True)
    odd = _run_prefill(case, store=False)
    assert A.prefill_workspace_errors()[key] == 0
    assert float(np.abs(odd - clean).max()) <= 1e-2
    _assert_ws_consistent(ws)
    assert_attn_close(odd, ref, what="key halves with the arrival count out of step")


@pytest.mark.parametrize("prefix", [0, 256])
def test_prefill_more_sequences_than_the_persistent_tables(dev, prefix):
    """Over 1024 sequences the persistent grid's tables do not fit its LDS and
    the direct grid serves the call: 1100 short ragged sequences, some empty."""
    from nanovllm_amd import workloads as W
    gen = torch.Generator().manual_seed(1100 + prefix)
    S = 1100
    lens = torch.randint(0, 41, (S,), generator=gen).tolist()
    for i in range(0, S, 97):
        lens[i] = 0
    lens[S - 1] = 300
    pages = (S if prefix else 0) + sum(-(-x // 256) for x in lens) + 4
    case = W.make_prefill_case(lens, 16, 8, pages, prefix_len=prefix, seed=1101 + prefix, bulk_device=dev,
                               shared_prefix=False)
    got = _run_prefill(case)
    seqs = list(range(0, S, 53)) + [S - 1]
    ref = prefill_reference(case, seqs)
    assert_attn_close(got[rows_of(case, seqs)], ref, what=f"{S} sequences prefix={prefix}")


@pytest.mark.parametrize("block_size,prefix_pages", [(64, 3), (128, 2), (512, 1), (768, 1)])
def test_prefill_paged_block_sizes(dev, block_size, prefix_pages):
    """Prefix-cached prefill over caches paged at block sizes other than 256: the
    kernel walks a sequence's tiles page by page (one tile per page at 64, a
    first tile in the middle of a page at 768), direct grid."""
    from nanovllm_amd import workloads as W
    lens = [1, 100, 333, 64, 0, 700]
    prefix = prefix_pages * block_size
    pages = sum(-(-(prefix + x) // block_size) for x in lens) + 4
    case = W.make_prefill_case(lens, 16, 8, pages, prefix_len=prefix, block_size=block_size,
                               seed=block_size + prefix_pages, bulk_device=dev, shared_prefix=False)
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"block_size={block_size} prefix={prefix}")


@pytest.mark.parametrize("block_size", [64, 512])
def test_prefill_persistent_block_sizes(dev, block_size):
    """The persistent grid (more than twice the CU count of items) over caches
    paged at 64 and 512 keys, with a shared cached prefix."""
    from nanovllm_amd import workloads as W
    gen = torch.Generator().manual_seed(950 + block_size)
    S = 24
    lens = torch.randint(0, 401, (S,), generator=gen).tolist()
    lens[5] = 0
    lens[S - 1] = 900
    prefix = 512
    pages = sum(-(-(prefix + x) // block_size) for x in lens) + 4
    case = W.make_prefill_case(lens, 32, 8, pages, prefix_len=prefix, block_size=block_size,
                               seed=951 + block_size, bulk_device=dev, shared_prefix=True)
    assert S * 8 * -(-max(lens) // 64) > 2 * 256  # the persistent grid serves this call
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"persistent block_size={block_size}")


@pytest.mark.parametrize("prefix", [0, 256])
def test_prefill_head_dim_64(dev, prefix):
    from nanovllm_amd import workloads as W
    lens = [1, 63, 64, 65, 300, 0, 777]
    case = W.make_prefill_case(lens, 14, 2, 24, prefix_len=prefix, head_dim=64, seed=65 + prefix,
                               bulk_device=dev, shared_prefix=False)
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what=f"d=64 prefill prefix={prefix}")


def test_prefill_head_dim_64_score_outliers(dev):
    from nanovllm_amd import workloads as W
    lens = [200, 130]
    case = W.make_prefill_case(lens, 8, 2, 8, head_dim=64, seed=66, bulk_device=dev)
    case.q.fill_(1.0)
    cu = case.cu_seqlens_q.cpu().tolist()
    for s, L in enumerate(lens):
        for p in SPIKE_POSITIONS:
            if p < L:
                case.k[cu[s] + p] = 16.0  # 64 * 16 * scale(1/8) = 128 nats
    got = _run_prefill(case)
    assert_attn_close(got, prefill_reference(case), what="d=64 outliers")
