"""Decode under the reference's zero padding (reference quirk Q1) on the GPU.

run_model zero-fills the captured graph's static buffers and copies the live rows
in (nanovllm/engine/model_runner.py:271-280), so every padded row has slot 0,
context length 0 and a block table of zeros, and its store writes slot 0 of block
0 -- the first block the block manager hands out (block_manager.py:33,71), which
a live sequence may own.  The reference stores first (attention.py:65-66) and then
decodes, so that live sequence reads the padded row in place of its own key 0.

The checks, each on two steps in a row:
  * Attention.forward (default: the reference's two calls) replayed from a
    DecodeGraphs capture with pad_slot=0, and called eagerly with ctx-0 rows at
    slot 0: outputs and caches bit-identical to store_kvcache followed by
    flash_attn_with_kvcache on copies of the caches;
  * store_and_decode (the fused call) on the same batches: its caches equal the
    two calls', and its outputs equal the two calls' on a cache where the ctx-0
    rows are stored after the decode -- the order nva_store_decode defines for
    rows without keys (the merge kernel stores them after every read).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _helpers import FP8_MAX_ABS, assert_attn_close, bits8, bits16, decode_reference, f32

pytestmark = pytest.mark.gpu

BS_PAGE = 256


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()
    return torch.device("cuda:0")


def _padded_batch(dev, live_lens, n_pad, num_blocks, width, nh, nkv, d, seed, pad_kv="zeros"):
    """A decode batch of len(live_lens) live sequences followed by n_pad rows padded
    the reference's way (slot 0, length 0, table of zeros).  Live sequence 0 owns
    block 0 as its first page, so its key 0 sits in slot 0.  Padded rows carry one
    common key/value row (zeros, as the zeroed static buffers give, or one random
    row), so their stores to slot 0 agree with each other."""
    g = torch.Generator().manual_seed(seed)
    perm = [int(x) for x in torch.randperm(num_blocks - 1, generator=g) + 1]
    B = len(live_lens) + n_pad
    bt = torch.zeros(B, width, dtype=torch.int32)
    ctx = torch.zeros(B, dtype=torch.int32)
    slots = torch.zeros(B, dtype=torch.int32)
    at = 0
    for b, L in enumerate(live_lens):
        n = math.ceil(L / BS_PAGE)
        pages = ([0] + perm[at:at + n - 1]) if b == 0 else perm[at:at + n]
        at += n - 1 if b == 0 else n
        bt[b, :n] = torch.tensor(pages, dtype=torch.int32)
        bt[b, n:] = -1
        ctx[b] = L
        slots[b] = pages[-1] * BS_PAGE + (L - 1) % BS_PAGE
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    q = torch.randn(B, nh, d, generator=gd, device=dev).bfloat16()
    k = torch.randn(B, nkv, d, generator=gd, device=dev).bfloat16()
    v = torch.randn(B, nkv, d, generator=gd, device=dev).bfloat16()
    nl = len(live_lens)
    if n_pad:
        if pad_kv == "zeros":
            q[nl:] = 0
            k[nl:] = 0
            v[nl:] = 0
        else:
            k[nl:] = k[nl]
            v[nl:] = v[nl]
    return q, k, v, slots.to(dev), ctx.to(dev), bt.to(dev)


def _caches(dev, num_blocks, nkv, d, seed, fp8):
    from nanovllm_amd import workloads as W
    g = torch.Generator(device=dev).manual_seed(seed)
    kc = torch.randn(num_blocks, BS_PAGE, nkv, d, generator=g, device=dev).bfloat16()
    vc = torch.randn(num_blocks, BS_PAGE, nkv, d, generator=g, device=dev).bfloat16()
    if not fp8:
        return kc, vc, None, None
    kc, ks = W.quantize_cache_fp8(kc)
    vc, vs = W.quantize_cache_fp8(vc)
    # headroom for the new rows (|x| <= ~5 sigma) under the cache's amax / 448
    return kc, vc, ks * 1.5, vs * 1.5


def _view(fp8):
    return bits8 if fp8 else bits16


def _two_calls(m, q, k, v, kc, vc, slots, ctx, bt, ks=None, vs=None):
    m.store_kvcache(k, v, kc, vc, slots, ks, vs)
    return m.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, ctx, bt, q.shape[-1] ** -0.5, True,
                                     k_scale=ks, v_scale=vs)


def _step_lens(base, step):
    return [x + step for x in base]


# ----------------------------------------------------------------------------
# Attention.forward, eager: the reference's two calls, bit for bit
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("live", [[300, 1000, 17], [300] + [129 + 31 * i for i in range(47)]])
def test_forward_zero_padded_rows_match_two_calls(dev, fp8, live):
    import nanovllm_amd as m
    nh, nkv, d, nb = 16, 8, 128, 256
    kc, vc, ks, vs = _caches(dev, nb, nkv, d, seed=5, fp8=fp8)
    a = m.Attention(nh, d, d ** -0.5, nkv)
    a.k_cache, a.v_cache, a.k_scale, a.v_scale = kc.clone(), vc.clone(), ks, vs
    tk, tv = kc.clone(), vc.clone()
    for step in range(2):
        q, k, v, slots, ctx, bt = _padded_batch(dev, _step_lens(live, step), 5, nb, 8, nh, nkv, d, seed=40 + step)
        m.set_context(False, slot_mapping=slots, context_lens=ctx, block_tables=bt)
        try:
            got = a(q.view(q.shape[0], -1), k.view(k.shape[0], -1), v.view(v.shape[0], -1))
        finally:
            m.reset_context()
        ref = _two_calls(m, q, k, v, tk, tv, slots, ctx, bt, ks, vs)
        torch.cuda.synchronize()
        assert np.array_equal(bits16(got), bits16(ref.view(got.shape))), f"step {step}: forward != two calls"
        assert np.array_equal(_view(fp8)(a.k_cache), _view(fp8)(tk))
        assert np.array_equal(_view(fp8)(a.v_cache), _view(fp8)(tv))
        # the padded rows did write slot 0, which sequence 0 reads as its key 0
        assert bool((a.k_cache[0, 0] == 0).all()) if not fp8 else bool((a.k_cache.view(torch.uint8)[0, 0] == 0).all())


# ----------------------------------------------------------------------------
# store_and_decode: rows without keys stored after every read
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("live", [[300, 1000, 17], [300] + [129 + 31 * i for i in range(47)]],
                         ids=["spread", "balanced"])
def test_store_decode_stores_empty_rows_after_reads(dev, fp8, live):
    from types import SimpleNamespace
    import nanovllm_amd as m
    nh, nkv, d, nb = 16, 8, 128, 256
    kc, vc, ks, vs = _caches(dev, nb, nkv, d, seed=6, fp8=fp8)
    fk, fv = kc.clone(), vc.clone()      # fused call's caches
    tk, tv = kc.clone(), vc.clone()      # the two calls' caches
    ok_, ov = kc.clone(), vc.clone()     # live rows stored, decode, then the ctx-0 rows
    nl = len(live)
    balanced_fp8 = fp8 and nl > 32  # this plan runs the store kernel first: exactly the two calls
    for step in range(2):
        q, k, v, slots, ctx, bt = _padded_batch(dev, _step_lens(live, step), 5, nb, 8, nh, nkv, d, seed=60 + step,
                                                pad_kv="random")
        fused = m.store_and_decode(q.unsqueeze(1), k, v, fk, fv, slots, ctx, bt, d ** -0.5, k_scale=ks, v_scale=vs)
        two = _two_calls(m, q, k, v, tk, tv, slots, ctx, bt, ks, vs)
        live_slots = slots.clone()
        live_slots[nl:] = -1
        after = _two_calls(m, q, k, v, ok_, ov, live_slots, ctx, bt, ks, vs)
        read_k, read_v = ok_.clone(), ov.clone()  # the cache the fused decode reads
        m.store_kvcache(k, v, ok_, ov, slots, ks, vs)
        torch.cuda.synchronize()
        view = _view(fp8)
        assert np.array_equal(view(fk), view(tk)) and np.array_equal(view(fv), view(tv)), f"step {step}: cache"
        assert np.array_equal(view(ok_), view(tk)) and np.array_equal(view(ov), view(tv))
        want = two if balanced_fp8 else after
        assert np.array_equal(bits16(fused), bits16(want)), f"step {step}: fused output"
        # every sequence that does not read slot 0 gets the two calls' bits
        assert np.array_equal(bits16(fused[1:]), bits16(two[1:]))
        assert not bool(fused[nl:].any())  # padded rows: no keys, zeros
        tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if fp8 else {}
        src_k, src_v = (tk, tv) if balanced_fp8 else (read_k, read_v)
        case = SimpleNamespace(batch=q.shape[0], context_lens=ctx, block_tables=bt, q=q, num_heads=nh,
                               num_kv_heads=nkv, head_dim=d, block_size=BS_PAGE, scale=d ** -0.5,
                               k_cache=src_k, v_cache=src_v, k_scale=ks, v_scale=vs)
        assert_attn_close(f32(fused[:, 0]), decode_reference(case), what=f"fused step {step}", **tol)


# ----------------------------------------------------------------------------
# DecodeGraphs with the reference's padding
# ----------------------------------------------------------------------------

def test_graph_replay_zero_padding_matches_two_calls(dev):
    """Captured steps of two layers with pad_slot=0, replayed at batch 3 (graph 4),
    batch 13 (graph 16) and batch 3 again, with a live sequence owning block 0: every
    row of every layer's output (padded rows included) and both caches are
    bit-identical to the two calls over the padded batch the replay saw."""
    import nanovllm_amd as m
    from nanovllm_amd.engine.decode_graphs import DecodeGraphs
    nh, nkv, d, nb, width = 16, 8, 128, 96, 6
    layers, twins = [], []
    for li in range(2):
        kc, vc, _, _ = _caches(dev, nb, nkv, d, seed=70 + li, fp8=False)
        a = m.Attention(nh, d, d ** -0.5, nkv)
        a.k_cache, a.v_cache = kc, vc
        layers.append(a)
        twins.append((kc.clone(), vc.clone()))
    graphs = DecodeGraphs(layers, max_bs=16, max_num_blocks=width, pad_slot=0).capture()
    for li, a in enumerate(layers):  # capture's warm-up wrote slot 0 (zero rows): same on the twins
        twins[li][0].copy_(a.k_cache)
        twins[li][1].copy_(a.v_cache)
    for step, live in enumerate([[300, 1000, 17], [301] + [200 + 50 * i for i in range(12)], [302, 1001, 18]]):
        q, k, v, slots, ctx, bt = _padded_batch(dev, live, 0, nb, width - 1, nh, nkv, d, seed=80 + step)
        bs = len(live)
        outs = graphs.run(q.view(bs, -1), k.view(bs, -1), v.view(bs, -1), slots, ctx, bt)
        size = min(x for x in graphs.graph_bs if x >= bs)
        assert size > bs
        # the padded batch the replay saw: its static buffers
        pq = graphs.q[:size].view(size, nh, d)
        pk = graphs.k[:size].view(size, nkv, d)
        pv = graphs.v[:size].view(size, nkv, d)
        ps, pc, pb = graphs.slot_mapping[:size], graphs.context_lens[:size], graphs.block_tables[:size]
        assert int(ps[bs:].abs().sum()) == 0 and int(pc[bs:].abs().sum()) == 0
        for li, a in enumerate(layers):
            tk, tv = twins[li]
            ref = _two_calls(m, pq, pk, pv, tk, tv, ps, pc, pb)
            torch.cuda.synchronize()
            full = graphs.layer_outputs[size][li]
            assert np.array_equal(bits16(full), bits16(ref.view(full.shape))), f"step {step} layer {li}"
            assert torch.equal(outs[li], full[:bs])
            assert np.array_equal(bits16(a.k_cache), bits16(tk)) and np.array_equal(bits16(a.v_cache), bits16(tv))
            assert bool((a.k_cache[0, 0] == 0).all())  # the padded rows' zeros, read by sequence 0
