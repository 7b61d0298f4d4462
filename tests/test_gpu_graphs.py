"""The decode graph harness (nanovllm_amd.engine.decode_graphs) on the GPU: captured
steps of two Attention layers replayed at several batch sizes match the CPU oracle
on the caches as the replay left them (and eager execution), the padded rows of a
graph produce zeros and leave the cache alone (slot pad -1, reference quirk Q1),
and sizes beyond the largest graph run eagerly."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from types import SimpleNamespace

from _helpers import assert_attn_close, bits16, decode_reference, f32

pytestmark = pytest.mark.gpu

NH, NKV, D, BS_PAGE = 16, 8, 128, 256


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()
    return torch.device("cuda:0")


def _layers(dev, n_layers, num_blocks, seed):
    import nanovllm_amd as nva
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        a = nva.Attention(NH, D, D ** -0.5, NKV)
        a.k_cache = torch.randn(num_blocks, BS_PAGE, NKV, D, generator=g, device=dev).bfloat16()
        a.v_cache = torch.randn(num_blocks, BS_PAGE, NKV, D, generator=g, device=dev).bfloat16()
        layers.append(a)
    return layers


def _batch(dev, bs, max_blocks, num_blocks, seed):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, max_blocks * BS_PAGE, (bs,), generator=g)
    perm = torch.randperm(num_blocks, generator=g)
    bt = torch.full((bs, max_blocks), -1, dtype=torch.int32)
    slots = []
    at = 0
    for b in range(bs):
        n = math.ceil(int(ctx[b]) / BS_PAGE)
        bt[b, :n] = perm[at:at + n].to(torch.int32)
        at += n
        last = int(ctx[b]) - 1
        slots.append(int(bt[b, last // BS_PAGE]) * BS_PAGE + last % BS_PAGE)
    gd = torch.Generator(device=dev).manual_seed(seed + 1)
    q = torch.randn(bs, NH * D, generator=gd, device=dev).bfloat16()
    k = torch.randn(bs, NKV * D, generator=gd, device=dev).bfloat16()
    v = torch.randn(bs, NKV * D, generator=gd, device=dev).bfloat16()
    return (q, k, v, torch.tensor(slots, dtype=torch.int32, device=dev), ctx.to(torch.int32).to(dev),
            bt.to(dev))


def _eager(layers, q, k, v, slots, ctx, bt):
    import nanovllm_amd as nva
    nva.set_context(False, slot_mapping=slots, context_lens=ctx, block_tables=bt)
    try:
        return torch.stack([a(q, k, v) for a in layers])
    finally:
        nva.reset_context()


def _oracle(layer, q, ctx, bt):
    """Oracle decode of one layer on its cache as it is now (after the step's store)."""
    case = SimpleNamespace(batch=q.shape[0], context_lens=ctx, block_tables=bt, q=q.view(-1, NH, D),
                           num_heads=NH, num_kv_heads=NKV, head_dim=D, block_size=BS_PAGE, scale=D ** -0.5,
                           k_cache=layer.k_cache, v_cache=layer.v_cache, k_scale=None, v_scale=None)
    return decode_reference(case)


def test_replay_matches_eager_and_skips_padding(dev):
    from nanovllm_amd.engine.decode_graphs import DecodeGraphs
    max_blocks, num_blocks = 4, 160
    layers = _layers(dev, 2, num_blocks, seed=3)
    # page 0's first slot holds a sentinel a zero-padded slot mapping would overwrite
    for a in layers:
        a.k_cache[0, 0].fill_(7.0)
        a.v_cache[0, 0].fill_(-7.0)
    twins = _layers(dev, 2, num_blocks, seed=3)
    for a in twins:
        a.k_cache[0, 0].fill_(7.0)
        a.v_cache[0, 0].fill_(-7.0)
    graphs = DecodeGraphs(layers, max_bs=48, max_num_blocks=max_blocks).capture()
    assert sorted(graphs.graphs) == [1, 2, 4, 8, 16, 32, 48]
    # graphs 1, 4, 16, 32 and 48 replayed, 48 and 1 twice, with eager work between
    for i, bs in enumerate([1, 3, 16, 17, 40, 48, 2, 1]):
        batch = _batch(dev, bs, max_blocks - 1, num_blocks, seed=100 + i)
        got = torch.stack(graphs.run(*batch))
        torch.cuda.synchronize()
        assert got.shape == (2, bs, NH * D)
        q, _, _, slots, ctx, bt = batch
        for li, a in enumerate(layers):
            # the new token is in its slot, and the replay equals the oracle on that cache
            assert np.array_equal(bits16(a.k_cache.view(-1, NKV * D)[slots.long()]), bits16(batch[1]))
            assert np.array_equal(bits16(a.v_cache.view(-1, NKV * D)[slots.long()]), bits16(batch[2]))
            assert_attn_close(f32(got[li]).reshape(bs, NH, D), _oracle(a, q, ctx, bt),
                              what=f"graph bs={bs} layer {li} vs oracle")
        # rows of the graph beyond bs ran with zero context: zeros
        size = min(x for x in graphs.graph_bs if x >= bs)
        for out in graphs.layer_outputs[size]:
            assert not bool(out[bs:size].any())
        ref = _eager(twins, *batch)
        torch.cuda.synchronize()
        # the padded launch plans its split-K for the graph size, so sums may round differently
        assert_attn_close(f32(got), f32(ref), what=f"graph bs={bs}")
        for a, t in zip(layers, twins):  # same cache contents: the live rows' store
            assert torch.equal(a.k_cache, t.k_cache) and torch.equal(a.v_cache, t.v_cache)
        for a in layers:
            assert bool((a.k_cache[0, 0] == 7.0).all()) and bool((a.v_cache[0, 0] == -7.0).all())


def test_batches_beyond_the_graphs_run_eagerly(dev):
    from nanovllm_amd.engine.decode_graphs import DecodeGraphs
    layers = _layers(dev, 1, 40, seed=5)
    twins = _layers(dev, 1, 40, seed=5)
    graphs = DecodeGraphs(layers, max_bs=8, max_num_blocks=2).capture()
    batch = _batch(dev, 12, 2, 40, seed=9)
    got = torch.stack(graphs.run(*batch))
    ref = _eager(twins, *batch)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_fp8_cache_replay_matches_oracle(dev):
    """Captured decode over an fp8 e4m3fn cache (allocated and bound by
    engine.kv_cache.allocate_kv_cache, scales from amax): every replayed layer
    matches the oracle on the dequantised cache, and the new token's stored codes
    equal the oracle's quantisation -- at batches served by the spread mode, where
    the store runs (and quantises) inside the decode launch, and by the balanced
    mode (48 sequences x 8 kv heads)."""
    import nanovllm_amd as nva
    from nanovllm_amd.engine.decode_graphs import DecodeGraphs
    from nanovllm_amd.engine.kv_cache import allocate_kv_cache
    from oracle import attention_oracle as O
    from _helpers import FP8_MAX_ABS, bits8
    max_blocks, num_blocks = 4, 200
    layers = torch.nn.ModuleList([nva.Attention(NH, D, D ** -0.5, NKV) for _ in range(2)])
    kv = allocate_kv_cache(layers.modules(), 2, BS_PAGE, NKV, D, kv_dtype=torch.float8_e4m3fn,
                           num_blocks=num_blocks, device=dev)
    g = torch.Generator(device=dev).manual_seed(21)
    # Scales first, amax 8 (far beyond any N(0,1) draw of the new tokens, so x / scale stays
    # under 448 and no NaN code is stored), then random cache codes within range.
    for i in range(2):
        kv.set_scales_from_amax(i, torch.full((NKV,), 8.0, device=dev), torch.full((NKV,), 8.0, device=dev))
        for c, sc in ((kv.kv_cache[0, i], kv.kv_scale[0, i]), (kv.kv_cache[1, i], kv.kv_scale[1, i])):
            src = torch.randn(num_blocks, BS_PAGE, NKV, D, generator=g, device=dev).clamp_(-7.5, 7.5)
            c.copy_((src / sc[None, None, :, None]).to(torch.float8_e4m3fn))
    graphs = DecodeGraphs(list(layers), max_bs=48, max_num_blocks=max_blocks).capture()
    for i, bs in enumerate([1, 3, 16, 40, 2]):
        q, k, v, slots, ctx, bt = _batch(dev, bs, max_blocks - 1, num_blocks, seed=300 + i)
        got = torch.stack(graphs.run(q, k, v, slots, ctx, bt))
        torch.cuda.synchronize()
        for li, a in enumerate(layers):
            ek = O.quantize_e4m3fn(f32(k).reshape(bs, NKV, D), f32(a.k_scale))
            ev = O.quantize_e4m3fn(f32(v).reshape(bs, NKV, D), f32(a.v_scale))
            assert np.array_equal(bits8(a.k_cache).reshape(-1, NKV, D)[slots.long().cpu().numpy()], ek)
            assert np.array_equal(bits8(a.v_cache).reshape(-1, NKV, D)[slots.long().cpu().numpy()], ev)
            case = SimpleNamespace(batch=bs, context_lens=ctx, block_tables=bt, q=q.view(-1, NH, D),
                                   num_heads=NH, num_kv_heads=NKV, head_dim=D, block_size=BS_PAGE,
                                   scale=D ** -0.5, k_cache=a.k_cache, v_cache=a.v_cache, k_scale=a.k_scale,
                                   v_scale=a.v_scale)
            assert_attn_close(f32(got[li]).reshape(bs, NH, D), decode_reference(case), max_abs=FP8_MAX_ABS,
                              mean_abs=FP8_MAX_ABS, what=f"fp8 graph bs={bs} layer {li} vs oracle")
