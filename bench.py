"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline (`value`): paged decode attention throughput in algorithmic HBM GB/s on
the bench-shaped decode step (config 3: store_kvcache of the new token + paged
GQA decode, Qwen3-0.6B heads 16/8, head_dim 128, block_size 256, batch 256,
context U[100, 2048], 2048-page pool).  A step is one such pass with inputs
resident in HBM; consecutive steps alternate between independent cache pools so
the 256 MB Infinity Cache cannot serve them.  Alongside: prefill TFLOP/s
(config 4 prefix-cached, Qwen3-8B heads 32/8; config 2 varlen), fp8-KV decode
GB/s (config 5), the config 1 decode step (cache-resident, reported without a
roofline claim), the fused qk-RMSNorm + rotary producer step (GB/s), the captured
decode steps, the roofline of the dominant kernel (HIP events on the launch
stream), rocprofv3 HBM traffic from profiles/, and the reference's PyTorch CPU
path (store + gather + SDPA) timed on the host cores on a bounded sample of
every configuration (`cpu_baseline` is config 3's, `cpu_baselines` all five).

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--warm-seconds 1] [--no-cpu]
                       [--only decode|prefill|fp8|producer|graphs|tp8]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "nano-vllm_amd"))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "paged decode attn HBM GB/s (% of peak) + prefill TFLOP/s, 1×MI355X"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def profiled_traffic(key: str, summary: str = "decode_hbm_traffic.md"):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE (scaled by a
    plain copy of known size), as recorded in the committed profile summary."""
    path = ROOT / "profiles" / summary
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(f"traffic_bytes_per_launch {key}"):
            return int(float(line.split(":")[1].split()[0]))
    return None


def _warm(fn, warmup, seconds):
    """`warmup` untimed calls, then more until `seconds` of wall time have passed:
    the clocks of an idle MI355X take a while to reach their sustained level, and
    the timed steps should see that level, not the ramp."""
    import torch
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    i = warmup
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def _pools(case, n):
    """n independent (k_cache, v_cache) pools with identical contents."""
    pools = [(case.k_cache, case.v_cache)]
    for _ in range(n - 1):
        pools.append((case.k_cache.clone(), case.v_cache.clone()))
    return pools


def bench_decode(case, steps, warmup, n_pools=2, with_store=True, warm_s=1.0, fused=False):
    """A decode step over `steps` rotations of the cache pools.  fused: the step is
    one store_and_decode call (Attention.forward's decode branch); otherwise
    store_kvcache then flash_attn_with_kvcache, timed apart."""
    import torch
    import nanovllm_amd as nva
    pools = _pools(case, n_pools)
    q = case.q.unsqueeze(1)
    if fused:
        return _bench_decode_fused(case, pools, q, steps, warmup, warm_s)

    def store(i):
        kc, vc = pools[i % n_pools]
        nva.store_kvcache(case.k_new, case.v_new, kc, vc, case.slot_mapping, case.k_scale, case.v_scale)

    def attend(i):
        kc, vc = pools[i % n_pools]
        return nva.flash_attn_with_kvcache(q, kc, vc, case.context_lens, case.block_tables, case.scale,
                                           k_scale=case.k_scale, v_scale=case.v_scale)

    def one(i):
        if with_store:
            store(i)
        attend(i)

    _warm(one, warmup, warm_s)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        if with_store:
            store(i)
        ev[i][1].record()
        attend(i)
        ev[i][2].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = ev[0][0].elapsed_time(ev[-1][2]) / steps
    attn_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / steps
    store_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    B = case.batch
    D = case.num_kv_heads * case.head_dim
    store_bytes = 2 * B * D * 2 + 2 * B * D * case.k_cache.element_size() + 4 * B if with_store else 0
    attn_bytes = case.kv_bytes()
    return dict(step_ms=step_ms, attn_ms=attn_ms, store_ms=store_ms, wall_ms=wall * 1e3 / steps,
                attn_bytes=attn_bytes, store_bytes=store_bytes,
                step_gbs=(attn_bytes + store_bytes) / (step_ms * 1e-3) / 1e9,
                attn_gbs=attn_bytes / (attn_ms * 1e-3) / 1e9)


def _bench_decode_fused(case, pools, q, steps, warmup, warm_s):
    import torch
    import nanovllm_amd as nva
    n_pools = len(pools)

    def one(i):
        kc, vc = pools[i % n_pools]
        return nva.store_and_decode(q, case.k_new, case.v_new, kc, vc, case.slot_mapping, case.context_lens,
                                    case.block_tables, case.scale, k_scale=case.k_scale, v_scale=case.v_scale)

    _warm(one, warmup, warm_s)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        one(i)
        ev[i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = ev[0][0].elapsed_time(ev[-1][1]) / steps
    call_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    B = case.batch
    D = case.num_kv_heads * case.head_dim
    store_bytes = 2 * B * D * 2 + 2 * B * D * case.k_cache.element_size() + 4 * B
    attn_bytes = case.kv_bytes()
    return dict(step_ms=step_ms, call_ms=call_ms, wall_ms=wall * 1e3 / steps, attn_bytes=attn_bytes,
                store_bytes=store_bytes, step_gbs=(attn_bytes + store_bytes) / (step_ms * 1e-3) / 1e9,
                call_gbs=(attn_bytes + store_bytes) / (call_ms * 1e-3) / 1e9)


def bench_prefill(case, steps, warmup, warm_s=1.0):
    import torch
    import nanovllm_amd as nva
    nva.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
    if case.block_tables is None:
        k, v = case.k, case.v
    else:
        k, v = case.k_cache, case.v_cache

    def run():
        return nva.flash_attn_varlen_func(case.q, k, v, case.max_seqlen_q, case.cu_seqlens_q, case.max_seqlen_k,
                                          case.cu_seqlens_k, case.scale, True, case.block_tables)

    _warm(lambda i: run(), warmup, warm_s)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        run()
        ev[i][1].record()
    torch.cuda.synchronize()
    ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    flops = case.flops()
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12)


def bench_store(case, steps, warmup, warm_s=1.0, n_pools=8):
    """store_kvcache of a prefill case's fresh tokens (the bandwidth case of the
    scatter).  Calls rotate over n_pools copies of the sources (k, and v as the
    same strided view of a wider buffer) and of the destination caches, so the
    rotation's footprint exceeds the 256 MB Infinity Cache.  Per-call time is
    the replay time of a graph of n_pools calls divided by n_pools."""
    import torch
    import nanovllm_amd as nva
    pools = []
    for _ in range(n_pools):
        k = case.k.clone()
        v = torch.empty_strided(case.v.shape, case.v.stride(), dtype=case.v.dtype, device=case.v.device)
        v.copy_(case.v)
        pools.append((k, v, torch.empty_like(case.k_cache), torch.empty_like(case.v_cache)))

    def run(i):
        k, v, kc, vc = pools[i % n_pools]
        nva.store_kvcache(k, v, kc, vc, case.slot_mapping)

    # One call per pool captured in a HIP graph and replayed: a store of this
    # size takes less time on the GPU than the Python wrapper takes to issue
    # it, so timing eager calls would time the host.
    _warm(run, warmup, warm_s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_pools):
            run(i)
    reps = max(4, steps // n_pools)
    for _ in range(3):
        g.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * n_pools)
    del g
    nbytes = case.store_bytes()
    del pools
    return dict(ms=ms, tokens=sum(case.lens_q), bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9,
                frac=nbytes / (ms * 1e-3) / 8.0e12)


def bench_copy(dev, steps, warm_s=0.25, nbytes=1 << 30):
    """A plain device-to-device copy of 1 GiB (torch's copy kernel): the practical
    read + write ceiling the store's scatter is compared with.  The 2 GiB footprint
    exceeds the 256 MB Infinity Cache."""
    import torch
    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    _warm(lambda i: dst.copy_(src), 3, warm_s)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del src, dst
    return dict(ms=ms, bytes=2 * nbytes, gbs=2 * nbytes / (ms * 1e-3) / 1e9)


def bench_prefill_fp8(case, steps, warmup, warm_s=1.0):
    """A prefix-cached prefill over an fp8 e4m3fn cache (scales amax / 448 per kv head,
    the cached prefix and the suffix quantised by store_kvcache): one
    flash_attn_varlen_func call = nva_gather_kv of every sequence's pages into packed
    dequantised bf16 rows + the packed prefill over them.  The gather is also timed
    alone, on the same rows."""
    import torch
    import nanovllm_amd as nva
    from nanovllm_amd import _capi, workloads as W
    kc8, ks = W.quantize_cache_fp8(case.k_cache, extra=case.k)
    vc8, vs = W.quantize_cache_fp8(case.v_cache, extra=case.v)
    nva.store_kvcache(case.k, case.v, kc8, vc8, case.slot_mapping, ks, vs)
    bt = case.block_tables

    def run(i=0):
        return nva.flash_attn_varlen_func(case.q, kc8, vc8, case.max_seqlen_q, case.cu_seqlens_q, case.max_seqlen_k,
                                          case.cu_seqlens_k, case.scale, True, bt, k_scale=ks, v_scale=vs)

    _warm(run, warmup, warm_s)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        run()
        ev[i][1].record()
    torch.cuda.synchronize()
    ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    S = len(case.lens_q)
    nkv, d = case.num_kv_heads, case.head_dim
    rows = S * case.max_seqlen_k
    kp = torch.empty(rows, nkv, d, dtype=torch.bfloat16, device=case.q.device)
    vp = torch.empty_like(kp)
    lib = _capi.load()
    stream = torch.cuda.current_stream().cuda_stream

    def gather(i=0):
        _capi.check(lib.nva_gather_kv(kc8.data_ptr(), vc8.data_ptr(), _capi.NVA_DTYPE_FP8_E4M3, ks.data_ptr(),
                                      vs.data_ptr(), kc8.shape[0], bt.data_ptr(), bt.stride(0), bt.shape[1],
                                      case.block_size, case.cu_seqlens_k.data_ptr(), S, case.max_seqlen_k, nkv, d,
                                      kp.data_ptr(), vp.data_ptr(), rows, nkv * d, stream))

    _warm(gather, warmup, warm_s / 4)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        gather()
    e1.record()
    torch.cuda.synchronize()
    g_ms = e0.elapsed_time(e1) / steps
    keys = sum(case.lens_k)
    g_bytes = 2 * keys * nkv * d * (1 + 2) + 4 * sum(math.ceil(x / case.block_size) for x in case.lens_k)
    flops = case.flops()
    del kc8, vc8, kp, vp
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12, gather_ms=g_ms, gather_bytes=g_bytes,
                gather_gbs=g_bytes / (g_ms * 1e-3) / 1e9)


def bench_producer(case, steps, warmup, warm_s=1.0):
    """The fused qk-RMSNorm + rotary step (nva_qk_norm_rope) over config 4's tokens."""
    import torch
    from nanovllm_amd.layers.qk_norm_rope import qk_norm_rope

    def run(i=0):
        return qk_norm_rope(case.positions, case.q, case.k, case.cos_sin_cache, case.num_heads,
                            case.num_kv_heads, case.head_dim, case.q_norm_weight, case.k_norm_weight, case.eps)

    _warm(run, warmup, warm_s)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        run()
        ev[i][1].record()
    torch.cuda.synchronize()
    ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    nbytes = case.bytes()
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9)


def bench_graph_decode(dev, steps, warmup, warm_s=1.0, layers=28, ctx=1024, batch_sizes=(1, 16, 64, 256)):
    """Captured decode steps (nanovllm_amd.engine.decode_graphs, the capture_cudagraph /
    run_model mirror) of `layers` Qwen3-0.6B attention layers (heads 16/8, head_dim 128)
    at a fixed context: one run() = buffer refresh + one graph replay of store + decode
    for every layer.  Caches are zero-filled (the timing does not depend on values)."""
    import torch
    import nanovllm_amd as nva
    from nanovllm_amd.engine.decode_graphs import DecodeGraphs
    nh, nkv, d, bsz = 16, 8, 128, 256
    max_bs = max(batch_sizes)
    pages_per_seq = ctx // bsz + 1
    num_blocks = max_bs * pages_per_seq
    attn = []
    for _ in range(layers):
        a = nva.Attention(nh, d, d ** -0.5, nkv)
        a.k_cache = torch.zeros(num_blocks, bsz, nkv, d, dtype=torch.bfloat16, device=dev)
        a.v_cache = torch.zeros_like(a.k_cache)
        attn.append(a)
    graphs = DecodeGraphs(attn, max_bs=max_bs, max_num_blocks=pages_per_seq).capture()
    res = {}
    for bs in batch_sizes:
        q = torch.randn(bs, nh * d, device=dev).bfloat16()
        k = torch.randn(bs, nkv * d, device=dev).bfloat16()
        v = torch.randn(bs, nkv * d, device=dev).bfloat16()
        bt = torch.arange(bs * pages_per_seq, dtype=torch.int32, device=dev).view(bs, pages_per_seq)
        ctx_t = torch.full((bs,), ctx, dtype=torch.int32, device=dev)
        slots = (bt[:, (ctx - 1) // bsz] * bsz + (ctx - 1) % bsz).contiguous()
        _warm(lambda i: graphs.run(q, k, v, slots, ctx_t, bt), warmup, warm_s / len(batch_sizes))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            graphs.run(q, k, v, slots, ctx_t, bt)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        kv = bs * ctx * nkv * d * 2 * 2 * layers
        res[bs] = dict(step_us=round(us, 1), layer_us=round(us / layers, 2), kv_gbs=round(kv / (us * 1e-6) / 1e9, 1))
    del graphs, attn
    return res


def _cpu_time(fn, budget_s):
    """Median wall time of fn() on the host, repeated until about half the budget
    is spent (at least 3 runs); returns (seconds, runs)."""
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s / 2 and len(times) < 500):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def _decode_bytes(case, n):
    """Algorithmic bytes of a decode step (store of the new token + attention) over
    the first n sequences of a decode case."""
    L = sum(case.lengths[:n])
    D = case.num_kv_heads * case.head_dim
    elem = case.k_cache.element_size()
    b = L * D * 2 * elem + n * case.num_heads * case.head_dim * 2 * 2 + 4 * n
    b += 4 * sum(math.ceil(x / case.block_size) for x in case.lengths[:n])
    return b + 2 * n * D * 2 + 2 * n * D * elem


def cpu_baseline_decode(case, name, budget_s):
    """Reference-semantics PyTorch CPU decode step (store + gather + SDPA; fp8 pages
    dequantised per sequence) on the first n sequences of a host copy of `case`, n
    chosen from a probe so the timed work fits the budget."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle import cpu_baseline as CB
    B = case.batch
    kw = dict(k_scale=case.k_scale, v_scale=case.v_scale)
    fp8 = case.k_scale is not None
    probe = min(B, 2 if fp8 else 8)
    t0 = time.perf_counter()
    CB.decode(case.q[:probe], case.k_cache, case.v_cache, case.context_lens[:probe], case.block_tables[:probe],
              case.scale, **kw)
    per_seq = (time.perf_counter() - t0) / probe
    n = max(probe, min(B, int(budget_s / 3 / max(per_seq, 1e-6))))

    def step():
        k_new, v_new = case.k_new[:n], case.v_new[:n]
        if fp8:  # e4m3fn(x / scale), torch's cast (bit-identical to the kernel's)
            CB.store_kvcache_fp8(k_new, v_new, case.k_cache, case.v_cache, case.slot_mapping[:n],
                                 case.k_scale, case.v_scale)
        else:
            CB.store_kvcache(k_new, v_new, case.k_cache, case.v_cache, case.slot_mapping[:n])
        CB.decode(case.q[:n], case.k_cache, case.v_cache, case.context_lens[:n], case.block_tables[:n],
                  case.scale, **kw)

    t, reps = _cpu_time(step, budget_s)
    what = "fp8 e4m3fn decode step (store + gather + dequantise + SDPA)" if fp8 else \
        "decode step (index_copy_ store + block-table gather + SDPA, bf16)"
    return dict(value=round(_decode_bytes(case, n) / t / 1e9, 3), unit="GB/s", cores=torch.get_num_threads(),
                kind="port", sample=f"{name} {what} over the first {n} of {B} sequences, median of {reps}, "
                                    f"{t:.3f} s each")


def cpu_baseline_prefill(case, name, budget_s):
    """Reference-semantics PyTorch CPU prefill (store + per-sequence SDPA with a
    bottom-right causal mask; prefix pages gathered through the block table) over
    the first n sequences of a host copy of `case`."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle import cpu_baseline as CB
    S = len(case.lens_q)
    paged = case.block_tables is not None

    def run(n):
        T = sum(case.lens_q[:n])
        CB.store_kvcache(case.k[:T], case.v[:T], case.k_cache, case.v_cache, case.slot_mapping[:T])
        k, v = (case.k_cache, case.v_cache) if paged else (case.k, case.v)
        CB.prefill(case.q[:T], k, v, case.cu_seqlens_q[:n + 1], case.cu_seqlens_k[:n + 1], case.scale,
                   case.block_tables[:n] if paged else None)

    t0 = time.perf_counter()
    run(1)
    per_seq = time.perf_counter() - t0
    n = max(1, min(S, int(budget_s / 3 / max(per_seq, 1e-6))))
    t, reps = _cpu_time(lambda: run(n), budget_s)
    flops = sum(4 * case.head_dim * case.num_heads * (lq * (lk - lq) + lq * (lq + 1) // 2)
                for lq, lk in zip(case.lens_q[:n], case.lens_k[:n]))
    return dict(value=round(flops / t / 1e12, 5), unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
                sample=f"{name} prefill (index_copy_ store + SDPA per sequence, bottom-right causal mask"
                       f"{', prefix pages gathered' if paged else ''}, bf16) over the first {n} of {S} sequences, "
                       f"median of {reps}, {t:.3f} s each")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warm-seconds", type=float, default=1.0,
                    help="after the warmup steps, keep running each workload untimed for this long")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["decode", "prefill", "fp8", "producer", "graphs", "tp8"], default=None)
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 1 GiB device copy (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the attention path has no cross-GPU step here "
              f"(--gpus {args.gpus} requested); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    import nanovllm_amd as nva
    from nanovllm_amd import workloads as W
    nva._capi.load()
    dev = torch.device("cuda:0")
    steps, warmup = args.steps, args.warmup
    out = {}
    host = {}  # host copies of the cases for the CPU baselines
    if args.copy_probe:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] copy probe: 3 x 1 GiB device-to-device copies")
        del src, dst

    if args.only in (None, "decode"):
        log("[bench] config 3: decode step (store + paged decode), B=256")
        c3 = W.config3(dev)
        d3 = bench_decode(c3, steps, warmup, warm_s=args.warm_seconds)
        log(f"[bench] cfg3 step {d3['step_ms']*1e3:.1f} us, attention {d3['attn_ms']*1e3:.1f} us "
            f"= {d3['attn_gbs']:.0f} GB/s, store {d3['store_ms']*1e3:.1f} us")
        out["cfg3"] = d3
        f3 = bench_decode(c3, steps, warmup, warm_s=args.warm_seconds, fused=True)
        log(f"[bench] cfg3 fused step {f3['step_ms']*1e3:.1f} us (store_and_decode: the store inside the "
            f"decode launch), call {f3['call_ms']*1e3:.1f} us")
        out["cfg3_fused"] = f3
        # the CPU baselines run last, so the GPU workloads follow each other
        # without the GPU idling (and its clocks dropping) for the CPU samples
        if not args.no_cpu:
            host["cfg3"] = c3.to("cpu")
        del c3
        log("[bench] config 1: decode step, B=4 (cache-resident: no roofline claim)")
        c1 = W.config1(dev)
        out["cfg1"] = bench_decode(c1, steps, warmup, n_pools=1, warm_s=args.warm_seconds, fused=True)
        log(f"[bench] cfg1 step {out['cfg1']['step_ms']*1e3:.1f} us (store_and_decode, store fused)")
        if not args.no_cpu:
            host["cfg1"] = c1.to("cpu")
        del c1
        torch.cuda.empty_cache()
    if args.only in (None, "prefill"):
        log("[bench] config 4: prefix-cached prefill (Qwen3-8B heads)")
        c4 = W.config4(dev)
        out["cfg4"] = bench_prefill(c4, max(10, steps // 2), warmup, args.warm_seconds)
        log(f"[bench] cfg4 {out['cfg4']['ms']*1e3:.1f} us = {out['cfg4']['tflops']:.0f} TFLOP/s")
        out["store4"] = bench_store(c4, steps, warmup, args.warm_seconds)
        log(f"[bench] cfg4 store_kvcache {out['store4']['tokens']} tokens {out['store4']['ms']*1e3:.1f} us "
            f"= {out['store4']['gbs']:.0f} GB/s ({out['store4']['frac']:.3f} of 8 TB/s)")
        if not args.no_cpu:
            host["cfg4"] = W.config4("cpu")
        del c4
        log("[bench] config 4 over an fp8 cache: gather + packed prefill")
        c4 = W.config4(dev)
        out["cfg4_fp8"] = bench_prefill_fp8(c4, max(10, steps // 2), warmup, args.warm_seconds)
        log(f"[bench] cfg4 fp8 cache {out['cfg4_fp8']['ms']*1e3:.1f} us = {out['cfg4_fp8']['tflops']:.0f} TFLOP/s "
            f"(gather alone {out['cfg4_fp8']['gather_ms']*1e3:.1f} us = {out['cfg4_fp8']['gather_gbs']:.0f} GB/s)")
        del c4
        torch.cuda.empty_cache()
        out["copy"] = bench_copy(dev, 20, args.warm_seconds / 4)
        log(f"[bench] plain 1 GiB device copy {out['copy']['ms']*1e3:.1f} us = {out['copy']['gbs']:.0f} GB/s "
            f"(read + write)")
        log("[bench] config 2: varlen prefill")
        c2 = W.config2(dev)
        out["cfg2"] = bench_prefill(c2, max(10, steps // 2), warmup, args.warm_seconds)
        log(f"[bench] cfg2 {out['cfg2']['ms']*1e3:.1f} us = {out['cfg2']['tflops']:.0f} TFLOP/s")
        out["store2"] = bench_store(c2, steps, warmup, args.warm_seconds)
        log(f"[bench] cfg2 store_kvcache {out['store2']['tokens']} tokens {out['store2']['ms']*1e3:.1f} us "
            f"= {out['store2']['gbs']:.0f} GB/s ({out['store2']['frac']:.3f} of 8 TB/s)")
        if not args.no_cpu:
            host["cfg2"] = W.config2("cpu")
        del c2
        # one fresh 2048-token prompt at Qwen3-8B heads (packed, direct grid): the
        # time-to-first-token case of a single request, no roofline claim
        c1p = W.make_prefill_case([2048], 32, 8, 12, seed=2048, bulk_device=dev, name="single_prompt")
        out["single_prompt"] = bench_prefill(c1p, max(10, steps // 2), warmup, args.warm_seconds)
        log(f"[bench] one 2048-token prompt (heads 32/8): {out['single_prompt']['ms']*1e3:.1f} us "
            f"= {out['single_prompt']['tflops']:.0f} TFLOP/s")
        del c1p
        torch.cuda.empty_cache()
    if args.only in (None, "producer"):
        log("[bench] producer: fused qk-RMSNorm + rotary over config 4's 8813 tokens (heads 32/8)")
        cp = W.producer_config4(dev)
        out["producer"] = bench_producer(cp, max(10, steps // 2), warmup, args.warm_seconds)
        log(f"[bench] producer {out['producer']['ms']*1e3:.1f} us = {out['producer']['gbs']:.0f} GB/s")
        del cp
        torch.cuda.empty_cache()
    if args.only in (None, "graphs"):
        log("[bench] graph decode: captured store + decode steps of 28 layers (heads 16/8), context 1024")
        out["graphs"] = bench_graph_decode(dev, max(10, steps // 5), warmup, args.warm_seconds)
        for bs, r in out["graphs"].items():
            log(f"[bench] graph decode bs={bs}: {r['step_us']} us/step ({r['layer_us']} us/layer, "
                f"{r['kv_gbs']} GB/s of KV)")
        torch.cuda.empty_cache()
    if args.only in (None, "tp8"):
        log("[bench] TP8 shares: config 5 at heads 8/1 (fp8 decode), config 4 at heads 4/1 (prefix prefill)")
        c5s = W.config5_tp8(dev)
        out["cfg5_tp8"] = bench_decode(c5s, max(10, steps // 2), warmup, warm_s=args.warm_seconds)
        log(f"[bench] cfg5 TP8 share attention {out['cfg5_tp8']['attn_ms']*1e3:.1f} us "
            f"= {out['cfg5_tp8']['attn_gbs']:.0f} GB/s")
        del c5s
        torch.cuda.empty_cache()
        c4s = W.config4_tp8(dev)
        out["cfg4_tp8"] = bench_prefill(c4s, max(10, steps // 2), warmup, args.warm_seconds)
        log(f"[bench] cfg4 TP8 share {out['cfg4_tp8']['ms']*1e3:.1f} us = {out['cfg4_tp8']['tflops']:.0f} TFLOP/s")
        del c4s
        torch.cuda.empty_cache()
    if args.only in (None, "fp8"):
        log("[bench] config 5: fp8 KV decode, B=64, ctx U[16k,32k]")
        c5 = W.config5(dev)
        out["cfg5"] = bench_decode(c5, max(10, steps // 2), warmup, warm_s=args.warm_seconds)
        log(f"[bench] cfg5 attention {out['cfg5']['attn_ms']*1e3:.1f} us = {out['cfg5']['attn_gbs']:.0f} GB/s")
        if not args.no_cpu:
            host["cfg5"] = c5.to("cpu")
        del c5
        torch.cuda.empty_cache()

    if host:
        torch.set_num_threads(os.cpu_count() or 1)
        cpu = {}
        budgets = {"cfg3": 16.0, "cfg1": 4.0, "cfg2": 8.0, "cfg4": 12.0, "cfg5": 12.0}
        for name in ("cfg3", "cfg1", "cfg2", "cfg4", "cfg5"):
            if name not in host:
                continue
            log(f"[bench] CPU baseline ({name} sample)")
            case = host.pop(name)
            fn = cpu_baseline_prefill if name in ("cfg2", "cfg4") else cpu_baseline_decode
            cpu[name] = fn(case, name.replace("cfg", "config "), budgets[name])
            log(f"[bench] cpu {name}: {cpu[name]['value']} {cpu[name]['unit']} on {cpu[name]['cores']} threads")
            del case
        out["cpu"] = cpu

    line = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic: seeded N(0,1) bf16 q/k/v, random page tables (no checkpoint)"}
    if "cfg3" in out:
        d3 = out["cfg3"]
        line["value"] = round(d3["step_gbs"], 1)
        line["ms_per_step"] = round(d3["step_ms"], 5)
        line["config"] = {"workload": "config 3: decode step = store_kvcache(new token) + paged GQA decode",
                          "batch": 256, "context": "U[100,2048]", "num_heads": 16, "num_kv_heads": 8,
                          "head_dim": 128, "block_size": 256, "pool_pages": 2048, "cache_pools_rotated": 2}
        line["roofline"] = {"kernel": "paged decode (paged_decode_balanced_kernel + decode_merge_kernel)",
                            "bound": "hbm", "achieved": round(d3["attn_gbs"], 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(d3["attn_gbs"] / HBM_PEAK_GBS, 4),
                            "traffic": profiled_traffic("config3"),
                            "traffic_source": "profiles/decode_hbm_traffic.md",
                            "bytes_per_launch": d3["attn_bytes"], "launch_us": round(d3["attn_ms"] * 1e3, 2)}
        line["store_kvcache_us"] = round(d3["store_ms"] * 1e3, 2)
        if "cfg3_fused" in out:
            f3 = out["cfg3_fused"]
            line["fused_step"] = {"note": "the same step as one store_and_decode call (Attention.forward's decode "
                                          "branch): the store runs inside the decode launch",
                                  "step_us": round(f3["step_ms"] * 1e3, 2), "call_us": round(f3["call_ms"] * 1e3, 2),
                                  "gbs": round(f3["step_gbs"], 1)}
    if "cpu" in out:
        if "cfg3" in out["cpu"]:
            line["cpu_baseline"] = out["cpu"]["cfg3"]
        line["cpu_baselines"] = out["cpu"]
    if "cfg1" in out:
        d1 = out["cfg1"]
        line["cfg1_decode"] = {"note": "cache-resident (5 MB): reported, no roofline claim; one store_and_decode "
                                       "call per step",
                               "step_us": round(d1["step_ms"] * 1e3, 2), "call_us": round(d1["call_ms"] * 1e3, 2),
                               "gbs": round(d1["call_gbs"], 1), "bytes": d1["attn_bytes"] + d1["store_bytes"]}
    if "cfg4" in out:
        p4 = out["cfg4"]
        line["prefill"] = {"config": "config 4: prefix-cached prefill, 16 sequences, 1024 cached + U[256,768] new "
                                     "tokens, heads 32/8, head_dim 128, block_size 256",
                           "tflops": round(p4["tflops"], 1), "ms": round(p4["ms"], 5),
                           "frac": round(p4["tflops"] / BF16_PEAK_TFLOPS, 4), "gflop": round(p4["flops"] / 1e9, 2),
                           "bound": "mfma", "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s"}
    if "cfg4" in out or "cfg2" in out:
        line["prefill_configs"] = {k: {"tflops": round(out[k]["tflops"], 1), "ms": round(out[k]["ms"], 5),
                                       "gflop": round(out[k]["flops"] / 1e9, 2),
                                       "frac_bf16_peak": round(out[k]["tflops"] / BF16_PEAK_TFLOPS, 4)}
                                   for k in ("cfg4", "cfg2") if k in out}
    if "cfg4_fp8" in out:
        f = out["cfg4_fp8"]
        line["prefill_fp8_cache"] = {"workload": "config 4 over an fp8 e4m3fn cache (per-kv-head scales): "
                                                 "nva_gather_kv into packed bf16 rows + packed prefill, one call",
                                     "us": round(f["ms"] * 1e3, 2), "tflops": round(f["tflops"], 1),
                                     "frac_bf16_peak": round(f["tflops"] / BF16_PEAK_TFLOPS, 4),
                                     "gather_us": round(f["gather_ms"] * 1e3, 2), "gather_bytes": f["gather_bytes"],
                                     "gather_gbs": round(f["gather_gbs"], 1),
                                     "gather_frac": round(f["gather_gbs"] / HBM_PEAK_GBS, 4)}
    if "cfg5_tp8" in out or "cfg4_tp8" in out:
        tp = {}
        if "cfg5_tp8" in out:
            r = out["cfg5_tp8"]
            tp["cfg5"] = {"workload": "config 5 at heads 8/1 (one kv head), fp8 cache, B=64, ctx U[16k,32k]",
                          "roofline": {"bound": "hbm", "achieved": round(r["attn_gbs"], 1), "peak": HBM_PEAK_GBS,
                                       "unit": "GB/s", "frac": round(r["attn_gbs"] / HBM_PEAK_GBS, 4)},
                          "attn_us": round(r["attn_ms"] * 1e3, 2), "bytes": r["attn_bytes"]}
        if "cfg4_tp8" in out:
            r = out["cfg4_tp8"]
            tp["cfg4"] = {"workload": "config 4 at heads 4/1 (one kv head), prefix 1024 + U[256,768]",
                          "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 1), "peak": BF16_PEAK_TFLOPS,
                                       "unit": "TFLOP/s", "frac": round(r["tflops"] / BF16_PEAK_TFLOPS, 4)},
                          "us": round(r["ms"] * 1e3, 2), "gflop": round(r["flops"] / 1e9, 2)}
        line["tp8_shares"] = tp
    if "single_prompt" in out:
        sp = out["single_prompt"]
        line["prefill_single_prompt"] = {"note": "one fresh 2048-token prompt, heads 32/8, head_dim 128 (packed): "
                                                 "time to first token of one request; no roofline claim",
                                         "us": round(sp["ms"] * 1e3, 2), "tflops": round(sp["tflops"], 1),
                                         "gflop": round(sp["flops"] / 1e9, 2)}
    if "store4" in out or "store2" in out:
        line["store_kvcache_prefill"] = {
            k: {"tokens": out[s]["tokens"], "us": round(out[s]["ms"] * 1e3, 2), "bytes": out[s]["bytes"],
                "gbs": round(out[s]["gbs"], 1), "frac": round(out[s]["frac"], 4),
                "traffic": profiled_traffic(f"store_{k}", "store_hbm_traffic.md"),
                "traffic_source": "profiles/store_hbm_traffic.md"}
            for k, s in (("cfg4", "store4"), ("cfg2", "store2")) if s in out}
        if "copy" in out:
            line["store_kvcache_prefill"]["copy_gbs"] = round(out["copy"]["gbs"], 1)
            line["store_kvcache_prefill"]["copy_note"] = ("plain 1 GiB device-to-device copy (read + write bytes): "
                                                          "the practical ceiling of a scatter")
    if "cfg5" in out:
        d5 = out["cfg5"]
        line["fp8_decode"] = {"cfg5": {"gbs": round(d5["attn_gbs"], 1), "frac": round(d5["attn_gbs"] / HBM_PEAK_GBS, 4),
                                       "attn_us": round(d5["attn_ms"] * 1e3, 2), "bytes": d5["attn_bytes"],
                                       "traffic": profiled_traffic("config5")}}
    if "graphs" in out:
        line["graph_decode"] = {"workload": "28 layers x (store + paged decode), heads 16/8, head_dim 128, "
                                            "context 1024, HIP graph per batch size",
                                "per_batch": {str(k): v for k, v in out["graphs"].items()}}
    if "producer" in out:
        dp = out["producer"]
        line["qk_norm_rope"] = {"workload": "config 4 tokens, heads 32/8, head_dim 128",
                                "gbs": round(dp["gbs"], 1), "frac": round(dp["gbs"] / HBM_PEAK_GBS, 4),
                                "us": round(dp["ms"] * 1e3, 2), "bytes": dp["bytes"]}
    if "value" not in line:
        k = next(iter(out))
        line["value"] = None
        line["config"] = {"workload": k}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
