"""Seeded synthetic inputs of the attention hot path (the five benchmark configs).

Each case reproduces what the reference's producers hand to Attention.forward:
  * decode: context_lens include the newest token, whose K/V are stored at
    slot block_table[-1]*bs + last_block_tokens - 1 before attending
    (model_runner.py:218-249);
  * prefill: cu_seqlens over the uncached tokens, slot_mapping over the
    uncached pages, block_tables only when a prefix is cached (model_runner.py:161-216);
  * block tables are int32, padded with -1 (model_runner.py:151-159); pages are
    whole block_size runs of slots (sequence.py:53-67);
  * v is a strided view of a fused qkv buffer, as qwen3.py:89 produces it.
Draw order: lengths -> block permutation -> q -> k -> v (all bf16 N(0, 1)).
Integer draws use a CPU generator; bulk tensors are drawn on `bulk_device`
(a CPU generator gives machine-independent values, a CUDA one is faster).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

BF16 = torch.bfloat16
FP8 = torch.float8_e4m3fn


@dataclass
class DecodeCase:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    scale: float
    q: torch.Tensor             # (B, nh, d) bf16
    k_new: torch.Tensor         # (B, nkv, d) bf16, newest token's key
    v_new: torch.Tensor         # (B, nkv, d) bf16 (strided view)
    k_cache: torch.Tensor       # (num_blocks, bs, nkv, d) bf16 or fp8
    v_cache: torch.Tensor
    context_lens: torch.Tensor  # (B,) int32
    block_tables: torch.Tensor  # (B, max_blocks) int32, -1 padded
    slot_mapping: torch.Tensor  # (B,) int32
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None
    seed: int = 0
    lengths: list = field(default_factory=list)

    @property
    def batch(self) -> int:
        return self.context_lens.shape[0]

    def kv_bytes(self) -> int:
        """Algorithmic HBM bytes of one decode: every visible K and V element once,
        plus q, o, block-table entries, lengths (and scales)."""
        elem = self.k_cache.element_size()
        L = sum(self.lengths)
        d, nkv, nh, B, bs = self.head_dim, self.num_kv_heads, self.num_heads, self.batch, self.block_size
        pages = sum(math.ceil(x / bs) for x in self.lengths)
        extra = 2 * nkv * 4 if self.k_scale is not None else 0
        return L * nkv * d * 2 * elem + B * nh * d * 2 * 2 + 4 * B + 4 * pages + extra

    def to(self, device) -> "DecodeCase":
        def mv(t):
            return None if t is None else t.to(device)
        return DecodeCase(self.name, self.num_heads, self.num_kv_heads, self.head_dim, self.block_size,
                          self.scale, mv(self.q), mv(self.k_new), mv(self.v_new), mv(self.k_cache),
                          mv(self.v_cache), mv(self.context_lens), mv(self.block_tables),
                          mv(self.slot_mapping), mv(self.k_scale), mv(self.v_scale), self.seed,
                          list(self.lengths))


@dataclass
class PrefillCase:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    scale: float
    q: torch.Tensor               # (Tq, nh, d) bf16
    k: torch.Tensor               # (Tq, nkv, d) bf16
    v: torch.Tensor               # (Tq, nkv, d) bf16, strided view of a qkv buffer
    cu_seqlens_q: torch.Tensor    # (S+1,) int32
    cu_seqlens_k: torch.Tensor
    max_seqlen_q: int
    max_seqlen_k: int
    slot_mapping: torch.Tensor    # (Tq,) int32
    k_cache: torch.Tensor         # (num_blocks, bs, nkv, d) bf16
    v_cache: torch.Tensor
    block_tables: torch.Tensor | None  # set only when a prefix is cached
    seed: int = 0
    lens_q: list = field(default_factory=list)
    lens_k: list = field(default_factory=list)
    # the pages the scheduler allocated to each sequence (model_runner.py:151-159),
    # -1 padded, kept on the host whether or not a prefix is cached, and the
    # cached tokens of each sequence: the inputs of the slot formula
    page_table: torch.Tensor | None = None
    prefix_lens: list = field(default_factory=list)

    def flops(self) -> int:
        pairs = sum(lq * (lk - lq) + lq * (lq + 1) // 2 for lq, lk in zip(self.lens_q, self.lens_k))
        return 4 * self.head_dim * self.num_heads * pairs

    def store_bytes(self) -> int:
        T = sum(self.lens_q)
        D = self.num_kv_heads * self.head_dim
        return 2 * T * D * 2 * 2 + 4 * T

    def to(self, device) -> "PrefillCase":
        def mv(t):
            return None if t is None else t.to(device)
        qkv_w = self.v.stride(0)
        # keep v a strided view on the new device
        T, nkv, d = self.v.shape
        buf = torch.empty((T, qkv_w), dtype=BF16, device=device)
        buf[:, qkv_w - nkv * d:] = self.v.reshape(T, nkv * d).to(device)
        v = buf[:, qkv_w - nkv * d:].view(T, nkv, d)
        return PrefillCase(self.name, self.num_heads, self.num_kv_heads, self.head_dim, self.block_size,
                           self.scale, mv(self.q), mv(self.k), v, mv(self.cu_seqlens_q),
                           mv(self.cu_seqlens_k), self.max_seqlen_q, self.max_seqlen_k,
                           mv(self.slot_mapping), mv(self.k_cache), mv(self.v_cache),
                           mv(self.block_tables), self.seed, list(self.lens_q), list(self.lens_k),
                           self.page_table, list(self.prefix_lens))


def _randn_bf16(shape, gen, device):
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(BF16)


def _bulk_gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed * 7919 + 17)


def _qkv_views(T, nh, nkv, d, gen, device):
    """q, k contiguous (as qk-norm + RoPE leave them) and v a strided view."""
    q = _randn_bf16((T, nh, d), gen, device)
    k = _randn_bf16((T, nkv, d), gen, device)
    qkv = torch.empty((T, (nh + 2 * nkv) * d), dtype=BF16, device=device)
    qkv[:, (nh + nkv) * d:] = _randn_bf16((T, nkv * d), gen, device)
    v = qkv[:, (nh + nkv) * d:].view(T, nkv, d)
    return q, k, v


def _fill_cache(num_blocks, bs, nkv, d, gen, device, chunk_pages=512):
    cache = torch.empty((num_blocks, bs, nkv, d), dtype=BF16, device=device)
    for p0 in range(0, num_blocks, chunk_pages):
        p1 = min(num_blocks, p0 + chunk_pages)
        cache[p0:p1] = _randn_bf16((p1 - p0, bs, nkv, d), gen, device)
    return cache


def quantize_cache_fp8(cache_bf16: torch.Tensor, chunk_pages=256, extra: torch.Tensor | None = None):
    """Per-kv-head scale = amax / 448 and e4m3fn codes of x / scale.
    `extra` (T, nkv, d): more source values that count towards the amax."""
    nkv = cache_bf16.shape[2]
    amax = torch.zeros(nkv, dtype=torch.float32, device=cache_bf16.device)
    if extra is not None:
        amax = torch.maximum(amax, extra.float().abs().amax(dim=(0, 2)).to(amax.device))
    for p0 in range(0, cache_bf16.shape[0], chunk_pages):
        blk = cache_bf16[p0:p0 + chunk_pages].float().abs()
        amax = torch.maximum(amax, blk.amax(dim=(0, 1, 3)))
    scale = (amax / 448.0).contiguous()
    out = torch.empty(cache_bf16.shape, dtype=FP8, device=cache_bf16.device)
    for p0 in range(0, cache_bf16.shape[0], chunk_pages):
        blk = cache_bf16[p0:p0 + chunk_pages].float() / scale.view(1, 1, nkv, 1)
        out[p0:p0 + chunk_pages] = blk.to(FP8)
    return out, scale


def make_decode_case(batch, num_heads, num_kv_heads, ctx_lo, ctx_hi, num_blocks, *, block_size=256,
                     head_dim=128, fp8=False, seed=0, bulk_device="cpu", name="decode",
                     table_width=None, lengths=None) -> DecodeCase:
    gen = torch.Generator().manual_seed(seed)
    if lengths is None:
        lengths = torch.randint(ctx_lo, ctx_hi + 1, (batch,), generator=gen).tolist()
    pages = [math.ceil(x / block_size) for x in lengths]
    if sum(pages) > num_blocks:
        raise ValueError(f"{sum(pages)} pages needed, pool has {num_blocks}")
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    width = table_width or max(max(pages), 1)
    bt = torch.full((batch, width), -1, dtype=torch.int32)
    slots = torch.empty(batch, dtype=torch.int32)
    at = 0
    for b in range(batch):
        row = perm[at:at + pages[b]]
        at += pages[b]
        bt[b, :pages[b]] = torch.tensor(row, dtype=torch.int32)
        L = lengths[b]
        if L > 0:
            last = L - (pages[b] - 1) * block_size
            slots[b] = row[pages[b] - 1] * block_size + last - 1
        else:
            slots[b] = -1
    q = k_new = v_new = k_cache = v_cache = k_scale = v_scale = None
    if bulk_device is None:  # the index tensors only (lengths, block tables, slots)
        return DecodeCase(name, num_heads, num_kv_heads, head_dim, block_size, head_dim ** -0.5, q, k_new, v_new,
                          k_cache, v_cache, torch.tensor(lengths, dtype=torch.int32), bt, slots, None, None, seed,
                          list(lengths))
    g = _bulk_gen(seed, bulk_device)
    q, k_new, v_new = _qkv_views(batch, num_heads, num_kv_heads, head_dim, g, bulk_device)
    k_cache = _fill_cache(num_blocks, block_size, num_kv_heads, head_dim, g, bulk_device)
    v_cache = _fill_cache(num_blocks, block_size, num_kv_heads, head_dim, g, bulk_device)
    if fp8:
        # the scale's amax covers every source value that enters the cache,
        # including the newest token, so x / scale never exceeds 448
        k_cache, k_scale = quantize_cache_fp8(k_cache, extra=k_new)
        v_cache, v_scale = quantize_cache_fp8(v_cache, extra=v_new)
    dev = bulk_device
    return DecodeCase(name, num_heads, num_kv_heads, head_dim, block_size, head_dim ** -0.5, q, k_new, v_new,
                      k_cache, v_cache, torch.tensor(lengths, dtype=torch.int32, device=dev), bt.to(dev),
                      slots.to(dev), k_scale, v_scale, seed, list(lengths))


def make_prefill_case(lens_q, num_heads, num_kv_heads, num_blocks, *, prefix_len=0, block_size=256,
                      head_dim=128, seed=0, bulk_device="cpu", name="prefill", shared_prefix=True,
                      gen=None) -> PrefillCase:
    """lens_q: fresh tokens per sequence.  prefix_len (an int, or one value per
    sequence): that many cached tokens, whole pages (block_manager.py:74),
    precede the sequence's fresh ones and are already in the cache.  With
    shared_prefix the cached pages are common to all sequences (a sequence with
    a shorter prefix uses the first of them).  Whenever any sequence has a
    cached prefix the whole batch gets block tables and takes the paged path,
    as model_runner.py:189-190 sets them; a sequence without one then reads all
    its keys back from the pages the store just wrote."""
    S = len(lens_q)
    pre_lens = list(prefix_len) if isinstance(prefix_len, (list, tuple)) else [prefix_len] * S
    if len(pre_lens) != S:
        raise ValueError("one prefix length per sequence")
    if any(x % block_size for x in pre_lens):
        raise ValueError("a cached prefix is whole pages (block_manager.py:74)")
    gen = gen or torch.Generator().manual_seed(seed)
    lens_k = [pre + x for pre, x in zip(pre_lens, lens_q)]
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    at = 0
    max_pre_pages = max(pre_lens, default=0) // block_size
    shared = perm[:max_pre_pages] if shared_prefix else None
    if shared_prefix:
        at = max_pre_pages
    rows = []
    for s in range(S):
        pre_pages = pre_lens[s] // block_size
        if shared_prefix:
            pre = list(shared[:pre_pages])
        else:
            pre = perm[at:at + pre_pages]
            at += pre_pages
        n_new = math.ceil(lens_k[s] / block_size) - pre_pages
        rows.append(pre + perm[at:at + n_new])
        at += n_new
    if at > num_blocks:
        raise ValueError(f"{at} pages needed, pool has {num_blocks}")
    width = max((len(r) for r in rows), default=1)
    bt = torch.full((S, max(width, 1)), -1, dtype=torch.int32)
    slots = []
    for s, r in enumerate(rows):
        bt[s, :len(r)] = torch.tensor(r, dtype=torch.int32)
        nb = len(r)
        for i in range(pre_lens[s] // block_size, nb):
            start = r[i] * block_size
            end = start + (block_size if i != nb - 1 else lens_k[s] - (nb - 1) * block_size)
            slots.extend(range(start, end))
    T = sum(lens_q)
    q = k = v = k_cache = v_cache = None
    if bulk_device is not None:  # None: the index tensors only
        g = _bulk_gen(seed, bulk_device)
        q, k, v = _qkv_views(T, num_heads, num_kv_heads, head_dim, g, bulk_device)
        k_cache = _fill_cache(num_blocks, block_size, num_kv_heads, head_dim, g, bulk_device)
        v_cache = _fill_cache(num_blocks, block_size, num_kv_heads, head_dim, g, bulk_device)
    cu_q = torch.zeros(S + 1, dtype=torch.int32)
    cu_k = torch.zeros(S + 1, dtype=torch.int32)
    cu_q[1:] = torch.cumsum(torch.tensor(lens_q), 0)
    cu_k[1:] = torch.cumsum(torch.tensor(lens_k), 0)
    dev = bulk_device or "cpu"
    return PrefillCase(name, num_heads, num_kv_heads, head_dim, block_size, head_dim ** -0.5, q, k, v,
                       cu_q.to(dev), cu_k.to(dev), max(lens_q) if S else 0, max(lens_k) if S else 0,
                       torch.tensor(slots, dtype=torch.int32, device=dev), k_cache, v_cache,
                       bt.to(dev) if any(pre_lens) else None, seed, list(lens_q), list(lens_k),
                       bt.clone(), list(pre_lens))


# ----------------------------------------------------------------------------
# The five benchmark configurations (heads nh/nkv, head_dim 128, block_size 256)
# ----------------------------------------------------------------------------

SEEDS = {1: 1001, 2: 1002, 3: 1003, 4: 1004, 5: 1005}


def config1(bulk_device="cpu", seed=SEEDS[1]) -> DecodeCase:
    """Qwen3-0.6B decode: B=4, ctx U[128,512], 16/8 heads, pool of 16 pages."""
    return make_decode_case(4, 16, 8, 128, 512, 16, seed=seed, bulk_device=bulk_device, name="cfg1")


def config2(bulk_device="cpu", seed=SEEDS[2]) -> PrefillCase:
    """Qwen3-0.6B varlen prefill + store: 8 seqs U[100,1024], 16/8 heads, 64-page pool."""
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(100, 1025, (8,), generator=gen).tolist()
    return make_prefill_case(lens, 16, 8, 64, seed=seed, bulk_device=bulk_device, name="cfg2", gen=gen)


def config3(bulk_device="cpu", seed=SEEDS[3]) -> DecodeCase:
    """Bench-shaped decode step: B=256, ctx U[100,2048], 16/8 heads, 2048-page pool."""
    return make_decode_case(256, 16, 8, 100, 2048, 2048, seed=seed, bulk_device=bulk_device, name="cfg3")


def config4(bulk_device="cpu", seed=SEEDS[4]) -> PrefillCase:
    """Qwen3-8B prefix-cached prefill: 16 seqs, shared 1024-token prefix (4 pages),
    suffix U[256,768], 32/8 heads."""
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(256, 769, (16,), generator=gen).tolist()
    return make_prefill_case(lens, 32, 8, 64, prefix_len=1024, seed=seed, bulk_device=bulk_device,
                             name="cfg4", gen=gen)


def config5(bulk_device="cpu", seed=SEEDS[5]) -> DecodeCase:
    """Qwen3-32B long-context fp8 decode: B=64, ctx U[16k,32k], 64/8 heads, e4m3 cache
    with per-kv-head scales amax/448, 8192-page pool."""
    return make_decode_case(64, 64, 8, 16384, 32768, 8192, fp8=True, seed=seed, bulk_device=bulk_device,
                            name="cfg5")


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


# One GPU's share of a tensor-parallel group of 8 (qwen3.py:33-43 divides the query
# and kv heads by the TP size, model_runner.py:117 sizes each rank's cache for its
# nkv / tp heads): the same draws of lengths, pages and values as configs 4 and 5,
# over one kv head.

def config4_tp8(bulk_device="cpu", seed=SEEDS[4]) -> PrefillCase:
    """Config 4 at Qwen3-8B's TP8 share: heads 4/1 (GQA 4), prefix 1024, suffix U[256,768]."""
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(256, 769, (16,), generator=gen).tolist()
    return make_prefill_case(lens, 4, 1, 64, prefix_len=1024, seed=seed, bulk_device=bulk_device,
                             name="cfg4-tp8", gen=gen)


def config5_tp8(bulk_device="cpu", seed=SEEDS[5]) -> DecodeCase:
    """Config 5 at Qwen3-32B's TP8 share: heads 8/1 (GQA 8), fp8 cache, B=64, ctx U[16k,32k]."""
    return make_decode_case(64, 8, 1, 16384, 32768, 8192, fp8=True, seed=seed, bulk_device=bulk_device,
                            name="cfg5-tp8")


@dataclass
class ProducerCase:
    """Inputs of the fused qk-RMSNorm + rotary step (qwen3.py:91-105): q and k are
    views into one fused qkv buffer, as the qkv projection leaves them."""
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    qkv: torch.Tensor              # (T, (nh + 2 nkv) d) bf16
    q: torch.Tensor                # (T, nh, d) view
    k: torch.Tensor                # (T, nkv, d) view
    positions: torch.Tensor        # (T,) int64
    cos_sin_cache: torch.Tensor    # (max_position, d) fp32
    q_norm_weight: torch.Tensor | None
    k_norm_weight: torch.Tensor | None
    eps: float = 1e-6

    @property
    def num_tokens(self) -> int:
        return self.q.shape[0]

    def bytes(self) -> int:
        """Algorithmic HBM bytes of one fused call: q and k rows read and written once
        (bf16), one cos/sin row (fp32) and one int64 position per token, the weights."""
        rows = self.num_tokens * (self.num_heads + self.num_kv_heads)
        w = 0 if self.q_norm_weight is None else 2 * self.head_dim * 2
        return rows * self.head_dim * 2 * 2 + self.num_tokens * (self.head_dim * 4 + 8) + w


def make_producer_case(num_tokens, num_heads, num_kv_heads, *, head_dim=128, max_position=40960,
                       rope_theta=1_000_000.0, norm=True, positions=None, seed=0, device="cpu",
                       name="producer") -> ProducerCase:
    """Qwen3 defaults (rope_theta 1e6, max_position 40960, eps 1e-6, qwen3.py:156-160);
    norm=False gives the Qwen2 rotary-only step.  Positions default to uniform random."""
    from .layers.qk_norm_rope import rope_cos_sin_cache
    gen = torch.Generator(device=device).manual_seed(seed * 7919 + 29)
    T, nh, nkv, d = num_tokens, num_heads, num_kv_heads, head_dim
    qkv = _randn_bf16((T, (nh + 2 * nkv) * d), gen, device)
    q = qkv[:, : nh * d].view(T, nh, d)
    k = qkv[:, nh * d:(nh + nkv) * d].view(T, nkv, d)
    if positions is None:
        positions = torch.randint(0, max_position, (T,), generator=gen, device=device, dtype=torch.int64)
    else:
        positions = torch.as_tensor(positions, dtype=torch.int64, device=device)
    cache = rope_cos_sin_cache(d, max_position, rope_theta, device=device)
    wq = wk = None
    if norm:
        wq = (1.0 + 0.2 * torch.randn(d, generator=gen, device=device)).to(BF16)
        wk = (1.0 + 0.2 * torch.randn(d, generator=gen, device=device)).to(BF16)
    return ProducerCase(name, nh, nkv, d, qkv, q, k, positions, cache, wq, wk)


def producer_config4(device="cpu", seed=SEEDS[4]) -> ProducerCase:
    """The producer step for config 4's suffix tokens: Qwen3-8B heads 32/8, positions
    1024 + i within each sequence (the cached prefix comes first)."""
    gen = torch.Generator().manual_seed(seed)
    lens = torch.randint(256, 769, (16,), generator=gen).tolist()
    pos = [1024 + i for L in lens for i in range(L)]
    return make_producer_case(len(pos), 32, 8, positions=pos, seed=seed, device=device, name="producer-cfg4")
