"""Attention hot path on MI355X, mirroring nanovllm/layers/attention.py:1-79.

The module keeps the reference's interface verbatim:
  * store_kvcache(key, value, k_cache, v_cache, slot_mapping)   attention.py:32-39
  * Attention(num_heads, head_dim, scale, num_kv_heads) with rebindable
    k_cache / v_cache attributes and forward(q, k, v) -> o     attention.py:42-79
and replaces the two flash-attn entry points it calls with functions of the same
names and argument meaning, backed by the gfx950 HIP library through its C ABI:
  * flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k,
    cu_seqlens_k, softmax_scale, causal=True, block_table=None)   attention.py:70-73
  * flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens, block_table,
    softmax_scale, causal=True)                                   attention.py:75-77

Extension (not in the reference): an fp8 e4m3fn KV cache.  A module whose
k_cache/v_cache are torch.float8_e4m3fn tensors must also carry k_scale/v_scale
(float32, one per kv head; engine/kv_cache.allocate_kv_cache owns and binds
them); store_kvcache then quantises x / scale, decode dequantises on the fly and a
prefix-cached prefill gathers the pages into dequantised packed rows first.  A
prefill without a cached prefix reads the fresh bf16 k/v, as in the reference.

Every launch goes to torch's current stream, nothing synchronises and the only
allocations are torch tensors (output, workspaces, fp8 gather rows), so decode can be
captured in a CUDA/HIP graph as model_runner.py:296-336 does.  There is no
fallback path: if the library is missing, calls raise.
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _capi
from ..utils.context import get_context

_BF16 = torch.bfloat16
_FP8 = torch.float8_e4m3fn


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


# One prefill workspace per (device, stream) -- the work queue, and the
# control words and partials of the key halves -- zeroed once: every completed
# nva_prefill call leaves its control words consistent for the next.  Calls on
# one stream run one after another, so they can share it; different streams
# get their own.
_PREFILL_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def prefill_workspace_errors() -> dict[tuple[int, int], int]:
    """Error bits each prefill workspace has collected since the last check, read
    and cleared (nva_prefill_workspace_errors; waits for each workspace's stream).
    Non-zero bits (NVA_PREFILL_ERR_SPLIT_WAIT) mean some prefill wrote NaN rows for
    an item whose key-half merge gave up waiting.  {(device, stream): bits}."""
    import ctypes
    lib = _capi.load()
    out = {}
    for (dev, stream), ws in _PREFILL_WORKSPACES.items():
        bits = ctypes.c_uint32(0)
        with torch.cuda.device(dev):
            _capi.check(lib.nva_prefill_workspace_errors(ws.data_ptr(), ws.numel(), ctypes.byref(bits), stream))
        out[(dev, stream)] = int(bits.value)
    return out


def _prefill_workspace(device: torch.device, stream: int) -> torch.Tensor | None:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _PREFILL_WORKSPACES.get(key)
    if ws is None:
        # A zero fill recorded into a graph under capture would not run until the
        # graph replays, so such a call takes the static item order instead.
        if torch.cuda.is_current_stream_capturing():
            return None
        ws = torch.zeros(int(_capi.load().nva_prefill_workspace_bytes()), dtype=torch.uint8, device=device)
        _PREFILL_WORKSPACES[key] = ws
    return ws


# Packed bf16 rows of the fp8 prefix-cached prefill's gather, one buffer per
# (device, stream), grown to the largest call seen and reused: calls on one stream
# run one after another, and the prefill that reads the rows is ordered before the
# next call's gather overwrites them.
_GATHER_BUFFERS: dict[tuple[int, int], torch.Tensor] = {}


def _gather_rows(device: torch.device, stream: int, rows: int, row_elems: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(k, v) views of rows x row_elems bf16 each.  Under graph capture a fresh
    tensor is taken from the graph's pool instead (its lifetime is the graph's)."""
    n = rows * row_elems
    if torch.cuda.is_current_stream_capturing():
        buf = torch.empty(2 * n, dtype=_BF16, device=device)
    else:
        key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
        buf = _GATHER_BUFFERS.get(key)
        if buf is None or buf.numel() < 2 * n:
            _GATHER_BUFFERS.pop(key, None)
            buf = torch.empty(2 * n, dtype=_BF16, device=device)
            _GATHER_BUFFERS[key] = buf
    return buf[:n], buf[n:2 * n]


def _check_device(device: torch.device, **tensors) -> None:
    """Every tensor handed to a kernel must live on the GPU the call runs on: a
    host pointer (or another GPU's) passed through the C ABI would be read by
    the kernel as a device address."""
    if device.type != "cuda":
        raise RuntimeError(f"the attention kernels run on a CUDA (HIP) device, got tensors on {device}")
    for name, t in tensors.items():
        if t is not None and t.device != device:
            raise RuntimeError(f"{name} must be on {device} (got {t.device})")


def _cache_dtype_code(cache: torch.Tensor) -> int:
    if cache.dtype == _BF16:
        return _capi.NVA_DTYPE_BF16
    if cache.dtype in (_FP8, torch.uint8):
        return _capi.NVA_DTYPE_FP8_E4M3
    raise RuntimeError(f"unsupported KV cache dtype {cache.dtype} (bfloat16 or float8_e4m3fn)")


def _check_scales(code: int, k_scale, v_scale, num_kv_heads: int, device) -> None:
    if code != _capi.NVA_DTYPE_FP8_E4M3:
        return
    for name, s in (("k_scale", k_scale), ("v_scale", v_scale)):
        if s is None:
            raise RuntimeError(f"fp8 KV cache needs {name}")
        if s.dtype != torch.float32 or s.numel() != num_kv_heads or not s.is_contiguous() or s.device != device:
            raise RuntimeError(f"{name} must be a contiguous float32 tensor of {num_kv_heads} values on {device}")


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor, k_scale: torch.Tensor | None = None,
                  v_scale: torch.Tensor | None = None):
    """Scatter key/value rows into the paged caches (attention.py:32-39).

    Same preconditions as the reference, raised as AssertionError like its asserts
    (attention.py:35-38).  Slots outside [0, num_blocks*block_size) are skipped.
    """
    N, num_heads, head_dim, code = _check_store(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale)
    num_slots = k_cache.numel() // (num_heads * head_dim)
    lib = _capi.load()
    _capi.check(lib.nva_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), num_slots,
        slot_mapping.data_ptr(), N, num_heads, head_dim, code,
        _ptr(k_scale), _ptr(v_scale), _stream(key)))


def _check_store(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale):
    """store_kvcache's preconditions (attention.py:35-38 asserts, then dtype,
    layout and device checks); returns (N, num_kv_heads, head_dim, cache dtype code)."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    if key.dtype != _BF16 or value.dtype != _BF16:
        raise RuntimeError("key/value must be bfloat16")
    if slot_mapping.dtype != torch.int32 or (N and not slot_mapping.is_contiguous()):
        raise RuntimeError("slot_mapping must be a contiguous int32 tensor")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or k_cache.shape != v_cache.shape:
        raise RuntimeError("k_cache/v_cache must be contiguous and of the same shape")
    code = _cache_dtype_code(k_cache)
    if _cache_dtype_code(v_cache) != code:
        raise RuntimeError("k_cache and v_cache must share a dtype")
    _check_scales(code, k_scale, v_scale, num_heads, k_cache.device)
    _check_device(key.device, value=value, k_cache=k_cache, v_cache=v_cache, slot_mapping=slot_mapping,
                  k_scale=k_scale, v_scale=v_scale)
    return N, num_heads, head_dim, code


def flash_attn_varlen_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, max_seqlen_q: int,
                           cu_seqlens_q: torch.Tensor, max_seqlen_k: int, cu_seqlens_k: torch.Tensor,
                           softmax_scale: float | None = None, causal: bool = True,
                           block_table: torch.Tensor | None = None, k_scale: torch.Tensor | None = None,
                           v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Varlen causal attention over packed K/V, or over the paged caches when
    block_table is given (attention.py:67-73).  q (total_q, nh, d) -> (total_q, nh, d).

    Extension: paged caches in fp8 e4m3fn (with k_scale/v_scale, one float32 per
    kv head) are first gathered into packed bf16 rows, dequantised
    (nva_gather_kv), and the packed prefill runs on those.  That needs
    cu_seqlens_k[s+1] - cu_seqlens_k[s] <= max_seqlen_k, as flash-attn does."""
    if not causal:
        raise RuntimeError("only causal=True is implemented (the only mode attention.py uses)")
    total_q, nh, d = q.shape
    if q.dtype != _BF16:
        raise RuntimeError("q must be bfloat16")
    if block_table is None and (k.dtype != _BF16 or v.dtype != _BF16):
        raise RuntimeError("packed k/v must be bfloat16 (an fp8 cache is read through block_table)")
    if softmax_scale is None:
        softmax_scale = d ** -0.5
    if q.stride(-1) != 1 or q.stride(1) != d:
        raise RuntimeError("q must have head stride head_dim and unit element stride")
    for t in (cu_seqlens_q, cu_seqlens_k):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise RuntimeError("cu_seqlens must be contiguous int32 tensors")
    num_seqs = cu_seqlens_q.numel() - 1
    if cu_seqlens_k.numel() != num_seqs + 1:
        raise RuntimeError("cu_seqlens_q and cu_seqlens_k must have the same length")
    out = torch.empty((total_q, nh, d), dtype=_BF16, device=q.device)
    if block_table is not None:
        if k.dim() != 4 or not k.is_contiguous() or not v.is_contiguous() or k.shape != v.shape:
            raise RuntimeError("paged k/v must be contiguous (num_blocks, block_size, nkv, d) caches")
        num_blocks, block_size, nkv, kd = k.shape
        if kd != d:
            raise RuntimeError(f"cache head_dim {kd} differs from q's {d}")
        if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(-1) != 1:
            raise RuntimeError("block_table must be a 2-d int32 tensor with unit column stride")
        if block_table.shape[0] != num_seqs:
            raise RuntimeError(f"block_table has {block_table.shape[0]} rows for {num_seqs} sequences")
        code = _cache_dtype_code(k)
        if _cache_dtype_code(v) != code:
            raise RuntimeError("k_cache and v_cache must share a dtype")
        _check_scales(code, k_scale, v_scale, nkv, k.device)
        k_row = v_row = nkv * d
        bt_ptr, bt_stride, max_blocks = block_table.data_ptr(), block_table.stride(0), block_table.shape[1]
        if code == _capi.NVA_DTYPE_FP8_E4M3:
            # dequantise each sequence's pages into packed rows, then the packed prefill
            _check_device(q.device, k=k, v=v, cu_seqlens_k=cu_seqlens_k, block_table=block_table,
                          k_scale=k_scale, v_scale=v_scale)
            # rows of every sequence's keys at cu_seqlens_k[s]: at most num_seqs *
            # max_seqlen_k (the total itself lives on the device)
            rows = num_seqs * int(max_seqlen_k)
            kf, vf = _gather_rows(q.device, _stream(q), rows, nkv * d)
            kp, vp = kf.view(rows, nkv, d), vf.view(rows, nkv, d)
            _capi.check(_capi.load().nva_gather_kv(
                k.data_ptr(), v.data_ptr(), code, _ptr(k_scale), _ptr(v_scale), num_blocks,
                bt_ptr, bt_stride, max_blocks, block_size, cu_seqlens_k.data_ptr(), num_seqs, int(max_seqlen_k),
                nkv, d, kp.data_ptr(), vp.data_ptr(), rows, nkv * d, _stream(q)))
            k, v, block_table = kp, vp, None
            bt_ptr, bt_stride, max_blocks, block_size, num_blocks = None, 0, 0, 0, 0
    else:
        if k.dim() != 3 or k.shape != v.shape or k.shape[2] != d:
            raise RuntimeError("packed k/v must both be (total_k, nkv, d) with q's head_dim")
        if k.stride(-1) != 1 or v.stride(-1) != 1 or k.stride(1) != d or v.stride(1) != d:
            raise RuntimeError("packed k/v must have head stride d and unit element stride")
        nkv = k.shape[1]
        k_row, v_row = k.stride(0), v.stride(0)
        bt_ptr, bt_stride, max_blocks, block_size, num_blocks = None, 0, 0, 0, 0
    _check_device(q.device, k=k, v=v, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k, block_table=block_table)
    lib = _capi.load()
    stream = _stream(q)
    ws = _prefill_workspace(q.device, stream)
    _capi.check(lib.nva_prefill(
        q.data_ptr(), q.stride(0), k.data_ptr(), k_row, v.data_ptr(), v_row,
        bt_ptr, bt_stride, max_blocks, block_size, num_blocks,
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), num_seqs, int(max_seqlen_q), int(max_seqlen_k),
        nh, nkv, d, float(softmax_scale), out.data_ptr(), out.stride(0),
        _ptr(ws), 0 if ws is None else ws.numel(), stream))
    return out


def flash_attn_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            cache_seqlens: torch.Tensor, block_table: torch.Tensor,
                            softmax_scale: float | None = None, causal: bool = True, num_splits: int = 0,
                            k_scale: torch.Tensor | None = None,
                            v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Paged decode, one query per sequence (attention.py:75-77).
    q (B, 1, nh, d) -> (B, 1, nh, d).  `causal` is accepted for signature parity
    and is a no-op for a single query; num_splits has flash-attn's meaning
    (0 = heuristic, n > 0 = about n splits per sequence), and -1 selects the
    balanced split-K whatever the sizes."""
    del causal
    a = _decode_args(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, num_splits, k_scale, v_scale)
    _capi.check(_capi.load().nva_decode(*a["decode"], _stream(q)))
    return a["out"]


def store_and_decode(q: torch.Tensor, key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                     v_cache: torch.Tensor, slot_mapping: torch.Tensor, cache_seqlens: torch.Tensor,
                     block_table: torch.Tensor, softmax_scale: float | None = None, num_splits: int = 0,
                     k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None) -> torch.Tensor:
    """The decode branch of Attention.forward as one call: store_kvcache of the new
    rows (attention.py:32-39), then flash_attn_with_kvcache (attention.py:75-77).
    The spread mode (small batches) and the balanced mode over a bf16 cache run the
    store inside the decode launch (nva_store_decode).  The result equals the two
    calls when slot_mapping[b] is the slot of key cache_seqlens[b]-1 for every
    sequence with keys, as prepare_decode (model_runner.py:218-229) produces it, and
    no sequence reads the slot of a row whose cache_seqlens is 0 (graph padding: use
    slot -1).  Such rows are stored after every read of the call, so a sequence that
    does read that slot sees its previous contents (the two calls would show it the
    padded row)."""
    N = key.shape[0]
    if N != q.shape[0]:
        raise RuntimeError("one new key/value row per sequence")
    _check_store(key, value, k_cache, v_cache, slot_mapping, k_scale, v_scale)
    a = _decode_args(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, num_splits, k_scale, v_scale)
    _check_device(q.device, key=key, value=value, slot_mapping=slot_mapping)
    _capi.check(_capi.load().nva_store_decode(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0), slot_mapping.data_ptr(),
        *a["decode"], _stream(q)))
    return a["out"]


def _decode_args(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, num_splits, k_scale, v_scale):
    """Checks of the decode call and its nva_decode arguments (all but the stream),
    with the output tensor and the workspace allocated."""
    if q.dim() != 4 or q.shape[1] != 1:
        raise RuntimeError("q must be (batch, 1, num_heads, head_dim)")
    B, _, nh, d = q.shape
    if q.dtype != _BF16:
        raise RuntimeError("q must be bfloat16")
    if q.stride(-1) != 1 or q.stride(2) != d:
        raise RuntimeError("q must have head stride head_dim and unit element stride")
    if softmax_scale is None:
        softmax_scale = d ** -0.5
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise RuntimeError("caches must be contiguous (num_blocks, block_size, nkv, d) of one shape")
    num_blocks, block_size, nkv, kd = k_cache.shape
    if kd != d:
        raise RuntimeError(f"cache head_dim {kd} differs from q's {d}")
    code = _cache_dtype_code(k_cache)
    if _cache_dtype_code(v_cache) != code:
        raise RuntimeError("k_cache and v_cache must share a dtype")
    _check_scales(code, k_scale, v_scale, nkv, k_cache.device)
    if cache_seqlens.dtype != torch.int32 or not cache_seqlens.is_contiguous() or cache_seqlens.numel() != B:
        raise RuntimeError("cache_seqlens must be a contiguous int32 tensor of batch size")
    if block_table.dtype != torch.int32 or block_table.stride(-1) != 1 or block_table.shape[0] != B:
        raise RuntimeError("block_table must be int32 (batch, max_blocks) with unit column stride")
    max_blocks = block_table.shape[1]
    _check_device(q.device, k_cache=k_cache, v_cache=v_cache, cache_seqlens=cache_seqlens, block_table=block_table,
                  k_scale=k_scale, v_scale=v_scale)
    out = torch.empty((B, 1, nh, d), dtype=_BF16, device=q.device)
    lib = _capi.load()
    ws_bytes = lib.nva_decode_workspace_bytes(B, nh, nkv, d, max_blocks, block_size, code, int(num_splits))
    ws = torch.empty(max(ws_bytes, 0), dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None
    args = (q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), code,
            _ptr(k_scale), _ptr(v_scale), num_blocks,
            cache_seqlens.data_ptr(), block_table.data_ptr(), block_table.stride(0), max_blocks, block_size,
            B, nh, nkv, d, float(softmax_scale), int(num_splits),
            out.data_ptr(), out.stride(0), _ptr(ws), ws_bytes)
    return {"decode": args, "out": out, "workspace": ws}


class Attention(nn.Module):
    """Drop-in for nanovllm.layers.attention.Attention (attention.py:42-79).

    fuse_decode_store (not in the reference, default False): when True the decode
    branch runs the store and the attention as one call (store_and_decode), one
    launch fewer per layer.  It equals the reference's store-then-decode only if no
    padded row (context length 0) carries a slot that a live sequence reads; the
    reference's run_model zero-fills slot_mapping (model_runner.py:271-273), so its
    padded rows write slot 0 of block 0, which a live sequence may own.  Set it only
    under a runner that pads slot_mapping with -1 (DecodeGraphs with pad_slot=-1)."""

    def __init__(self, num_heads, head_dim, scale, num_kv_heads):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        # fp8 cache extension: per-kv-head float32 scales, None for a bf16 cache
        self.k_scale = self.v_scale = None
        self.fuse_decode_store = False

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        q = q.view(-1, self.num_heads, self.head_dim)
        k = k.view(-1, self.num_kv_heads, self.head_dim)
        v = v.view(-1, self.num_kv_heads, self.head_dim)
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        bound = k_cache.numel() and v_cache.numel()
        if not context.is_prefill and bound and self.fuse_decode_store:  # store and attention as one call
            o = store_and_decode(q.unsqueeze(1), k, v, k_cache, v_cache, context.slot_mapping,
                                 context.context_lens, context.block_tables, softmax_scale=self.scale,
                                 k_scale=self.k_scale, v_scale=self.v_scale)
            return o.view(-1, self.num_heads * self.head_dim)
        if bound:
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping, self.k_scale, self.v_scale)
        if context.is_prefill:
            if context.block_tables is not None:  # prefix cache
                k, v = k_cache, v_cache
            o = flash_attn_varlen_func(q, k, v,
                                       max_seqlen_q=context.max_seqlen_q, cu_seqlens_q=context.cu_seqlens_q,
                                       max_seqlen_k=context.max_seqlen_k, cu_seqlens_k=context.cu_seqlens_k,
                                       softmax_scale=self.scale, causal=True, block_table=context.block_tables,
                                       k_scale=self.k_scale, v_scale=self.v_scale)
        else:  # decode
            o = flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
                                        cache_seqlens=context.context_lens, block_table=context.block_tables,
                                        softmax_scale=self.scale, causal=True,
                                        k_scale=self.k_scale, v_scale=self.v_scale)
        return o.view(-1, self.num_heads * self.head_dim)
