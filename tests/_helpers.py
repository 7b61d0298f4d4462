"""Shared helpers of the test suite: tensor <-> numpy conversion and the
tolerance checks the parity tests apply."""
from __future__ import annotations

import numpy as np
import torch

from oracle import attention_oracle as O

# bf16 attention outputs vs the fp32 oracle (the parity bar: max-abs 2e-2, mean-abs 2e-3)
BF16_MAX_ABS = 2e-2
BF16_MEAN_ABS = 2e-3
# fp8-KV outputs vs the fp32 oracle on the dequantised cache
FP8_MAX_ABS = 5e-2


def bits16(t: torch.Tensor) -> np.ndarray:
    """Raw 16-bit patterns of a bf16 tensor as uint16 numpy."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def bits8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.uint8).numpy()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_attn_close(got: np.ndarray, ref: np.ndarray, max_abs=BF16_MAX_ABS, mean_abs=BF16_MEAN_ABS, what=""):
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    mx, mn = float(err.max()) if err.size else 0.0, float(err.mean()) if err.size else 0.0
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})"
    return mx, mn


def decode_reference(case, seqs=None, dtype=np.float32):
    """Oracle decode outputs (len(seqs), nh, d) for the given sequence indices,
    gathering only those sequences' pages from the (device) cache."""
    B = case.batch
    seqs = list(range(B)) if seqs is None else list(seqs)
    lens = case.context_lens.cpu().tolist()
    bt = case.block_tables.cpu().numpy()
    q = f32(case.q)
    out = np.zeros((len(seqs), case.num_heads, case.head_dim), dtype=dtype)
    bs = case.block_size
    for r, b in enumerate(seqs):
        L = lens[b]
        if L <= 0:
            continue
        pages = torch.from_numpy(bt[b, : (L + bs - 1) // bs].astype(np.int64)).to(case.k_cache.device)
        kp = case.k_cache.index_select(0, pages)
        vp = case.v_cache.index_select(0, pages)
        if case.k_scale is not None:
            k = O.e4m3fn_to_f32(bits8(kp)) * f32(case.k_scale)[None, None, :, None]
            v = O.e4m3fn_to_f32(bits8(vp)) * f32(case.v_scale)[None, None, :, None]
        else:
            k, v = f32(kp), f32(vp)
        k = k.reshape(-1, case.num_kv_heads, case.head_dim)[:L]
        v = v.reshape(-1, case.num_kv_heads, case.head_dim)[:L]
        out[r] = O.attention(q[b][None], k, v, case.scale, True, dtype)[0]
    return out


def prefill_reference(case, seqs=None, dtype=np.float32):
    """Oracle prefill outputs for the given sequences, concatenated in order.
    Uses the case's current caches (after the store) for the paged case."""
    cu_q = case.cu_seqlens_q.cpu().numpy()
    cu_k = case.cu_seqlens_k.cpu().numpy()
    S = len(cu_q) - 1
    seqs = list(range(S)) if seqs is None else list(seqs)
    q = f32(case.q)
    outs = []
    bs = case.block_size
    for s in seqs:
        q0, q1 = cu_q[s], cu_q[s + 1]
        Lk = cu_k[s + 1] - cu_k[s]
        if case.block_tables is None:
            k = f32(case.k[cu_k[s]:cu_k[s + 1]])
            v = f32(case.v[cu_k[s]:cu_k[s + 1]])
        else:
            bt = case.block_tables[s].cpu().numpy()
            pages = torch.from_numpy(bt[: (Lk + bs - 1) // bs].astype(np.int64)).to(case.k_cache.device)
            k = f32(case.k_cache.index_select(0, pages)).reshape(-1, case.num_kv_heads, case.head_dim)[:Lk]
            v = f32(case.v_cache.index_select(0, pages)).reshape(-1, case.num_kv_heads, case.head_dim)[:Lk]
        outs.append(O.attention(q[q0:q1], k, v, case.scale, True, dtype))
    return np.concatenate(outs) if outs else np.zeros((0, case.num_heads, case.head_dim), dtype)


def rows_of(case, seqs):
    cu_q = case.cu_seqlens_q.cpu().tolist()
    idx = []
    for s in seqs:
        idx.extend(range(cu_q[s], cu_q[s + 1]))
    return idx
