"""CPU oracle for nano-vllm's attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or the timed CPU baseline), never as the
computation being measured or shipped.

It restates, in numpy, what the reference computes at nanovllm/layers/attention.py
(read-only reference tree):

  store_kvcache            attention.py:10-39   (cache.flat[slot*D : +D] = row)
  prefill_attention        attention.py:67-73   (flash_attn_varlen_func, causal=True,
                                                 block_table=None or the paged caches)
  decode_attention         attention.py:74-77   (flash_attn_with_kvcache, one query)
  paged_gather             model_runner.py:151-159 (int32 block tables, -1 padded) and
                           sequence.py:53-67 (key j lives in page j // block_size)
  prefill_slots / decode_slots  model_runner.py:180-188 and :226-229

flash-attn itself (Dao-AILab, unpinned at pyproject.toml:18, not installed here) is
not vendored in the reference; its published semantics are restated instead:
softmax(scale * Q K^T + M) V per sequence and query head, with GQA head h reading
kv head h // (num_heads // num_kv_heads), and M the causal mask aligned to the
bottom-right corner (query i of Lq sees keys j <= i + Lk - Lq).

Parity pinning (tests/test_oracle.py): brute-force pure-Python loops on tiny
inputs, torch.nn.functional.scaled_dot_product_attention on the same inputs,
closed forms (single key -> v0, q = 0 -> running mean of visible V rows, which pins
the mask alignment row by row), decode == last prefill row, prefix prefill == tail
of full prefill, GQA == MHA with repeated K/V, page-permutation invariance, the
e4m3fn table against its bit-level definition and torch's float8_e4m3fn cast.
Planted mistakes (top-left mask, wrong GQA index, missing scale, transposed
operand) are shown to fail those checks.
"""
from __future__ import annotations

import math

import numpy as np

# ----------------------------------------------------------------------------
# bf16 / fp8 element formats
# ----------------------------------------------------------------------------


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 stored as uint16 bit patterns -> float32 (exact)."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even, NaN kept quiet."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(x)
    out = rounded.astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def e4m3fn_table() -> np.ndarray:
    """Float value of every OCP e4m3fn code 0..255 from the bit layout.

    sign(1) exponent(4, bias 7) mantissa(3); exponent 0 is subnormal
    (m/8 * 2^-6); code 0x7f / 0xff is NaN; no infinities.
    """
    vals = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            vals[code] = np.nan
        elif e == 0:
            vals[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


def f32_to_e4m3fn(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn codes: round-to-nearest-even on the e4m3fn grid.

    The grid is extended by 480 (the NaN code 0x7f read as 1.111b * 2^8): a
    magnitude above 464, the midpoint of 448 and 480, rounds there and gives NaN
    (0x7f | sign), as do infinities and NaNs; exactly 464 ties to even, 448.
    This is what torch's float8_e4m3fn cast does.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = (np.signbit(x)).astype(np.uint8) << 7
    a = np.abs(x).astype(np.float64)
    overflow = ~(a <= 464.0)  # also catches NaN
    a = np.where(overflow, 0.0, a)
    sub = a < 2.0 ** -6
    # subnormal grid: multiples of 2^-9
    q_sub = np.rint(a * 2.0 ** 9)  # numpy rint = round half to even
    # normal grid: mantissa 3 bits at exponent floor(log2 a)
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(sub | overflow, 1.0, a)))
    frac = np.where(sub | overflow, 1.0, a) / 2.0 ** e  # in [1, 2)
    qm = np.rint((frac - 1.0) * 8.0)
    carry = qm >= 8
    e = e + carry
    qm = np.where(carry, 0, qm)
    normal_code = ((e + 7).astype(np.int64) << 3) | qm.astype(np.int64)
    codes = np.where(sub, q_sub.astype(np.int64), normal_code)
    codes = np.where(overflow, 0x7F, codes).astype(np.uint8)
    return codes | sign


def e4m3fn_to_f32(codes: np.ndarray) -> np.ndarray:
    return e4m3fn_table()[np.asarray(codes, dtype=np.uint8)].astype(np.float32)


# ----------------------------------------------------------------------------
# store_kvcache (attention.py:10-39)
# ----------------------------------------------------------------------------


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """In-place restatement of store_kvcache_kernel on numpy arrays.

    key/value: (T, nkv, d) arrays of any dtype (bf16 kept as uint16 bits);
    caches: (num_blocks, block_size, nkv, d) of the same dtype.  Each token's row
    of D = nkv*d elements is copied to flat slot `slot_mapping[i]`
    (attention.py:22-29).  Slots outside [0, num_slots) are skipped, the
    documented extension of the unguarded reference.
    """
    T = key.shape[0]
    D = key.shape[1] * key.shape[2]
    kf = k_cache.reshape(-1, D)
    vf = v_cache.reshape(-1, D)
    for i in range(T):
        s = int(slot_mapping[i])
        if 0 <= s < kf.shape[0]:
            kf[s] = key[i].reshape(D)
            vf[s] = value[i].reshape(D)


def quantize_e4m3fn(x_f32: np.ndarray, scale_per_head: np.ndarray) -> np.ndarray:
    """(..., nkv, d) float32 -> e4m3fn codes of x / scale[h] (float32 division)."""
    s = np.asarray(scale_per_head, dtype=np.float32).reshape((1,) * (x_f32.ndim - 2) + (-1, 1))
    return f32_to_e4m3fn((x_f32.astype(np.float32) / s).astype(np.float32))


# ----------------------------------------------------------------------------
# page math (model_runner.py:151-249, sequence.py:53-67)
# ----------------------------------------------------------------------------


def paged_gather(cache: np.ndarray, block_table_row: np.ndarray, length: int) -> np.ndarray:
    """First `length` slots of a sequence: key j lives at page block_table_row[j // bs],
    offset j % bs.  cache: (num_blocks, bs, ...)."""
    bs = cache.shape[1]
    npages = (length + bs - 1) // bs
    pages = np.asarray(block_table_row[:npages], dtype=np.int64)
    if np.any(pages < 0):
        raise ValueError("block table row has -1 padding inside the sequence")
    g = cache[pages].reshape((npages * bs,) + cache.shape[2:])
    return g[:length]


def prefill_slots(block_table_row, num_cached_tokens: int, seqlen: int, block_size: int) -> list[int]:
    """Slots of the uncached tokens of one sequence (model_runner.py:180-188)."""
    out = []
    nblocks = (seqlen + block_size - 1) // block_size
    for i in range(num_cached_tokens // block_size, nblocks):
        start = int(block_table_row[i]) * block_size
        end = start + (block_size if i != nblocks - 1 else seqlen - (nblocks - 1) * block_size)
        out.extend(range(start, end))
    return out


def decode_slot(block_table_row, seqlen: int, block_size: int) -> int:
    """Slot of the newest token (model_runner.py:227-229)."""
    nblocks = (seqlen + block_size - 1) // block_size
    last = seqlen - (nblocks - 1) * block_size
    return int(block_table_row[nblocks - 1]) * block_size + last - 1


# ----------------------------------------------------------------------------
# attention (attention.py:67-77, flash-attn semantics)
# ----------------------------------------------------------------------------


def attention(q, k, v, scale: float, causal: bool = True, dtype=np.float32) -> np.ndarray:
    """One sequence.  q (Lq, nh, d), k/v (Lk, nkv, d) -> (Lq, nh, d).

    Explicit gather-then-softmax: per kv head, the group of nh/nkv query heads
    is contracted against that head's keys; the causal mask is bottom-right
    aligned; rows with no visible key give zeros.
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    Lq, nh, d = q.shape
    Lk, nkv, _ = k.shape
    grp = nh // nkv
    out = np.zeros((Lq, nh, d), dtype=dtype)
    if Lq == 0:
        return out
    if causal:
        i = np.arange(Lq)[:, None]
        j = np.arange(Lk)[None, :]
        visible = j <= i + (Lk - Lq)
    else:
        visible = np.ones((Lq, Lk), dtype=bool)
    any_vis = visible.any(axis=1)
    for kh in range(nkv):
        kk = k[:, kh, :]  # (Lk, d)
        vv = v[:, kh, :]
        for hg in range(grp):
            h = kh * grp + hg
            s = (q[:, h, :] @ kk.T) * dtype(scale)  # (Lq, Lk)
            s = np.where(visible, s, -np.inf)
            m = np.max(s, axis=1, keepdims=True)
            m = np.where(np.isfinite(m), m, 0)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            o = (p @ vv) / np.where(l > 0, l, 1)
            out[:, h, :] = np.where(any_vis[:, None], o, 0)
    return out


def prefill_attention(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, block_table=None,
                      dtype=np.float32) -> np.ndarray:
    """Varlen causal prefill (attention.py:67-73).

    Without a block table k/v are packed (total_k, nkv, d) rows delimited by
    cu_seqlens_k.  With one, k/v are the paged caches (num_blocks, bs, nkv, d) and
    sequence s's Lk keys are gathered through block_table[s] (prefix-cache case).
    """
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    cu_k = np.asarray(cu_seqlens_k, dtype=np.int64)
    out = np.zeros(q.shape, dtype=dtype)
    for s in range(len(cu_q) - 1):
        q0, q1 = cu_q[s], cu_q[s + 1]
        Lk = cu_k[s + 1] - cu_k[s]
        if block_table is None:
            ks = k[cu_k[s]:cu_k[s + 1]]
            vs = v[cu_k[s]:cu_k[s + 1]]
        else:
            ks = paged_gather(k, block_table[s], Lk)
            vs = paged_gather(v, block_table[s], Lk)
        out[q0:q1] = attention(q[q0:q1], ks, vs, scale, True, dtype)
    return out


def decode_attention(q, k_cache, v_cache, cache_seqlens, block_table, scale,
                     k_scale=None, v_scale=None, dtype=np.float32) -> np.ndarray:
    """Paged decode (attention.py:74-77): q (B, nh, d), one query per sequence over
    cache_seqlens[b] keys gathered through block_table[b].  Caches are float
    arrays (bf16 already widened) or e4m3fn codes (uint8) dequantised with the
    per-kv-head scales."""
    B, nh, d = q.shape
    out = np.zeros((B, nh, d), dtype=dtype)
    for b in range(B):
        L = int(cache_seqlens[b])
        if L <= 0:
            continue
        ks = paged_gather(k_cache, block_table[b], L)
        vs = paged_gather(v_cache, block_table[b], L)
        if k_scale is not None:
            ks = e4m3fn_to_f32(ks) * np.asarray(k_scale, np.float32)[None, :, None]
            vs = e4m3fn_to_f32(vs) * np.asarray(v_scale, np.float32)[None, :, None]
        out[b] = attention(q[b][None], ks, vs, scale, True, dtype)[0]
    return out


def prefill_flops(cu_seqlens_q, cu_seqlens_k, num_heads: int, head_dim: int) -> int:
    """Causal-visible multiply-adds x 2 for QK^T and PV: 4*d*nh*sum of visible pairs."""
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    cu_k = np.asarray(cu_seqlens_k, dtype=np.int64)
    lq = np.diff(cu_q)
    lk = np.diff(cu_k)
    pairs = lq * (lk - lq) + lq * (lq + 1) // 2
    return int(4 * head_dim * num_heads * pairs.sum())


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
