"""CPU oracle for the producer step feeding the attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker, never as the computation being measured
or shipped.

It restates, in numpy float32 with bf16 roundings where the reference rounds,
what nanovllm/models/qwen3.py:91-105 computes between the qkv projection and
Attention.forward (read-only reference tree):

  rms_norm_bf16   RMSNorm.rms_forward, layernorm.py:17-27, eager op sequence:
                  x.float(); var = mean(x^2); x *= rsqrt(var + eps);
                  x = x.to(bf16) * weight (bf16 product, rounded to bf16)
  rope_bf16       apply_rotary_emb, rotary_embedding.py:6-17, with cos/sin rows of
                  cos_sin_cache[positions] (rotary_embedding.py:47-49):
                  x1, x2 = halves of x.float(); y1 = x1 cos - x2 sin;
                  y2 = x2 cos + x1 sin; cat -> bf16 (each product and sum rounded)
  qk_norm_rope    q_norm / k_norm per head, then the rotary embedding of both
                  (qwen3.py:92-105); without weights, the rotary embedding alone
                  (qwen2.py:91-92)
  rope_cos_sin    the cache RotaryEmbedding.__init__ builds (rotary_embedding.py:29-35)

Parity pinning (tests/test_producer_oracle.py): the rotation against numpy complex
multiplication (x1 + i x2) * exp(i p f), norm preservation of every pair,
position 0 = identity, rotate(p1) then rotate(p2) = rotate(p1 + p2) in float64,
the RMS of a normalised row = 1 (unit weight), RMSNorm of a constant row, and
torch.nn.functional.rms_norm / torch float32 ops on the same inputs; planted
mistakes (halves swapped, sin sign flipped, mean over the wrong axis, missing
eps) fail them.

Not pinned: the reference runs both functions under @torch.compile
(layernorm.py:17, rotary_embedding.py:39), and this module follows the eager
op sequence.  Inductor may fuse the rotation's products and sums (fused
multiply-adds round once where eager rounds twice in float32) and may keep
an intermediate in float32 where eager rounds it to bf16.  The compiled
reference's bits can therefore differ from this restatement by a bf16 ulp in
rare elements; no check here (torch is eager, flash-attn and the compiled
graph are absent) fixes which.
"""
from __future__ import annotations

import numpy as np

from oracle.attention_oracle import bf16_bits_to_f32, f32_to_bf16_bits


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 (RNE), returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def rope_cos_sin(head_dim: int, max_position: int, base: float) -> np.ndarray:
    """(max_position, head_dim) float32: [cos(p f) | sin(p f)], f = base^(-2i/d)
    (rotary_embedding.py:29-35, computed here in float64 then rounded)."""
    inv_freq = 1.0 / (base ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    freqs = np.arange(max_position, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.concatenate([np.cos(freqs), np.sin(freqs)], axis=-1).astype(np.float32)


def rms_norm_bf16(x_bf16: np.ndarray, weight_bf16: np.ndarray, eps: float) -> np.ndarray:
    """x: (..., d) float32 holding bf16 values; weight: (d,) likewise.  layernorm.py:21-27."""
    x = np.asarray(x_bf16, dtype=np.float32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    y = bf16_round(x * r)
    return bf16_round(y * np.asarray(weight_bf16, dtype=np.float32))


def rope_bf16(x_bf16: np.ndarray, positions: np.ndarray, cos_sin: np.ndarray) -> np.ndarray:
    """x: (T, heads, d) float32 holding bf16 values; rotary_embedding.py:6-17, 44-55."""
    x = np.asarray(x_bf16, dtype=np.float32)
    d = x.shape[-1]
    cs = cos_sin[np.asarray(positions, dtype=np.int64)]            # (T, d)
    cos = cs[:, None, : d // 2]
    sin = cs[:, None, d // 2:]
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    y1 = (x1 * cos).astype(np.float32) - (x2 * sin).astype(np.float32)
    y2 = (x2 * cos).astype(np.float32) + (x1 * sin).astype(np.float32)
    return bf16_round(np.concatenate([y1, y2], axis=-1))


def qk_norm_rope(q_bf16, k_bf16, positions, cos_sin, q_weight=None, k_weight=None, eps=1e-6):
    """q: (T, nh, d), k: (T, nkv, d) float32 holding bf16 values -> (q, k) as bf16 values.
    qwen3.py:91-105 (with weights) / qwen2.py:91-92 (without)."""
    q = np.asarray(q_bf16, dtype=np.float32)
    k = np.asarray(k_bf16, dtype=np.float32)
    if q_weight is not None:
        q = rms_norm_bf16(q, q_weight, eps)
        k = rms_norm_bf16(k, k_weight, eps)
    return rope_bf16(q, positions, cos_sin), rope_bf16(k, positions, cos_sin)


def producer_bytes(num_tokens: int, num_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """Algorithmic HBM bytes of one fused call: q and k read and written once (bf16),
    one cos/sin row (fp32) and one int64 position per token, two bf16 weights."""
    rows = num_tokens * (num_heads + num_kv_heads)
    return rows * head_dim * 2 * 2 + num_tokens * (head_dim * 4 + 8) + 2 * head_dim * 2
