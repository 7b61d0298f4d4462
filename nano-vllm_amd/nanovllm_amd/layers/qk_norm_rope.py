"""Fused per-head RMSNorm + rotary embedding, the producer step feeding the path.

In the reference, Qwen3Attention.forward (nanovllm/models/qwen3.py:91-105) runs
  q = q_norm(q.view(-1, nh, d)).view(q.shape)      RMSNorm, layernorm.py:17-27
  k = k_norm(k.view(-1, nkv, d)).view(k.shape)
  q, k = rotary_emb(positions, q, k)               rotary_embedding.py:37-55
as three torch.compile'd graphs.  qk_norm_rope does all of it in one gfx950
kernel (nva_qk_norm_rope): one read and one write of q and k.  Without norm
weights it is the rotary embedding alone, as Qwen2 uses it (qwen2.py:91-92).

cos_sin_cache is the fp32 buffer RotaryEmbedding registers
(rotary_embedding.py:29-35): row p = [cos(p * inv_freq) | sin(p * inv_freq)].
rope_cos_sin_cache builds it the same way on the caller's device.
"""
from __future__ import annotations

import torch

from .. import _capi

_BF16 = torch.bfloat16


def rope_cos_sin_cache(head_dim: int, max_position: int, base: float, device=None) -> torch.Tensor:
    """The cos/sin table of RotaryEmbedding.__init__ (rotary_embedding.py:29-35)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float, device=device) / head_dim))
    t = torch.arange(max_position, dtype=torch.float, device=device)
    freqs = torch.einsum("i,j -> ij", t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def _rows(x: torch.Tensor, heads: int, head_dim: int, what: str) -> tuple[int, int]:
    """(num_tokens, row stride in elements) of a (T, heads*d) or (T, heads, d) view."""
    if x.dtype != _BF16 or not x.is_cuda:
        raise RuntimeError(f"{what} must be a bf16 device tensor")
    if x.dim() == 2:
        ok = x.shape[1] == heads * head_dim and x.stride(1) == 1
    elif x.dim() == 3:
        ok = x.shape[1:] == (heads, head_dim) and x.stride(2) == 1 and x.stride(1) == head_dim
    else:
        ok = False
    if not ok:
        raise RuntimeError(f"{what} must be (T, {heads}*{head_dim}) or (T, {heads}, {head_dim}) with contiguous heads")
    return x.shape[0], x.stride(0)


def qk_norm_rope(positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor, cos_sin_cache: torch.Tensor,
                 num_heads: int, num_kv_heads: int, head_dim: int,
                 q_norm_weight: torch.Tensor | None = None, k_norm_weight: torch.Tensor | None = None,
                 eps: float = 1e-6, inplace: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Returns (q, k) after the per-head RMSNorm (when weights are given) and the
    rotary embedding, in q's and k's shapes.  inplace=True writes into q and k."""
    T, q_rs = _rows(q, num_heads, head_dim, "q")
    Tk, k_rs = _rows(k, num_kv_heads, head_dim, "k")
    if Tk != T or positions.shape != (T,) or positions.dtype != torch.int64:
        raise RuntimeError("positions must be int64 (T,) with T matching q and k")
    if cos_sin_cache.dtype != torch.float32 or cos_sin_cache.dim() != 2 or cos_sin_cache.shape[1] != head_dim \
            or not cos_sin_cache.is_contiguous():
        raise RuntimeError("cos_sin_cache must be a contiguous float32 (max_position, head_dim) tensor")
    if (q_norm_weight is None) != (k_norm_weight is None):
        raise RuntimeError("pass both norm weights or neither")
    for w in (q_norm_weight, k_norm_weight):
        if w is not None and (w.dtype != _BF16 or w.shape != (head_dim,) or not w.is_contiguous()):
            raise RuntimeError(f"norm weights must be contiguous bf16 ({head_dim},)")
    if inplace:
        q_out, k_out = q, k
    else:
        q_out = torch.empty((T, num_heads * head_dim), dtype=_BF16, device=q.device).view(q.shape)
        k_out = torch.empty((T, num_kv_heads * head_dim), dtype=_BF16, device=k.device).view(k.shape)
    lib = _capi.load()
    rc = lib.nva_qk_norm_rope(
        q.data_ptr(), q_rs, k.data_ptr(), k_rs, q_out.data_ptr(), q_out.stride(0), k_out.data_ptr(),
        k_out.stride(0), None if q_norm_weight is None else q_norm_weight.data_ptr(),
        None if k_norm_weight is None else k_norm_weight.data_ptr(), float(eps), cos_sin_cache.data_ptr(),
        cos_sin_cache.shape[0], positions.data_ptr(), T, num_heads, num_kv_heads, head_dim,
        torch.cuda.current_stream(q.device).cuda_stream)
    _capi.check(rc)
    return q_out, k_out
