"""Golden cases of the attention hot path: seeded inputs, their digest, and the
oracle's expected outputs.

A fixture (tests/golden/*.npz, written by make_golden.py) holds the case's
parameters, the SHA-256 of its regenerated inputs, the expected attention
outputs (all rows, or a stated subset for the larger prefill case) and the
SHA-256 of the paged caches after store_kvcache (bit-exact).  Inputs are not
stored: they are rebuilt from the seed with torch's CPU generator, which is
deterministic for a given torch build, and the digest proves the rebuild is the
same data the expected values were computed from.

The expected values come from oracle/attention_oracle.py (numpy, float32), the
restatement of nanovllm/layers/attention.py:10-79 that tests/test_oracle.py pins
against brute force, torch's SDPA and closed forms.  The reference ships no
golden vectors of its own for this path.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import torch

from nanovllm_amd import workloads as W
from oracle import attention_oracle as O

HERE = Path(__file__).resolve().parent

# name -> parameters.  kind: decode (store of the newest token, then paged
# decode) or prefill (store of the fresh tokens, then varlen prefill, paged
# when prefix_len > 0).  rows: every `row_step`-th output row is kept.
CASES = {
    "decode_cfg1": dict(kind="decode", config=1),
    "prefill_cfg2": dict(kind="prefill", config=2, row_step=64),
    "decode_fp8_g8": dict(kind="decode", batch=3, num_heads=8, num_kv_heads=1, lengths=[300, 513, 17],
                          num_blocks=8, fp8=True, seed=71),
    "prefix_g4": dict(kind="prefill", lens_q=[40, 90], num_heads=8, num_kv_heads=2, num_blocks=8,
                      prefix_len=256, seed=72, row_step=1),
    "decode_d64_g7": dict(kind="decode", batch=4, num_heads=14, num_kv_heads=2, lengths=[1, 63, 256, 700],
                          num_blocks=12, head_dim=64, seed=73),
}


def build(name: str):
    """The case's inputs on the CPU, exactly as the fixture was made from."""
    m = CASES[name]
    if m.get("config"):
        return W.CONFIGS[m["config"]]("cpu")
    if m["kind"] == "decode":
        return W.make_decode_case(m["batch"], m["num_heads"], m["num_kv_heads"], 0, 0, m["num_blocks"],
                                  head_dim=m.get("head_dim", 128), fp8=m.get("fp8", False), seed=m["seed"],
                                  lengths=m["lengths"], name=name)
    return W.make_prefill_case(m["lens_q"], m["num_heads"], m["num_kv_heads"], m["num_blocks"],
                               prefix_len=m.get("prefix_len", 0), head_dim=m.get("head_dim", 128),
                               seed=m["seed"], name=name)


def _tensors(case) -> list[torch.Tensor]:
    if isinstance(case, W.DecodeCase):
        ts = [case.q, case.k_new, case.v_new, case.k_cache, case.v_cache, case.context_lens, case.block_tables,
              case.slot_mapping]
        if case.k_scale is not None:
            ts += [case.k_scale, case.v_scale]
        return ts
    ts = [case.q, case.k, case.v, case.cu_seqlens_q, case.cu_seqlens_k, case.slot_mapping, case.k_cache,
          case.v_cache]
    if case.block_tables is not None:
        ts.append(case.block_tables)
    return ts


def _sha(arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def _raw(t: torch.Tensor) -> np.ndarray:
    """Raw bytes of a tensor as numpy (bf16 / fp8 reinterpreted as integers)."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def input_digest(case) -> str:
    return _sha(_raw(t) for t in _tensors(case))


def cache_digest(k_cache: torch.Tensor, v_cache: torch.Tensor) -> str:
    return _sha([_raw(k_cache), _raw(v_cache)])


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def oracle_expected(case, name: str) -> dict:
    """Oracle store (bit patterns) then oracle attention; returns the fixture body."""
    m = CASES[name]
    if isinstance(case, W.DecodeCase):
        kc, vc = _raw(case.k_cache).copy(), _raw(case.v_cache).copy()
        if case.k_scale is not None:
            kn = O.quantize_e4m3fn(_f32(case.k_new), _f32(case.k_scale))
            vn = O.quantize_e4m3fn(_f32(case.v_new), _f32(case.v_scale))
        else:
            kn, vn = _raw(case.k_new), _raw(case.v_new)
        O.store_kvcache(kn, vn, kc, vc, case.slot_mapping.numpy())
        if case.k_scale is not None:
            kf = O.e4m3fn_to_f32(kc) * _f32(case.k_scale)[None, None, :, None]
            vf = O.e4m3fn_to_f32(vc) * _f32(case.v_scale)[None, None, :, None]
        else:
            kf, vf = O.bf16_bits_to_f32(kc.view(np.uint16)), O.bf16_bits_to_f32(vc.view(np.uint16))
        out = O.decode_attention(_f32(case.q), kf, vf, case.context_lens.numpy(), case.block_tables.numpy(),
                                 case.scale)
        rows = np.arange(out.shape[0])
    else:
        kc, vc = _raw(case.k_cache).copy(), _raw(case.v_cache).copy()
        O.store_kvcache(_raw(case.k), _raw(case.v), kc, vc, case.slot_mapping.numpy())
        if case.block_tables is None:
            out = O.prefill_attention(_f32(case.q), _f32(case.k), _f32(case.v), case.cu_seqlens_q.numpy(),
                                      case.cu_seqlens_k.numpy(), case.scale)
        else:
            kf, vf = O.bf16_bits_to_f32(kc.view(np.uint16)), O.bf16_bits_to_f32(vc.view(np.uint16))
            out = O.prefill_attention(_f32(case.q), kf, vf, case.cu_seqlens_q.numpy(), case.cu_seqlens_k.numpy(),
                                      case.scale, block_table=case.block_tables.numpy())
        rows = np.arange(0, out.shape[0], m.get("row_step", 1))
    return dict(rows=rows.astype(np.int64), expected=out[rows].astype(np.float32),
                store_sha256=np.array(_sha([kc, vc])))


def fixture_path(name: str) -> Path:
    return HERE / f"{name}.npz"


def load_fixture(name: str) -> dict:
    with np.load(fixture_path(name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def meta_json(name: str) -> str:
    return json.dumps(CASES[name], sort_keys=True)
