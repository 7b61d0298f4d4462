"""The C ABI without a GPU: the library loads, exports every symbol that
include/nva_attention.h declares, and rejects bad arguments with the documented
error codes before any HIP call (so rejected calls are safe on a CPU host)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from nanovllm_amd import _capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "nva_attention.h"

# fake, suitably aligned device addresses: validation rejects before dereferencing
A = 0x10000
B = 0x20000
C = 0x30000


@pytest.fixture(scope="module")
def lib():
    return _capi.load()


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(nva_\w+)\s*\(", text, flags=re.M)))


def test_header_lists_entry_points():
    names = declared_functions()
    assert {"nva_store_kvcache", "nva_prefill", "nva_prefill_workspace_bytes", "nva_decode",
            "nva_decode_workspace_bytes",
            "nva_last_error", "nva_version", "nva_qk_norm_rope"} <= set(names)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(declared_functions()) <= set(_capi.SIGNATURES)


def test_version(lib):
    assert lib.nva_version() >= 100


def store(lib, **kw):
    args = dict(key=A, key_row_stride=1024, value=B, value_row_stride=4096, k_cache=C, v_cache=C + 0x100000,
                num_slots=4096, slot_mapping=A + 0x8000, num_tokens=4, num_kv_heads=8, head_dim=128,
                cache_dtype=0, k_scale=None, v_scale=None, stream=None)
    args.update(kw)
    return lib.nva_store_kvcache(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(num_tokens=-1), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(num_kv_heads=0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(cache_dtype=7), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(key=None), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(slot_mapping=None), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(key_row_stride=1000), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(num_slots=0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(slot_mapping=A + 2), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(cache_dtype=1), _capi.NVA_ERR_INVALID_ARGUMENT),           # fp8 without scales
    (dict(cache_dtype=1, k_scale=A, v_scale=B, key=A + 8), _capi.NVA_ERR_UNSUPPORTED),
    (dict(key=A + 1), _capi.NVA_ERR_INVALID_ARGUMENT),               # bf16 misaligned
])
def test_store_rejects(lib, kw, code):
    assert store(lib, **kw) == code
    assert lib.nva_last_error().decode()


def test_store_zero_tokens_is_noop(lib):
    assert store(lib, num_tokens=0, key=None, value=None) == _capi.NVA_OK
    assert lib.nva_last_error().decode() == ""


def prefill(lib, **kw):
    args = dict(q=A, q_row_stride=2048, k=B, k_row_stride=1024, v=C, v_row_stride=4096, block_table=None,
                bt_row_stride=0, max_blocks=0, block_size=0, num_blocks=0, cu_q=A + 0x9000, cu_k=A + 0xA000,
                num_seqs=2, max_seqlen_q=100, max_seqlen_k=100, num_heads=16, num_kv_heads=8, head_dim=128,
                scale=0.088, out=C + 0x200000, out_row_stride=2048, workspace=None, workspace_bytes=0,
                stream=None)
    args.update(kw)
    return lib.nva_prefill(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(head_dim=96), _capi.NVA_ERR_UNSUPPORTED),
    (dict(num_heads=12), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(num_seqs=-1), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(q=None), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(cu_k=None), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(q_row_stride=1024), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(v_row_stride=1000), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(q=A + 2), _capi.NVA_ERR_UNSUPPORTED),
    (dict(scale=0.0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(block_table=A, bt_row_stride=8, max_blocks=8, block_size=32, num_blocks=10), _capi.NVA_ERR_UNSUPPORTED),
    (dict(block_table=A, bt_row_stride=4, max_blocks=8, block_size=256, num_blocks=10), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(workspace=A + 0x100000, workspace_bytes=128), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(workspace=A + 0x100040, workspace_bytes=256), _capi.NVA_ERR_INVALID_ARGUMENT),
])
def test_prefill_rejects(lib, kw, code):
    assert prefill(lib, **kw) == code


def test_prefill_empty_is_noop(lib):
    assert prefill(lib, num_seqs=0, q=None) == _capi.NVA_OK
    assert prefill(lib, max_seqlen_q=0) == _capi.NVA_OK


def test_prefill_workspace_bytes(lib):
    n = lib.nva_prefill_workspace_bytes()
    assert n >= 4 * 9 and n % 256 == 0


def test_prefill_workspace_errors_rejects(lib):
    """Bad workspaces are refused before any HIP call (no GPU here)."""
    import ctypes
    bits = ctypes.c_uint32(7)
    n = lib.nva_prefill_workspace_bytes()
    assert lib.nva_prefill_workspace_errors(None, n, ctypes.byref(bits), None) == _capi.NVA_ERR_INVALID_ARGUMENT
    assert lib.nva_prefill_workspace_errors(A, n, None, None) == _capi.NVA_ERR_INVALID_ARGUMENT
    assert lib.nva_prefill_workspace_errors(A, n - 256, ctypes.byref(bits), None) == _capi.NVA_ERR_INVALID_ARGUMENT
    assert lib.nva_prefill_workspace_errors(A + 64, n, ctypes.byref(bits), None) == _capi.NVA_ERR_INVALID_ARGUMENT
    assert bits.value == 7


def decode(lib, **kw):
    args = dict(q=A, q_row_stride=2048, k_cache=B, v_cache=C, kv_dtype=0, k_scale=None, v_scale=None,
                num_blocks=2048, seqlens=A + 0x9000, block_table=A + 0xA000, bt_row_stride=8, max_blocks=8,
                block_size=256, batch=256, num_heads=16, num_kv_heads=8, head_dim=128, scale=0.088,
                num_splits=0, out=C + 0x200000, out_row_stride=2048, workspace=None, workspace_bytes=0,
                stream=None)
    args.update(kw)
    return lib.nva_decode(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(head_dim=96), _capi.NVA_ERR_UNSUPPORTED),
    (dict(num_heads=24), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(num_heads=136), _capi.NVA_ERR_UNSUPPORTED),              # group 17
    (dict(kv_dtype=3), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(kv_dtype=1), _capi.NVA_ERR_INVALID_ARGUMENT),            # fp8 without scales
    (dict(batch=-2), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(block_size=48), _capi.NVA_ERR_UNSUPPORTED),
    (dict(bt_row_stride=4), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(num_blocks=0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(q=None), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(out=C + 8), _capi.NVA_ERR_UNSUPPORTED),
    (dict(num_splits=-2), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(scale=-1.0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(), _capi.NVA_ERR_WORKSPACE),                               # split-K needs a workspace
    (dict(workspace=A, workspace_bytes=16), _capi.NVA_ERR_WORKSPACE),
])
def test_decode_rejects(lib, kw, code):
    assert decode(lib, **kw) == code


def test_decode_workspace_plan(lib):
    f = lib.nva_decode_workspace_bytes
    rnd = lambda x: (x + 255) // 256 * 256
    # fixed mode, one split: no workspace
    assert f(4, 16, 8, 128, 1, 256, 0, 1) == 0
    assert f(256, 16, 8, 128, 8, 256, 0, 1) == 0
    # fixed mode: ceil(8 / 2) = 4 pages per split -> 2 splits per sequence
    assert f(256, 16, 8, 128, 8, 256, 0, 2) == rnd(256 * 2 * 16 * (128 + 2) * 4)
    # balanced mode (num_splits = 0): B + P slots plus the step prefix, where
    # P ranges of 4 kv-head waves (two head groups) make about 1024 bf16 waves
    assert f(256, 16, 8, 128, 8, 256, 0, 0) == rnd((256 + 128) * 16 * 130 * 4 + 257 * 4)
    # fp8: ranges of 8 kv-head waves, about 2048 waves
    assert f(64, 64, 8, 128, 128, 256, 1, 0) == rnd((64 + 256) * 64 * 130 * 4 + 65 * 4)
    # never more ranges than steps: 2 sequences x 1 page x 8 steps (balanced forced with -1)
    assert f(2, 16, 8, 128, 1, 256, 0, -1) == rnd((2 + 16) * 16 * 130 * 4 + 3 * 4)
    # small batch, table of at most 64 blocks (batch * nkv <= 256): spread mode,
    # S = min(1024 / (batch * nkv), table steps, 16) shares per sequence, B * S slots
    spread = lambda B, S: rnd(B * S * 16 * 130 * 4)
    assert f(2, 16, 8, 128, 1, 256, 0, 0) == spread(2, 8)      # 8 table steps
    assert f(32, 16, 8, 128, 16, 256, 0, 0) == spread(32, 4)   # 1024 / 256 pairs
    assert f(32, 16, 8, 128, 16, 256, 1, 0) == spread(32, 4)
    assert f(4, 16, 8, 128, 17, 256, 0, 0) == spread(4, 16)     # at most 16 shares
    assert f(1, 16, 8, 128, 1, 32, 0, 0) == 0                  # one share: written directly
    assert f(33, 16, 8, 128, 16, 256, 0, 0) == rnd((33 + 128) * 16 * 130 * 4 + 34 * 4)  # 264 pairs: balanced
    assert f(4, 16, 8, 128, 65, 256, 0, 0) > spread(4, 16)     # 65-block table: balanced
    # deterministic, and nothing for an empty batch
    assert f(64, 64, 8, 128, 128, 256, 1, 0) == f(64, 64, 8, 128, 128, 256, 1, 0) > 0
    assert f(0, 16, 8, 128, 8, 256, 0, 0) == 0


def store_decode(lib, **kw):
    st = dict(key=A + 0x100000, key_row_stride=1024, value=A + 0x180000, value_row_stride=1024,
              slot_mapping=A + 0xB000)
    dec = dict(q=A, q_row_stride=2048, k_cache=B, v_cache=C, kv_dtype=0, k_scale=None, v_scale=None,
               num_blocks=2048, seqlens=A + 0x9000, block_table=A + 0xA000, bt_row_stride=8, max_blocks=8,
               block_size=256, batch=256, num_heads=16, num_kv_heads=8, head_dim=128, scale=0.088,
               num_splits=0, out=C + 0x200000, out_row_stride=2048, workspace=None, workspace_bytes=0,
               stream=None)
    for d in (st, dec):
        for k in list(kw):
            if k in d:
                d[k] = kw.pop(k)
    assert not kw, kw
    return lib.nva_store_decode(*st.values(), *dec.values())


@pytest.mark.parametrize("kw,code", [
    (dict(key_row_stride=512), _capi.NVA_ERR_INVALID_ARGUMENT),      # < nkv * d
    (dict(key=None), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(slot_mapping=A + 0xB002), _capi.NVA_ERR_INVALID_ARGUMENT),  # misaligned
    (dict(kv_dtype=1), _capi.NVA_ERR_INVALID_ARGUMENT),              # fp8 without scales
    (dict(num_blocks=0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(head_dim=96, key_row_stride=768, value_row_stride=768), _capi.NVA_ERR_UNSUPPORTED),
    (dict(workspace=A, workspace_bytes=16), _capi.NVA_ERR_WORKSPACE),
])
def test_store_decode_rejects(lib, kw, code):
    """Both halves are validated (the store's, then the decode's) before any launch."""
    assert store_decode(lib, **kw) == code


def test_store_decode_batch_zero_is_noop(lib):
    assert store_decode(lib, batch=0) == _capi.NVA_OK


def test_decode_batch_zero_is_noop(lib):
    assert decode(lib, batch=0, workspace=None) == _capi.NVA_OK


def test_error_raises_runtime_error(lib):
    assert decode(lib, head_dim=96) != 0
    with pytest.raises(RuntimeError, match="head_dim"):
        _capi.check(_capi.NVA_ERR_UNSUPPORTED)


def qk_norm_rope(lib, **kw):
    args = dict(q=A, q_row_stride=6144, k=A + 0x1000, k_row_stride=6144, q_out=B, q_out_row_stride=4096,
                k_out=C, k_out_row_stride=1024, q_w=A + 0x20000, k_w=A + 0x20100, eps=1e-6,
                cos_sin=A + 0x40000, max_position=4096, positions=A + 0x80000, num_tokens=5, num_heads=32,
                num_kv_heads=8, head_dim=128, stream=None)
    args.update(kw)
    return lib.nva_qk_norm_rope(*args.values())


@pytest.mark.parametrize("kw,code", [
    (dict(num_tokens=-1), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(num_heads=0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(head_dim=96), _capi.NVA_ERR_UNSUPPORTED),
    (dict(k_w=None), _capi.NVA_ERR_INVALID_ARGUMENT),               # one weight without the other
    (dict(eps=-1.0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(max_position=0), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(positions=None), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(q_row_stride=4000), _capi.NVA_ERR_INVALID_ARGUMENT),       # < num_heads * head_dim
    (dict(k_out_row_stride=1000), _capi.NVA_ERR_INVALID_ARGUMENT),
    (dict(q=A + 4), _capi.NVA_ERR_UNSUPPORTED),                      # head_dim 128 needs 8-byte rows
    (dict(positions=A + 0x80004), _capi.NVA_ERR_INVALID_ARGUMENT),
])
def test_qk_norm_rope_rejects(lib, kw, code):
    assert qk_norm_rope(lib, **kw) == code
    assert lib.nva_last_error().decode()


def test_qk_norm_rope_zero_tokens_is_noop(lib):
    assert qk_norm_rope(lib, num_tokens=0, q=None) == _capi.NVA_OK
    # rotary embedding only (no weights) and head_dim 64 validate too
    assert qk_norm_rope(lib, num_tokens=0, q_w=None, k_w=None, head_dim=64) == _capi.NVA_OK


def test_decode_refuses_fp8_head_dim_64(lib):
    assert decode(lib, head_dim=64, kv_dtype=1, k_scale=A, v_scale=B) == _capi.NVA_ERR_UNSUPPORTED
    assert "head_dim" in lib.nva_last_error().decode()


def test_decode_noalloc_refuses_above_its_scratch(lib):
    """nva_decode_noalloc serves workspaces up to its static scratch and refuses a
    larger one with NVA_ERR_WORKSPACE before any HIP call (so this runs without a
    GPU)."""
    cap = lib.nva_decode_noalloc_max_workspace_bytes()
    assert cap == 32 << 20
    assert lib.nva_decode_workspace_bytes(4096, 128, 8, 128, 64, 256, 0, 8) > cap
    rc = lib.nva_decode_noalloc(A, 128 * 128, B, C, 0, None, None, 100, A + 0x8000, A + 0x9000, 64, 64, 256, 4096,
                                128, 8, 128, 0.1, 8, B + 0x40000, 128 * 128, None)
    assert rc == _capi.NVA_ERR_WORKSPACE
    assert b"static scratch" in lib.nva_last_error()
    # argument checks run first, as in nva_decode
    rc = lib.nva_decode_noalloc(A, 128, B, C, 0, None, None, 100, A, A, 64, 64, 256, 4, 16, 8, 96, 0.1, 0,
                                B, 128, None)
    assert rc == _capi.NVA_ERR_UNSUPPORTED
