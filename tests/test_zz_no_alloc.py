"""nva_decode_noalloc (the decode entry point that allocates nothing: its
split-K partials live in the library's static device scratch) against
nva_decode with a caller-allocated workspace, through the C ABI: bit-identical
outputs on two calls in a row, the second with a smaller input (so a stale
first-call scratch would show), in bf16 and fp8, and an oversized request
refused before any launch."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    return _capi.load()


def _noalloc(lib, case, num_splits=0):
    from nanovllm_amd import _capi
    q = case.q.unsqueeze(1)
    B, _, nh, d = q.shape
    nb, bs, nkv, _ = case.k_cache.shape
    code = _capi.NVA_DTYPE_FP8_E4M3 if case.k_scale is not None else _capi.NVA_DTYPE_BF16
    out = torch.empty((B, 1, nh, d), dtype=torch.bfloat16, device=q.device)
    bt = case.block_tables
    _capi.check(lib.nva_decode_noalloc(
        q.data_ptr(), q.stride(0), case.k_cache.data_ptr(), case.v_cache.data_ptr(), code,
        case.k_scale.data_ptr() if case.k_scale is not None else None,
        case.v_scale.data_ptr() if case.v_scale is not None else None, nb,
        case.context_lens.data_ptr(), bt.data_ptr(), bt.stride(0), bt.shape[1], bs,
        B, nh, nkv, d, float(case.scale), int(num_splits), out.data_ptr(), out.stride(0),
        torch.cuda.current_stream().cuda_stream))
    return out


def _reference(case, num_splits=0):
    import nanovllm_amd as nva
    return nva.flash_attn_with_kvcache(case.q.unsqueeze(1), case.k_cache, case.v_cache, case.context_lens,
                                       case.block_tables, case.scale, True, num_splits=num_splits,
                                       k_scale=case.k_scale, v_scale=case.v_scale)


@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_matches_decode_two_calls(lib, fp8):
    from nanovllm_amd import workloads as W
    dev = torch.device("cuda:0")
    big = W.make_decode_case(96, 32, 8, 100, 3000, 1400, fp8=fp8, seed=31, bulk_device=dev)
    small = W.make_decode_case(5, 32, 8, 1, 700, 40, fp8=fp8, seed=32, bulk_device=dev)
    for case in (big, small):
        for ns in (0, 3):
            got = _noalloc(lib, case, ns)
            ref = _reference(case, ns)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"batch {case.batch} splits {ns}"


def test_noalloc_refuses_above_its_scratch(lib):
    from nanovllm_amd import _capi
    cap = lib.nva_decode_noalloc_max_workspace_bytes()
    assert cap == 32 << 20
    # 4096 sequences x 8 fixed splits x 128 heads of partials: far above the scratch
    assert lib.nva_decode_workspace_bytes(4096, 128, 8, 128, 64, 256, 0, 8) > cap
    A = 0x10000
    rc = lib.nva_decode_noalloc(A, 128 * 128, A, A, 0, None, None, 100, A, A, 64, 64, 256, 4096, 128, 8, 128, 0.1, 8,
                                A, 128 * 128, None)
    assert rc == _capi.NVA_ERR_WORKSPACE
    assert b"static scratch" in lib.nva_last_error()
