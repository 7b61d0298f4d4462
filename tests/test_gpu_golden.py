"""The golden fixtures on the GPU: store_kvcache then attention through the C ABI
on the rebuilt seeded inputs, against the recorded oracle outputs (bf16: max-abs
2e-2, mean-abs 2e-3; fp8 KV: 5e-2) and the recorded post-store cache digest
(bit-exact)."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

from _helpers import FP8_MAX_ABS, assert_attn_close, f32

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import golden_cases as G  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    from nanovllm_amd import _capi
    _capi.load()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")


@pytest.mark.parametrize("name", list(G.CASES))
def test_fixture_on_gpu(dev, name):
    import nanovllm_amd as nva
    from nanovllm_amd import workloads as W
    fx = G.load_fixture(name)
    cpu_case = G.build(name)
    assert str(fx["input_sha256"]) == G.input_digest(cpu_case)
    case = cpu_case.to(dev)
    if isinstance(case, W.DecodeCase):
        nva.store_kvcache(case.k_new, case.v_new, case.k_cache, case.v_cache, case.slot_mapping,
                          case.k_scale, case.v_scale)
        o = nva.flash_attn_with_kvcache(case.q.unsqueeze(1), case.k_cache, case.v_cache, case.context_lens,
                                        case.block_tables, case.scale, True, k_scale=case.k_scale,
                                        v_scale=case.v_scale)[:, 0]
    else:
        nva.store_kvcache(case.k, case.v, case.k_cache, case.v_cache, case.slot_mapping)
        k, v = (case.k, case.v) if case.block_tables is None else (case.k_cache, case.v_cache)
        o = nva.flash_attn_varlen_func(case.q, k, v, case.max_seqlen_q, case.cu_seqlens_q, case.max_seqlen_k,
                                       case.cu_seqlens_k, case.scale, True, case.block_tables)
    torch.cuda.synchronize()
    assert G.cache_digest(case.k_cache, case.v_cache) == str(fx["store_sha256"]), "cache contents differ after the store"
    got = f32(o)[fx["rows"]]
    tol = dict(max_abs=FP8_MAX_ABS, mean_abs=FP8_MAX_ABS) if case.k_cache.element_size() == 1 else {}
    mx, mn = assert_attn_close(got, fx["expected"], what=name, **tol)
    print(f"{name}: max-abs {mx:.3e} mean-abs {mn:.3e}")
