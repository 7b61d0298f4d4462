"""engine.kv_cache on the CPU: the block-size formula of model_runner.py:123-130,
the (2, L, num_blocks, block_size, nkv, d) layout, and the binding of k_cache /
v_cache (and, for fp8, k_scale / v_scale) on every module that has the
attributes, in module order (model_runner.py:144-149).  No kernel runs here."""
from __future__ import annotations

import pytest
import torch

from nanovllm_amd import Attention
from nanovllm_amd.engine.kv_cache import allocate_kv_cache, kv_block_bytes


class _Model(torch.nn.Module):
    def __init__(self, n):
        super().__init__()
        self.proj = torch.nn.Linear(2, 2)  # no cache attributes: skipped
        self.layers = torch.nn.ModuleList([Attention(16, 128, 128 ** -0.5, 8) for _ in range(n)])


def test_block_bytes():
    # 2 (K, V) * layers * block_size * nkv * d * itemsize
    assert kv_block_bytes(28, 256, 8, 128, torch.bfloat16) == 2 * 28 * 256 * 8 * 128 * 2
    assert kv_block_bytes(28, 256, 8, 128, torch.float8_e4m3fn) == 2 * 28 * 256 * 8 * 128


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_binding_in_module_order(dtype):
    m = _Model(3)
    kv = allocate_kv_cache(m.modules(), 3, 64, 8, 128, kv_dtype=dtype, num_blocks=5, device="cpu")
    assert kv.kv_cache.shape == (2, 3, 5, 64, 8, 128) and kv.kv_cache.dtype == dtype
    for i, a in enumerate(m.layers):
        assert a.k_cache.data_ptr() == kv.kv_cache[0, i].data_ptr()
        assert a.v_cache.data_ptr() == kv.kv_cache[1, i].data_ptr()
        assert a.k_cache.is_contiguous() and a.k_cache.stride(1) == 8 * 128  # the store's layout assert
        if dtype == torch.float8_e4m3fn:
            assert a.k_scale.shape == (8,) and a.k_scale.dtype == torch.float32 and a.k_scale.is_contiguous()
            assert a.v_scale.data_ptr() == kv.kv_scale[1, i].data_ptr()
        else:
            assert a.k_scale is None and a.v_scale is None


def test_scales_from_amax():
    m = _Model(2)
    kv = allocate_kv_cache(m.modules(), 2, 64, 8, 128, kv_dtype=torch.float8_e4m3fn, num_blocks=2, device="cpu")
    amax = torch.arange(1, 9, dtype=torch.float32)
    kv.set_scales_from_amax(1, amax, 2 * amax)
    assert torch.equal(m.layers[1].k_scale, amax / 448)
    assert torch.equal(m.layers[1].v_scale, 2 * amax / 448)
    assert torch.equal(m.layers[0].k_scale, torch.ones(8))  # untouched layer


def test_layer_count_must_match():
    with pytest.raises(ValueError, match="layers"):
        allocate_kv_cache(_Model(2).modules(), 3, 64, 8, 128, num_blocks=2, device="cpu")
