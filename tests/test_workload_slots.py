"""The synthetic producers (nanovllm_amd/workloads.py) write the cache slots the
reference's producers would: every configuration's slot_mapping equals the
oracle's slot formulas, which tests/test_oracle.py pins to
model_runner.py:180-188 (prefill) and model_runner.py:227-229 (decode).
Only the index tensors are built (no q/k/v or caches), so this runs on the CPU
at the full configuration sizes."""
from __future__ import annotations

import numpy as np
import pytest

from nanovllm_amd import workloads as W
from oracle import attention_oracle as O


def _check_prefill(case):
    bt = case.page_table.numpy()
    expect = []
    for s, (pre, lk) in enumerate(zip(case.prefix_lens, case.lens_k)):
        expect += O.prefill_slots(bt[s], pre, lk, case.block_size)
    assert case.slot_mapping.tolist() == expect
    # the cached prefix is whole pages and the paged path gets the same table
    if case.block_tables is not None:
        assert np.array_equal(case.block_tables.numpy(), bt)
    assert case.cu_seqlens_q.tolist() == list(np.cumsum([0] + case.lens_q))
    assert case.cu_seqlens_k.tolist() == list(np.cumsum([0] + case.lens_k))


def _check_decode(case):
    bt = case.block_tables.numpy()
    lens = case.context_lens.tolist()
    assert len(lens) == case.slot_mapping.numel()
    for b, L in enumerate(lens):
        if L > 0:
            assert int(case.slot_mapping[b]) == O.decode_slot(bt[b], L, case.block_size)
        # pages of one sequence are distinct and inside the pool
        pages = bt[b, : -(-L // case.block_size)]
        assert len(set(pages.tolist())) == len(pages) and (pages >= 0).all()
    # no two sequences share a page (the decode caches are not prefix-shared)
    used = np.concatenate([bt[b, : -(-L // case.block_size)] for b, L in enumerate(lens)])
    assert len(np.unique(used)) == len(used)


@pytest.mark.parametrize("cfg", [2, 4])
def test_prefill_config_slots(cfg):
    _check_prefill(W.CONFIGS[cfg](None))


@pytest.mark.parametrize("cfg", [1, 3, 5])
def test_decode_config_slots(cfg):
    _check_decode(W.CONFIGS[cfg](None))


def test_mixed_prefix_slots():
    case = W.make_prefill_case([100, 300, 5, 256, 0], 16, 8, 40, prefix_len=[0, 256, 1024, 0, 512], seed=2,
                               bulk_device=None)
    _check_prefill(case)
    assert case.block_tables is not None  # one cached prefix puts the whole batch on the paged path
