"""The parts of bench.py's contract that need no GPU: the one-GPU refusal, and the
profiled HBM traffic it copies into its JSON line from profiles/ -- present, parsed,
and within a few percent of the algorithmic bytes of the launch each figure describes
(a profile edited out of step with the workload, or a line the parser no longer
reads, fails here rather than as a silent null in the bench line)."""
import math
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "nano-vllm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import bench  # noqa: E402
from nanovllm_amd import workloads as W  # noqa: E402


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU only" in capsys.readouterr().err


def _decode_launch_bytes(case, elem):
    """Every visible K and V byte once, plus q and o (bf16), the lengths and the
    block-table entries of the visible pages (and the fp8 scales)."""
    L = sum(case.lengths)
    B = len(case.lengths)
    pages = sum(math.ceil(x / case.block_size) for x in case.lengths)
    scales = 2 * case.num_kv_heads * 4 if elem == 1 else 0
    return (L * case.num_kv_heads * case.head_dim * 2 * elem + B * case.num_heads * case.head_dim * 2 * 2
            + 4 * B + 4 * pages + scales)


@pytest.mark.parametrize("key,make,elem", [("config3", W.config3, 2), ("config5", W.config5, 1)])
def test_profiled_decode_traffic_matches_its_launch(key, make, elem):
    traffic = bench.profiled_traffic(key)
    assert traffic is not None, f"profiles/decode_hbm_traffic.md has no {key} line"
    ratio = traffic / _decode_launch_bytes(make(bulk_device=None), elem)
    assert 1.0 <= ratio <= 1.05, ratio


@pytest.mark.parametrize("key,make", [("store_cfg4", W.config4), ("store_cfg2", W.config2)])
def test_profiled_store_traffic_matches_its_launch(key, make):
    traffic = bench.profiled_traffic(key, "store_hbm_traffic.md")
    assert traffic is not None, f"profiles/store_hbm_traffic.md has no {key} line"
    case = make(bulk_device=None)
    tokens = sum(case.lens_q)
    # each new token's K and V rows of every kv head read once and written once, plus its slot
    per_token = 2 * case.num_kv_heads * case.head_dim * 2 * 2 + 4
    ratio = traffic / (tokens * per_token)
    assert 1.0 <= ratio <= 1.05, ratio
