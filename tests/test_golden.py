"""The golden fixtures (tests/golden/*.npz) on the CPU: the seeded inputs rebuild
to the recorded digest, and the oracle reproduces the recorded outputs and
post-store cache digest.  This pins the oracle against drift; the GPU side of
the same fixtures is tests/test_gpu_golden.py."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import golden_cases as G  # noqa: E402


@pytest.mark.parametrize("name", list(G.CASES))
def test_fixture_matches_oracle(name):
    fx = G.load_fixture(name)
    assert str(fx["meta"]) == G.meta_json(name), "case parameters changed since the fixture was written"
    case = G.build(name)
    assert str(fx["input_sha256"]) == G.input_digest(case), "seeded inputs no longer rebuild to the recorded data"
    body = G.oracle_expected(case, name)
    assert str(body["store_sha256"]) == str(fx["store_sha256"])
    np.testing.assert_array_equal(body["rows"], fx["rows"])
    np.testing.assert_allclose(body["expected"], fx["expected"], rtol=1e-5, atol=1e-6)


def test_fixtures_are_small_and_cover_the_path():
    kinds = {G.CASES[n]["kind"] for n in G.CASES}
    assert kinds == {"decode", "prefill"}
    assert any(G.CASES[n].get("fp8") for n in G.CASES)
    assert any(G.CASES[n].get("prefix_len") for n in G.CASES)
    assert sum(G.fixture_path(n).stat().st_size for n in G.CASES) < 2 << 20
