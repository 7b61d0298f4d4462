"""Write the golden fixtures tests/golden/*.npz from the oracle.

Usage (repository root):  python tests/golden/make_golden.py [name ...]

Each fixture: the case parameters (JSON), the SHA-256 of the regenerated
inputs, the expected outputs (float32) at the stored row indices and the SHA-256
of the caches after the store.  See golden_cases.py.
"""
from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
for p in (ROOT, ROOT / "nano-vllm_amd", Path(__file__).resolve().parent):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import numpy as np  # noqa: E402

import golden_cases as G  # noqa: E402


def main(names: list[str]) -> int:
    for name in names or list(G.CASES):
        case = G.build(name)
        body = G.oracle_expected(case, name)
        np.savez_compressed(G.fixture_path(name), meta=np.array(G.meta_json(name)),
                            input_sha256=np.array(G.input_digest(case)), **body)
        size = G.fixture_path(name).stat().st_size
        print(f"{name}: {body['expected'].shape} expected rows, {size / 1024:.0f} KiB")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
