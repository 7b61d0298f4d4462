"""Build the gfx950 attention library (libnva_attn.so) in-tree with hipcc.

Usage:  python nano-vllm_amd/build.py [--jobs N] [--verbose]

Every .hip file under csrc/ is compiled to an object under _build/ and the
objects are linked into nanovllm_amd/_lib/libnva_attn.so, which the Python
host side loads with ctypes.  No GPU is needed to build.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
BUILD = HERE / "_build"
LIB_DIR = HERE / "nanovllm_amd" / "_lib"
LIB = LIB_DIR / "libnva_attn.so"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled: the kernels are written with scalar and
# float2 arithmetic and rely on the compiler not fusing them into v_pk_* forms.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


# Per-file extras.  The prefill kernel's softmax never relies on NaN
# propagation (masked scores are -inf, not NaN), so max() can skip the
# IEEE quieting of its operands.  Its atomics are single-lane (the work-queue
# claims, the key-half arrivals), so the compiler's atomic optimizer only adds
# a wait for the result right after each one; without it the wait moves to the
# result's first use, which lets the first claim overlap the table loads.
FILE_FLAGS = {
    "varlen_prefill.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), f"-I{CSRC}", f"-I{INCLUDE}", "-c", str(src),
           "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    warn = (res.stderr or "").strip()
    # hipcc's host pass does not know the -packed-fp32-ops feature and says so.
    lines = [ln for ln in warn.splitlines() if "packed-fp32-ops" not in ln and "not a recognized feature" not in ln]
    if verbose and lines:
        print("\n".join(lines), flush=True)
    return obj


def build(jobs: int = 4, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no .hip sources under {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    lib = build(args.jobs, args.verbose)
    print(f"built {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
