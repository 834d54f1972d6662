"""Build recipe for libtaomate_ltx.so (hipcc, gfx950 only).

    python -m taomate_amd.build          # compiles every csrc/*.hip, links lib/libtaomate_ltx.so

Objects are compiled in parallel into ``taomate_amd/_build/`` and linked into
``taomate_amd/lib/``.  The library is always rebuilt when this runs.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libtaomate_ltx.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 VALU ops are disabled for every HIP object on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmd):
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    return out


# per-source extra flags: the attention kernels' slot programs are fully
# unrolled (#pragma unroll) and larger than LLVM's default limit for a
# requested full unroll (16384), which would leave the fp8 instance rolled
PER_SOURCE = {"flash_attn.hip": ["-mllvm", "-pragma-unroll-threshold=200000"]}


def build(verbose: bool = False) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = []
    for src in sources:
        obj = BUILD / (src.stem + ".o")
        jobs.append((obj, [HIPCC, *FLAGS, *PER_SOURCE.get(src.name, []), "-c", str(src), "-o", str(obj)]))
    workers = min(len(jobs), max(1, (os.cpu_count() or 2) // 2))
    with cf.ThreadPoolExecutor(workers) as ex:
        outs = list(ex.map(lambda j: _run(j[1]), jobs))
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for o, _ in jobs]])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
