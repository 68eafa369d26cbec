"""Build libstrim_sampler.so in-tree with hipcc for gfx950.

    python strim-engine_amd/build.py

Always recompiles. Every translation unit is compiled to an object in parallel (the
k_stream variants are split over one object per (dtype, penalties, segments) triple), then the
objects are linked into strim-engine_amd/strim_amd/libstrim_sampler.so, next to the
Python binding, so the library travels with the tree. Objects go to a temporary
directory that is removed afterwards.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "strim_amd" / "libstrim_sampler.so"

# (source, extra defines): k_stream variants per (dtype, penalties, segments) triple
# (k_stream's ten leading arguments, the fields its first loads need, arrive preloaded in
# SGPRs, so those loads are issued before any wait for the argument block)
UNITS = [
    ("stream_kernels.hip", [f"-DSTRIM_DT={dt}", f"-DSTRIM_PEN={pen}", f"-DSTRIM_SSEG={sseg}",
                            "-mllvm", "-amdgpu-kernarg-preload-count=10"])
    for dt in (1, 0) for pen in (2, 1, 0) for sseg in (1, 4)
] + [
    ("finalize_kernels.hip", []),
    # k_gfinal's five leading arguments (the chunk statistics', lattice words' and slots'
    # addresses, the chunk stride and count) arrive preloaded in SGPRs, so its first load
    # is issued before any wait for the argument block
    ("gfinal_kernels.hip", ["-mllvm", "-amdgpu-kernarg-preload-count=5"]),
    ("sample_kernels.hip", []),
    ("qres_kernels.hip", []),
    ("aux_kernels.hip", []),
    ("head_kernels.hip", []),
    ("grammar_kernels.hip", []),
    ("capi.hip", []),
]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # every float32 step is one IEEE rounding (the parity contract relies on it)
    "-ffp-contract=off",
    # no packed fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed: " + " ".join(cmd))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    cc = hipcc()
    jobs = jobs or min(len(UNITS), os.cpu_count() or 1, 16)
    with tempfile.TemporaryDirectory(prefix="strim_build_") as tmpdir:
        objs, cmds = [], []
        for i, (src, defs) in enumerate(UNITS):
            obj = str(Path(tmpdir) / f"{i}_{Path(src).stem}.o")
            objs.append(obj)
            cmds.append([cc, *HIPCC_FLAGS, *defs, f"-I{ROOT / 'include'}", "-c",
                         str(CSRC / src), "-o", obj])
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            for f in [ex.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp = OUT.with_suffix(".so.tmp")
        _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", str(tmp)], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
