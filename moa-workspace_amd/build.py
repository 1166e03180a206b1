#!/usr/bin/env python3
"""Build libmoa_gfx950.so in-tree with hipcc (cross-compiles without a GPU).

    python moa-workspace_amd/build.py [--verbose]

Flags:
  --offload-arch=gfx950                  MI355X only
  -ffp-contract=off                      every multiply/add rounds on its own, as the
                                         reference's torch ops do; kernels call fmaf()
                                         explicitly where the product is exact
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                         no packed-FP32 VALU instructions
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmoa_gfx950.so"
SOURCES = ["moa_api.hip", "moa_decode.hip", "moa_chunk.hip", "moa_attention.hip", "moa_logits.hip", "moa_ckpt.hip", "moa_full_attention.hip", "moa_rows.hip", "moa_bench.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)


def build(verbose: bool = False) -> Path:
    """Compiles every source to an object (in parallel: the translation units are independent),
    then links the shared library. Objects and the linked file go to a directory of this build's
    own, so builds that run at the same time never read each other's half-written files; the
    library is then replaced in one step."""
    import shutil
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    srcs = [CSRC / s for s in SOURCES if (CSRC / s).exists()]
    (PKG / "_build").mkdir(exist_ok=True)
    objdir = Path(tempfile.mkdtemp(prefix="build-", dir=PKG / "_build"))
    try:
        objs = [objdir / (s.stem + ".o") for s in srcs]
        compile_flags = [f for f in FLAGS if f != "-shared"]
        jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
        with ThreadPoolExecutor(jobs) as ex:
            for f in [ex.submit(_run, [HIPCC, *compile_flags, "-c", "-o", str(o), str(s)], verbose)
                      for s, o in zip(srcs, objs)]:
                f.result()
        tmp = objdir / LIB.name
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
        os.replace(tmp, LIB)
    finally:
        shutil.rmtree(objdir, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
