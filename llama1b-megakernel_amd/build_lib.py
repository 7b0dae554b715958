"""Build ``libmk.so`` (the HIP megakernel + C ABI) in-tree for gfx950.

Usage: ``python build_lib.py`` or ``build_lib.build()``. Always recompiles.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
SOURCES = [HERE / "csrc" / "mk_decode.hip", HERE / "csrc" / "mk_decode_step.hip", HERE / "csrc" / "mk_batch.hip",
           HERE / "csrc" / "mk_batch_tile2.hip",
           HERE / "csrc" / "mk_sample.hip", HERE / "csrc" / "mk_prefill.hip"]
LIB = HERE / "libmk.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # no packed fp32 instructions anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(REPO / "include"),
]


# Extra flags per source (each source is compiled to an object, then linked). The prefill
# GEMMs keep their MFMA accumulators in VGPRs (the VGPR form of the MFMA):
# with the default AGPR form the compiler copies every accumulator between the
# two register files around each k-step of the LDS pipeline.
SEPARATE = {HERE / "csrc" / "mk_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {LIB.name}")


def build(verbose: bool = False) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB.with_suffix(".so.tmp")
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    objs = []
    try:
        for src in SOURCES:
            obj = src.with_suffix(".o")
            _run([hipcc, *compile_flags, *SEPARATE.get(src, []), "-c", str(src), "-o", str(obj)], verbose)
            objs.append(obj)
        _run([hipcc, "--hip-link", "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)],
             verbose)
    finally:
        for obj in objs:
            if obj.exists():
                obj.unlink()
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
