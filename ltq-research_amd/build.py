"""Builds libltq_hip.so for gfx950 in-tree (ltq_amd/libltq_hip.so) from csrc/*.hip.

Flags: -ffp-contract=off (no FMA contraction: the quantizer's fp32 arithmetic must match the reference's
torch order of operations bit for bit), packed-fp32 instructions disabled, and -fno-honor-nans for the
Viterbi units (see EXTRA)."""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "ltq_amd" / "libltq_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", str(CSRC),
         "-I", str(HERE.parent / "include")]


# the Viterbi kernels compare and add path metrics that are never NaN or -0 (sums of squared errors >= +0
# under a 3.4e38 sentinel): without NaN semantics the compiler keeps v_min_f32 operands as they are instead of
# canonicalizing each one first, with bit-identical results
EXTRA = {"tcq_inst_": ["-fno-honor-nans"]}


def _extra(name: str):
    return [f for k, v in EXTRA.items() if name.startswith(k) for f in v]


def build(verbose: bool = False) -> Path:
    srcs = sorted(CSRC.glob("*.hip"))
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [HIPCC, *FLAGS, *_extra(src.name), "-c", str(src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
        if verbose:
            print(f"compiled {src.name}", flush=True)
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    tmp.replace(OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
