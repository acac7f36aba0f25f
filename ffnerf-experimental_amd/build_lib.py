"""Build libffnerf_hip.so (gfx950) in-tree with hipcc.

Every HIP source is compiled with -ffp-contract=off (the sampler, hash and
occupancy outputs must be reproducible operation for operation) and with the
packed-fp32 target feature disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libffnerf_hip.so"
ARCH = os.environ.get("FFN_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["ffn_capi.hip", "ffn_sample.hip", "ffn_hash.hip", "ffn_mlp.hip", "ffn_optim.hip", "ffn_march.hip", "ffn_mlp16.hip", "ffn_batch.hip"]

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    # MFMA results in VGPRs: the MLP chains every layer's accumulator into the next layer's operand, and the
    # AGPR form costs a v_accvgpr_read per value (and spills at the cfg2 shape)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def build(verbose: bool = False, jobs: int = 8) -> Path:
    hipcc = HIPCC
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        objs.append(obj)
        cmd = [hipcc, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        if len(procs) >= jobs:
            _drain(procs, verbose)
    _drain(procs, verbose)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def _drain(procs, verbose):
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        lines = [l for l in (out or "").splitlines() if "packed-fp32-ops" not in l]
        if p.returncode != 0:
            failed.append(src)
            print("\n".join(lines), file=sys.stderr)
        elif verbose and lines:
            print("\n".join(lines))
    procs.clear()
    if failed:
        raise RuntimeError(f"hipcc failed for: {', '.join(failed)}")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
