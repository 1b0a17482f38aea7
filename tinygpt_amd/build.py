"""Builds libtgs_sampler.so in-tree with hipcc for gfx950.

    python -m tinygpt_amd.build

Flags: -ffp-contract=off (each float operation is the single IEEE operation
the source writes: the sampling contract is bit-exact), correctly rounded
fp32 division, IEEE denormals, and packed-fp32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libtgs_sampler.so")
# the plain-read floor kernel of bench.py --workload read (measurement only,
# its own library: not part of the sampler's C ABI)
FLOOR_SRC = "tgs_floor.hip"
FLOOR_OUT = os.path.join(HERE, "libtgs_floor.so")
SOURCES = ["tgs_kernels.hip", "tgs_k64.hip", "tgs_spec.hip", "tgs_topp.hip", "tgs_topk.hip", "tgs_logprob.hip",
           "tgs_mask.hip", "tgs_api.hip"]
ARCH = os.environ.get("TGS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep single-lane atomics as written: the wave-aggregating rewrite
    # consumes an atomic's result right after it, which would stall the
    # loads issued behind the fused kernel's arrival count
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    return "hipcc"


def build(verbose: bool = False) -> str:
    """Compiles every source to an object in parallel, then links the library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    comp = [f for f in HIPCC_FLAGS if f != "-shared"]

    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc(), *comp, "-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        return src, obj, cmd, r

    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES) + 1)) as ex:
        results = list(ex.map(compile_one, SOURCES + [FLOOR_SRC]))
    floor = results.pop()
    msgs = []
    for src, obj, cmd, r in results:
        errors = "\n".join(l for l in (r.stderr or "").splitlines() if "packed-fp32-ops" not in l)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed ({r.returncode}):\n{' '.join(cmd)}\n{errors}")
        if errors.strip():
            msgs.append(errors)
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[o for _, o, _, _ in results], "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed ({r.returncode}):\n{' '.join(cmd)}\n{r.stderr}")
    _, fobj, fcmd, fr = floor
    if fr.returncode != 0:
        raise RuntimeError(f"hipcc failed ({fr.returncode}):\n{' '.join(fcmd)}\n{fr.stderr}")
    ftmp = FLOOR_OUT + ".tmp"
    r2 = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", fobj, "-o", ftmp], capture_output=True,
                        text=True)
    if r2.returncode != 0:
        raise RuntimeError(f"link failed ({r2.returncode}):\n{r2.stderr}")
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)
    os.replace(tmp, OUT)
    os.replace(ftmp, FLOOR_OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
