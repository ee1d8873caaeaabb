"""Build libgllm_hip.so (the C-ABI library of include/gllm_hip.h) for gfx950.

One hipcc invocation over csrc/*.hip, output in-tree next to this file so the
built library travels with the repository snapshot.  Flags:

* ``-ffp-contract=off``: the kernels place every fused multiply-add
  explicitly (fmaf) where the reference's AVX2 code uses VFMADD, and nowhere
  else, so float results are bit-identical to the reference's amd64 order.
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: IEEE division (the Q8K scale
  amax/127 and the softmax 1/denom must round exactly like the CPU).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 math.
* ``-mllvm -amdgpu-kernarg-preload-count=8``: the leading eight dwords of a
  kernel's plain (non-aggregate) arguments are preloaded into SGPRs by the
  command processor, so such a kernel issues its first loads without waiting
  for scalar loads of its arguments (the code keeps the loads as a fallback
  prologue for firmware without preloading).
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgllm_hip.so")
# measurement probes (bench.py --read-ceiling), a library of their own so the
# product library's exports stay exactly include/gllm_hip.h
PROBE_LIB = os.path.join(HERE, "libgllm_probe.so")
ARCH = os.environ.get("GLLM_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=8",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libgllm_hip)")


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compile every HIP source into libgllm_hip.so; returns its path.  Each
    source is compiled to an object in parallel (no device code crosses
    translation units), then one link step writes the library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    cc = hipcc()
    compile_flags = [f for f in FLAGS if f != "-shared"]

    def compile_one(src):
        obj = os.path.join(objdir, os.path.basename(src)[:-4] + ".o")
        cmd = [cc] + compile_flags + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        return obj, res

    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(compile_one, srcs))
    failed = [(o, r) for o, r in results if r.returncode != 0]
    for o, r in failed:
        sys.stderr.write(r.stdout + r.stderr)
    if failed:
        raise RuntimeError(f"hipcc failed for {[os.path.basename(o) for o, _ in failed]}")
    tmp = LIB + ".tmp"
    cmd = [cc] + FLAGS + [o for o, _ in results] + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc link failed with exit code {res.returncode}")
    os.replace(tmp, LIB)
    probe_srcs = sorted(glob.glob(os.path.join(CSRC, "probe", "*.hip")))
    if probe_srcs:
        tmp = PROBE_LIB + ".tmp"
        cmd = [cc] + FLAGS + probe_srcs + ["-o", tmp]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed for the probe library ({res.returncode})")
        os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
