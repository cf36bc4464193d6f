"""Compile the gfx950 HIP kernels of this package into ``lib/libsymbiote_mi355x.so``.

The library is a plain C-ABI shared object (see ``include/symbiote_mi355x.h``) built with
``hipcc`` for ``--offload-arch=gfx950`` only. Each ``csrc/*.hip`` file compiles to its own
object in parallel; the objects are linked into one ``.so`` that is loaded with ``ctypes``
after ``torch`` (so the process keeps a single HIP runtime: torch's ``libamdhip64.so.7``).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libsymbiote_mi355x.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # IEEE fp32 division and denormals on the device: the router's integer outputs depend on
    # exact fp32 arithmetic matching the CPU oracle.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    # never emit packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: AGPRs are allocated from the same register file in addition
    # to the VGPRs' peak, so keeping them out raises occupancy (the decode attention kernels
    # from 3 to 4 waves per SIMD; no kernel loses occupancy)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-pass-failed",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")


def _compile_one(hipcc: str, src: str, obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
    cmd = [hipcc, *HIP_FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False, out: str = LIB_PATH) -> str:
    """Compile every ``csrc/*.hip`` and link the shared library. Returns the library path."""
    hipcc = _hipcc()
    obj_dir = OBJ_DIR
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
    sources = sorted(
        os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip")
    )
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC_DIR}")
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile_one(hipcc, s, obj_dir), sources))
    tmp = out + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(sources)} sources", file=sys.stderr)
    return out


if __name__ == "__main__":
    build(verbose=True)
