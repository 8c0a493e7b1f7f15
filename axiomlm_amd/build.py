"""Ahead-of-time build of libaxm.so (HIP kernels + C ABI) for gfx950.

Every ``csrc/*.hip`` file is compiled by ``hipcc`` to an object (in parallel)
and linked into ``axiomlm_amd/libaxm.so``.  The library links against the HIP
runtime by its SONAME (libamdhip64.so.7); inside a process that already
imported torch it binds to torch's copy of the runtime, so device pointers and
streams are shared with torch.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(REPO_DIR, "_build", "axm")
LIB_PATH = os.path.join(PKG_DIR, "libaxm.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Contraction into multiply-adds everywhere except code marked
    # "#pragma clang fp contract(off)" (the rounded helpers of axm_common.h).
    "-ffp-contract=fast-honor-pragmas",
    # Packed-fp32 VALU ops are disabled for all device code on this target.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{os.path.join(REPO_DIR, 'include')}",
    f"-I{CSRC}",
]


# Per-file code generation options.  attention.hip: MFMA accumulators in VGPRs
# (with them in AGPRs the compiler copied every output accumulator out and back
# on each key block of the decode kernel).
FILE_FLAGS = {
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # q4_tile16.hip: the same; with AGPR accumulators every GEMV chunk copied all
    # sixteen accumulator values out (7B decode step 758.7 -> 763.3 tok/s).
    "q4_tile16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form",
                      # The GEMV's leading scalar arguments land in SGPRs before the wave
                      # starts: its first requests do not wait for an argument load.
                      "-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "lowbit_gemv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "q2k_gguf.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    # AXM_HIPCC_EXTRA adds flags to every compile (diagnostic builds, e.g. -DAXM_STEP_STAMPS).
    extra = FILE_FLAGS.get(os.path.basename(src), []) + os.environ.get("AXM_HIPCC_EXTRA", "").split()
    cmd = [os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, *extra, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link libaxm.so; returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources found")
    workers = min(len(sources), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH + ".tmp"
    link = [
        os.path.join(ROCM, "bin", "hipcc"),
        f"--offload-arch={ARCH}",
        "-shared",
        "-fPIC",
        "-o",
        tmp,
        *objs,
        f"-L{os.path.join(ROCM, 'lib')}",
        "-lamdhip64",
        f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
    ]
    res = subprocess.run(link, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
