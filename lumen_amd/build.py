"""Builds the engine in-tree.

  lumen_amd/lib/lumen_sampler_gfx950.hsaco   gfx950 code object (hipcc --genco)
  lumen_amd/lib/liblumen_sampler.so           C-ABI host library with the code
                                              object embedded (.incbin)

Run `python -m lumen_amd.build` (or __graft_entry__.build()).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
ROOT = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HSACO = os.path.join(LIB, "lumen_sampler_gfx950.hsaco")
SO = os.path.join(LIB, "liblumen_sampler.so")

# Device flags: gfx950 only; every f32 operation stays a single IEEE operation
# (no contraction into FMA), f32 denormals are kept (as on the x86 host the
# reference runs on), no packed-FP32 instructions, SGPR spills kept in VGPRs.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "--offload-device-only", "--no-gpu-bundle-output", "-O3",
    "-std=c++17",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # SGPR spills go to VGPR lanes reserved up front, so the lane-holding VGPR
    # is never itself spilled to scratch (whose reloads wait on every vector
    # memory load in flight): -3 us on the mixed config-3 batch
    "-mllvm", "--amdgpu-prealloc-sgpr-spill-vgprs",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout)
        raise RuntimeError("build step failed: " + " ".join(cmd))
    return r.stdout


def build(verbose: bool = False) -> str:
    os.makedirs(LIB, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(hipcc):
        hipcc = shutil.which("hipcc") or hipcc
    tmp_hsaco = HSACO + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, "-o", tmp_hsaco, os.path.join(CSRC, "sampler_kernels.hip")])
    os.replace(tmp_hsaco, HSACO)
    obj = os.path.join(LIB, "code_object.o")
    _run(["gcc", "-c", f'-DLUMEN_HSACO_PATH="{HSACO}"', "-o", obj,
          os.path.join(CSRC, "code_object.S")])
    # the no-allocation entry point's device array lives in a HIP source of
    # the host library (its own gfx950 device code, registered by HIP)
    na_obj = os.path.join(LIB, "noalloc.o")
    _run([hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-c",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-o", na_obj, os.path.join(CSRC, "noalloc.hip")])
    tmp_so = SO + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{ROOT}/include",
          "-o", tmp_so, os.path.join(CSRC, "sampler_host.cpp"), obj, na_obj,
          f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp_so, SO)
    os.remove(obj)
    os.remove(na_obj)
    if verbose:
        print("built", SO)
    return SO


if __name__ == "__main__":
    build(verbose=True)
