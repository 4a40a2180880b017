"""Builds the gfx950 HIP library and the runner in-tree (velox_amd/lib/).

    python -m velox_amd.build        # or: from velox_amd.build import build; build()

hipcc cross-compiles for gfx950 without a GPU. Every HIP translation unit is built with
packed-FP32 instruction selection disabled (-packed-fp32-ops): the hardware's v_pk_*_f32 forms
are avoided on purpose.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libvelox_hip.so")
RUNNER = os.path.join(LIBDIR, "velox_hip_runner")
ARCH = "gfx950"

HIP_SOURCES = ["vx_kernels.hip", "vx_gemv_g64.hip", "vx_gemv_f.hip", "vx_batch.hip", "vx_mgemm.hip", "vx_mla.hip", "vx_noalloc.hip", "vx_host.cpp", "vx_mla_host.cpp", "vx_gguf.cpp", "vx_safetensors.cpp", "vx_vlx.cpp"]


def _hipcc() -> str:
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc") or ""):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP backend cannot be built")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function", "-Wno-unused-value",
        f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
    ]


# Per-file code generation flags. The batched Q4_0 GEMM and the fp8 GEMMs of the MLA layer keep MFMA
# results in VGPRs: their scale FMAs read every MFMA result, and the AGPR form cost four
# v_accvgpr_read per MFMA (a quarter of the Q4_0 GEMM's loop, a fifth of the fp8 GEMM's).
_VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
FILE_FLAGS = {"vx_mgemm.hip": _VGPR_MFMA, "vx_mla.hip": _VGPR_MFMA}


def build(verbose: bool = False) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    hipcc = _hipcc()
    tmp = LIB + ".tmp"
    with tempfile.TemporaryDirectory(prefix="velox_hip_build_") as objdir:
        cmds, objs = [], []
        for s in HIP_SOURCES:
            obj = os.path.join(objdir, s + ".o")
            objs.append(obj)
            cmds.append([hipcc, *common_flags(), *FILE_FLAGS.get(s, []), "-c", "-o", obj, os.path.join(CSRC, s)])
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(cmds))) as pool:
            for cmd in cmds:
                if verbose:
                    print(" ".join(cmd), flush=True)
            for r in pool.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds):
                if r.stderr:
                    sys.stderr.write(r.stderr)
                if r.returncode != 0:
                    raise subprocess.CalledProcessError(r.returncode, r.args, r.stdout, r.stderr)
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    runner_src = os.path.join(CSRC, "vx_runner_main.cpp")
    if os.path.exists(runner_src):
        cmd = [hipcc, *common_flags(), "-o", RUNNER + ".tmp", runner_src, f"-L{LIBDIR}", "-lvelox_hip",
               f"-Wl,-rpath,$ORIGIN"]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(RUNNER + ".tmp", RUNNER)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
