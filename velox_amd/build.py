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

HIP_SOURCES = ["vx_kernels.hip", "vx_gemv_g64.hip", "vx_gemv_f.hip", "vx_batch.hip", "vx_mgemm.hip", "vx_mla.hip", "vx_noalloc.hip", "vx_qkv_attn.hip", "vx_host.cpp", "vx_mla_host.cpp", "vx_gguf.cpp", "vx_safetensors.cpp", "vx_vlx.cpp", "vx_runner.cpp"]


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


def _compile_library(lib: str, extra: list[str], verbose: bool) -> None:
    """Every HIP_SOURCES unit (common flags + extra) linked into the shared library `lib`."""
    os.makedirs(os.path.dirname(lib), exist_ok=True)
    hipcc = _hipcc()
    tmp = lib + ".tmp"
    with tempfile.TemporaryDirectory(prefix="velox_hip_build_") as objdir:
        cmds, objs = [], []
        for s in HIP_SOURCES:
            obj = os.path.join(objdir, s + ".o")
            objs.append(obj)
            cmds.append([hipcc, *common_flags(), *extra, *FILE_FLAGS.get(s, []), "-c", "-o", obj, os.path.join(CSRC, s)])
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
    os.replace(tmp, lib)


def _link_program(src: str, exe: str, extra: list[str], verbose: bool) -> None:
    """A program on the library beside it (rpath $ORIGIN)."""
    cmd = [_hipcc(), *common_flags(), *extra, "-o", exe + ".tmp", src, f"-L{os.path.dirname(exe)}", "-lvelox_hip",
           "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(exe + ".tmp", exe)


def build(verbose: bool = False) -> str:
    _compile_library(LIB, [], verbose)
    runner_src = os.path.join(CSRC, "vx_runner_main.cpp")
    if os.path.exists(runner_src):
        _link_program(runner_src, RUNNER, [], verbose)
    return LIB


TIMELINE_DIR = os.path.join(LIBDIR, "timeline")


def build_timeline(verbose: bool = False) -> str:
    """The timeline build (-DVX_TIMELINE) of the library and its velox_hip_timeline program under
    velox_amd/lib/timeline/: the single-sequence decode step's GEMV and attention workgroups stamp
    s_memrealtime at their start, staging / first barrier and end. A measuring tool only: the
    product library (build()) holds no stamps. Returns the program's path."""
    lib = os.path.join(TIMELINE_DIR, "libvelox_hip.so")
    _compile_library(lib, ["-DVX_TIMELINE"], verbose)
    exe = os.path.join(TIMELINE_DIR, "velox_hip_timeline")
    _link_program(os.path.join(CSRC, "vx_timeline_main.cpp"), exe, ["-DVX_TIMELINE"], verbose)
    return exe


# ---------------------------------------------------------------------------------------------
# `velox build model.vlx`: the per-model module and runner
# ---------------------------------------------------------------------------------------------
# The reference's `velox build` compiles a .vlx source into an emitted module whose extern "C" entry
# points are named for the model (velox_<Model>_{decode,prefill}{_graph_step,}_cuda,
# src/codegen.rs:2803-2808, 3243-3253) with its constants baked in (src/codegen.rs:936-1102), and
# builds a runner around it (src/cli.rs:1367-1388). Here the kernels are generic over the model, so
# the generated translation unit holds the model's configuration as read from the source and the
# four named entry points, each checking the arena's plan against that configuration before it runs
# the library's step; the runner is the library's runner program bound to that model and step.

_DENSE_TEMPLATE = """// {file} -- generated by `python -m velox_amd.build --model {src}`; do not edit.
// Model {name}: the emitted-runner ABI (velox_<Model>_{{decode,prefill}}{{_graph_step,}}_hip) of the
// MI355X decode backend (libvelox_hip.so), with the model's configuration baked in.
#include "velox_hip.h"

static const VeloxHipModelConfig kModel = {{
    "{name}", {vocab_size}u, {hidden_dim}u, {intermediate_dim}u, {num_layers}u, {num_heads}u, {num_kv_heads}u,
    {head_dim}u, {max_seq_len}u, {rms_norm_eps!r}f, {rope_theta!r}f, {qkv_bias}u, {tied_lm_head}u,
    {quant_mode}u, 0u, {vram_budget_bytes}ull, 0u, 0u}};

static int vx_is_model(const VeloxHipArena* ctx) {{
    if (velox_hip_arena_check(ctx, &kModel) == VELOX_HIP_OK) return 1;
    velox_hip_record_error(VELOX_HIP_EINVAL);
    return 0;
}}

extern "C" {{
int velox_{name}_model_config(VeloxHipModelConfig* out) {{
    if (!out) return VELOX_HIP_EINVAL;
    *out = kModel;
    return VELOX_HIP_OK;
}}
void velox_{name}_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_decode_graph_step(ctx, active_mask, stream);
}}
void velox_{name}_decode_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                             hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_decode(ctx, token_in, step, active_mask, stream);
}}
void velox_{name}_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_prefill_graph_step(ctx, active_mask, stream);
}}
void velox_{name}_prefill_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                              hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_prefill(ctx, token_in, step, active_mask, stream);
}}
}}  // extern "C"

#ifdef VELOX_BUILD_RUNNER
int main(int argc, char** argv) {{
    return velox_hip_runner_main(argc, argv, &kModel, velox_{name}_decode_graph_step_hip);
}}
#endif
"""

_MLA_TEMPLATE = """// {file} -- generated by `python -m velox_amd.build --model {src}`; do not edit.
// Model {name}: the absorbed-MLA attention stack under the emitted-runner ABI
// (velox_<Model>_{{decode,prefill}}{{_graph_step,}}_hip over an MLA arena, velox_hip_mla_arena) of the
// MI355X decode backend (libvelox_hip.so), with the model's configuration baked in.
#include "velox_hip.h"

static const VeloxHipMlaConfig kModel = {{
    {hidden_dim}u, {num_heads}u, {q_lora_rank}u, {kv_lora_rank}u, {qk_nope_dim}u, {qk_rope_dim}u, {v_head_dim}u,
    {num_layers}u, {max_seq_len}u, {max_batch}u, {kv_norm}u, 0u, {rms_norm_eps!r}f, {rope_theta!r}f,
    {softmax_scale!r}f, 0u, {vram_budget_bytes}ull}};

static int vx_is_model(const VeloxHipArena* ctx) {{
    if (velox_hip_mla_arena_check(ctx, &kModel) == VELOX_HIP_OK) return 1;
    velox_hip_record_error(VELOX_HIP_EINVAL);
    return 0;
}}

extern "C" {{
int velox_{name}_mla_config(VeloxHipMlaConfig* out) {{
    if (!out) return VELOX_HIP_EINVAL;
    *out = kModel;
    return VELOX_HIP_OK;
}}
void velox_{name}_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_mla_graph_step(ctx, active_mask, stream);
}}
void velox_{name}_decode_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                             hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_mla_decode(ctx, token_in, step, active_mask, stream);
}}
void velox_{name}_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_mla_graph_step(ctx, active_mask, stream);
}}
void velox_{name}_prefill_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                              hipStream_t stream) {{
    if (vx_is_model(ctx)) velox_hip_mla_decode(ctx, token_in, step, active_mask, stream);
}}
}}  // extern "C"
"""


def _fields(struct) -> dict:
    return {f: getattr(struct, f) for f, _ in struct._fields_}


def generate_model_source(vlx_path: str, max_seq_len: int = 0) -> tuple[str, str, bool]:
    """(model name, generated C++ source, is_mla) for a .vlx model source, read by the library's
    .vlx reader (dense models: velox_hip_vlx_load; MLA models, LATENT_KV_DIM: velox_hip_vlx_mla_config)."""
    import ctypes as C

    from . import _lib as L

    lib = L.load()
    cfg, tgt = L.ModelConfig(), L.VlxTarget()
    rc = lib.velox_hip_vlx_load(vlx_path.encode(), max_seq_len, C.byref(cfg), C.byref(tgt))
    src_name = os.path.basename(vlx_path)
    if rc == 0:
        d = _fields(cfg)
        name = cfg.name.decode()
        text = _DENSE_TEMPLATE.format(file=f"velox_{name}.cpp", src=src_name, **dict(d, name=name))
        return name, text, False
    with open(vlx_path) as f:
        source = f.read()
    mla = L.MlaConfig()
    rc2 = lib.velox_hip_vlx_mla_config(source.encode(), max_seq_len, 0, C.byref(mla), C.byref(tgt))
    if rc2 != 0:
        raise RuntimeError(f"{vlx_path}: not a model source this backend reads (status {rc} / {rc2})")
    import re

    m = re.search(r"\bmodel\s+([A-Za-z_][A-Za-z0-9_]*)\s*<", source)
    name = m.group(1)
    text = _MLA_TEMPLATE.format(file=f"velox_{name}.cpp", src=src_name, name=name, **_fields(mla))
    return name, text, True


def build_model(vlx_path: str, out_dir: str | None = None, max_seq_len: int = 0, runner: bool = True,
                verbose: bool = False) -> dict:
    """Generates velox_<Model>.cpp from a .vlx source and compiles it against libvelox_hip.so into
    libvelox_<Model>.so (the named entry points) and, for decoder models, velox_<Model>_runner (the
    reference runner's argv and report, bound to the model). Returns the paths."""
    if not os.path.exists(LIB):
        build(verbose)
    name, text, is_mla = generate_model_source(vlx_path, max_seq_len)
    out_dir = os.path.abspath(out_dir or os.path.join(LIBDIR, "models", name))
    os.makedirs(out_dir, exist_ok=True)
    src = os.path.join(out_dir, f"velox_{name}.cpp")
    with open(src, "w") as f:
        f.write(text)
    hipcc = _hipcc()
    rpath = ["-Wl,-rpath," + os.path.join("$ORIGIN", os.path.relpath(LIBDIR, out_dir)), f"-Wl,-rpath,{LIBDIR}"]
    base = [hipcc, "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{os.path.join(ROOT, 'include')}"]
    out = {"name": name, "source": src, "mla": is_mla}
    lib = os.path.join(out_dir, f"libvelox_{name}.so")
    cmd = [*base, "-shared", "-o", lib, src, f"-L{LIBDIR}", "-lvelox_hip", *rpath]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    out["library"] = lib
    if runner and not is_mla:  # the MLA stack emits no token: a module only
        exe = os.path.join(out_dir, f"velox_{name}_runner")
        cmd = [*base, "-DVELOX_BUILD_RUNNER", "-o", exe, src, f"-L{LIBDIR}", "-lvelox_hip", *rpath]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        out["runner"] = exe
    return out


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="Build the HIP library, or (--model) a model's module and runner.")
    ap.add_argument("--model", help=".vlx model source: generate and build velox_<Model>.cpp")
    ap.add_argument("--out", help="output directory (default velox_amd/lib/models/<Model>)")
    ap.add_argument("--max-seq-len", type=int, default=0)
    ap.add_argument("--no-runner", action="store_true")
    ap.add_argument("--timeline", action="store_true",
                    help="build the timeline build and velox_hip_timeline under velox_amd/lib/timeline/")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    if args.timeline:
        print(build_timeline(verbose=args.verbose))
    elif args.model:
        res = build_model(args.model, args.out, args.max_seq_len, not args.no_runner, args.verbose)
        for k in ("library", "runner"):
            if k in res:
                print(res[k])
    else:
        build(verbose=args.verbose)
        print(LIB)
