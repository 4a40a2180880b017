"""CPU tests of the C ABI library: it loads, exports every declared symbol, and its planner (pure
host code, no GPU needed) sizes the benchmark configurations by their published shapes."""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import make_config

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol(hiplib):
    names = L.header_exports()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(hiplib, n)]
    assert not missing, missing


def _plan(cfg):
    m = C.c_void_p()
    rc = L.load().velox_hip_model_create(C.byref(cfg), C.byref(m))
    return rc, m


def test_builtin_configs_match_baseline():
    c = L.builtin_config("llama3_8b")
    assert (c.vocab_size, c.hidden_dim, c.intermediate_dim, c.num_layers, c.num_heads, c.num_kv_heads,
            c.head_dim) == (128256, 4096, 14336, 32, 32, 8, 128)
    assert c.rope_theta == 500000.0 and abs(c.rms_norm_eps - 1e-5) < 1e-12 and c.tied_lm_head == 0
    q = L.builtin_config("qwen2_5_7b")
    assert (q.hidden_dim, q.intermediate_dim, q.num_layers, q.num_heads, q.num_kv_heads, q.vocab_size,
            q.qkv_bias, q.tied_lm_head) == (3584, 18944, 28, 28, 4, 152064, 1, 1)
    s = L.builtin_config("smollm_135m")
    assert (s.hidden_dim, s.num_layers, s.num_heads, s.num_kv_heads, s.head_dim, s.tied_lm_head) == (576, 30, 9, 3,
                                                                                                     64, 1)
    b = L.builtin_config("qwen2_72b")
    assert (b.hidden_dim, b.intermediate_dim, b.num_layers, b.num_heads, b.num_kv_heads) == (8192, 29568, 80, 64, 8)
    with pytest.raises(RuntimeError):
        L.builtin_config("no_such_model")


def test_step_bytes_match_baseline_llama():
    """Llama-3-8B Q4_0 algorithmic bytes per decode step: 4,221,370,368 weight bytes + 2,304
    embedding row + 1,064,960 norm bytes + 131,072*(pos+1) KV read + 131,072 KV write."""
    rc, m = _plan(make_config("llama3_8b", max_seq_len=385))
    assert rc == 0
    lib = L.load()
    for pos in (0, 128, 383):
        want = 4_221_370_368 + 2_304 + 1_064_960 + 131_072 * (pos + 1) + 131_072
        assert lib.velox_hip_model_step_bytes(m, pos) == want
    mean = np.mean([lib.velox_hip_model_step_bytes(m, p) for p in range(128, 384)])
    assert mean == 4_222_437_632 + 131_072 * 257.5  # = 4.256 GB over positions 128..383
    lib.velox_hip_model_destroy(m)


def test_arena_plan_sizes_and_budget():
    lib = L.load()
    rc, m = _plan(make_config("llama3_8b", max_seq_len=385))
    assert rc == 0
    v = [C.c_uint64() for _ in range(5)]
    lib.velox_hip_model_arena_bytes(m, *[C.byref(x) for x in v])
    codes, scales, norms, kv, act = [x.value for x in v]
    # codes + scales hold exactly 18 B per 32 weights of every matrix (embedding and head included)
    weights = (32 * (6144 * 4096 + 4096 * 4096 + 2 * 14336 * 4096 + 4096 * 14336) + 2 * 128256 * 4096)
    assert codes == weights // 2 and scales == weights // 32 * 2
    # bf16 K and V of every layer; the position capacity rounds up to whole 32-position V blocks
    assert kv == 32 * 2 * 8 * 416 * 128 * 2
    lib.velox_hip_model_destroy(m)
    # Qwen2-72B Q4_0 with an 8448-token context fits the 288 GB budget of one MI355X
    rc, m = _plan(make_config("qwen2_72b"))
    assert rc == 0
    lib.velox_hip_model_destroy(m)
    # ... and not a 40 GB budget: reference diagnostic E002 (src/memory_planner.rs:398-420)
    cfg = make_config("qwen2_72b")
    cfg.vram_budget_bytes = 40 * 10 ** 9
    rc, _ = _plan(cfg)
    assert rc == -2


def test_float_row_plan_sizes():
    """quant_mode 0 / 1: every matrix as fp32 / fp16 rows (gate and up as one 2F-row matrix), no
    scales; the single-sequence decode only."""
    lib = L.load()
    smollm = dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_layers=30, num_heads=9,
                  num_kv_heads=3, head_dim=64, max_seq_len=64, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0,
                  tied_lm_head=1)
    weights = 30 * ((576 + 2 * 192) * 576 + 576 * 576 + 2 * 1536 * 576 + 576 * 1536) + 49152 * 576
    for quant, elt in ((L.QUANT_F32, 4), (L.QUANT_F16, 2)):
        rc, m = _plan(make_config(dict(smollm, quant_mode=quant)))
        assert rc == 0
        v = [C.c_uint64() for _ in range(5)]
        lib.velox_hip_model_arena_bytes(m, *[C.byref(x) for x in v])
        assert v[1].value == 0
        # each matrix starts 256-aligned: at most 255 padding bytes per matrix
        assert weights * elt <= v[0].value < weights * elt + 256 * (4 * 30 + 1)
        assert lib.velox_hip_model_step_bytes(m, 0) >= weights * elt
        lib.velox_hip_model_destroy(m)
        for field, value in (("max_batch", 8), ("prefill_chunk", 16), ("intermediate_dim", 32768 + 32)):
            rc, _ = _plan(make_config(dict(smollm, quant_mode=quant, **{field: value})))
            assert rc == -1, field


def test_group64_plan_sizes():
    """quant_mode 2 (the reference's group-64 format): the tiled layout of GGML Q4_0, the same bytes
    per weight (16-byte codes and a 16-bit slot per 32 weights); single-sequence decode only, and
    whole 64-weight groups along every row."""
    lib = L.load()
    base = make_config("smollm_135m", max_seq_len=64)
    sizes = {}
    for quant in (L.QUANT_GGML_Q4_0, L.QUANT_G64):
        cfg = make_config("smollm_135m", max_seq_len=64)
        cfg.quant_mode = quant
        rc, m = _plan(cfg)
        assert rc == 0
        v = [C.c_uint64() for _ in range(5)]
        lib.velox_hip_model_arena_bytes(m, *[C.byref(x) for x in v])
        sizes[quant] = (v[0].value, v[1].value, lib.velox_hip_model_step_bytes(m, 0))
        lib.velox_hip_model_destroy(m)
    assert sizes[L.QUANT_GGML_Q4_0] == sizes[L.QUANT_G64]
    for field, value in (("max_batch", 8), ("prefill_chunk", 16), ("intermediate_dim", 1568)):
        cfg = make_config("smollm_135m", max_seq_len=64)
        cfg.quant_mode = L.QUANT_G64
        setattr(cfg, field, value)
        rc, _ = _plan(cfg)
        assert rc == -1, field
    assert base.quant_mode == L.QUANT_GGML_Q4_0


@pytest.mark.parametrize("field,value", [("head_dim", 96), ("num_kv_heads", 5), ("hidden_dim", 4100),
                                         ("quant_mode", 3), ("num_layers", 0)])
def test_plan_rejects_unsupported_shapes(field, value):
    cfg = make_config("llama3_8b", max_seq_len=64)
    setattr(cfg, field, value)
    rc, _ = _plan(cfg)
    assert rc == -1


def test_attention_split_choices():
    """The planner's split-K count over the sequence: up to 1024 positions a power of two >= 2 of
    up to 256 positions (merged in the o_proj prologue); beyond, 8 splits up to 3072 positions (o_proj
    still merges them), then 256-position splits, or 256 / KV heads longer ones when
    splits x KV heads would exceed 256 workgroups (two rounds of the one-workgroup-per-CU attention
    kernel), as long as no split exceeds 512 positions."""
    lib = L.load()
    cases = [("llama3_8b", 130, 2), ("llama3_8b", 385, 2), ("llama3_8b", 512, 2), ("llama3_8b", 513, 4),
             ("llama3_8b", 1024, 4), ("llama3_8b", 1025, 8), ("qwen2_5_7b", 1535, 8), ("qwen2_5_7b", 2080, 8), ("qwen2_5_7b", 2304, 8),
             ("qwen2_5_7b", 3072, 8), ("qwen2_5_7b", 3073, 13), ("llama3_8b", 2048, 8), ("qwen2_72b", 8216, 32), ("qwen2_72b", 8192, 32),
             ("llama3_8b", 20000, 64)]
    for name, max_seq, want in cases:
        cfg = L.builtin_config(name, max_seq)
        rc, m = _plan(cfg)
        assert rc == 0, (name, max_seq, rc)
        out = L.ModelConfig()
        assert lib.velox_hip_model_config(m, C.byref(out)) == 0
        lib.velox_hip_model_destroy(m)
        assert out.attn_splits == want, (name, max_seq, out.attn_splits)
    cfg = L.builtin_config("llama3_8b", 385)
    cfg.attn_splits = 3  # an explicit count is kept
    rc, m = _plan(cfg)
    out = L.ModelConfig()
    assert rc == 0 and lib.velox_hip_model_config(m, C.byref(out)) == 0 and out.attn_splits == 3
    lib.velox_hip_model_destroy(m)


def test_tiled_layout_choices():
    """Lanes per row for the benchmark shapes: the largest S padding a row by at most 1/32 of its
    blocks (padded blocks are streamed, so padding costs bandwidth), else the least padding."""
    lib = L.load()
    expect = {(6144, 4096): 32, (4096, 14336): 32, (960, 576): 4, (576, 1536): 16,
              (3584, 18944): 32, (8192, 29568): 32, (1000, 64): 4, (4096, 3584): 16}
    for (n, k), s in expect.items():
        m = L.Q4Matrix()
        cb, sb = C.c_uint64(), C.c_uint64()
        assert lib.velox_hip_q4_layout(n, k, 0, 0, C.byref(m), C.byref(cb), C.byref(sb)) == 0
        assert m.s_lanes == s, (n, k, m.s_lanes)
        assert m.n_iter * m.s_lanes >= k // 32 and (m.n_iter - 1) * m.s_lanes < k // 32
        assert cb.value == m.n_tiles * m.n_iter * 64 * 16 and sb.value == m.n_tiles * m.n_iter * 64 * 2
    m = L.Q4Matrix()
    assert lib.velox_hip_q4_layout(10, 33, 0, 0, C.byref(m), None, None) == -1
    assert lib.velox_hip_q4_layout(10, 64, 64, 1, C.byref(m), None, None) == -1


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_runner_rejects_unsupported_arguments():
    runner = os.path.join(ROOT, "velox_amd", "lib", "velox_hip_runner")
    # a checkpoint that is not there ends the run with the reference runner's message
    # (velox_cuda_runner.cu:391-394)
    r = subprocess.run([runner, "--weights", "/nonexistent/x.safetensors"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 1 and "failed to open weights file" in r.stderr
    r = subprocess.run([runner, "--bogus"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1
    # argv of src/cli.rs:653-675: token lists are parsed strictly; speculative flags are refused
    r = subprocess.run([runner, "--weights", "synthetic", "--tokens", "1,x,3"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 1 and "bad token id 'x'" in r.stderr
    r = subprocess.run([runner, "--speculative"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "not supported" in r.stderr


def test_arena_struct_is_the_reference_layout():
    """VeloxHipArena is VeloxCudaArena (src/codegen.rs:1032-1041): six pointers then quant_mode and
    tied_lm_head, nothing after them, in the header and in the Python mirror."""
    import re

    want = ["weight_arena", "kv_cache_pool", "activation_arena", "host_pinned_ring", "norm_weight_arena",
            "weight_scales", "quant_mode", "tied_lm_head"]
    assert [f for f, _ in L.Arena._fields_] == want
    assert C.sizeof(L.Arena) == 6 * 8 + 2 * 4
    assert [getattr(L.Arena, f).offset for f in want] == [0, 8, 16, 24, 32, 40, 48, 52]
    hdr = open(L.HEADER).read()
    body = re.search(r"typedef struct VeloxHipArena \{(.*?)\} VeloxHipArena;", hdr, re.S).group(1)
    assert re.findall(r"(\w+);", body) == want
