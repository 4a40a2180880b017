"""CPU tests of the .vlx model-source reader (velox_hip_vlx_config / _load / _mla_config): the
reference's example models yield the benchmark configurations' shapes, the planner's budget follows
the `target hardware` block as src/memory_planner.rs:372-488 computes it, and the reference's own
fallbacks (theta and eps by model name) apply where a file is silent."""
import ctypes as C
import math
import os

import pytest

from velox_amd import _lib as L

EXAMPLES = "/root/reference/examples"
GIB = 1024 ** 3


def _cfg(src: str, max_seq: int = 0):
    c, t = L.ModelConfig(), L.VlxTarget()
    rc = L.load().velox_hip_vlx_config(src.encode(), max_seq, C.byref(c), C.byref(t))
    return rc, c, t


def _file(name: str, max_seq: int = 0):
    c, t = L.ModelConfig(), L.VlxTarget()
    rc = L.load().velox_hip_vlx_load(os.path.join(EXAMPLES, name).encode(), max_seq, C.byref(c), C.byref(t))
    return rc, c, t


def _budget(vram: int, sf: float) -> int:
    reserve = 512 * 1024 ** 2 if vram >= 24 * GIB else (256 * 1024 ** 2 if vram >= 2 * GIB else vram // 32)
    return math.floor(vram * sf) - reserve


def _shape(c):
    return (c.vocab_size, c.hidden_dim, c.intermediate_dim, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim)


MINI = """
// a comment with model Fake<const X: usize = 1> inside it
target hardware {
    device: "amd_mi355x";
    vram_capacity: 2 * 144 * GB;   /* block comment */
    compute_capability: 9.5;
    safety_factor: 0.5;
}
model Tiny_Llama<
    const B_MAX: usize = 4, const S_MAX: usize = 0x400, const VOCAB: usize = 1_000,
    const HIDDEN_DIM: usize = 256, const INTERMEDIATE_DIM: usize = 4 * 128, const NUM_LAYERS: usize = 2,
    const NUM_HEADS: usize = 4, const NUM_KV_HEADS: usize = 2
> {
    @vram_immutable weight w_embed: Tensor<[VOCAB, HIDDEN_DIM], f16> = safetensors("x", "y");
    @vram_immutable weight w_lm_head: Tensor<[HIDDEN_DIM, VOCAB], f16> = safetensors("x", "z");
    scope decode<const B: usize>(t: Tensor<[B, 1], u32>, step: usize) -> Tensor<[B, 1], u32> {
        let n = rmsnorm(h, w_n[l], eps = 2.5e-6);
    }
}
"""


def test_reader_on_a_source_of_its_own():
    rc, c, t = _cfg(MINI)
    assert rc == 0
    assert c.name.decode() == "Tiny_Llama"
    assert _shape(c) == (1000, 256, 512, 2, 4, 2, 64)  # HEAD_DIM defaults to HIDDEN_DIM / NUM_HEADS
    assert c.max_seq_len == 1024 and c.qkv_bias == 0 and c.tied_lm_head == 0
    assert c.rope_theta == 500000.0  # "llama" in the name (src/codegen.rs:962-975)
    # eps by the model's name, as the reference's lowering sets it (src/ir.rs:549-553), not the
    # source's `eps = 2.5e-6`, which its emitted kernels do not receive either
    assert abs(c.rms_norm_eps - 1e-5) < 1e-12
    assert t.weights_file.decode() == "x"  # the first safetensors("x", ...) binding
    assert t.device.decode() == "amd_mi355x" and t.vram_capacity_bytes == 288 * 10 ** 9
    assert t.safe_budget_bytes == 144 * 10 ** 9 and t.b_max == 4 and t.s_max == 1024
    assert c.vram_budget_bytes == _budget(288 * 10 ** 9, 0.5)
    rc, c, _ = _cfg(MINI, 77)
    assert rc == 0 and c.max_seq_len == 77


@pytest.mark.parametrize("bad", [
    MINI.replace("/* block comment */", "/* unterminated"),
    MINI.replace("const NUM_LAYERS: usize = 2,", ""),          # a dimension missing
    MINI.replace("= 4 * 128", "= 4 * lots"),                     # unknown identifier in a constant
    MINI.replace("model Tiny_Llama<", "model <"),                # no model name
    "target hardware { device: \"x\"; }",                        # no model at all
])
def test_reader_rejects_malformed_sources(bad):
    assert _cfg(bad)[0] == L.EINVAL


@pytest.mark.parametrize("bad", [
    MINI.replace("const NUM_LAYERS: usize = 2,", "const NUM_LAYERS: usize = 0 - 2,"),     # negative
    MINI.replace("const NUM_LAYERS: usize = 2,", "const NUM_LAYERS: usize = 2.5,"),       # fractional
    MINI.replace("const B_MAX: usize = 4,", "const B_MAX: usize = 9000000000,"),           # past 2^32
    MINI.replace("const S_MAX: usize = 0x400,", "const S_MAX: usize = 0 - 1,"),
])
def test_reader_rejects_constants_out_of_range(bad):
    assert _cfg(bad)[0] == L.EINVAL


def test_eps_follows_the_model_name():
    for name, want in (("Qwen_Tiny", 1e-6), ("Tiny_K2", 1e-6), ("Horizon_X", 1e-6), ("Mistral_Tiny", 1e-5)):
        rc, c, _ = _cfg(MINI.replace("model Tiny_Llama<", f"model {name}<"))
        assert rc == 0 and abs(c.rms_norm_eps - want) < 1e-12, name


def test_missing_file_is_not_loaded():
    c = L.ModelConfig()
    assert L.load().velox_hip_vlx_load(b"/nonexistent/model.vlx", 0, C.byref(c), None) == L.ENOTLOADED


def test_builtins_are_vlx_sources_with_the_baseline_shapes():
    want = {
        "smollm_135m": ((49152, 576, 1536, 30, 9, 3, 64), 10000.0, 1e-5, 0, 1, 2048),
        "llama3_8b": ((128256, 4096, 14336, 32, 32, 8, 128), 500000.0, 1e-5, 0, 0, 8192),
        "qwen2_5_7b": ((152064, 3584, 18944, 28, 28, 4, 128), 1000000.0, 1e-6, 1, 1, 4096),
        "qwen2_72b": ((152064, 8192, 29568, 80, 64, 8, 128), 1000000.0, 1e-6, 1, 0, 8448),
    }
    for name, (shape, theta, eps, bias, tied, smax) in want.items():
        c = L.builtin_config(name)
        assert c.name.decode() == name and _shape(c) == shape
        assert c.rope_theta == theta and abs(c.rms_norm_eps - eps) < 1e-12
        assert (c.qkv_bias, c.tied_lm_head, c.max_seq_len) == (bias, tied, smax)
        assert c.vram_budget_bytes == _budget(288 * 10 ** 9, 1.0)


needs_ref = pytest.mark.skipif(not os.path.isdir(EXAMPLES), reason="reference examples absent")


@needs_ref
@pytest.mark.parametrize("name,shape,theta,eps,bias,tied,smax,vram", [
    # declares w_head = "lm_head.weight": a separate head as far as the source says (the reference ties
    # it only when the checkpoint lacks that tensor, src/runners/velox_cuda_runner.cu:132-135)
    ("tinystories_smollm.vlx", (49152, 576, 1536, 30, 9, 3, 64), 10000.0, 1e-5, 0, 0, 2048, 4096 * 1024 ** 2),
    ("llama3_8b.vlx", (128256, 4096, 14336, 32, 32, 8, 128), 500000.0, 1e-5, 0, 0, 4096, 80 * GIB),
    ("qwen2_5_7b.vlx", (152064, 3584, 18944, 28, 28, 4, 128), 1000000.0, 1e-6, 1, 1, 8192, 24 * GIB),
    ("qwen2_72b.vlx", (152064, 8192, 29568, 80, 64, 8, 128), 1000000.0, 1e-6, 1, 1, 8192, 640 * GIB),
])
def test_reference_examples_yield_baseline_shapes(name, shape, theta, eps, bias, tied, smax, vram):
    """BASELINE configurations 1, 2, 3 and 5 from the reference's own model sources."""
    rc, c, t = _file(name)
    assert rc == 0, name
    assert _shape(c) == shape and c.max_seq_len == smax
    assert c.rope_theta == theta and abs(c.rms_norm_eps - eps) < 1e-12
    assert (c.qkv_bias, c.tied_lm_head) == (bias, tied)
    assert t.vram_capacity_bytes == vram and abs(t.safety_factor - 0.95) < 1e-12
    assert c.vram_budget_bytes == _budget(vram, 0.95)


@needs_ref
def test_reference_mla_example_yields_config_4():
    c, t = L.MlaConfig(), L.VlxTarget()
    src = open(os.path.join(EXAMPLES, "deepseek_v3_mla.vlx")).read()
    assert L.load().velox_hip_vlx_mla_config(src.encode(), 4096 + 256, 16, C.byref(c), C.byref(t)) == 0
    assert (c.hidden_dim, c.num_heads, c.q_lora_rank, c.kv_lora_rank, c.qk_nope_dim, c.qk_rope_dim,
            c.v_head_dim) == (7168, 128, 1536, 512, 128, 64, 128)
    assert (c.num_layers, c.max_seq_len, c.max_batch, c.kv_norm) == (61, 4352, 16, 1)
    assert t.vram_capacity_bytes == 1280 * GIB and t.b_max == 32 and t.s_max == 8192
    # the dense reader refuses an MLA model
    assert _cfg(src)[0] == L.EINVAL


@needs_ref
def test_planner_refuses_a_plan_beyond_the_files_budget():
    """k2_horizon_3_7b.vlx targets a 4 GiB laptop GPU with S_MAX 524288: its bf16 KV cache alone is
    77 GB, so planning at the file's S_MAX fails as the reference's E002 does
    (src/memory_planner.rs:398-420); a short context fits."""
    rc, c, _ = _file("k2_horizon_3_7b.vlx")
    assert rc == 0 and c.max_seq_len == 524288 and c.rope_theta == 10000000.0 and abs(c.rms_norm_eps - 1e-6) < 1e-12
    m = C.c_void_p()
    assert L.load().velox_hip_model_create(C.byref(c), C.byref(m)) == L.ENOMEM
    rc, c, _ = _file("k2_horizon_3_7b.vlx", 256)
    assert rc == 0
    assert L.load().velox_hip_model_create(C.byref(c), C.byref(m)) == 0
    L.load().velox_hip_model_destroy(m)
