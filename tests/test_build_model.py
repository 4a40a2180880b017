"""`velox build model.vlx` on the CPU: velox_amd.build --model generates velox_<Model>.cpp from a
.vlx source and compiles the module (the four named entry points plus the baked configuration) and
the runner, as the reference's build emits velox_<Model>_{decode,prefill}{_graph_step,}_cuda
(src/codegen.rs:2803-2808, 3243-3253) and builds its runner (src/cli.rs:1367-1388). No GPU call."""
import ctypes as C
import os
import subprocess

import pytest

from velox_amd import _lib as L
from velox_amd import build as B

HERE = os.path.dirname(os.path.abspath(__file__))
EXAMPLES = "/root/reference/examples"

TINY = """
target hardware { device: "amd_mi355x"; vram_capacity: 288 * GB; safety_factor: 0.9; }
model Tiny_Mistral<const B_MAX: usize = 2, const S_MAX: usize = 512, const VOCAB: usize = 49152,
    const HIDDEN_DIM: usize = 576, const INTERMEDIATE_DIM: usize = 1536, const NUM_LAYERS: usize = 2,
    const NUM_HEADS: usize = 9, const NUM_KV_HEADS: usize = 3, const HEAD_DIM: usize = 64> {
    @vram_immutable weight w_embed: Tensor<[VOCAB, HIDDEN_DIM], f32> = safetensors("tiny.safetensors", "e");
    scope decode<const B: usize>(t: Tensor<[B, 1], u32>, step: usize) -> Tensor<[B, 1], u32> {
        let x = rmsnorm(h, w_attn_norm[l], eps = 1e-5);
    }
}
"""

TINY_MLA = """
model Tiny_MLA<const B_MAX: usize = 2, const S_MAX: usize = 256, const HIDDEN_DIM: usize = 1024,
    const NUM_HEADS: usize = 64, const NUM_LAYERS: usize = 2, const LATENT_KV_DIM: usize = 512,
    const Q_LATENT_DIM: usize = 512, const ROPE_DIM: usize = 64, const HEAD_DIM: usize = 128> {
    @vram_immutable weight w_dkv: Tensor<[NUM_LAYERS, HIDDEN_DIM, 576], f8> = safetensors("m.safetensors", "kv");
}
"""

ENTRY = ["decode_graph_step_hip", "decode_hip", "prefill_graph_step_hip", "prefill_hip"]


def _exports(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_build_from_a_renamed_source(tmp_path):
    src = tmp_path / "tiny.vlx"
    src.write_text(TINY)
    res = B.build_model(str(src), str(tmp_path / "out"))
    assert res["name"] == "Tiny_Mistral" and not res["mla"]
    syms = _exports(res["library"])
    assert {f"velox_Tiny_Mistral_{e}" for e in ENTRY} | {"velox_Tiny_Mistral_model_config"} <= syms
    assert not any(s.startswith("velox_hip_") for s in syms)  # the module holds the model's names only
    # the baked configuration is what the library's .vlx reader reads from the source
    mod = C.CDLL(res["library"])
    got = L.ModelConfig()
    assert mod.velox_Tiny_Mistral_model_config(C.byref(got)) == 0
    want = L.ModelConfig()
    assert L.load().velox_hip_vlx_load(str(src).encode(), 0, C.byref(want), None) == 0
    for f, _ in L.ModelConfig._fields_:
        assert getattr(got, f) == getattr(want, f), f
    assert got.name == b"Tiny_Mistral" and got.num_layers == 2 and got.max_seq_len == 512
    # the runner is bound to its model: it takes the reference runner's argv but no other model
    r = subprocess.run([res["runner"], "--model", "llama3_8b"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "built for model Tiny_Mistral" in r.stderr
    r = subprocess.run([res["runner"], "--weights", str(tmp_path / "absent.safetensors"), "--tokens", "1,2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "failed to open weights file" in r.stderr


def test_build_an_mla_model_source(tmp_path):
    src = tmp_path / "mla.vlx"
    src.write_text(TINY_MLA)
    res = B.build_model(str(src), str(tmp_path / "out"))
    assert res["name"] == "Tiny_MLA" and res["mla"] and "runner" not in res
    syms = _exports(res["library"])
    assert {f"velox_Tiny_MLA_{e}" for e in ENTRY} | {"velox_Tiny_MLA_mla_config"} <= syms
    got = L.MlaConfig()
    assert C.CDLL(res["library"]).velox_Tiny_MLA_mla_config(C.byref(got)) == 0
    assert (got.hidden_dim, got.num_heads, got.q_lora_rank, got.kv_lora_rank, got.qk_nope_dim, got.qk_rope_dim,
            got.v_head_dim, got.num_layers, got.max_seq_len, got.max_batch) == (1024, 64, 512, 512, 128, 64, 128, 2,
                                                                                 256, 2)


def test_malformed_source_is_refused(tmp_path):
    src = tmp_path / "bad.vlx"
    src.write_text(TINY.replace("const NUM_LAYERS: usize = 2,", ""))
    with pytest.raises(RuntimeError):
        B.build_model(str(src), str(tmp_path / "out"))


@pytest.mark.skipif(not os.path.isdir(EXAMPLES), reason="reference examples absent")
@pytest.mark.parametrize("example,name", [("mistral_7b.vlx", "Mistral_7B"), ("llama3_8b.vlx", "Llama3_8B"),
                                          ("deepseek_v3_mla.vlx", "DeepSeek_V3_MLA")])
def test_build_the_reference_examples(tmp_path, example, name):
    """Every model the reference's own sources declare gets its named symbols (Mistral-7B has no
    builtin configuration here)."""
    res = B.build_model(os.path.join(EXAMPLES, example), str(tmp_path / name), runner=False)
    assert res["name"] == name
    assert {f"velox_{name}_{e}" for e in ENTRY} <= _exports(res["library"])
