"""End-to-end decode parity: the HIP decode step (C ABI, eager and hipGraph) vs the CPU oracle.

Teacher forcing: both paths consume the same token sequence, so one argmax
flip on a near-tie cannot desynchronise the comparison. Bars: logits max-abs <= 2e-2 against
the oracle with bf16 KV (the bf16 parity bar), and the
GPU argmax equal to the exact argmax of the GPU's own logits.
"""
import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import HipDecodeEngine, run

from test_gpu_kernels import kv_from_device

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2

SMOLLM = dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_layers=30, num_heads=9, num_kv_heads=3,
              head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
LLAMA = dict(vocab_size=128256, hidden_dim=4096, intermediate_dim=14336, num_layers=32, num_heads=32, num_kv_heads=8,
             head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, qkv_bias=0, tied_lm_head=0)
QWEN7 = dict(vocab_size=152064, hidden_dim=3584, intermediate_dim=18944, num_layers=28, num_heads=28, num_kv_heads=4,
             head_dim=128, rms_norm_eps=1e-6, rope_theta=1000000.0, qkv_bias=1, tied_lm_head=1)


def _compare(oracle, name, cfg, layers, max_seq, n_steps, seed, norm_sigma, threads=8, attn_splits=0):
    ocfg = dict(cfg, num_layers=layers, max_seq_len=max_seq)
    ref = oracle.Engine(ocfg, seed=seed, sigma=0.02, norm_sigma=norm_sigma, q4_0=True, kv_bf16=True,
                        threads=threads)
    gpu = HipDecodeEngine(name, seed=seed, sigma=0.02, norm_sigma=norm_sigma, max_seq_len=max_seq,
                          num_layers=layers, attn_splits=attn_splits)
    toks = list(oracle.prompt_tokens(seed, n_steps, cfg["vocab_size"]))
    worst = 0.0
    for pos, tok in enumerate(toks):
        t_ref = ref.forward(int(tok), pos)
        t_gpu = gpu.forward_step(int(tok), pos)
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        worst = max(worst, d)
        print(f"[{name}] pos={pos} tok={tok} gpu={t_gpu} ref={t_ref} maxabs={d:.3e}", flush=True)
        assert t_gpu == oracle.argmax(gpu.logits)
        srt = np.sort(ref.logits)
        if srt[-1] - srt[-2] > 2 * LOGIT_TOL:
            assert t_gpu == t_ref
        assert d < LOGIT_TOL, (pos, d)
    gpu.close()
    ref.close()
    return worst


def test_decode_smollm_q4_vs_oracle(oracle):
    _compare(oracle, "smollm_135m", SMOLLM, 30, 48, 12, seed=11, norm_sigma=0.1)


def test_decode_llama_shapes_2_layers_vs_oracle(oracle):
    _compare(oracle, "llama3_8b", LLAMA, 2, 32, 4, seed=12, norm_sigma=0.1, threads=16)


def test_decode_qwen_bias_tied_2_layers_vs_oracle(oracle):
    _compare(oracle, "qwen2_5_7b", QWEN7, 2, 24, 3, seed=13, norm_sigma=0.1, threads=16)


@pytest.mark.parametrize("splits", [2, 8, 3])
def test_decode_split_k_attention_vs_oracle(oracle, splits):
    """Split-K attention over the sequence: 2 and 8 splits are merged in the o_proj GEMV prologue,
    3 splits by the separate LSE merge kernel; 20 positions leave some splits empty early on."""
    _compare(oracle, "smollm_135m", SMOLLM, 4, 24, 20, seed=17, norm_sigma=0.1, attn_splits=splits)


def test_graph_replay_matches_eager(oracle):
    """hipGraph replays (device-driven state, teacher-forced prompt) == eager per-step calls."""
    seed, P, n = 21, 6, 10
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, 49152)]
    eager = HipDecodeEngine("smollm_135m", seed=seed, max_seq_len=32, num_layers=4)
    want = eager.generate_greedy_into(prompt, n)
    eager.close()
    rep, toks = run("smollm_135m", prompt_len=P, warmup=2, steps=n - 3, seed=seed, num_layers=4, max_seq_len=32)
    assert rep["status"] == 0
    # ring[p] = argmax after position p; generated tokens are ring[P-1 ...]
    assert toks[P - 1:P - 1 + n] == want
    assert rep["first_token"] == want[0]


def test_state_advances_and_ring(oracle):
    g = HipDecodeEngine("smollm_135m", seed=3, max_seq_len=16, num_layers=2)
    g.set_prompt([5, 6, 7])
    g.set_state(0, 5)
    for _ in range(5):
        g.graph_step()
    g.sync()
    step, tok = g.state()
    assert step == 5
    assert tok == g.ring(4)
    g.close()


def test_active_mask_predication(oracle):
    g = HipDecodeEngine("smollm_135m", seed=3, max_seq_len=16, num_layers=2)
    g.set_state(0, 5)
    g.lib.velox_hip_decode_graph_step(__import__("ctypes").byref(g.arena), 0, None)  # bit 0 clear: no-op
    g.sync()
    assert g.state() == (0, 5)
    g.close()


def test_run_with_explicit_prompt_tokens(oracle):
    """velox_hip_run with explicit ids (the runner's --tokens) equals the seeded-prompt run when the
    ids are the seeded ones, and refuses an id outside the vocabulary."""
    seed, P = 23, 5
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, 49152)]
    rep_a, toks_a = run("smollm_135m", prompt_len=P, warmup=0, steps=4, seed=seed, num_layers=3, max_seq_len=16)
    rep_b, toks_b = run("smollm_135m", prompt=prompt, warmup=0, steps=4, seed=seed, num_layers=3, max_seq_len=16)
    assert rep_a["status"] == rep_b["status"] == 0 and toks_a == toks_b
    with pytest.raises(RuntimeError):
        run("smollm_135m", prompt=[1, 49152], warmup=0, steps=1, seed=seed, num_layers=1, max_seq_len=8)


def test_runner_binary_stdout_contract(oracle):
    """velox_hip_runner as src/cli.rs:640-770 spawns it: --weights/--tokens/--steps/--verbose, one
    "[Step N] Token: id" line per generated token (parsed at src/cli.rs:706-733) and the report
    block; the tokens equal the library's own greedy decode of the same prompt."""
    import os
    import re
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    runner = os.path.join(root, "velox_amd", "lib", "velox_hip_runner")
    prompt = [int(t) for t in oracle.prompt_tokens(31, 5, 49152)]
    r = subprocess.run([runner, "--model", "smollm_135m", "--weights", "synthetic", "--tokens",
                        ",".join(map(str, prompt)), "--steps", "6", "--seed", "31", "--verbose"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    steps = re.findall(r"^\[Step (\d+)\] Token: (\d+)$", r.stdout, re.M)
    assert [int(s) for s, _ in steps] == list(range(6))
    assert re.search(r"Decode Latency \(\d+ tok\): [\d.]+ ms \([\d.]+ tok/s", r.stdout)
    _, toks = run("smollm_135m", prompt=prompt, warmup=0, steps=5, seed=31)
    assert [int(t) for _, t in steps] == toks[len(prompt) - 1:len(prompt) - 1 + 6]


LONG = dict(vocab_size=4096, hidden_dim=8192, intermediate_dim=2048, num_heads=64, num_kv_heads=8, head_dim=128,
            rms_norm_eps=1e-6, rope_theta=1000000.0, qkv_bias=1, tied_lm_head=0)


@pytest.mark.parametrize("splits", [0, 8])
def test_decode_long_context_vs_oracle(oracle, splits):
    """Qwen2-72B attention shape (64 q / 8 kv heads, D 128, hidden 8192, QKV bias) after a seeded
    2048-position context already in the KV cache (the benchmark long-context setup): automatic
    256-position splits with the merge kernel, and 8 splits merged in the o_proj prologue."""
    ctx, max_seq, seed = 2048, 2064, 41
    gpu = HipDecodeEngine(dict(LONG, num_layers=1), seed=seed, norm_sigma=0.1, max_seq_len=max_seq,
                          attn_splits=splits)
    gpu.fill_kv(0, ctx, seed=9, sigma=1.0)
    kvd = LONG["num_kv_heads"] * LONG["head_dim"]
    cap = (max_seq + 31) // 32 * 32
    raw = np.zeros(2 * kvd * cap, np.uint16)
    L.memcpy_dtoh(raw.ctypes.data, gpu.arena.kv_cache_pool, raw.nbytes)
    kv = (kv_from_device(raw, LONG["num_kv_heads"], max_seq, LONG["head_dim"]).astype(np.uint32) << 16).view(np.float32)
    ref = oracle.Engine(dict(LONG, num_layers=1, max_seq_len=max_seq), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=True, kv_bf16=True, threads=16)
    kr, vr = ref.kv_cache(0)
    kr[:ctx] = kv[0, :, :ctx, :].transpose(1, 0, 2).reshape(ctx, kvd)
    vr[:ctx] = kv[1, :, :ctx, :].transpose(1, 0, 2).reshape(ctx, kvd)
    for i, tok in enumerate(oracle.prompt_tokens(seed, 3, LONG["vocab_size"])):
        pos = ctx + i
        t_ref = ref.forward(int(tok), pos)
        t_gpu = gpu.forward_step(int(tok), pos)
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        print(f"[long ctx splits={splits}] pos={pos} gpu={t_gpu} ref={t_ref} maxabs={d:.3e}", flush=True)
        assert t_gpu == oracle.argmax(gpu.logits)
        assert d < LOGIT_TOL, (pos, d)
    gpu.close()
    ref.close()


def test_caller_allocated_arena_bind(hiplib):
    """The reference runner's allocation pattern (velox_cuda_runner.cu:417-431): the caller allocates
    every buffer itself, fills the eight VeloxCudaArena fields and binds the plan. Decoding through
    the model-named entry point on that arena equals decoding on an arena the library created, bit
    for bit; a second bind of the same buffers and mismatching flags are refused."""
    import ctypes as C

    h = L.hip()
    h.hipMalloc.restype = C.c_int
    h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    h.hipHostMalloc.restype = C.c_int
    h.hipHostMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t, C.c_uint]
    h.hipFree.argtypes = [C.c_void_p]
    h.hipHostFree.argtypes = [C.c_void_p]
    seed = 41
    ref = HipDecodeEngine("smollm_135m", seed=seed, max_seq_len=16, num_layers=2, norm_sigma=0.1)
    sizes = ref.arena_bytes()
    bufs = {}
    for k in ("weights", "scales", "norms", "kv", "activations"):
        p = C.c_void_p()
        assert h.hipMalloc(C.byref(p), sizes[k]) == 0
        bufs[k] = p.value
    ring = C.c_void_p()
    assert h.hipHostMalloc(C.byref(ring), L.RING_SIZE * 4, 0x2) == 0  # mapped
    a = L.Arena()
    a.weight_arena, a.weight_scales, a.norm_weight_arena = bufs["weights"], bufs["scales"], bufs["norms"]
    a.kv_cache_pool, a.activation_arena = bufs["kv"], bufs["activations"]
    a.host_pinned_ring = C.cast(ring, C.POINTER(C.c_uint32))
    a.quant_mode, a.tied_lm_head = L.QUANT_GGML_Q4_0, 0  # SmolLM's head is tied: refused
    assert hiplib.velox_hip_arena_bind(ref._model, C.byref(a)) == L.EINVAL
    a.tied_lm_head = 1
    L.check(hiplib.velox_hip_arena_bind(ref._model, C.byref(a)), "arena_bind")
    assert hiplib.velox_hip_arena_model(C.byref(a)) == ref._model.value
    assert hiplib.velox_hip_arena_bind(ref._model, C.byref(a)) == L.EINVAL  # already bound
    L.check(hiplib.velox_hip_synthesize_model(C.byref(a), seed, 0.02, 0.1, None), "synthesize")
    logits_off = hiplib.velox_hip_model_logits_offset(ref._model)
    V = ref.cfg.vocab_size
    tok = 17
    for pos in range(4):
        want = ref.forward_step(tok, pos)
        hiplib.velox_SmolLM_135M_decode_hip(C.byref(a), tok, pos, 1, None)
        assert h.hipDeviceSynchronize() == 0 and hiplib.velox_hip_last_error() == 0
        got = np.empty(V, np.float32)
        L.memcpy_dtoh(got.ctypes.data, bufs["activations"] + logits_off, got.nbytes)
        assert np.array_equal(got.view(np.uint32), ref.logits.view(np.uint32))
        assert C.cast(ring, C.POINTER(C.c_uint32))[pos] == want
        tok = want
    L.check(hiplib.velox_hip_arena_destroy(C.byref(a)), "destroy")  # forgets it, frees nothing
    assert hiplib.velox_hip_arena_model(C.byref(a)) is None
    for p in bufs.values():
        assert h.hipFree(p) == 0
    assert h.hipHostFree(ring) == 0
    ref.close()


def test_run_drains_the_ring_past_1024_positions(oracle):
    """velox_hip_run over more positions than the 1024-entry ring (a regression test: tokens read only
    at the end of the run came out shifted once positions wrapped): every position's token is the
    engine's own greedy decode of the same prompt, from position 0 on."""
    seed, P, steps = 29, 6, 1100
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, 49152)]
    rep, toks = run("smollm_135m", prompt=prompt, warmup=3, steps=steps, seed=seed, num_layers=1,
                    max_seq_len=P + 3 + steps + 1, max_tokens=2048)
    assert rep["status"] == 0 and rep["first_position"] == 0 and rep["n_tokens"] == P + 3 + steps
    eng = HipDecodeEngine("smollm_135m", seed=seed, max_seq_len=P + 3 + steps + 1, num_layers=1)
    want = eng.generate_greedy_into(prompt, 3 + steps + 1)
    eng.close()
    assert rep["first_token"] == want[0]
    assert toks[P - 1:] == want[:len(toks) - (P - 1)]


SMOLLM_VLX = """
target hardware { device: "amd_mi355x"; vram_capacity: 8 * GiB; safety_factor: 0.95; }
model SmolLM_135M<const B_MAX: usize = 1, const S_MAX: usize = 64, const VOCAB: usize = 49152,
    const HIDDEN_DIM: usize = 576, const INTERMEDIATE_DIM: usize = 1536, const NUM_LAYERS: usize = 30,
    const NUM_HEADS: usize = 9, const NUM_KV_HEADS: usize = 3, const HEAD_DIM: usize = 64> {
    @vram_immutable weight w_embed: Tensor<[VOCAB, HIDDEN_DIM], f32> = safetensors("m.safetensors", "e");
    scope decode<const B: usize>(t: Tensor<[B, 1], u32>, step: usize) -> Tensor<[B, 1], u32> {
        let x = rmsnorm(h, w_attn_norm[l], eps = 1e-5);
    }
}
"""


def test_run_from_a_vlx_model_source(oracle, tmp_path):
    """`velox build model.vlx` flow: the runner reads the model from its .vlx source
    (velox_hip_run's model_file, the runner binary's --model-file) and decodes exactly what the
    builtin configuration with the same shapes decodes; the named entry points accept the
    source's model name."""
    import os
    import re
    import subprocess

    path = tmp_path / "smollm.vlx"
    path.write_text(SMOLLM_VLX)
    seed, P = 37, 4
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, 49152)]
    _, want = run("smollm_135m", prompt=prompt, warmup=0, steps=5, seed=seed, num_layers=2, max_seq_len=32)
    rep, got = run("", prompt=prompt, warmup=0, steps=5, seed=seed, num_layers=2, max_seq_len=32,
                   model_file=str(path))
    assert rep["status"] == 0 and got == want
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    runner = os.path.join(root, "velox_amd", "lib", "velox_hip_runner")
    r = subprocess.run([runner, "--model-file", str(path), "--tokens", ",".join(map(str, prompt)), "--steps", "4",
                        "--seed", str(seed), "--layers", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    steps = [int(t) for t in re.findall(r"^\[Step \d+\] Token: (\d+)$", r.stdout, re.M)]
    _, want4 = run("smollm_135m", prompt=prompt, warmup=0, steps=3, seed=seed, num_layers=2)
    assert steps == want4[P - 1:P - 1 + 4]
    eng = HipDecodeEngine(str(path), seed=seed, max_seq_len=16, num_layers=2)
    assert eng.cfg.name.decode() == "SmolLM_135M"
    import ctypes as C

    eng.lib.velox_SmolLM_135M_decode_hip(C.byref(eng.arena), prompt[0], 0, 1, None)
    eng.sync()  # raises if the named entry point refused the arena
    eng.close()
