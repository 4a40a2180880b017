"""Batched prefill (velox_hip_prefill_batch): a staged prompt's positions run as the rows of one
batched step per chunk, against the oracle's token-by-token forward of the same seeded model and
prompt (the reference prefills token by token through its decode graph, velox_cuda_runner.cu:493-512).

Tolerances: logits within 2e-2 absolute of the oracle (the bound of the batched decode tests: the
batched GEMMs take fp16 activations); ring entries equal the argmax of the device's own logits row,
and the oracle's argmax wherever its top-2 margin exceeds twice that bound; every layer's K/V rows
agree with the oracle's cache to one bf16 ulp plus what the layers before it propagate."""
import ctypes as C

import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import HipBatchEngine, HipDecodeEngine

from test_gpu_kernels import kv_from_device

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
SMOLLM = dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_heads=9, num_kv_heads=3, head_dim=64,
              rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
QWEN_SMALL_VOCAB = dict(vocab_size=4096, hidden_dim=3584, intermediate_dim=18944, num_heads=28, num_kv_heads=4,
                        head_dim=128, rms_norm_eps=1e-6, rope_theta=1000000.0, qkv_bias=1, tied_lm_head=1)
LLAMA_SMALL_VOCAB = dict(vocab_size=4096, hidden_dim=4096, intermediate_dim=14336, num_heads=32, num_kv_heads=8,
                         head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, qkv_bias=0, tied_lm_head=0)


def _margin(logits):
    top = np.sort(logits)[-2:]
    return float(top[1] - top[0])


def _device_kv(gpu, layer, n_pos):
    """Layer `layer`'s K/V rows [0, n_pos) of sequence 0 as fp32, [2][hkv][n_pos][D]."""
    c = gpu.cfg
    cap = (c.max_seq_len + 31) // 32 * 32
    elems = 2 * c.num_kv_heads * cap * c.head_dim
    layer_bytes = (elems * 2 + 255) // 256 * 256
    raw = np.zeros(elems, np.uint16)
    L.memcpy_dtoh(raw.ctypes.data, gpu.arena.kv_cache_pool + layer * layer_bytes, raw.nbytes)
    kv = kv_from_device(raw, c.num_kv_heads, c.max_seq_len, c.head_dim)[:, :, :n_pos]
    return (kv.astype(np.uint32) << 16).view(np.float32)


def _prefill_vs_oracle(oracle, cfg, layers, chunk, prompt_len, prefill_spans, max_seq, seed, decode_steps=3):
    """prefill_spans: [(pos0, n)] covering [0, P) in order; then decode_steps graph steps."""
    V = cfg["vocab_size"]
    prompt = [int(t) for t in oracle.prompt_tokens(seed + 7, prompt_len, V)]
    gpu = HipDecodeEngine(cfg, seed=seed, norm_sigma=0.1, max_seq_len=max_seq, num_layers=layers,
                          prefill_chunk=chunk)
    gpu.set_prompt(prompt)
    for pos0, n in prefill_spans:
        gpu.prefill_batch(pos0, n)
    P = sum(n for _, n in prefill_spans)
    last_n = prefill_spans[-1][1] % chunk or chunk
    rows = gpu.chunk_logits(last_n)
    ref = oracle.Engine(dict(cfg, num_layers=layers, max_seq_len=max_seq), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=True, kv_bf16=True, threads=16)
    worst = 0.0
    for pos in range(P):
        ref.forward(prompt[pos], pos)
        ring = gpu.ring(pos)
        if _margin(ref.logits) > 2 * LOGIT_TOL:
            assert ring == oracle.argmax(ref.logits), pos
        r = pos - (P - last_n)
        if r >= 0:
            d = float(np.max(np.abs(rows[r] - ref.logits)))
            worst = max(worst, d)
            assert d < LOGIT_TOL, (pos, d)
            assert ring == oracle.argmax(rows[r]), pos
    want_tok = prompt[P] if P < prompt_len else oracle.argmax(rows[-1])
    assert gpu.state() == (P, want_tok)
    # every layer's cache as the oracle's (rows written by the chunks, read by later chunks)
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    for layer in range(layers):
        kv = _device_kv(gpu, layer, P)
        kr, vr = ref.kv_cache(layer)
        for t, (dev, want) in enumerate(((kv[0], kr), (kv[1], vr))):
            want = want[:P].reshape(P, cfg["num_kv_heads"], cfg["head_dim"]).transpose(1, 0, 2)
            err = float(np.max(np.abs(dev - want)))
            scale = float(np.max(np.abs(want)))
            assert err <= (2 ** -7 + 0.01 * layer) * scale, (layer, t, err, scale)
    # decode continues from the prefilled caches through the single-token graph step
    for i in range(decode_steps):
        pos = P + i
        step, tok = gpu.state()
        assert step == pos
        gpu.graph_step()
        gpu.sync()
        gpu.read_logits()
        ref.forward(tok, pos)
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        worst = max(worst, d)
        assert d < LOGIT_TOL, ("decode", pos, d)
    print(f"[prefill chunk={chunk} P={P} layers={layers}] worst logits maxabs {worst:.3e}", flush=True)
    gpu.close()
    ref.close()
    return prompt


def test_prefill_smollm_chunks_vs_oracle(oracle):
    """45 positions in chunks of 16 (16, 16, 13), 4 layers of SmolLM (G = 3, D = 64)."""
    _prefill_vs_oracle(oracle, SMOLLM, 4, 16, 45, [(0, 45)], 64, seed=71)


def test_prefill_spans_and_partial_prompt(oracle):
    """Two calls (positions 0..9, then 10..30 with a 1-row tail chunk) inside a longer prompt: the
    state's next token is the prompt's; single-row chunks; a chunk equal to the prefill size."""
    _prefill_vs_oracle(oracle, SMOLLM, 2, 10, 40, [(0, 10), (10, 21)], 48, seed=72)
    _prefill_vs_oracle(oracle, SMOLLM, 2, 8, 8, [(0, 1), (1, 7)], 16, seed=73, decode_steps=2)


def test_prefill_qwen_bias_32_rows_vs_oracle(oracle):
    """Qwen2.5-7B's layer shapes (q/k/v biases, G = 7, D = 128), 32-row chunks, a context crossing
    several attention splits."""
    _prefill_vs_oracle(oracle, QWEN_SMALL_VOCAB, 1, 32, 70, [(0, 70)], 96, seed=74, decode_steps=2)


def test_prefill_llama_gqa_vs_oracle(oracle):
    """Llama-3-8B's layer shapes (G = 4, D = 128, untied head), 2 layers, 24-row chunks."""
    _prefill_vs_oracle(oracle, LLAMA_SMALL_VOCAB, 2, 24, 50, [(0, 50)], 64, seed=75, decode_steps=2)


def test_prefill_64_and_48_row_chunks_vs_oracle(oracle):
    """Chunks of 64 rows (four MFMA row tiles) and of 48 (three), Llama-shaped and SmolLM layers."""
    _prefill_vs_oracle(oracle, LLAMA_SMALL_VOCAB, 2, 64, 100, [(0, 100)], 128, seed=79, decode_steps=2)
    _prefill_vs_oracle(oracle, SMOLLM, 2, 48, 60, [(0, 60)], 64, seed=80, decode_steps=1)


def test_prefill_128_and_100_row_chunks_vs_oracle(oracle):
    """Chunks of 128 rows (eight MFMA row tiles: a 128-token prompt reads the weights once) and a
    100-row tail; Llama-shaped layers, then SmolLM layers in 100-row chunks."""
    _prefill_vs_oracle(oracle, LLAMA_SMALL_VOCAB, 2, 128, 228, [(0, 228)], 256, seed=81, decode_steps=2)
    _prefill_vs_oracle(oracle, SMOLLM, 2, 100, 130, [(0, 130)], 160, seed=82, decode_steps=1)


def test_prefill_four_and_eight_wave_attention_agree(oracle):
    """Llama-3-8B layer shapes (8 KV heads), a 100-token prompt: 64-row chunks run the prefill
    attention on 4-wave workgroups (64 x 8 = 512 workgroups, rows attending <= 128 positions), 16-row
    chunks on 8-wave ones (128 workgroups). Each row's attention differs only in how its 32-position
    chunks are dealt to waves, so the logits and the K/V rows agree to fp32 accumulation order."""
    seed, P = 81, 100
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, LLAMA_SMALL_VOCAB["vocab_size"])]
    outs = []
    for chunk in (64, 16):
        b = HipDecodeEngine(LLAMA_SMALL_VOCAB, seed=seed, norm_sigma=0.1, max_seq_len=128, num_layers=2,
                            prefill_chunk=chunk)
        b.set_prompt(prompt)
        b.prefill_batch(0, P)
        outs.append((b.chunk_logits(P % chunk)[-1], b.state(), _device_kv(b, 1, P)))
        b.close()
    (la, sa, ka), (lb, sb, kb) = outs
    assert sa == sb and sa[0] == P
    d = float(np.max(np.abs(la - lb)))
    print(f"[prefill 4/8-wave attention] logits maxabs {d:.3e} of {np.max(np.abs(la)):.3e}", flush=True)
    assert d < 1e-3 * max(1.0, float(np.max(np.abs(la))))
    # layer 1's K/V rows come from layer 0's attention output: the fp32 differences can move a
    # bf16 rounding by an ulp or two (2^-9 at values near 0.12), far below a wrong row's error
    assert np.all(np.abs(ka - kb) <= 2 ** -7 * np.abs(kb) + 1e-3 * np.max(np.abs(kb)))


def test_prefill_chunking_invariance(oracle):
    """The same prompt in chunks of 32 and of 7 (and, for layer 0, token by token): each row's
    arithmetic does not depend on the chunk it is in, up to fp32 accumulation order, so the final
    logits agree far inside the oracle bound and layer 0's K/V rows to about one bf16 ulp."""
    seed, P = 76, 37
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, SMOLLM["vocab_size"])]
    a = HipDecodeEngine(SMOLLM, seed=seed, norm_sigma=0.1, max_seq_len=64, num_layers=2)
    a.set_prompt(prompt)
    for pos in range(P):
        a.forward_step(prompt[pos], pos)
    outs = []
    for chunk in (32, 7):
        b = HipDecodeEngine(SMOLLM, seed=seed, norm_sigma=0.1, max_seq_len=64, num_layers=2, prefill_chunk=chunk)
        b.set_prompt(prompt)
        b.prefill_batch(0, P)
        outs.append((b.chunk_logits(P % chunk)[-1], b.state(), _device_kv(b, 0, P)))
        b.close()
    (la, sa, ka), (lb, sb, kb) = outs
    assert sa == sb and sa[0] == a.state()[0] == P
    d = float(np.max(np.abs(la - lb)))
    print(f"[prefill chunking] logits maxabs {d:.3e}, identical {np.array_equal(la, lb)}", flush=True)
    assert d < 1e-3
    # the batched GEMMs round their inputs to fp16 (2^-12 relative), the decode GEMV keeps them to
    # 2^-22: one bf16 step of each value plus 2e-3 of the largest, where rows cancel towards zero
    kt = _device_kv(a, 0, P)
    for k in (ka, kb):
        assert np.all(np.abs(k - kt) <= 2 ** -7 * np.abs(kt) + 2e-3 * np.max(np.abs(kt)))
    a.close()


def test_prefill_in_batch_arena_keeps_sequence_states(oracle):
    """An arena planned for 4 sequences and 12-row prefill chunks: prefill leaves the batched
    sequences' states alone and the batched step still runs after it."""
    seed = 77
    gpu = HipBatchEngine(SMOLLM, max_batch=4, seed=seed, max_seq_len=32, num_layers=2, prefill_chunk=12)
    prompt = [int(t) for t in oracle.prompt_tokens(seed, 20, SMOLLM["vocab_size"])]
    for s in range(4):
        gpu.set_prompt_seq(s, prompt)
        gpu.set_state_seq(s, s, prompt[s])
    gpu.set_prompt(prompt)
    gpu.prefill_batch(0, 20)
    for s in range(4):
        assert gpu.state_seq(s) == (s, prompt[s])
    gpu.batch_step(4)
    gpu.sync()
    for s in range(4):
        assert gpu.state_seq(s) == (s + 1, prompt[s + 1])
    gpu.close()


def test_prefill_rejects_bad_arguments():
    lib = L.load()
    a = HipDecodeEngine(SMOLLM, max_seq_len=32, num_layers=1)  # no prefill_chunk
    assert lib.velox_hip_prefill_batch(C.byref(a.arena), 0, 4, 1, None) == L.EINVAL
    a.close()
    b = HipDecodeEngine(SMOLLM, max_seq_len=32, num_layers=1, prefill_chunk=8)
    for pos0, n in ((0, 0), (30, 3), (32, 1)):
        assert lib.velox_hip_prefill_batch(C.byref(b.arena), pos0, n, 1, None) == L.EINVAL, (pos0, n)
    b.close()
    c = L.ModelConfig()
    L.check(lib.velox_hip_builtin_config(b"smollm_135m", 32, C.byref(c)))
    c.prefill_chunk = 129
    m = C.c_void_p()
    assert lib.velox_hip_model_create(C.byref(c), C.byref(m)) == L.EINVAL


def test_run_with_batched_prefill_matches_engine(oracle):
    """velox_hip_run with prefill_chunk (batched prefill, then the captured decode graph) emits the
    tokens of the same flow driven step by step through the engine."""
    from velox_amd.engine import run
    seed, P, n = 78, 21, 5
    rep, toks = run("smollm_135m", prompt_len=P, warmup=0, steps=n - 1, seed=seed, num_layers=3, max_seq_len=40,
                    prefill_chunk=8)
    assert rep["status"] == 0 and rep["prefill_ms"] > 0
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, 49152)]
    gpu = HipDecodeEngine("smollm_135m", seed=seed, max_seq_len=40, num_layers=3, prefill_chunk=8)
    gpu.set_prompt(prompt)
    gpu.prefill_batch(0, P)
    for _ in range(n - 1):
        gpu.graph_step()
    gpu.sync()
    assert toks[:P + n - 1] == [gpu.ring(p) for p in range(P + n - 1)]
    gpu.close()
    with pytest.raises(RuntimeError):
        run("smollm_135m", prompt_len=1, warmup=0, steps=2, context_len=8, num_layers=1, prefill_chunk=8)


def test_prefill_rejects_positions_past_the_staged_prompt():
    """Every row reads its token from the staged prompt: positions past it are refused (EINVAL)
    instead of reading stale prompt memory."""
    lib = L.load()
    b = HipDecodeEngine(SMOLLM, max_seq_len=32, num_layers=1, prefill_chunk=8)
    b.set_prompt([1, 2, 3, 4])
    assert lib.velox_hip_prefill_batch(C.byref(b.arena), 0, 6, 1, None) == L.EINVAL
    assert lib.velox_hip_prefill_batch(C.byref(b.arena), 3, 2, 1, None) == L.EINVAL
    b.prefill_batch(0, 4)
    b.close()


def test_prefill_llama3_8b_full_depth_128_rows_vs_oracle(oracle):
    """The bench's TTFT path at full size: Llama-3-8B (32 layers, untied 128256-row head) prefills a
    128-token prompt as one 128-row chunk of velox_hip_prefill_batch. At sampled rows the oracle
    recomputes that position on the GPU's K/V rows of every layer (its own row included), so the
    two sides attend over the same values; the chunk's logits rows must be within the bf16 bar."""
    from test_gpu_configs import _device_kv as kv_rows

    seed, P = 97, 128
    max_seq = P + 8
    gpu = HipDecodeEngine("llama3_8b", seed=seed, max_seq_len=max_seq, prefill_chunk=128)
    c = gpu.cfg
    nl, hkv, D = c.num_layers, c.num_kv_heads, c.head_dim
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, c.vocab_size)]
    gpu.set_prompt(prompt)
    gpu.prefill_batch(0, P)
    rows = gpu.chunk_logits(P)
    kv = [kv_rows(gpu.arena, layer, hkv, max_seq, D, P) for layer in range(nl)]
    for pos in range(P):
        assert gpu.ring(pos) == oracle.argmax(rows[pos]), pos
    assert gpu.state() == (P, oracle.argmax(rows[-1]))
    gpu.close()
    ref = oracle.Engine(dict(c.as_dict(), max_seq_len=max_seq), seed=seed, sigma=0.02, norm_sigma=0.0, q4_0=True,
                        kv_bf16=True, threads=16)
    caches = [ref.kv_cache(layer) for layer in range(nl)]
    worst = 0.0
    for pos in (0, 1, 63, 126, 127):
        for layer, (kr, vr) in enumerate(caches):
            kr[:pos], vr[:pos] = kv[layer][0][:pos], kv[layer][1][:pos]
        t_ref, _, _ = ref.forward_forced(prompt[pos], pos, np.stack([kv[layer][0][pos] for layer in range(nl)]),
                                         np.stack([kv[layer][1][pos] for layer in range(nl)]))
        d = float(np.max(np.abs(rows[pos] - ref.logits)))
        worst = max(worst, d)
        print(f"[llama3_8b prefill 128 rows, 32 layers] pos={pos} gpu={oracle.argmax(rows[pos])} ref={t_ref} "
              f"maxabs={d:.3e}", flush=True)
        if _margin(ref.logits) > 2 * LOGIT_TOL:
            assert oracle.argmax(rows[pos]) == t_ref, pos
        assert d < LOGIT_TOL, (pos, d)
    print(f"[llama3_8b prefill 128 rows, 32 layers] worst logits maxabs {worst:.3e}", flush=True)
    ref.close()
