"""The fused QKV + attention launch of the single-sequence step (vx_qkv_attn.hip: one kernel per layer,
each KV head's q/k/v rows and attention splits on one XCD) against the CPU oracle and against the
two-launch step it replaces.

Bars: logits within the bf16 bar of 2e-2 of the oracle (teacher forcing, bf16 KV); against the
two-launch step, layer 0's K/V rows bit for bit (the same GEMV rows, RoPE and bf16 rounding) and
logits within 1e-3 (the two attentions sum the same exact products in different orders); graph
replays equal eager steps bit for bit; the launches' error word stays 0 (every workgroup on its
expected XCD, every wait ended)."""
import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import HipDecodeEngine, run, set_fused_attention

from test_gpu_kernels import kv_from_device

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
LLAMA = dict(vocab_size=128256, hidden_dim=4096, intermediate_dim=14336, num_layers=32, num_heads=32, num_kv_heads=8,
             head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, qkv_bias=0, tied_lm_head=0)
LONG = dict(vocab_size=4096, hidden_dim=8192, intermediate_dim=2048, num_heads=64, num_kv_heads=8, head_dim=128,
            rms_norm_eps=1e-6, rope_theta=1000000.0, qkv_bias=1, tied_lm_head=0)


@pytest.fixture(autouse=True)
def _fused_on():
    set_fused_attention(True)
    yield
    set_fused_attention(True)


def _layer_kv(arena, layer, hkv, max_seq, d):
    cap = (max_seq + 31) // 32 * 32
    layer_bytes = (2 * hkv * cap * d * 2 + 255) // 256 * 256
    raw = np.zeros(2 * hkv * cap * d, np.uint16)
    L.memcpy_dtoh(raw.ctypes.data, arena.kv_cache_pool + layer * layer_bytes, raw.nbytes)
    return raw


def test_fused_plan():
    """Llama-3-8B shapes take it (4 splits up to 512 positions, 8 up to 2048); 4 KV heads (Qwen2.5-7B),
    an explicit split count, a context past 2048 positions or the switch turned off do not."""
    g = HipDecodeEngine("llama3_8b", seed=1, max_seq_len=400, num_layers=1)
    assert g.fused_status() == (4, 0)
    g.close()
    g = HipDecodeEngine("llama3_8b", seed=1, max_seq_len=2048, num_layers=1)
    assert g.fused_status() == (8, 0)
    g.close()
    for kw in (dict(model="qwen2_5_7b", max_seq_len=400), dict(model="llama3_8b", max_seq_len=400, attn_splits=2),
               dict(model="llama3_8b", max_seq_len=4096)):
        g = HipDecodeEngine(kw.pop("model"), seed=1, num_layers=1, **kw)
        assert g.fused_status()[0] == 0, kw
        g.close()
    set_fused_attention(False)
    g = HipDecodeEngine("llama3_8b", seed=1, max_seq_len=400, num_layers=1)
    assert g.fused_status()[0] == 0
    g.close()


def test_fused_llama_vs_oracle(oracle):
    """Llama-3-8B layer shapes (2 layers, the full 128256-word head) over 70 teacher-forced positions:
    the 4 splits' chunks rotate through every split, and positions 0, 31, 32, 64 put the new position
    first in a chunk, last in one, and in a chunk with no cached positions."""
    seed, n, max_seq = 31, 70, 200
    ref = oracle.Engine(dict(LLAMA, num_layers=2, max_seq_len=max_seq), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=True, kv_bf16=True, threads=16)
    gpu = HipDecodeEngine("llama3_8b", seed=seed, norm_sigma=0.1, max_seq_len=max_seq, num_layers=2)
    assert gpu.fused_status()[0] == 4
    worst = 0.0
    for pos, tok in enumerate(oracle.prompt_tokens(seed, n, LLAMA["vocab_size"])):
        t_ref = ref.forward(int(tok), pos)
        t_gpu = gpu.forward_step(int(tok), pos)
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        worst = max(worst, d)
        assert t_gpu == oracle.argmax(gpu.logits)
        srt = np.sort(ref.logits)
        if srt[-1] - srt[-2] > 2 * LOGIT_TOL:
            assert t_gpu == t_ref, pos
        assert d < LOGIT_TOL, (pos, d)
    print(f"[fused llama] worst max-abs {worst:.3e}", flush=True)
    assert gpu.fused_status() == (4, 0)
    gpu.close()
    ref.close()


def test_fused_matches_two_launches(oracle):
    """The same model stepped fused and as two launches: layer 0's K/V rows bit for bit (identical
    GEMV rows, RoPE and bf16 rounding), logits within 1e-3 at every position."""
    seed, n, max_seq = 5, 140, 160
    toks = [int(t) for t in oracle.prompt_tokens(seed, n, LLAMA["vocab_size"])]
    out = {}
    for fused in (True, False):
        set_fused_attention(fused)
        g = HipDecodeEngine("llama3_8b", seed=seed, norm_sigma=0.1, max_seq_len=max_seq, num_layers=2)
        assert (g.fused_status()[0] > 0) == fused
        logits = []
        for pos, t in enumerate(toks):
            g.forward_step(t, pos)
            logits.append(g.logits.copy())
        out[fused] = (np.stack(logits), _layer_kv(g.arena, 0, 8, max_seq, 128))
        if fused:
            assert g.fused_status() == (4, 0)
        g.close()
    assert np.array_equal(out[True][1], out[False][1])
    d = float(np.max(np.abs(out[True][0] - out[False][0])))
    print(f"[fused vs two launches] max-abs {d:.3e}", flush=True)
    assert d < 1e-3


def test_fused_long_context_8_splits_vs_oracle(oracle):
    """Qwen2-72B attention shape (64 q / 8 KV heads: 8 q heads per XCD, hidden 8192: two activation
    register groups) after a seeded 1500-position context: 8 splits of 47 chunks between them."""
    ctx, max_seq, seed = 1500, 2048, 43
    gpu = HipDecodeEngine(dict(LONG, num_layers=1), seed=seed, norm_sigma=0.1, max_seq_len=max_seq)
    assert gpu.fused_status()[0] == 8
    gpu.fill_kv(0, ctx, seed=9, sigma=1.0)
    kvd = LONG["num_kv_heads"] * LONG["head_dim"]
    raw = _layer_kv(gpu.arena, 0, 8, max_seq, 128)
    kv = (kv_from_device(raw, LONG["num_kv_heads"], max_seq, LONG["head_dim"]).astype(np.uint32) << 16).view(np.float32)
    ref = oracle.Engine(dict(LONG, num_layers=1, max_seq_len=max_seq), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=True, kv_bf16=True, threads=16)
    kr, vr = ref.kv_cache(0)
    kr[:ctx] = kv[0, :, :ctx, :].transpose(1, 0, 2).reshape(ctx, kvd)
    vr[:ctx] = kv[1, :, :ctx, :].transpose(1, 0, 2).reshape(ctx, kvd)
    for i, tok in enumerate(oracle.prompt_tokens(seed, 3, LONG["vocab_size"])):
        pos = ctx + i
        ref.forward(int(tok), pos)
        t_gpu = gpu.forward_step(int(tok), pos)
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        print(f"[fused long ctx] pos={pos} maxabs={d:.3e}", flush=True)
        assert t_gpu == oracle.argmax(gpu.logits)
        assert d < LOGIT_TOL, (pos, d)
    assert gpu.fused_status() == (8, 0)
    gpu.close()
    ref.close()


def test_fused_graph_replay_matches_eager(oracle):
    """Replays of one captured fused step (the counters re-armed by each launch) decode exactly the
    tokens eager fused steps do, across a masked-off step (bit 0 clear: no launch counts)."""
    seed, P, n = 27, 8, 24
    prompt = [int(t) for t in oracle.prompt_tokens(seed, P, LLAMA["vocab_size"])]
    eager = HipDecodeEngine("llama3_8b", seed=seed, max_seq_len=64, num_layers=2)
    eager.lib.velox_hip_decode_graph_step(__import__("ctypes").byref(eager.arena), 0, None)  # masked: no-op
    want = eager.generate_greedy_into(prompt, n)
    assert eager.fused_status() == (4, 0)
    eager.close()
    rep, toks = run("llama3_8b", prompt_len=P, warmup=2, steps=n - 3, seed=seed, num_layers=2, max_seq_len=64)
    assert rep["status"] == 0
    assert toks[P - 1:P - 1 + n] == want
