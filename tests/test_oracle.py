"""CPU tests pinning the oracle (oracle/velox_oracle.c) before it is trusted as the checker.

Each group names what fixes it: the reference's own known answers, the reference's compiled C99
module (oracle/_ref, plus its golden fixture for machines without /root/reference), closed forms
and exhaustive enumeration, or an independent library routine (numpy.float16, torch.bfloat16).
"""
import hashlib
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SMOLLM = dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_layers=30, num_heads=9, num_kv_heads=3,
              head_dim=64, max_seq_len=2048, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)


# ---- reference known answers ------------------------------------------------------------------
def test_rmsnorm_known_answers(oracle):
    # src/runtime.rs:1552-1557
    out = oracle.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 1e-5)
    assert abs(out[0] - 1.0 / np.sqrt(np.float32(7.50001))) < 1e-6
    # tests/test_runtime_e2e.rs:40-48 (uniform input returns the gain)
    out = oracle.rmsnorm(np.full(4, 2.0, np.float32), np.array([1, 0.5, -1, 2], np.float32), 1e-5)
    np.testing.assert_allclose(out, [1, 0.5, -1, 2], atol=1e-5)


def test_matmul_known_answer(oracle):
    # tests/test_runtime_e2e.rs:82-86
    out = oracle.matmul_transposed(np.array([2, 3], np.float32), np.array([[1, 2], [3, 4]], np.float32))
    np.testing.assert_allclose(out, [8, 18], atol=1e-6)


def test_matmul_tail_and_accumulation_order(oracle):
    # in_dim not a multiple of 8 exercises the scalar tail of the AVX2 path (src/runtime.rs:663-673)
    rng = np.random.default_rng(0)
    for k in (1, 7, 8, 13, 576, 4099):
        w = rng.standard_normal((5, k)).astype(np.float32)
        x = rng.standard_normal(k).astype(np.float32)
        got = oracle.matmul_transposed(x, w)
        np.testing.assert_allclose(got, w.astype(np.float64) @ x.astype(np.float64), rtol=1e-5, atol=1e-5)


def test_rope_identity_at_pos0_and_norm_invariance(oracle):
    q = np.array([1.25, -0.75, 0.5, 2.5], np.float32)
    assert np.array_equal(oracle.rope(q, 1, 4, 0, 10000.0), q)  # tests/test_runtime_e2e.rs:50-56
    rng = np.random.default_rng(1)
    t = rng.standard_normal(8 * 128).astype(np.float32)
    r = oracle.rope(t, 8, 128, 4095, 500000.0)
    # rotation preserves each pair's norm, hence each head's norm
    np.testing.assert_allclose(np.linalg.norm(r.reshape(8, 128), axis=1), np.linalg.norm(t.reshape(8, 128), axis=1),
                               rtol=1e-5)
    # closed form for one pair against float64: angle = pos * theta^(-2j/D)
    D, pos, theta = 4, 3, 10000.0
    v = np.array([1.0, 0.0, 0.0, 0.0], np.float32)
    r = oracle.rope(v, 1, D, pos, theta)
    assert abs(r[0] - np.cos(pos)) < 1e-6 and abs(r[2] - np.sin(pos)) < 1e-6


def test_attention_known_answers(oracle):
    # tests/test_runtime_e2e.rs:58-66: at pos 0 both q heads copy v
    q = np.array([1, 0, 0, 1, 0.5, 0.5, -0.5, 0.5], np.float32)
    k = np.array([1, 0, 0, 1], np.float32)
    v = np.array([3.5, -1.5, 0.25, 7.0], np.float32)
    out = oracle.attention(q, k, v, 2, 1, 4, 0)
    assert np.array_equal(out[:4], v) and np.array_equal(out[4:], v)
    # two positions against a float64 softmax
    rng = np.random.default_rng(2)
    q = rng.standard_normal(4 * 8).astype(np.float32)
    kc = rng.standard_normal((6, 2 * 8)).astype(np.float32)
    vc = rng.standard_normal((6, 2 * 8)).astype(np.float32)
    out = oracle.attention(q, kc, vc, 4, 2, 8, 5).reshape(4, 8)
    for h in range(4):
        g = h // 2
        s = kc[:, g * 8:(g + 1) * 8].astype(np.float64) @ q[h * 8:(h + 1) * 8] / np.sqrt(8)
        p = np.exp(s - s.max())
        p /= p.sum()
        np.testing.assert_allclose(out[h], p @ vc[:, g * 8:(g + 1) * 8], rtol=1e-5, atol=1e-6)


def test_swiglu_known_answer(oracle):
    # tests/test_runtime_e2e.rs:68-80 with identity weights: res + silu(1) * 1
    silu1 = 1.0 / (1.0 + np.exp(-1.0))
    act = oracle.swiglu(np.ones(2, np.float32), np.ones(2, np.float32))
    np.testing.assert_allclose(act, [silu1, silu1], rtol=1e-6)


def test_argmax_known_answers_and_ties(oracle):
    assert oracle.argmax(np.array([-1.0, 3.5, 2.1, 0.4], np.float32)) == 1  # src/runtime.rs:1559-1560
    assert oracle.argmax(np.array([-2.0, 0.5, 9.2, 3.1], np.float32)) == 2  # tests/test_runtime_e2e.rs:88-90
    assert oracle.argmax(np.array([1.0, 5.0, 5.0, 5.0], np.float32)) == 1  # strict '>' keeps the first
    assert oracle.argmax(np.array([np.nan, -np.inf, 2.0], np.float32)) == 2
    assert oracle.argmax(np.full(3, -np.inf, np.float32)) == 0


def test_mla_two_step_closed_form(oracle):
    """tests/test_runtime_e2e.rs:100-201 (absorbed MLA, online softmax over latents)."""
    import ctypes as C

    L = oracle.lib()
    fp = oracle.fptr
    w_norm = np.ones(4, np.float32)
    w_dkv = np.array([[1, 0, 0, 0], [0, 1, 0, 0]], np.float32)
    w_q = w_dkv.copy()
    w_o = np.array([[1, 0], [0, 1], [0, 0], [0, 0]], np.float32)
    pool = np.zeros(4 * 2, np.float32)
    dst = np.zeros(4, np.float32)
    x0 = np.full(4, 2.0, np.float32)
    L.vxo_mla_absorbed_step(fp(dst), fp(x0), fp(w_norm), fp(w_dkv), fp(w_q), fp(w_o), fp(pool), 4, 2, 4, 0,
                            C.c_float(1e-5))
    np.testing.assert_allclose(pool[:2], [1, 1], atol=1e-4)
    np.testing.assert_allclose(dst, [3, 3, 2, 2], atol=1e-4)
    x1 = np.array([2, -2, 2, -2], np.float32)
    L.vxo_mla_absorbed_step(fp(dst), fp(x1), fp(w_norm), fp(w_dkv), fp(w_q), fp(w_o), fp(pool), 4, 2, 4, 1,
                            C.c_float(1e-5))
    k0, k1 = pool[0:2].astype(np.float64), pool[2:4].astype(np.float64)
    s = np.array([k1 @ k0, k1 @ k1]) / np.sqrt(2.0)
    p = np.exp(s - s.max())
    p /= p.sum()
    ctx = p[0] * k0 + p[1] * k1
    np.testing.assert_allclose(dst, [2 + ctx[0], -2 + ctx[1], 2, -2], atol=1e-4)


# ---- the reference's own compiled C99 module -----------------------------------------------------
def _golden():
    with open(os.path.join(HERE, "golden", "smollm_ref_fp32.json")) as f:
        return json.load(f)


def test_oracle_matches_reference_golden_bitexact(oracle):
    """The oracle reproduces velox_SmolLM_135M_prefill (the reference's emitted C99 decode step,
    tinystories_smollm.c:532) bit for bit: every logit of 4 consecutive positions."""
    g = _golden()
    eng = oracle.Engine(dict(SMOLLM, max_seq_len=64), seed=g["seed"], sigma=g["sigma"], norm_sigma=g["norm_sigma"],
                        q4_0=False, kv_bf16=False, threads=8)
    for st in g["steps"]:
        tok = eng.forward(st["token_in"], st["pos"])
        assert tok == st["argmax"]
        assert eng.logits[:16].tolist() == st["logits_head"]
        assert hashlib.sha256(eng.logits.tobytes()).hexdigest() == st["logits_sha256"]
    eng.close()


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(HERE), "oracle", "_ref",
                                                    "libvelox_ref_smollm.so")),
                    reason="oracle/_ref not built (needs /root/reference)")
def test_oracle_matches_reference_module_live(oracle):
    """Live comparison with a different seed than the fixture, where oracle/_ref is built."""
    ref = oracle.RefSmolLM(seed=99, sigma=0.02, norm_sigma=0.05)
    eng = oracle.Engine(dict(SMOLLM, max_seq_len=64), seed=99, sigma=0.02, norm_sigma=0.05, q4_0=False,
                        kv_bf16=False, threads=8)
    for pos, tok in enumerate(oracle.prompt_tokens(99, 3, 49152)):
        assert ref.step(int(tok), pos) == eng.forward(int(tok), pos)
        assert np.array_equal(ref.logits.view(np.uint32), eng.logits.view(np.uint32))
    ref.close()
    eng.close()


# ---- scalar conversions ------------------------------------------------------------------------
def test_f16_conversion_matches_numpy(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, np.inf, -np.inf, 2 ** -24, 2 ** -25,
                  3 * 2 ** -26, 2 ** -14, 2 ** -14 - 2 ** -25, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32)])
    vals = vals.astype(np.float32)
    got = np.array([L.vxo_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = np.array([L.vxo_f16_to_f32(int(h)) for h in range(0, 65536, 7) if (h & 0x7C00) != 0x7C00], np.float32)
    ref = np.arange(0, 65536, 7, dtype=np.uint32)
    ref = ref[(ref & 0x7C00) != 0x7C00].astype(np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(back, ref)


def test_bf16_conversion_matches_torch(oracle):
    import torch

    L = oracle.lib()
    rng = np.random.default_rng(4)
    vals = (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32)
    vals = np.concatenate([vals, np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, np.inf], np.float32)])
    vals = vals.astype(np.float32)
    got = np.array([L.vxo_f32_to_bf16(float(v)) for v in vals], np.uint16)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


# ---- Q4_0 codec --------------------------------------------------------------------------------
def test_q4_0_offset_exact_all_nibbles(oracle):
    """(q - 8) * d is exact in fp32 for all 16 nibbles (cf. the reference's exhaustive nibble
    check, tests/empirical_challenge_step2/test_03_marlin_bit_arithmetic.py:52-75)."""
    for dh in (0x3C00, 0x2E66, 0x0001, 0x7BFF, 0x8400 | 0x123):
        d = np.array([dh], np.uint16).view(np.float16).astype(np.float64)[0]
        for q in range(16):
            blk = np.zeros(18, np.uint8)
            blk[0], blk[1] = dh & 0xFF, dh >> 8
            blk[2:18] = q | (q << 4)
            out = oracle.q4_0_dequant(blk.reshape(1, 18), 32)[0]
            assert np.all(out.astype(np.float64) == (q - 8) * d)


def test_q4_0_nibble_order_roundtrip(oracle):
    """Values (q - 8) with d = 1 quantize back to exactly q; element j sits in the low nibble of
    qs[j] and element j + 16 in its high nibble (GGML block_q4_0)."""
    rng = np.random.default_rng(5)
    for _ in range(50):
        q = rng.integers(0, 16, 32)
        q[rng.integers(0, 32)] = 0  # an element at -8 fixes d = (-8) / -8 = 1
        x = (q - 8).astype(np.float32).reshape(1, 32)
        blk = oracle.q4_0_quantize(x)[0]
        assert blk[0] == 0x00 and blk[1] == 0x3C  # fp16 1.0
        assert np.array_equal(blk[2:] & 15, q[:16]) and np.array_equal(blk[2:] >> 4, q[16:])
        assert np.array_equal(oracle.q4_0_dequant(blk.reshape(1, 18), 32)[0], x[0])


def test_q4_0_quantizer_error_bound_and_extreme(oracle):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((500, 64)) * 0.02).astype(np.float32)
    blk = oracle.q4_0_quantize(x)
    deq = oracle.q4_0_dequant(blk, 64)
    for r in range(50):
        for b in range(2):
            xb = x[r, b * 32:(b + 1) * 32].astype(np.float64)
            db = deq[r, b * 32:(b + 1) * 32].astype(np.float64)
            d = abs(np.frombuffer(blk[r, b * 18:b * 18 + 2].tobytes(), np.float16)[0])
            i = np.argmax(np.abs(xb))
            # the extreme element maps to code 0, i.e. -8 * d = x_max up to fp16 rounding of d
            assert abs(db[i] - xb[i]) <= abs(xb[i]) * 2 ** -11 + 1e-12
            # every element within one step (the clamp of q to 15 costs at most one step)
            assert np.max(np.abs(db - xb)) <= d * (1 + 2 ** -10) + 1e-12
    assert np.all(oracle.q4_0_quantize(np.zeros((1, 32), np.float32))[0, 2:] == 0x88)


def test_g64_reference_codec(oracle):
    """The reference's group-64 format (src/codegen.rs:2337-2370): scale (max-min)/15, min, and
    the interleaved word q0|q2<<4|q4<<8|q6<<12|q1<<16|q3<<20|q5<<24|q7<<28."""
    import ctypes as C

    L = oracle.lib()
    # scale 0.03125 and zero point 8 of tests/empirical_challenge_phase2/test3_marlin_lop3_dequant.cu
    q = np.arange(64) % 16
    x = ((q - 8) * 0.03125).astype(np.float32)
    packed = np.zeros(8, np.uint32)
    sm = np.zeros(2, np.uint16)
    L.vxo_g64_quantize(oracle.fptr(x), 1, packed.ctypes.data_as(C.POINTER(C.c_uint32)),
                       sm.ctypes.data_as(C.POINTER(C.c_uint16)))
    # scale = (max - min) / 15 = (0.21875 + 0.25) / 15 = 0.03125, min = -0.25, both exact in fp16
    assert sm.view(np.float16)[0] == np.float16(0.03125) and sm.view(np.float16)[1] == np.float16(-0.25)
    w0 = [q[i] for i in (0, 2, 4, 6, 1, 3, 5, 7)]
    assert packed[0] == sum(int(v) << (4 * i) for i, v in enumerate(w0))
    out = np.zeros(64, np.float32)
    L.vxo_g64_dequant(packed.ctypes.data_as(C.POINTER(C.c_uint32)), sm.ctypes.data_as(C.POINTER(C.c_uint16)), 1,
                      oracle.fptr(out))
    np.testing.assert_allclose(out, x, atol=1e-4)  # the reference test's tolerance


def test_g64_codec_picks_the_nearest_level(oracle):
    """Random groups of every sign and scale: each value decodes to the level q s + m (q in 0..15)
    nearest to it, brute-forced over all 16 levels in float64 (ties and fp32 rounding of the
    quantizer's own arithmetic within 1e-5 s); a constant group has scale 0 and decodes exactly to
    its value rounded to fp16."""
    rng = np.random.default_rng(64)
    groups = [rng.standard_normal(64) * sc + off for sc, off in ((0.02, 0.0), (1.0, 3.0), (1e-3, -0.5), (40.0, 0.0))]
    x = np.concatenate(groups).astype(np.float32)
    packed, sm = oracle.g64_quantize(x)
    got = oracle.g64_dequant(packed, sm).astype(np.float64)
    s = sm[:, 0].view(np.float16).astype(np.float64).repeat(64)
    m = sm[:, 1].view(np.float16).astype(np.float64).repeat(64)
    levels = m[:, None] + s[:, None] * np.arange(16)[None, :]
    best = np.min(np.abs(levels - x[:, None]), axis=1)
    assert np.all(np.abs(got - x) <= best + 1e-5 * s + 1e-12)
    # the decoded values are the levels themselves (fmaf(q, s, m) within one fp32 rounding)
    q = np.rint((got - m) / s)
    assert np.all((q >= 0) & (q <= 15)) and np.allclose(got, m + q * s, rtol=2 ** -23, atol=0)
    c = np.full(64, 0.3, np.float32)
    packed, sm = oracle.g64_quantize(c)
    assert sm[0, 0] == 0 and np.all(oracle.g64_dequant(packed, sm) == np.float32(np.float16(0.3)))


# ---- synthetic recipe ---------------------------------------------------------------------------
def test_rng_statistics_and_determinism(oracle):
    a = oracle.fill_normal(400000, 1, 2, 0.02)
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4
    assert np.array_equal(a, oracle.fill_normal(400000, 1, 2, 0.02))
    assert not np.array_equal(a[:100], oracle.fill_normal(100, 1, 3, 0.02))
    t = oracle.prompt_tokens(5, 1000, 128256)
    assert t.max() < 128256 and len(set(t.tolist())) > 900


def test_q4_0_engine_matches_dequantized_fp32_engine(oracle):
    """Q4_0 GEMV path == fp32 path run on the dequantized weights (dequant-on-the-fly is exact)."""
    cfg = dict(SMOLLM, num_layers=2, max_seq_len=8)
    q = oracle.Engine(cfg, seed=3, q4_0=True, kv_bf16=False, threads=4)
    blocks = q.tensor(oracle.T_Q, 0).reshape(576, -1)
    x = np.random.default_rng(7).standard_normal(576).astype(np.float32)
    w = oracle.q4_0_dequant(blocks, 576)
    assert np.array_equal(oracle.matmul_q4_0(x, blocks, 576), oracle.matmul_transposed(x, w))
    assert np.array_equal(oracle.matmul_q4_0(x, blocks, 576, threads=4), oracle.matmul_transposed(x, w))
    q.close()


# ---- QKV bias and theta-dependent RoPE (the Qwen and Llama-3 configurations) -------------------------
def _rope64(v: np.ndarray, pos: int, theta: float) -> np.ndarray:
    """Rotate-half RoPE of one head in float64: pair (j, j + D/2) turns by pos * theta^(-2j/D)."""
    d = v.shape[0]
    j = np.arange(d // 2, dtype=np.float64)
    ang = pos * theta ** (-2.0 * j / d)
    x1, x2 = v[:d // 2].astype(np.float64), v[d // 2:].astype(np.float64)
    return np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang), x2 * np.cos(ang) + x1 * np.sin(ang)])


@pytest.mark.parametrize("theta", [500000.0, 1000000.0])
def test_rope_theta_closed_form_all_pairs(oracle, theta):
    """Every pair j of a D = 128 head at positions up to 8191 against float64 cos/sin of
    pos * theta^(-2j/D). The bound is what fp32 rounding of the angle allows (a few ulp of pos *
    freq); a wrong exponent (-j/D, D/2), a swapped pair or a wrong theta misses by orders more."""
    rng = np.random.default_rng(8)
    d = 128
    for pos in (1, 7, 300, 4095, 8191):
        v = rng.standard_normal(d).astype(np.float32)
        got = oracle.rope(v, 1, d, pos, theta).astype(np.float64)
        want = _rope64(v, pos, theta)
        tol = (8.0 * pos * 2.0 ** -24 + 1e-6) * np.abs(v).max() * 2
        assert np.max(np.abs(got - want)) <= tol, (pos, np.max(np.abs(got - want)), tol)
    # pair j = 1 at pos 1 turns by exactly theta^(-2/D): two thetas must give two different rotations
    e = np.zeros(d, np.float32)
    e[1] = 1.0
    r = oracle.rope(e, 1, d, 1, theta)
    assert abs(float(r[1]) - np.cos(theta ** (-2.0 / d))) < 1e-6
    assert abs(float(r[1 + d // 2]) - np.sin(theta ** (-2.0 / d))) < 1e-6


def test_qkv_bias_added_before_rope_closed_form(oracle):
    """Qwen's q/k/v biases (HF semantics: q = W_q x + b_q, then RoPE; the reference drops the bias,
    src/runtime.rs:1368-1370). One layer with W_q = W_k = 0, O = identity and a zero FFN, so that
    at position p: the K cache slot is rope(b_k, p), the V slot W_v rmsnorm(x) + b_v, and the
    hidden state minus the embedding row is softmax_t(rope(b_q, p) . rope(b_k, t) / sqrt(D)) v_t
    per head, all computed here in float64. Bias after RoPE (K slot b_k), a dropped bias (K slot
    0) or a q bias missing from the scores each fail."""
    H, hq, hkv, d, theta = 64, 4, 2, 16, 1000000.0
    cfg = dict(vocab_size=16, hidden_dim=H, intermediate_dim=32, num_layers=1, num_heads=hq, num_kv_heads=hkv,
               head_dim=d, max_seq_len=8, rms_norm_eps=1e-5, rope_theta=theta, qkv_bias=1, tied_lm_head=1)
    eng = oracle.Engine(cfg, seed=21, q4_0=False, kv_bf16=False, threads=1)
    f32 = lambda kind: eng.tensor_view(kind, 0).view(np.float32)  # noqa: E731
    rng = np.random.default_rng(9)
    f32(oracle.T_Q)[:] = 0.0
    f32(oracle.T_K)[:] = 0.0
    wv = rng.standard_normal((hkv * d, H)).astype(np.float32) * np.float32(0.5)
    f32(oracle.T_V)[:] = wv.ravel()
    f32(oracle.T_O)[:] = np.eye(H, hq * d, dtype=np.float32).ravel()
    for k in (oracle.T_GATE, oracle.T_UP, oracle.T_DOWN):
        f32(k)[:] = 0.0
    bq = rng.standard_normal(hq * d).astype(np.float32)
    bk = rng.standard_normal(hkv * d).astype(np.float32)
    bv = rng.standard_normal(hkv * d).astype(np.float32)
    f32(oracle.T_BQ)[:] = bq
    f32(oracle.T_BK)[:] = bk
    f32(oracle.T_BV)[:] = bv
    embed = f32(oracle.T_EMBED).reshape(16, H).astype(np.float64)
    gain = f32(oracle.T_ATTN_NORM).astype(np.float64)
    kc, vc = eng.kv_cache(0)
    vs = []
    for pos, tok in enumerate((3, 11, 5, 7)):
        eng.forward(tok, pos)
        x = embed[tok]
        xn = x / np.sqrt(np.mean(x * x) + 1e-5) * gain
        want_k = np.concatenate([_rope64(bk[g * d:(g + 1) * d], pos, theta) for g in range(hkv)])
        want_v = wv.astype(np.float64) @ xn + bv
        vs.append(want_v)
        np.testing.assert_allclose(kc[pos], want_k, rtol=0, atol=2e-5)
        np.testing.assert_allclose(vc[pos], want_v, rtol=0, atol=2e-5)
        attn = eng.hidden().astype(np.float64) - x
        for h in range(hq):
            g = h // (hq // hkv)
            q = _rope64(bq[h * d:(h + 1) * d], pos, theta)
            s = np.array([q @ _rope64(bk[g * d:(g + 1) * d], t, theta) for t in range(pos + 1)]) / np.sqrt(d)
            p = np.exp(s - s.max())
            p /= p.sum()
            want_o = sum(p[t] * vs[t][g * d:(g + 1) * d] for t in range(pos + 1))
            np.testing.assert_allclose(attn[h * d:(h + 1) * d], want_o, rtol=0, atol=5e-5)
        if pos == 0:  # one position: every head of a group returns its V row
            for h in range(hq):
                g = h // (hq // hkv)
                np.testing.assert_allclose(attn[h * d:(h + 1) * d], want_v[g * d:(g + 1) * d], atol=5e-5)
    eng.close()


def test_forced_kv_step_attends_with_the_given_rows(oracle):
    """The one-step K/V forcing of the oracle (the harness of the full-depth GPU comparison, which
    recomputes a step on the GPU's cache rows): forcing the rows an engine computes itself changes
    nothing, bit for bit, and reports those rows; and the forced rows are the ones attended: one
    layer with O = identity and a zero FFN at position 0 (a single position, so each head's attention
    output is its group's V row) leaves hidden - embedding equal to the forced V rows."""
    cfg = dict(vocab_size=64, hidden_dim=64, intermediate_dim=96, num_layers=2, num_heads=4, num_kv_heads=2,
               head_dim=16, max_seq_len=8, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
    a = oracle.Engine(cfg, seed=5, sigma=0.2, q4_0=False, kv_bf16=True, threads=1)
    b = oracle.Engine(cfg, seed=5, sigma=0.2, q4_0=False, kv_bf16=True, threads=1)
    for pos, tok in enumerate((7, 19)):
        a.forward(tok, pos)
    rows = [np.stack([a.kv_cache(layer)[i][1] for layer in range(2)]) for i in (0, 1)]
    b.forward(7, 0)
    t, seen_k, seen_v = b.forward_forced(19, 1, rows[0], rows[1])
    assert t == oracle.argmax(a.logits) and np.array_equal(b.logits, a.logits)
    assert np.array_equal(seen_k, rows[0]) and np.array_equal(seen_v, rows[1])
    a.forward(33, 2)
    b.forward(33, 2)  # the forcing lasts one step
    assert np.array_equal(b.logits, a.logits)
    a.close()
    b.close()

    H, hq, hkv, d = 64, 4, 2, 16
    one = dict(cfg, num_layers=1)
    eng = oracle.Engine(one, seed=6, q4_0=False, kv_bf16=False, threads=1)
    f32 = lambda kind: eng.tensor_view(kind, 0).view(np.float32)  # noqa: E731
    f32(oracle.T_O)[:] = np.eye(H, hq * d, dtype=np.float32).ravel()
    for k in (oracle.T_GATE, oracle.T_UP, oracle.T_DOWN):
        f32(k)[:] = 0.0
    rng = np.random.default_rng(4)
    fk = rng.standard_normal((1, hkv * d)).astype(np.float32)
    fv = rng.standard_normal((1, hkv * d)).astype(np.float32)
    _, seen_k, seen_v = eng.forward_forced(9, 0, fk, fv)
    assert not np.array_equal(seen_v, fv)
    x = f32(oracle.T_EMBED).reshape(64, H)[9].astype(np.float64)
    want = np.concatenate([fv[0, (h // (hq // hkv)) * d:(h // (hq // hkv) + 1) * d] for h in range(hq)])
    np.testing.assert_allclose(eng.hidden().astype(np.float64) - x, want, rtol=0, atol=1e-6)
    kc, vc = eng.kv_cache(0)
    assert np.array_equal(kc[0], fk[0]) and np.array_equal(vc[0], fv[0])
    eng.close()


def test_fp16_weight_mode_rounds_the_fp32_weights(oracle):
    """w_f16 (the reference's quant_mode 1): every linear weight and embedding value is the fp32
    engine's value rounded to fp16 (numpy's round-to-nearest-even cast); vectors stay fp32."""
    cfg = dict(vocab_size=64, hidden_dim=64, intermediate_dim=96, num_layers=1, num_heads=4, num_kv_heads=2,
               head_dim=16, max_seq_len=8, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
    a = oracle.Engine(cfg, seed=4, sigma=0.5, norm_sigma=0.1, q4_0=False, threads=1)
    b = oracle.Engine(cfg, seed=4, sigma=0.5, norm_sigma=0.1, q4_0=False, w_f16=True, threads=1)
    for kind in (oracle.T_EMBED, oracle.T_Q, oracle.T_GATE, oracle.T_DOWN):
        wa, wb = a.tensor(kind, 0).view(np.float32), b.tensor(kind, 0).view(np.float32)
        assert np.array_equal(wb, wa.astype(np.float16).astype(np.float32)) and not np.array_equal(wa, wb)
    assert np.array_equal(a.tensor(oracle.T_ATTN_NORM, 0), b.tensor(oracle.T_ATTN_NORM, 0))
    a.close()
    b.close()
