"""The absorbed MLA layer on the GPU (benchmark configuration 4; the full form of src/runtime.rs:845-1044)
against the oracle's vxo_mla_layer_step on the same seeded fp8 weights and latent context.

Tolerance: the device computes every projection with fp16 activations against exactly converted
fp8 weights and the attention on bf16 MFMA operands (the cached latent rows, q and P rounded to
bf16; fp32 accumulation), the oracle in fp32; the
layer's update (h_out - h) must agree to 2e-2 of its largest magnitude (the bf16 bound), and the
appended latent row to bf16 rounding of the same value."""
import ctypes as C

import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import MlaEngine

pytestmark = pytest.mark.gpu

SMALL = dict(hidden_dim=256, num_heads=16, q_lora_rank=128, kv_lora_rank=128, qk_nope_dim=128, qk_rope_dim=64,
             v_head_dim=128, kv_norm=1, rms_norm_eps=1e-6, rope_theta=10000.0)
GOLDEN = 0x9E3779B97F4A7C15
TOL = 2e-2


def _oracle_cfg(oracle, c, max_seq):
    return oracle.mla_config(c.hidden_dim, c.num_heads, c.q_lora_rank, c.kv_lora_rank, c.qk_nope_dim, c.qk_rope_dim,
                             c.v_head_dim, kv_norm=c.kv_norm, max_seq=max_seq, eps=c.rms_norm_eps,
                             rope_theta=c.rope_theta)


def _check_layer(oracle, cfg_name, batch, ctxs, steps=2, max_seq=96, seed=5, norm_sigma=0.1, splits=0):
    gpu = MlaEngine(cfg_name, max_seq_len=max_seq, max_batch=batch, seed=seed, norm_sigma=norm_sigma,
                    attn_splits=splits)
    c = gpu.cfg
    ocfg = _oracle_cfg(oracle, c, max_seq)
    w = oracle.mla_synth_weights(ocfg, seed, 0.02, norm_sigma)
    R = gpu.R
    rng = np.random.default_rng(seed + batch)
    caches = []
    for b, n in enumerate(ctxs):
        gpu.fill_cache(0, b, n, seed=77, sigma=1.0)
        gpu.set_position(b, n)
        cache = np.zeros((max_seq, R), np.float32)
        cache[:n] = gpu.cache(0, b, n)
        # the device fill is the seeded N(0, 1) of the oracle's stream, rounded to bf16
        want = oracle.fill_normal(n * R, (77 + b * GOLDEN) % (1 << 64), oracle.tag(0, oracle.MLA_TAGS["cache"]), 1.0)
        want16 = (want.view(np.uint32) + 0x7FFF + ((want.view(np.uint32) >> 16) & 1)) >> 16 << 16
        assert np.array_equal(cache[:n].ravel().view(np.uint32), want16.astype(np.uint32)), b
        caches.append(cache)
    for s in range(steps):
        h = rng.standard_normal((batch, c.hidden_dim)).astype(np.float32)
        gpu.set_hidden(h)
        if s:
            for b, n in enumerate(ctxs):
                gpu.set_position(b, n + s)
        gpu.step(0, batch)
        got = gpu.hidden(batch)
        for b, n in enumerate(ctxs):
            pos = n + s
            ref = oracle.mla_layer_step(ocfg, w, caches[b], h[b], pos, cache_bf16=True)
            d_ref, d_got = ref - h[b], got[b] - h[b]
            err = float(np.max(np.abs(d_got - d_ref)))
            scale = float(np.max(np.abs(d_ref)))
            print(f"[mla {cfg_name if isinstance(cfg_name, str) else 'small'} b={b} pos={pos}] update max "
                  f"{scale:.3e} err {err:.3e}", flush=True)
            assert err <= TOL * scale, (b, pos, err, scale)
            row = gpu.cache(0, b, pos + 1)[pos]
            assert np.max(np.abs(row - caches[b][pos])) <= 2 ** -7 * np.max(np.abs(caches[b][pos])), (b, pos)
            caches[b][pos] = row  # continue from the device's bf16 row
    gpu.close()


def test_mla_small_vs_oracle(oracle):
    _check_layer(oracle, SMALL, batch=3, ctxs=[5, 40, 70])


def test_mla_small_one_split_and_many(oracle):
    _check_layer(oracle, SMALL, batch=2, ctxs=[33, 64], splits=1, steps=1)
    _check_layer(oracle, SMALL, batch=2, ctxs=[0, 64], splits=3, steps=1)


def test_mla_deepseek_shape_vs_oracle(oracle):
    """Config 4's shapes (hidden 7168, 128 heads, q LoRA 1536, latent 512 + rope 64) on a short context."""
    _check_layer(oracle, "deepseek_v3_mla", batch=2, ctxs=[37, 100], steps=1, max_seq=160, norm_sigma=0.0)


def test_mla_deepseek_shape_batched_vs_oracle(oracle):
    """17 sequences: two 16-row activation tiles per GEMM wave, and GEMM waves over 4, 2 or 1 row tiles
    (the launcher takes fewer row tiles per wave where 4 would leave fewer than 256 workgroups)."""
    _check_layer(oracle, "deepseek_v3_mla", batch=17, ctxs=[1 + 9 * i for i in range(17)], steps=1, max_seq=160,
                 norm_sigma=0.0)


def test_mla_deepseek_shape_many_splits_vs_oracle(oracle):
    """16 sequences x 8 position splits x 2 head groups = 256 attention workgroups (the config-4 B=16
    grid), every split non-empty, merged over 8 splits."""
    _check_layer(oracle, "deepseek_v3_mla", batch=16, ctxs=[200 + 19 * i for i in range(16)], steps=1,
                 max_seq=520, norm_sigma=0.0)


def test_mla_deepseek_shape_one_sequence_vs_oracle(oracle):
    """Config 4's B=1 step: [W_qa; W_kva] over the whole K normalizing h itself, W_qb's GEMV normalizing
    the q latent (its extra workgroup appending the latent row), W_uk^T, the W_uv GEMV merging the
    attention splits, W_o adding to h -- two steps against the oracle."""
    _check_layer(oracle, "deepseek_v3_mla", batch=1, ctxs=[100], steps=2, max_seq=160, norm_sigma=0.0)


def test_mla_synthesized_weights_equal_loaded_codes(oracle):
    """The device quantizer and tile maps: loading the oracle's fp8 codes and block scales through the
    checkpoint entry point gives bit-identical layer outputs to the device-synthesized weights."""
    seed, max_seq = 9, 48
    a = MlaEngine(SMALL, max_seq_len=max_seq, max_batch=1, seed=seed)
    b = MlaEngine(SMALL, max_seq_len=max_seq, max_batch=1, synthesize=False)
    c = a.cfg
    ocfg = _oracle_cfg(oracle, c, max_seq)
    H, nh, ql, lr, dq = c.hidden_dim, c.num_heads, c.q_lora_rank, c.kv_lora_rank, c.qk_nope_dim + c.qk_rope_dim
    mats = {L.MLA_Q_A: ("q_a", ql, H), L.MLA_Q_B: ("q_b", nh * dq, ql), L.MLA_KV_A: ("kv_a", lr + c.qk_rope_dim, H),
            L.MLA_KV_B: ("kv_b", nh * (c.qk_nope_dim + c.v_head_dim), lr), L.MLA_O: ("o", H, nh * c.v_head_dim)}
    for kind, (name, r, k) in mats.items():
        codes, scales, _ = oracle.fp8_synth_matrix(seed, oracle.tag(0, oracle.MLA_TAGS[name]), r, k, 0.02)
        b.load_fp8(kind, 0, codes, scales)
    b.load_f32(L.MLA_NORM, 0, np.ones(H, np.float32))
    b.load_f32(L.MLA_Q_A_NORM, 0, np.ones(ql, np.float32))
    b.load_f32(L.MLA_KV_A_NORM, 0, np.ones(lr, np.float32))
    h = np.random.default_rng(1).standard_normal((1, H)).astype(np.float32)
    outs = []
    for e in (a, b):
        e.fill_cache(0, 0, 20, seed=3)
        e.set_position(0, 20)
        e.set_hidden(h)
        e.step(0, 1)
        outs.append(e.hidden(1))
    assert np.array_equal(outs[0], outs[1])
    a.close()
    b.close()


@pytest.mark.parametrize("batch", [1, 16])
def test_mla_decode_step_equals_layer_steps(batch):
    """velox_hip_mla_decode_step over a 3-layer DeepSeek-V3-shaped stack (each layer's W_o partials
    folded into the next layer's RMSNorm: 5 of them at B=1, 19 at B=16) ends with the hidden state
    and appended latent rows of three successive layer steps, bit for bit; the layers' own weights
    and contexts differ, so a wrong layer index or a dropped partial changes the result."""
    layers, max_seq = 3, 96
    eng = [MlaEngine("deepseek_v3_mla", max_seq_len=max_seq, max_batch=batch, num_layers=layers, seed=9,
                     norm_sigma=0.1) for _ in range(2)]
    h = np.random.default_rng(batch).standard_normal((batch, eng[0].cfg.hidden_dim)).astype(np.float32)
    ctx = [40 + 3 * s for s in range(batch)]
    for e in eng:
        for layer in range(layers):
            for s in range(batch):
                e.fill_cache(layer, s, ctx[s], seed=3 + layer)
        for s in range(batch):
            e.set_position(s, ctx[s])
        e.set_hidden(h)
    eng[0].decode_step(batch)
    for layer in range(layers):
        eng[1].step(layer, batch)
    got, want = eng[0].hidden(batch), eng[1].hidden(batch)
    assert np.all(np.isfinite(got)) and not np.array_equal(got, h)
    assert np.array_equal(got, want)
    for layer in range(layers):
        for s in range(batch):
            assert np.array_equal(eng[0].cache(layer, s, ctx[s] + 1), eng[1].cache(layer, s, ctx[s] + 1)), (layer, s)
    for e in eng:
        e.close()


def test_mla_bad_arguments():
    lib = L.load()
    c = L.MlaConfig()
    L.check(lib.velox_hip_mla_builtin_config(b"deepseek_v3_mla", 64, 1, C.byref(c)))
    c.num_heads = 100  # not a multiple of 16
    m = C.c_void_p()
    assert lib.velox_hip_mla_create(C.byref(c), C.byref(m)) == L.ESHAPE
    assert lib.velox_hip_mla_builtin_config(b"nope", 64, 1, C.byref(L.MlaConfig())) == L.EINVAL
