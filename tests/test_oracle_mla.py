"""CPU pins of the oracle's fp8 e4m3fn block format and absorbed MLA layer (benchmark configuration 4).

The reference's MLA (src/runtime.rs:845-1044) is a simplified single-latent-head form; config 4 asks
for the DeepSeek-V3 form (128 heads, q LoRA, a RoPE part, fp8 weights with 128x128 block scales).
The oracle's full form is pinned by: reduction to the reference's own step (bit for bit), the
absorption identity against textbook attention over decompressed keys and values (float64), and
the reference's two-step closed form through that reduction. The fp8 codec is pinned against an
independent closed-form decode of all 256 codes and torch's float8_e4m3fn rounding.
"""
import numpy as np
import pytest
import torch


def _decode_closed_form(b):
    s = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 15, b & 7
    if e == 15 and m == 7:
        return np.nan
    return s * (np.ldexp(1.0 + m / 8.0, e - 7) if e else np.ldexp(m / 8.0, -6))


def test_e4m3_decode_all_codes(oracle):
    codes = np.arange(256, dtype=np.uint8)
    got = oracle.e4m3_decode(codes)
    want = np.array([_decode_closed_form(int(b)) for b in codes], np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_e4m3_encode_roundtrip_and_rounding(oracle):
    codes = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], np.uint8)
    assert np.array_equal(oracle.e4m3_encode(oracle.e4m3_decode(codes)), codes)
    # round to nearest even against torch's float8_e4m3fn cast, across normals, subnormals and ties
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-448, 448, 4000), rng.uniform(-0.02, 0.02, 4000),
                        (oracle.e4m3_decode(codes[:-1]) + oracle.e4m3_decode(codes[1:])) / 2]).astype(np.float32)
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.e4m3_encode(x), want)
    # saturation (the block quantizer never exceeds 448, but the encoder clamps)
    assert list(oracle.e4m3_encode(np.array([1000.0, -1e9, 448.0, 460.0], np.float32))) == [0x7E, 0xFE, 0x7E, 0x7E]


def test_fp8_block_quantize(oracle):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((200, 300)) * 0.02).astype(np.float32)
    w[3, 7] = 0.5  # one block with a large outlier
    codes, scales = oracle.fp8_quantize(w)
    assert scales.shape == (2, 3)
    for i in range(2):
        for j in range(3):
            blk = w[i * 128:(i + 1) * 128, j * 128:(j + 1) * 128]
            assert scales[i, j] == np.float32(np.max(np.abs(blk))) / np.float32(448.0)
            # the block maximum lands on the largest code
            r, c = np.unravel_index(np.argmax(np.abs(blk)), blk.shape)
            assert codes[i * 128 + r, j * 128 + c] & 0x7F == 0x7E
    deq = oracle.fp8_dequant(codes, scales)
    srow = np.repeat(np.repeat(scales, 128, 0), 128, 1)[:200, :300]
    # 3 mantissa bits: |error| <= 2^-4 of the value's binade, or half the subnormal step
    assert np.all(np.abs(deq - w) <= np.maximum(np.abs(w) * 2.0 ** -4, srow * 2.0 ** -10) * 1.0001)


def _reduced_step_inputs(rng, H=96, lr=128, S=8):
    return dict(norm=(1 + 0.1 * rng.standard_normal(H)).astype(np.float32),
                dkv=(0.1 * rng.standard_normal((lr, H))).astype(np.float32),
                qabs=(0.1 * rng.standard_normal((lr, H))).astype(np.float32),
                oabs=(0.1 * rng.standard_normal((H, lr))).astype(np.float32))


def test_mla_full_form_reduces_to_reference_step(oracle):
    """n_heads 1, no q LoRA, no RoPE part, no latent norm, W_kvb = [I; I]: bit-identical to the
    reference's simplified step (src/runtime.rs:944-1044) over several positions."""
    L = oracle.lib()
    rng = np.random.default_rng(11)
    H, lr, S = 96, 128, 8
    w = _reduced_step_inputs(rng, H, lr, S)
    cfg = oracle.mla_config(H, 1, 0, lr, lr, 0, lr, kv_norm=0, max_seq=S, eps=1e-5,
                            scale=np.float32(1.0) / np.sqrt(np.float32(128.0)))
    full = dict(norm=w["norm"], q_b=w["qabs"], kv_a=w["dkv"], kv_b=np.concatenate([np.eye(lr), np.eye(lr)]),
                o=w["oabs"])
    pool_ref = np.zeros(S * lr, np.float32)
    cache = np.zeros((S, lr), np.float32)
    fp = oracle.fptr
    for pos in range(5):
        h = rng.standard_normal(H).astype(np.float32)
        ref = np.zeros(H, np.float32)
        L.vxo_mla_absorbed_step(fp(ref), fp(h), fp(w["norm"]), fp(w["dkv"]), fp(w["qabs"]), fp(w["oabs"]),
                                fp(pool_ref), H, lr, S, pos, 1e-5)
        got = oracle.mla_layer_step(cfg, full, cache, h, pos, cache_bf16=False)
        assert np.array_equal(got, ref), pos
        assert np.array_equal(cache.ravel(), pool_ref)


def _rope_np(x, pos, theta):
    d = x.shape[-1]
    half = d // 2
    j = np.arange(half)
    freq = 1.0 / np.power(np.float64(theta), (2 * j) / d)
    ang = pos * freq
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang), x2 * np.cos(ang) + x1 * np.sin(ang)], -1)


def _rms_np(x, g, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * g


def test_mla_absorbed_equals_decompressed_attention(oracle):
    """The absorbed step equals textbook MLA: per-head keys [W_uk c_t ; rope(kr_t)] and values
    W_uv c_t decompressed from the latent cache, softmax attention, then W_o (float64)."""
    rng = np.random.default_rng(12)
    H, nh, ql, lr, dn, dr, dv, S = 64, 4, 48, 32, 16, 8, 24, 8
    theta, eps = 10000.0, 1e-6
    cfg = oracle.mla_config(H, nh, ql, lr, dn, dr, dv, kv_norm=1, max_seq=S, eps=eps, rope_theta=theta)
    w = dict(norm=(1 + 0.1 * rng.standard_normal(H)), q_a=0.2 * rng.standard_normal((ql, H)),
             q_a_norm=(1 + 0.1 * rng.standard_normal(ql)), q_b=0.2 * rng.standard_normal((nh * (dn + dr), ql)),
             kv_a=0.2 * rng.standard_normal((lr + dr, H)), kv_a_norm=(1 + 0.1 * rng.standard_normal(lr)),
             kv_b=0.2 * rng.standard_normal((nh * (dn + dv), lr)), o=0.2 * rng.standard_normal((H, nh * dv)))
    w = {k: v.astype(np.float32) for k, v in w.items()}
    W = {k: v.astype(np.float64) for k, v in w.items()}
    cache = np.zeros((S, lr + dr), np.float32)
    lat = []
    for pos in range(6):
        h = rng.standard_normal(H).astype(np.float32)
        got = oracle.mla_layer_step(cfg, w, cache, h, pos, cache_bf16=False)
        x = _rms_np(h.astype(np.float64), W["norm"], eps)
        q = W["q_b"] @ _rms_np(W["q_a"] @ x, W["q_a_norm"], eps)
        ckr = W["kv_a"] @ x
        lat.append((_rms_np(ckr[:lr], W["kv_a_norm"], eps), _rope_np(ckr[lr:], pos, theta)))
        out = np.zeros(nh * dv)
        for hh in range(nh):
            wk = W["kv_b"][hh * (dn + dv):hh * (dn + dv) + dn]
            wv = W["kv_b"][hh * (dn + dv) + dn:(hh + 1) * (dn + dv)]
            qh = q[hh * (dn + dr):(hh + 1) * (dn + dr)]
            qf = np.concatenate([qh[:dn], _rope_np(qh[dn:], pos, theta)])
            keys = np.stack([np.concatenate([wk @ c, kr]) for c, kr in lat])
            vals = np.stack([wv @ c for c, _ in lat])
            s = keys @ qf * cfg.scale
            p = np.exp(s - s.max())
            out[hh * dv:(hh + 1) * dv] = (p / p.sum()) @ vals
        want = h + W["o"] @ out
        assert np.max(np.abs(got - want)) < 1e-4 * max(1.0, np.max(np.abs(want))), pos


def test_mla_synth_weights_are_fp8_blocks(oracle):
    """The seeded MLA weights are exactly representable as e4m3 codes times their block scale."""
    codes, scales, deq = oracle.fp8_synth_matrix(7, oracle.tag(0, oracle.MLA_TAGS["kv_b"]), 256, 192, 0.02)
    assert np.array_equal(oracle.fp8_dequant(codes, scales), deq)
    assert np.all(np.abs(deq) <= np.repeat(np.repeat(scales, 128, 0), 128, 1)[:256, :192] * 448)
