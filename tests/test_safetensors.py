"""The safetensors reader (velox_amd/csrc/vx_safetensors.cpp) on the CPU: no GPU call is made.

Malformed-input cases follow the reference's own adversarial tests of its reader
(tests/test_adversarial_runtime.rs:145-400): missing keys and the tied-head fallback, data_offsets
past the end of the file or inverted (E013 -> VELOX_HIP_ETENSOR), dtype mismatches for every stored
type (E014 -> VELOX_HIP_EDTYPE), files under 8 bytes, a header length past the end, invalid UTF-8
and malformed JSON (refused, never a crash), and a metadata-only header (no tensors). The runner
refuses the same files before it touches the GPU."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import Safetensors

import st_writer as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUNNER = os.path.join(ROOT, "velox_amd", "lib", "velox_hip_runner")
SMOLLM_LAYER = dict(vocab_size=64, hidden_dim=576, intermediate_dim=1536, num_layers=2, num_heads=9, num_kv_heads=3,
                    head_dim=64, qkv_bias=0, tied_lm_head=1)


def _open(path):
    h = C.c_void_p()
    rc = L.load().velox_hip_st_open(path.encode(), C.byref(h))
    return rc, h


def _data(h, name, dtype):
    p, n = C.c_void_p(), C.c_uint64()
    rc = L.load().velox_hip_st_tensor_data(h, name.encode(), dtype.encode(), C.byref(p), C.byref(n))
    return rc, (C.string_at(p.value, n.value) if rc == 0 else None)


def test_round_trip_of_every_float_dtype(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    path = str(tmp_path / "rt.safetensors")
    W.write(path, [("a.f32", "F32", (3, 5), W.to_dtype(a, "F32")), ("b.f16", "F16", (7,), W.to_dtype(b, "F16")),
                   ("c.bf16", "BF16", (7,), W.to_dtype(b, "BF16"))], metadata={"format": "pt"})
    with Safetensors(path) as st:
        assert st.names() == ["a.f32", "b.f16", "c.bf16"]
        rc, raw = _data(st.handle, "a.f32", "F32")
        assert rc == 0 and np.array_equal(np.frombuffer(raw, np.float32).reshape(3, 5), a)
        rc, raw = _data(st.handle, "b.f16", "F16")
        assert rc == 0 and np.array_equal(np.frombuffer(raw, np.float16), b.astype(np.float16))
        rc, raw = _data(st.handle, "c.bf16", "BF16")
        assert rc == 0 and np.allclose(W.from_bf16(raw), b, rtol=2 ** -8, atol=0)
        shape, nd, beg, end = (C.c_uint64 * 8)(), C.c_uint32(), C.c_uint64(), C.c_uint64()
        dt = C.create_string_buffer(16)
        assert L.load().velox_hip_st_tensor_info(st.handle, 1, None, 0, dt, shape, C.byref(nd), C.byref(beg),
                                                 C.byref(end)) == 0
        assert (dt.value, nd.value, shape[0], beg.value, end.value) == (b"F16", 1, 7, 60, 74)


def test_bf16_writer_rounds_to_nearest_even():
    # 1 + 2^-8 is halfway between two bf16 values: ties go to the even one (1.0); 1 + 3*2^-8 rounds up
    x = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0], np.float32)
    assert list(W.from_bf16(W.to_dtype(x, "BF16"))) == [1.0, 1.0 + 2 ** -6, -2.5, 0.0]


def test_missing_keys_and_the_tied_head_fallback(tmp_path):
    """E013 for a missing name; lm_head.weight resolves to the embedding when absent
    (tests/test_adversarial_runtime.rs:145-175)."""
    path = str(tmp_path / "e013.safetensors")
    W.write(path, [("model.embed_tokens.weight", "F32", (2, 2), W.to_dtype(np.arange(4.0), "F32"))])
    rc, h = _open(path)
    assert rc == 0
    lib = L.load()
    idx = C.c_uint64()
    assert lib.velox_hip_st_find(h, b"non_existent.weight", C.byref(idx)) == L.ETENSOR
    assert _data(h, "non_existent.weight", "F32")[0] == L.ETENSOR
    assert lib.velox_hip_st_find(h, b"lm_head.weight", C.byref(idx)) == 0 and idx.value == 0
    rc, raw = _data(h, "lm_head.weight", "F32")
    assert rc == 0 and list(np.frombuffer(raw, np.float32)) == [0.0, 1.0, 2.0, 3.0]
    lib.velox_hip_st_close(h)


@pytest.mark.parametrize("offsets,payload", [((1000, 2000), 100), ((50, 10), 100), ((0, 101), 100)])
def test_offsets_outside_the_file_or_inverted(tmp_path, offsets, payload):
    """Header accepted at open; the tensor's data refused with E013
    (tests/test_adversarial_runtime.rs:177-232)."""
    path = str(tmp_path / "trunc.safetensors")
    hdr = '{"bad.tensor":{"dtype":"F32","shape":[250],"data_offsets":[%d,%d]}}' % offsets
    while (8 + len(hdr)) % 8:
        hdr += " "
    W.write_raw(path, hdr, bytes(payload))
    rc, h = _open(path)
    assert rc == 0
    assert _data(h, "bad.tensor", "F32")[0] == L.ETENSOR
    L.load().velox_hip_st_close(h)


def test_dtype_mismatch_for_every_stored_type(tmp_path):
    """E014 whenever the stored dtype is not the one asked for (tests/test_adversarial_runtime.rs:256-320)."""
    path = str(tmp_path / "dt.safetensors")
    hdr = ('{"tensor_f16":{"dtype":"F16","shape":[4],"data_offsets":[0,8]},'
           '"tensor_bf16":{"dtype":"BF16","shape":[4],"data_offsets":[8,16]},'
           '"tensor_fp8":{"dtype":"F8_E4M3","shape":[4],"data_offsets":[16,20]},'
           '"tensor_i8":{"dtype":"I8","shape":[4],"data_offsets":[20,24]},'
           '"tensor_f32":{"dtype":"F32","shape":[4],"data_offsets":[24,40]}}')
    while (8 + len(hdr)) % 8:
        hdr += " "
    W.write_raw(path, hdr, bytes(64))
    rc, h = _open(path)
    assert rc == 0
    for name in ("tensor_f16", "tensor_bf16", "tensor_fp8", "tensor_i8"):
        assert _data(h, name, "F32")[0] == L.EDTYPE, name
    assert _data(h, "tensor_f32", "F32")[0] == 0
    assert _data(h, "tensor_f32", "F16")[0] == L.EDTYPE
    L.load().velox_hip_st_close(h)


def test_byte_count_must_match_the_shape(tmp_path):
    path = str(tmp_path / "shape.safetensors")
    W.write_raw(path, '{"t":{"dtype":"F32","shape":[3,3],"data_offsets":[0,32]}}      ', bytes(32))
    rc, h = _open(path)
    assert rc == 0 and _data(h, "t", "F32")[0] == L.ESHAPE
    L.load().velox_hip_st_close(h)


def test_corrupt_containers_are_refused(tmp_path):
    """tests/test_adversarial_runtime.rs:328-400: a missing file, files under 8 bytes, a header length
    past the end, invalid UTF-8, malformed JSON; a metadata-only header parses to no tensors."""
    assert _open(str(tmp_path / "none.safetensors"))[0] == L.ENOTLOADED
    for size in range(8):
        p = tmp_path / f"tiny{size}.safetensors"
        p.write_bytes(bytes(size))
        assert _open(str(p))[0] == L.EINVAL, size
    p = str(tmp_path / "huge.safetensors")
    W.write_raw(p, b"short", header_len=10_000_000)
    assert _open(p)[0] == L.EINVAL
    p = str(tmp_path / "utf8.safetensors")
    W.write_raw(p, bytes([0xFF, 0xFE, 0xFD, 0xFC]))
    assert _open(p)[0] == L.EINVAL
    for bad in ["", "not json", "[]", "{", '{"unclosed"', '{"foo": 123}', '{"foo": {"dtype": 123}}',
                '{"a":{"dtype":"F32","shape":[1],"data_offsets":[0]}}',
                '{"a":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}',
                '{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"a":{"dtype":"F32","shape":[1],'
                '"data_offsets":[0,4]}}',
                '{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}} trailing',
                '{"a":{"dtype":"F32","shape":[99999999999999999999],"data_offsets":[0,4]}}',
                "{" * 100 + "}" * 100]:
        p = str(tmp_path / "bad.safetensors")
        W.write_raw(p, bad, bytes(8))
        assert _open(p)[0] == L.EINVAL, bad
    p = str(tmp_path / "meta.safetensors")
    W.write_raw(p, '{"__metadata__": {"meta": "data", "nested": [1, {"x": null}]}}')
    rc, h = _open(p)
    assert rc == 0 and L.load().velox_hip_st_tensor_count(h) == 0
    L.load().velox_hip_st_close(h)


def _smollm_like(path, dtype="F16", drop=None, reshape=None, bad_dtype=None, lm_head=False):
    """A 2-layer checkpoint with SmolLM-135M's layer shapes and a 64-word vocabulary (zero weights)."""
    tensors = []
    names = W.hf_names(dict(SMOLLM_LAYER, tied_lm_head=0 if lm_head else 1))
    for name, _, _, shape in names:
        if name == drop:
            continue
        if name == reshape:
            shape = (shape[0] + 1,) + tuple(shape[1:])
        dt = bad_dtype if (bad_dtype and name.endswith("o_proj.weight")) else dtype
        eb = {"F32": 4, "F16": 2, "BF16": 2, "F8_E4M3": 1}[dt]
        tensors.append((name, dt, shape, bytes(int(np.prod(shape)) * eb)))
    W.write(path, tensors)


def test_config_from_tensor_shapes(tmp_path):
    """Vocabulary, depth and head tying come from the file, head count and size from the builtin
    configuration with the same layer shapes (SmolLM-135M), eps/theta with them; fp32 rows by default."""
    path = str(tmp_path / "m.safetensors")
    _smollm_like(path)
    with Safetensors(path) as st:
        c = st.config(32)
    assert (c.vocab_size, c.hidden_dim, c.intermediate_dim, c.num_layers, c.num_heads, c.num_kv_heads,
            c.head_dim) == (64, 576, 1536, 2, 9, 3, 64)
    assert c.tied_lm_head == 1 and c.qkv_bias == 0 and c.quant_mode == L.QUANT_F32 and c.max_seq_len == 32
    assert c.rope_theta == 10000.0 and abs(c.rms_norm_eps - 1e-5) < 1e-12
    _smollm_like(path, lm_head=True)
    with Safetensors(path) as st:
        assert st.config(32).tied_lm_head == 0
    W.write(path, [("model.embed_tokens.weight", "F32", (4, 8), bytes(128))])
    with Safetensors(path) as st:
        c = L.ModelConfig()
        assert L.load().velox_hip_st_config(st.handle, 0, C.byref(c)) == L.ETENSOR


@pytest.mark.parametrize("case,want", [
    (dict(), 0),
    (dict(drop="model.layers.1.mlp.up_proj.weight"), L.ETENSOR),
    (dict(drop="model.norm.weight"), L.ETENSOR),
    (dict(reshape="model.layers.0.self_attn.k_proj.weight"), L.ESHAPE),
    (dict(bad_dtype="F8_E4M3"), L.EDTYPE),
    (dict(dtype="BF16"), 0),
    (dict(dtype="F32"), 0),
])
def test_check_against_a_plan(tmp_path, case, want):
    path = str(tmp_path / "c.safetensors")
    _smollm_like(path, **case)
    cfg = L.builtin_config("smollm_135m", 32)
    cfg.vocab_size, cfg.num_layers = 64, 2
    with Safetensors(path) as st:
        assert L.load().velox_hip_st_check(st.handle, C.byref(cfg)) == want


@pytest.mark.skipif(not os.path.exists(RUNNER), reason="runner not built")
@pytest.mark.parametrize("case,msg", [
    ("missing", "failed to open weights file"),
    ("truncated", "[E013]"),
    ("incomplete", "[E013]"),
    ("fp8", "[E014]"),
])
def test_runner_refuses_bad_checkpoints_before_the_gpu(tmp_path, case, msg):
    """The reference CLI passes --weights on every run (src/cli.rs:653-654); a checkpoint the model
    cannot load ends the runner with exit 1 and the reference's diagnostic, before any HIP call."""
    path = str(tmp_path / "w.safetensors")
    if case == "truncated":
        _smollm_like(path)
        raw = open(path, "rb").read()
        open(path, "wb").write(raw[:len(raw) // 2])
    elif case == "incomplete":
        W.write(path, [("model.embed_tokens.weight", "F32", (2, 2), bytes(16))])
    elif case == "fp8":
        _smollm_like(path, bad_dtype="F8_E4M3")
    # the CLI's own argv (src/cli.rs:653-660): the model comes from the file
    r = subprocess.run([RUNNER, "--weights", path, "--tokens", "1,2", "--steps", "2", "--verbose"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1, (r.stdout, r.stderr)
    assert msg in r.stderr, r.stderr
    assert "[Step" not in r.stdout
