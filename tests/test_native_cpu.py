"""CPU tests of the native libraries: the C ABI loads and exports every declared symbol, and the
host side (synthetic generator, f16/bf16 rounding, GGUF metadata -> config, XoshiroRandom,
SamplerPipeline on host logits) matches the oracle / numpy. No GPU calls."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import dotnetfoundryllm_amd._native as N
import oracle_bind as O
from dotnetfoundryllm_amd.configs import CONFIGS, desc_of
from dotnetfoundryllm_amd.gguf import GgufWriter, write_synthetic_gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    return re.findall(r"FLLM_API\s+[\w\s\*]+?\b(fllmh?_\w+)\s*\(", src)


def test_every_declared_symbol_is_exported():
    names = declared("fllm.h") + declared("fllm_host.h")
    assert len(names) > 45
    missing = [n for n in names if not (hasattr(N.dev, n) or hasattr(N.host, n))]
    assert not missing
    # and the binding covers all of them
    bound = set(N.DEVICE_SIGS) | set(N.HOST_SIGS)
    assert set(names) <= bound, set(names) - bound


def test_null_handles_and_pure_functions():
    out = C.c_int64()
    assert N.dev.fllm_element_count(N.Q6_K, 420, C.byref(out)) == 0 and out.value == 512
    assert N.dev.fllm_element_count(99, 4, C.byref(out)) == N.E_NOT_SUPPORTED
    assert N.dev.fllm_forward(None, 0, 0) == N.E_NULL
    assert N.dev.fllm_model_finalize(None) == N.E_NULL
    assert N.dev.fllm_dequantize(None, 0, None, 0, None, 0) == N.E_NULL
    assert b"must not be null" in N.dev.fllm_last_error()


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_context_fails_loudly_without_gpu():
    with pytest.raises(F.FoundryError):
        F.Context(0)


def test_f16_bf16_rounding():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-8, 5, 20000),
                         np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8, 3e-5, np.inf, -np.inf], np.float32)])
    xs = xs.astype(np.float32)
    got = np.array([N.host.fllmh_f32_to_f16(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, xs.astype(np.float16).view(np.uint16))
    b = np.array([N.host.fllmh_f32_to_bf16(float(x)) for x in xs[:5000]], dtype=np.uint16)
    back = (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x64 = xs[:5000].astype(np.float64)
    fin = np.isfinite(x64)
    ulp = np.abs(back[fin]) * 2.0 ** -7 + 1e-45
    assert np.all(np.abs(back[fin] - x64[fin]) <= ulp * 0.5 * 1.0001 + 1e-40)


def test_synth_deterministic_and_in_range():
    a = F.synth_tensor(N.Q4_K, 7, 3, 256 * 64, 0, 1e-3, 4e-3)
    b = F.synth_tensor(N.Q4_K, 7, 3, 256 * 64, 0, 1e-3, 4e-3)
    c = F.synth_tensor(N.Q4_K, 7, 4, 256 * 64, 0, 1e-3, 4e-3)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    t = F.synth_tensor(N.Q4_K, 7, 3, 256 * 64, 0, 1e-3, 4e-3, threads=5)
    assert np.array_equal(a, t)  # thread count does not change the bytes
    blocks = a.reshape(64, 144)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    assert np.all((d >= np.float32(np.float16(1e-3))) & (d <= np.float32(np.float16(4e-3))))
    nib = np.concatenate([blocks[:, 16:] & 15, blocks[:, 16:] >> 4]).ravel()
    assert set(np.unique(nib)) == set(range(16))
    q8 = F.synth_tensor(N.Q8_0, 1, 1, 32 * 1000, 0, 1e-3, 1e-2).reshape(1000, 34)
    qs = q8[:, 2:].view(np.int8)
    assert qs.min() >= -127 and qs.max() <= 127 and qs.min() < -120 and qs.max() > 120
    emb = F.synth_tensor(N.F32, 2, 0, 100000, 0, 0.0, 0.02).view(np.float32)
    assert abs(emb.mean()) < 1e-3 and abs(emb.std() - 0.02) < 1e-3
    q6 = F.synth_tensor(N.Q6_K, 3, 0, 256 * 100, 0, 1e-3, 4e-3).reshape(100, 210)
    assert q6[:, 192:208].max() <= 63
    toks = F.synth_tokens(5, 0, 1000, 500)
    assert toks.min() >= 0 and toks.max() < 1000 and np.array_equal(toks, F.synth_tokens(5, 0, 1000, 500))


def test_xoshiro_host_known_answers():
    """The host XoshiroRandom against the published SplitMix64 and xoshiro256** vectors
    (the same literals that pin the oracle)."""
    from test_oracle_ops import SPLITMIX64_0, SPLITMIX64_1234567, XOSHIRO256SS_1234, next_float_of
    for seed, want in ((1234567, SPLITMIX64_1234567), (0, SPLITMIX64_0)):
        r = F.XoshiroRandom(seed)
        assert [r.s.s0, r.s.s1, r.s.s2, r.s.s3] == want[:4]
    s = N.Xoshiro(1, 2, 3, 4)
    assert [N.host.fllmh_xoshiro_next(C.byref(s)) for _ in range(10)] == XOSHIRO256SS_1234
    s = N.Xoshiro(1, 2, 3, 4)
    assert [N.host.fllmh_xoshiro_next_float(C.byref(s)) for _ in range(10)] == \
        [next_float_of(v) for v in XOSHIRO256SS_1234]


def test_xoshiro_host_matches_oracle():
    for seed in (1, 42, 2 ** 63 + 5):
        a, b = F.XoshiroRandom(seed), O.Xoshiro(seed)
        for _ in range(100):
            assert a.next_uint64() == b.next()
        for _ in range(100):
            assert a.next_float() == b.next_float()


@pytest.mark.parametrize("temp,k", [(0.0, 0), (1.0, 0), (0.8, 40), (1.0, 1), (0.7, 5), (1.3, 0)])
def test_host_sampler_matches_oracle_pipeline(temp, k):
    rng = np.random.default_rng(11)
    s = F.SamplerPipeline(temp, k, 1.0, 77)
    r = O.Xoshiro(77)
    for i in range(60):
        lg = (rng.standard_normal(3000) * 3).astype(np.float32)
        if i % 3 == 0:
            lg = np.round(lg, 1)  # ties at the top-k threshold
        assert s.sample_host(lg) == O.sampler_pipeline(lg, temp, k, r)
    s.close()


@pytest.mark.parametrize("temp,k,top_p", [(1.0, 0, 0.9), (0.8, 40, 0.5), (1.2, 0, 0.05), (0.7, 200, 0.95)])
def test_host_top_p_pipeline_matches_oracle(temp, k, top_p):
    """The host pipeline (what runs over the device's top-k survivors) with top-p: the same tokens
    as the oracle's SamplerPipeline for the same seed, bit for bit (both sum in index order and
    order equal probabilities by index)."""
    rng = np.random.default_rng(12)
    s = F.SamplerPipeline(temp, k, top_p, 91)
    r = O.Xoshiro(91)
    for i in range(60):
        lg = (rng.standard_normal(3000) * 3).astype(np.float32)
        if i % 3 == 0:
            lg = np.round(lg, 1)  # ties, also at the nucleus edge
        assert s.sample_host(lg) == O.sampler_pipeline_p(lg, temp, k, top_p, r)
    s.close()


def test_sampler_argument_checks():
    with pytest.raises(F.ArgumentOutOfRangeException):
        F.SamplerPipeline(-1.0)
    for p in (0.0, 1.1):
        with pytest.raises(F.ArgumentOutOfRangeException):
            F.SamplerPipeline(1.0, 0, p)


@pytest.mark.parametrize("name", ["test-llama", "test-mistral", "test-qwen2", "test-gemma2", "test-llama-straddle"])
def test_gguf_metadata_builds_the_config(tmp_path, name):
    cfg = CONFIGS[name]
    path = str(tmp_path / f"{name}.gguf")
    write_synthetic_gguf(path, cfg)
    info = F.GgufModelLoader.read_info(path)
    want = desc_of(cfg)
    for f, _ in N.ModelDesc._fields_:
        assert getattr(info.desc, f) == pytest.approx(getattr(want, f), rel=1e-7), f
    assert info.gguf_version == 3 and info.bos_token_id == 1 and info.eos_token_id == 2
    assert info.data_offset % 32 == 0


def test_gguf_errors(tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + bytes(40))
    with pytest.raises(F.ModelLoadException):
        F.GgufModelLoader.read_info(str(bad))
    v1 = tmp_path / "v1.gguf"
    v1.write_bytes(b"GGUF" + struct.pack("<IQQ", 1, 0, 0))
    with pytest.raises(F.ModelLoadException):
        F.GgufModelLoader.read_info(str(v1))
    with pytest.raises(F.ModelLoadException):
        F.GgufModelLoader.read_info(str(tmp_path / "missing.gguf"))
    w = GgufWriter(str(tmp_path / "phi.gguf"))
    w.add("general.architecture", 8, "phi3")
    w.write()
    with pytest.raises(F.NotSupportedException):
        F.GgufModelLoader.read_info(str(tmp_path / "phi.gguf"))
    # defaults: no head_count_kv -> head_count, no context_length -> 4096, vocab from the token list
    w = GgufWriter(str(tmp_path / "min.gguf"))
    w.add("general.architecture", 8, "llama")
    for k, v in [("llama.block_count", 2), ("llama.embedding_length", 64), ("llama.feed_forward_length", 128),
                 ("llama.attention.head_count", 4)]:
        w.add(k, 4, v)
    w.add_array("tokenizer.ggml.tokens", 8, ["a", "b", "c"])
    w.write()
    info = F.GgufModelLoader.read_info(str(tmp_path / "min.gguf"))
    d = info.desc
    assert (d.n_kv_heads, d.max_ctx, d.vocab, d.head_dim, d.rope_base) == (4, 4096, 3, 16, 10000.0)
    assert d.norm_eps == pytest.approx(1e-5) and d.sliding_window == 0x7FFFFFFF
