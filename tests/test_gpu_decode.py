"""GPU parity of the decode step (IForwardPass.Forward on the device) against the oracle.

Bars (float32 accumulation): per-layer hidden states and logits within normwise relative error
1e-3; greedy token sequences identical; KV cache contents within 1e-3; graph replay
bit-identical to eager launches; error codes as the reference's exceptions.
"""
import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import dotnetfoundryllm_amd._native as N
import oracle_bind as O
from dotnetfoundryllm_amd.configs import CONFIGS, desc_of, synth_bytes, tensor_plan
from fixtures import REF_TOKENS, reference_fixture, synthetic, upload

pytestmark = pytest.mark.gpu
TOL = 1e-3


def device_model(ctx, desc, tensors):
    m = F.Model(ctx, desc)
    upload(m, tensors)
    return m


@pytest.mark.parametrize("arch", [N.ARCH_LLAMA, N.ARCH_MISTRAL, N.ARCH_QWEN2, N.ARCH_GEMMA2])
def test_reference_fixtures(ctx, arch):
    desc, tensors = reference_fixture(arch)
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    try:
        for tok, pos in REF_TOKENS:
            fwd.forward(tok, pos, kv)
            assert orc.forward(tok, pos) == 0
            got, want = fwd.logits, orc.logits()
            assert got.shape == (16,) and np.all(np.isfinite(got))
            assert O.normwise_rel_err(got, want) <= TOL
        assert kv.current_length == 3
        for l in range(desc.n_layers):
            assert O.normwise_rel_err(kv.get_keys(l), orc.kv(l, 0)) <= TOL
            assert O.normwise_rel_err(kv.get_values(l), orc.kv(l, 1)) <= TOL
    finally:
        orc.close()
        kv.close()
        m.close()


SMALL = ["test-llama", "test-llama-straddle", "test-mistral", "test-qwen2", "test-gemma2", "test-gemma2-hd256",
         "test-mixed", "test-ragged"]


@pytest.mark.parametrize("name", SMALL)
def test_small_models_hidden_logits_and_greedy(ctx, name):
    cfg, desc, tensors = synthetic(name)
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    F.set_debug(kv, True)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 1, desc.vocab, 12)
    worst = 0.0
    try:
        pos = 0
        for t in prompt:
            fwd.forward(int(t), pos, kv)
            assert orc.forward(int(t), pos) == 0
            for l in range(desc.n_layers + 1):
                worst = max(worst, O.normwise_rel_err(fwd.hidden(l), orc.hidden(l)))
            worst = max(worst, O.normwise_rel_err(fwd.logits, orc.logits()))
            pos += 1
        # greedy decode: identical tokens
        nxt_d = nxt_o = int(prompt[-1])
        for step in range(min(24, desc.max_ctx - pos)):
            fwd.forward(nxt_d, pos, kv)
            assert orc.forward(nxt_o, pos) == 0
            lg = orc.logits()
            worst = max(worst, O.normwise_rel_err(fwd.logits, lg))
            nxt_d = fwd.sample_greedy()
            nxt_o = int(O.lib.orc_argmax(O.fp(lg), lg.size))
            assert nxt_d == nxt_o, f"step {step}"
            pos += 1
        print(f"{name}: worst normwise rel err {worst:.2e}")
        assert worst <= TOL
    finally:
        orc.close()
        kv.close()
        m.close()


def test_tiny_llama_64_greedy_tokens(ctx):
    """The tiny Llama Q4_K workload: 128-token prompt, then greedy decode; the first 64 tokens
    equal the oracle's."""
    cfg, desc, tensors = synthetic("tiny-llama-q4k")
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 0, desc.vocab, 128)
    lm = F.LlamaLanguageModel(m, kv)
    sampler = F.SamplerPipeline(0.0)
    try:
        toks, stats = lm.generate(prompt, 64, sampler, stop_at_eos=False)
        assert len(toks) == 64 and stats.completion_tokens == 64
        pos = 0
        for t in prompt[:-1]:
            assert orc.forward(int(t), pos) == 0
            pos += 1
        nxt = int(prompt[-1])
        ref = []
        for _ in range(64):
            assert orc.forward(nxt, pos) == 0
            pos += 1
            lg = orc.logits()
            nxt = int(O.lib.orc_argmax(O.fp(lg), lg.size))
            ref.append(nxt)
        assert list(toks) == ref
    finally:
        sampler.close()
        orc.close()
        kv.close()
        m.close()


def test_graph_replay_matches_eager(ctx):
    cfg, desc, tensors = synthetic("test-qwen2")
    m = device_model(ctx, desc, tensors)
    kv_g, kv_e = F.HipKvCache(m), F.HipKvCache(m)
    F.set_graph(kv_e, False)
    fg, fe = F.HipForwardPass(m), F.HipForwardPass(m)
    try:
        for pos, t in enumerate(F.synth_tokens(3, 3, desc.vocab, 20)):
            fg.forward(int(t), pos, kv_g)
            fe.forward(int(t), pos, kv_e)
            assert np.array_equal(fg.logits, fe.logits)
    finally:
        kv_g.close()
        kv_e.close()
        m.close()


def test_forward_error_contract(ctx):
    cfg, desc, tensors = synthetic("test-llama")
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m, 4)
    fwd = F.HipForwardPass(m)
    try:
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.forward(desc.vocab, 0, kv)
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.forward(-1, 0, kv)
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.forward(3, 1, kv)  # position beyond the cached length: layer 0 appended, then the Slice throws
        with pytest.raises(F.InvalidOperationException):
            fwd.forward(3, 0, kv)  # the cache now expects layer 1 (KvCache.cs:69-74)
        kv.clear()
        for p in range(4):
            fwd.forward(3 + p, p, kv)
        assert kv.current_length == 4 and kv.max_sequence_length == 4 and not kv.was_evicted
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.forward(3, 4, kv)  # full: evicts the oldest half, then position 4 is past the 2 kept
        assert kv.was_evicted and kv.current_length == 2
        kv.clear()
        assert kv.current_length == 0 and not kv.was_evicted
        fwd.forward(3, 0, kv)
        assert np.all(np.isfinite(fwd.logits))
        with pytest.raises(F.ArgumentNullException):
            fwd.forward(3, 0, None)
    finally:
        kv.close()
        m.close()


def test_model_upload_contract(ctx):
    cfg, desc, tensors = synthetic("test-llama")
    m = F.Model(ctx, desc)
    try:
        entry, data = tensors["blk.0.attn_q.weight"]
        with pytest.raises(F.ArgumentException):
            m.upload(entry[1], 0, entry[3], data[:-1])
        with pytest.raises(F.ArgumentOutOfRangeException):
            m.upload(entry[1], desc.n_layers, entry[3], data)
        with pytest.raises(F.NotSupportedException):
            m.upload(entry[1], 0, 3, data)
        with pytest.raises(F.InvalidOperationException):
            m.finalize()  # required tensors missing
    finally:
        m.close()
    bad = N.ModelDesc.from_buffer_copy(desc)
    bad.n_kv_heads = 3
    with pytest.raises(F.ArgumentOutOfRangeException):
        F.Model(ctx, bad)


def test_device_sampling_matches_oracle(ctx):
    cfg, desc, tensors = synthetic("test-llama")
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    fwd.forward(1, 0, kv)
    rng = np.random.default_rng(5)
    try:
        for i in range(40):
            lg = (rng.standard_normal(desc.vocab) * 3).astype(np.float32)
            if i % 2:
                lg = np.round(lg, 1)  # ties
            if i == 7:
                lg[[3, 9]] = lg.max() + 1  # tie at the maximum: first index wins
            fwd.write_logits(lg)
            assert fwd.sample_greedy() == int(O.lib.orc_argmax(O.fp(lg), lg.size))
            for inv, k in ((1.0, 40), (1.25, 40), (2.0, 1), (0.5, 7)):
                fwd.write_logits(lg)
                ids, vals = fwd.sample_topk(inv, k, cap=desc.vocab)
                scaled = lg * np.float32(inv) if inv != 1.0 else lg.copy()
                ref = scaled.copy()
                O.lib.orc_apply_topk(O.fp(ref), ref.size, k)
                keep = np.nonzero(ref != -np.inf)[0]
                assert np.array_equal(ids, keep)
                assert np.array_equal(vals, scaled[keep])
        # the whole pipeline on device candidates draws the same tokens as the oracle
        for temp, k in ((0.8, 40), (1.0, 5), (0.0, 0)):
            sp = F.SamplerPipeline(temp, k, 1.0, 1234)
            r = O.Xoshiro(1234)
            for j in range(50):
                lg = np.round(rng.standard_normal(desc.vocab) * 2, 2).astype(np.float32)
                fwd.write_logits(lg)
                assert sp.sample(kv) == O.sampler_pipeline(lg, temp, k, r)
            sp.close()
    finally:
        kv.close()
        m.close()


@pytest.mark.parametrize("name", ["test-llama", "test-qwen2", "test-gemma2", "test-mistral"])
def test_gguf_load_path(ctx, tmp_path, name):
    from dotnetfoundryllm_amd.gguf import write_synthetic_gguf
    cfg = CONFIGS[name]
    path = str(tmp_path / f"{name}.gguf")
    write_synthetic_gguf(path, cfg)
    m1, info = F.GgufModelLoader.load(ctx, path)
    _, desc, tensors = synthetic(name)
    m2 = device_model(ctx, desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 2, desc.vocab, 10)
    outs = []
    try:
        for m in (m1, m2):
            kv = F.HipKvCache(m)
            sp = F.SamplerPipeline(0.0)
            toks, st = F.LlamaLanguageModel(m, kv).generate(prompt, 16, sp, stop_at_eos=False)
            outs.append(list(toks))
            sp.close()
            kv.close()
        assert outs[0] == outs[1]
    finally:
        m1.close()
        m2.close()


def test_llama3_8b_shape_two_layers(ctx):
    """Full Llama-3-8B shapes (dim 4096, 32/8 heads x 128, FFN 14336, vocab 128256, Q4_K + Q6_K),
    two decoder layers: logits and greedy tokens against the oracle."""
    cfg, desc, tensors = synthetic("llama3-8b-q4km", n_layers=2)
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m, 64)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors, 64)
    try:
        nxt_d = nxt_o = 1234
        for pos in range(4):
            fwd.forward(nxt_d, pos, kv)
            assert orc.forward(nxt_o, pos) == 0
            lg = orc.logits()
            err = O.normwise_rel_err(fwd.logits, lg)
            print(f"pos {pos}: normwise rel err {err:.2e}")
            assert err <= TOL
            nxt_d = fwd.sample_greedy()
            nxt_o = int(O.lib.orc_argmax(O.fp(lg), lg.size))
            assert nxt_d == nxt_o
    finally:
        orc.close()
        kv.close()
        m.close()


@pytest.mark.parametrize("name", ["qwen2-7b-q5k", "gemma2-9b-q8"])
def test_full_width_shapes_two_layers(ctx, name):
    """The other full-size configurations at full width, two decoder layers: Qwen2-7B (dim 3584,
    28/4 heads, FFN 18944, Q5_K with q/k/v bias, vocab 152064) and Gemma-2-9B (16/8 heads x 256,
    GeGLU FFN 14336, Q8_0, BF16 embedding as the tied LM head, attention and final softcaps,
    vocab 256000). A 24-token prompt through the batched prefill, then 4 decode steps: logits,
    K/V and greedy tokens against the oracle."""
    cfg, desc, tensors = synthetic(name, n_layers=2)
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m, 64)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors, 64)
    prompt = F.synth_tokens(cfg["seed"], 6, desc.vocab, 24)
    try:
        fwd.prefill(prompt[:-1], 0, kv)
        for pos, t in enumerate(prompt[:-1]):
            assert orc.forward(int(t), pos) == 0
        for l in range(desc.n_layers):
            assert O.normwise_rel_err(kv.get_keys(l), orc.kv(l, 0)) <= TOL, l
            assert O.normwise_rel_err(kv.get_values(l), orc.kv(l, 1)) <= TOL, l
        nxt_d = nxt_o = int(prompt[-1])
        for pos in range(23, 27):
            fwd.forward(nxt_d, pos, kv)
            assert orc.forward(nxt_o, pos) == 0
            lg = orc.logits()
            err = O.normwise_rel_err(fwd.logits, lg)
            print(f"{name} pos {pos}: normwise rel err {err:.2e}")
            assert err <= TOL
            nxt_d = fwd.sample_greedy()
            nxt_o = int(O.lib.orc_argmax(O.fp(lg), lg.size))
            assert nxt_d == nxt_o
    finally:
        orc.close()
        kv.close()
        m.close()


def test_profile_mode_reports_kernels(ctx):
    cfg, desc, tensors = synthetic("test-llama")
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    F.set_profile(kv, True)
    fwd = F.HipForwardPass(m)
    try:
        for p in range(3):
            fwd.forward(5, p, kv)
        ents = {e["name"]: e for e in F.profile_entries(kv)}
        # fused launches: [norm+QKV+RoPE+KV], attention, [Wo+residual], [norm+gate/up+act],
        # [down+residual] per layer, then [norm+LM head] and the argmax over its workgroups
        for name in ("attention", "attn_output", "ffn_gate_up", "ffn_down"):
            assert ents[name]["launches"] == 3 * desc.n_layers, name
        # q, k and v go out as one launch (Q4_K q, k with a Q6_K v here)
        assert ents["qkv_rope_kv"]["launches"] == 3 * desc.n_layers
        assert ents["lm_head"]["launches"] == 3 and ents["argmax"]["launches"] == 3
        assert all(e["ms"] > 0 for e in ents.values())
    finally:
        kv.close()
        m.close()


def _oracle_greedy(orc, prompt, n):
    pos = 0
    for t in prompt[:-1]:
        assert orc.forward(int(t), pos) == 0
        pos += 1
    nxt, out = int(prompt[-1]), []
    for _ in range(n):
        assert orc.forward(nxt, pos) == 0
        pos += 1
        lg = orc.logits()
        nxt = int(O.lib.orc_argmax(O.fp(lg), lg.size))
        out.append(nxt)
    return out


@pytest.mark.parametrize("name", ["test-llama", "test-qwen2", "test-gemma2", "test-mixed", "test-llama-straddle"])
@pytest.mark.parametrize("graph", [True, False])
def test_device_greedy_loop(ctx, name, graph):
    """fllm_decode_greedy (each step's argmax fed to the next step on the device) produces the
    tokens of stepwise Forward + greedy sampling, and the oracle's."""
    cfg, desc, tensors = synthetic(name)
    m = device_model(ctx, desc, tensors)
    kv_a, kv_b = F.HipKvCache(m), F.HipKvCache(m)
    F.set_graph(kv_a, graph)
    F.set_graph(kv_b, graph)
    fa, fb = F.HipForwardPass(m), F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 7, desc.vocab, 10)
    n = 20
    try:
        fa.prefill(prompt[:-1], 0, kv_a)
        fb.prefill(prompt[:-1], 0, kv_b)
        toks = fa.decode_greedy(int(prompt[-1]), len(prompt) - 1, n, kv_a)
        assert kv_a.current_length == len(prompt) - 1 + n
        step, nxt, pos = [], int(prompt[-1]), len(prompt) - 1
        for _ in range(n):
            fb.forward(nxt, pos, kv_b)
            nxt = fb.sample_greedy()
            step.append(nxt)
            pos += 1
        assert list(toks) == step
        # logits of the last step are the same as the stepwise path's
        assert np.array_equal(fa.logits, fb.logits)
        assert fa.sample_greedy() == step[-1]
        assert list(toks) == _oracle_greedy(orc, prompt, n)
    finally:
        orc.close()
        kv_a.close()
        kv_b.close()
        m.close()


def test_device_greedy_loop_errors(ctx):
    cfg, desc, tensors = synthetic("test-llama")
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m, 16)
    fwd = F.HipForwardPass(m)
    try:
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.decode_greedy(desc.vocab, 0, 4, kv)       # token outside the vocabulary
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.decode_greedy(1, 1, 4, kv)                # position beyond the cached length
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.decode_greedy(1, 0, 17, kv)               # more steps than the cache holds
        assert kv.current_length == 0
        assert len(fwd.decode_greedy(1, 0, 16, kv)) == 16
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.forward(1, 16, kv)                        # cache full
    finally:
        kv.close()
        m.close()


def test_long_context_windowed_attention(ctx):
    """Mistral-style 1000-position window over a 3000-position context with 8 KV heads: the window
    is split into position chunks whose partials the merge kernel combines; logits, K/V and greedy
    tokens against the oracle."""
    from dotnetfoundryllm_amd.configs import _cfg, _types
    cfg = _cfg("long-mistral", N.ARCH_MISTRAL, 1, 512, 8, 8, 512, 512, 4096, 10000.0,
               _types(*([N.Q4_K] * 7), N.Q6_K), window=1000, norm_std=0.1, seed=21)
    desc = desc_of(cfg)
    tensors = {e[0]: (e, synth_bytes(cfg, e)) for e in tensor_plan(cfg)}
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 2, desc.vocab, 3000)
    try:
        fwd.prefill(prompt, 0, kv)
        for pos, t in enumerate(prompt):
            assert orc.forward(int(t), pos) == 0
        assert O.normwise_rel_err(fwd.logits, orc.logits()) <= TOL
        assert O.normwise_rel_err(kv.get_keys(0), orc.kv(0, 0)) <= TOL
        assert O.normwise_rel_err(kv.get_values(0), orc.kv(0, 1)) <= TOL
        toks = fwd.decode_greedy(int(prompt[-1]), 3000, 8, kv)
        ref, pos = [], 3000
        nxt = int(prompt[-1])
        for _ in range(8):
            assert orc.forward(nxt, pos) == 0
            pos += 1
            lg = orc.logits()
            nxt = int(O.lib.orc_argmax(O.fp(lg), lg.size))
            ref.append(nxt)
        assert list(toks) == ref
    finally:
        orc.close()
        kv.close()
        m.close()



@pytest.mark.parametrize("arch", ["llama-hd128", "gemma2-hd256", "llama-g7"])
def test_long_context_many_chunks(ctx, arch):
    """More than 32 position chunks per kv head (one or two KV heads at a 4096-position capacity: 128
    chunk slots, 79 live over 2500 positions), so the four-wave merge runs: head_dim 128 in one pass
    over its streams; head_dim 256 (Gemma-2 softcaps) in two on its full-range odd layer and one on
    its even layer's 1500-position window (47 chunks); and 7 query heads per kv head.
    Logits, K/V and 8 greedy tokens against the oracle."""
    from dotnetfoundryllm_amd.configs import _cfg, _types
    if arch == "llama-hd128":
        cfg = _cfg("long-llama", N.ARCH_LLAMA, 1, 512, 4, 2, 512, 512, 4096, 10000.0,
                   _types(*([N.Q4_K] * 7), N.Q6_K), norm_std=0.1, seed=22)
    elif arch == "llama-g7":
        # 7 query heads per kv head in one attention workgroup
        cfg = _cfg("long-llama-g7", N.ARCH_LLAMA, 1, 1792, 14, 2, 512, 512, 4096, 10000.0,
                   _types(*([N.Q4_K] * 7), N.Q6_K), norm_std=0.1, seed=24)
    else:
        cfg = _cfg("long-gemma2", N.ARCH_GEMMA2, 2, 512, 2, 1, 512, 512, 4096, 10000.0,
                   _types(*([N.Q8_0] * 8)), head_dim=256, emb_type=N.BF16, window=1500, attn_softcap=50.0,
                   final_softcap=30.0, norm_std=0.1, seed=23)
    desc = desc_of(cfg)
    tensors = {e[0]: (e, synth_bytes(cfg, e)) for e in tensor_plan(cfg)}
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    n = 2500
    prompt = F.synth_tokens(cfg["seed"], 2, desc.vocab, n)
    try:
        fwd.prefill(prompt, 0, kv)
        for pos, t in enumerate(prompt):
            assert orc.forward(int(t), pos) == 0
        assert O.normwise_rel_err(fwd.logits, orc.logits()) <= TOL
        assert O.normwise_rel_err(kv.get_keys(0), orc.kv(0, 0)) <= TOL
        assert O.normwise_rel_err(kv.get_values(0), orc.kv(0, 1)) <= TOL
        toks = fwd.decode_greedy(int(prompt[-1]), n, 8, kv)
        ref, pos = [], n
        nxt = int(prompt[-1])
        for _ in range(8):
            assert orc.forward(nxt, pos) == 0
            pos += 1
            lg = orc.logits()
            nxt = int(O.lib.orc_argmax(O.fp(lg), lg.size))
            ref.append(nxt)
        assert list(toks) == ref
        assert O.normwise_rel_err(fwd.logits, lg) <= TOL
    finally:
        orc.close()
        kv.close()
        m.close()