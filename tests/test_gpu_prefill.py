"""GPU parity of the batched prefill (fllm_prefill with a prompt that continues the cache).

The contract is that of n consecutive Forward calls (LlamaLanguageModel.cs:133-137): the K/V rows
of every position, the last position's logits and its greedy token. The batched path runs the
projections as matrix-core GEMMs over all tokens and a causal attention over the cache, so its
results are compared with the oracle and with the per-token path within the f32 bar (normwise
relative error 1e-3), and the greedy tokens that follow must be the oracle's.
"""
import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import dotnetfoundryllm_amd._native as N
import oracle_bind as O
from dotnetfoundryllm_amd.configs import desc_of, synth_bytes, tensor_plan
from fixtures import synthetic, upload

pytestmark = pytest.mark.gpu
TOL = 1e-3


def device_model(ctx, desc, tensors):
    m = F.Model(ctx, desc)
    upload(m, tensors)
    return m


def _oracle_prefill(orc, prompt):
    for pos, t in enumerate(prompt):
        assert orc.forward(int(t), pos) == 0


def _oracle_continue(orc, first, pos, n):
    nxt, out = int(first), []
    for _ in range(n):
        assert orc.forward(nxt, pos) == 0
        pos += 1
        lg = orc.logits()
        nxt = int(O.lib.orc_argmax(O.fp(lg), lg.size))
        out.append(nxt)
    return out


SMALL = ["test-llama", "test-llama-straddle", "test-mistral", "test-qwen2", "test-gemma2", "test-gemma2-hd256",
         "test-mixed", "test-ragged", "test-wide-ffn"]


@pytest.mark.parametrize("name", SMALL)
def test_batched_prefill_matches_oracle_and_stepwise(ctx, name):
    cfg, desc, tensors = synthetic(name)
    m = device_model(ctx, desc, tensors)
    kv_b, kv_s = F.HipKvCache(m), F.HipKvCache(m)
    fb, fs = F.HipForwardPass(m), F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    n = min(40, desc.max_ctx - 10)
    prompt = F.synth_tokens(cfg["seed"], 5, desc.vocab, n)
    try:
        fb.prefill(prompt, 0, kv_b)  # batched
        for pos, t in enumerate(prompt):
            fs.forward(int(t), pos, kv_s)  # one step per token
        _oracle_prefill(orc, prompt)
        assert kv_b.current_length == n == kv_s.current_length
        want = orc.logits()
        assert O.normwise_rel_err(fb.logits, want) <= TOL
        assert O.normwise_rel_err(fb.logits, fs.logits) <= TOL
        for l in range(desc.n_layers):
            for kind, get in ((0, kv_b.get_keys), (1, kv_b.get_values)):
                got = get(l)
                assert O.normwise_rel_err(got, orc.kv(l, kind)) <= TOL, (l, kind)
        assert fb.sample_greedy() == int(O.lib.orc_argmax(O.fp(want), want.size))
        # decoding after the batched prefill gives the oracle's greedy tokens
        steps = min(8, desc.max_ctx - n - 1)
        toks = fb.decode_greedy(int(prompt[-1]), n, steps, kv_b)
        assert list(toks) == _oracle_continue(orc, prompt[-1], n, steps)
    finally:
        orc.close()
        kv_b.close()
        kv_s.close()
        m.close()


@pytest.mark.parametrize("name,cap,n", [("test-llama", 256, 200), ("test-qwen2", 256, 200), ("test-gemma2", 256, 200),
                                        ("test-gemma2", 1280, 1100), ("test-gemma2-hd256", 256, 200),
                                        ("test-mistral", 256, 200)])
def test_batched_prefill_split_attention(ctx, name, cap, n):
    """A prompt of several query blocks with a partial last one (200 tokens: blocks of 64, 64, 64,
    8; 1100: 17 blocks and 12) into a 256- (1280-) position cache: the prefill attention runs every
    block but the first as two halves of its key range plus a merge when all halves fit the
    resident workgroups, as here. Head dim 64 (Llama; Qwen2 with its q/k/v bias; Mistral with its
    window) on the f32 kernel, 128 (Gemma-2: softcaps, window on the even layer; also over 1100
    keys) and 256 on the fp16 kernel over the K / V planes. Logits and every K/V row against the
    oracle, then greedy decode."""
    cfg, desc, tensors = synthetic(name)
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m, cap)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors, cap)
    prompt = F.synth_tokens(cfg["seed"], 7, desc.vocab, n)
    try:
        fwd.prefill(prompt, 0, kv)
        _oracle_prefill(orc, prompt)
        want = orc.logits()
        err = O.normwise_rel_err(fwd.logits, want)
        print(f"{name}: {n} tokens, logits normwise rel err {err:.2e}")
        assert err <= TOL
        for l in range(desc.n_layers):
            assert O.normwise_rel_err(kv.get_keys(l), orc.kv(l, 0)) <= TOL, l
            assert O.normwise_rel_err(kv.get_values(l), orc.kv(l, 1)) <= TOL, l
        toks = fwd.decode_greedy(int(prompt[-1]), n, 4, kv)
        assert list(toks) == _oracle_continue(orc, prompt[-1], n, 4)
    finally:
        orc.close()
        kv.close()
        m.close()


def test_prefill_chunk_contract(ctx):
    """fllm_seq_set_prefill_chunk: tokens < 1 is out of range; a chunk of 24 tokens takes a 61-token
    prompt in passes of 24, 24 and 13 (logits, K/V and the greedy token against the oracle); after
    it, a chunk of 40 makes the next prefill replace the 24-row scratch with a 40-row one, and a
    30-token prompt in one pass stores the same K/V rows as the oracle's first 30 positions."""
    cfg, desc, tensors = synthetic("test-llama")
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 5, desc.vocab, 61)
    try:
        for bad in (0, -5):
            with pytest.raises(F.ArgumentOutOfRangeException):
                F.set_prefill_chunk(kv, bad)
        F.set_prefill_chunk(kv, 100)
        F.set_prefill_chunk(kv, 24)  # another value before the first prefill
        fwd.prefill(prompt, 0, kv)
        _oracle_prefill(orc, prompt)
        want = orc.logits()
        assert O.normwise_rel_err(fwd.logits, want) <= TOL
        for l in range(desc.n_layers):
            assert O.normwise_rel_err(kv.get_keys(l), orc.kv(l, 0)) <= TOL
            assert O.normwise_rel_err(kv.get_values(l), orc.kv(l, 1)) <= TOL
        assert fwd.sample_greedy() == int(O.lib.orc_argmax(O.fp(want), want.size))
        F.set_prefill_chunk(kv, 40)
        kv.clear()
        fwd.prefill(prompt[:30], 0, kv)
        assert kv.current_length == 30
        kvdim = desc.n_kv_heads * desc.head_dim
        for l in range(desc.n_layers):
            for got, kind in ((kv.get_keys(l), 0), (kv.get_values(l), 1)):
                assert O.normwise_rel_err(got, orc.kv(l, kind)[: 30 * kvdim]) <= TOL, (l, kind)
    finally:
        orc.close()
        kv.close()
        m.close()


@pytest.mark.parametrize("chunk", [512, None], ids=["chunk-512", "chunk-default"])
def test_batched_prefill_several_chunks(ctx, chunk):
    """1100 tokens go through the layers in chunks of 512, 512 and 76: every chunk attends to the
    rows the earlier chunks stored (and, with the default chunk, in one pass). No window; K/V of the
    first, a middle and the last position and the logits against the oracle."""
    from dotnetfoundryllm_amd.configs import _cfg, _types
    cfg = _cfg("chunks-llama", N.ARCH_LLAMA, 2, 256, 4, 2, 512, 512, 1200, 10000.0,
               _types(N.Q4_K, N.Q4_K, N.Q6_K, N.Q4_K, N.Q4_K, N.Q4_K, N.Q6_K, N.Q6_K), norm_std=0.1, seed=23)
    desc = desc_of(cfg)
    tensors = {e[0]: (e, synth_bytes(cfg, e)) for e in tensor_plan(cfg)}
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 3, desc.vocab, 1100)
    try:
        if chunk:
            F.set_prefill_chunk(kv, chunk)
        fwd.prefill(prompt, 0, kv)
        _oracle_prefill(orc, prompt)
        assert kv.current_length == 1100
        assert O.normwise_rel_err(fwd.logits, orc.logits()) <= TOL
        for l in range(desc.n_layers):
            k, v = kv.get_keys(l), kv.get_values(l)
            kr, vr = orc.kv(l, 0), orc.kv(l, 1)
            assert O.normwise_rel_err(k, kr) <= TOL and O.normwise_rel_err(v, vr) <= TOL
            kvdim = desc.n_kv_heads * desc.head_dim
            for pos in (0, 600, 1099):
                row = slice(pos * kvdim, (pos + 1) * kvdim)
                assert O.normwise_rel_err(k[row], kr[row]) <= TOL, (l, pos)
        toks = fwd.decode_greedy(int(prompt[-1]), 1100, 6, kv)
        assert list(toks) == _oracle_continue(orc, prompt[-1], 1100, 6)
    finally:
        orc.close()
        kv.close()
        m.close()


@pytest.mark.parametrize("chunk", [512, None], ids=["chunk-512", "chunk-default"])
@pytest.mark.parametrize("arch", [N.ARCH_MISTRAL, N.ARCH_GEMMA2])
def test_batched_prefill_window_across_chunks(ctx, arch, chunk):
    """A sliding window of 700 over a 1100-token prompt (chunks of 512, 512, 76, or one pass with the
    default chunk): from position 700 on, the first keys a row may attend are in an earlier chunk, so
    the window start of the batched attention is checked against keys other chunks stored (Mistral:
    every layer windowed; Gemma-2: the even layer, with softcaps). Logits, K/V rows on both sides of
    the edge and the greedy tokens after it against the oracle."""
    from dotnetfoundryllm_amd.configs import _cfg, _types
    if arch == N.ARCH_MISTRAL:
        cfg = _cfg("window-mistral", arch, 2, 256, 4, 2, 512, 512, 1200, 10000.0, _types(*([N.Q8_0] * 8)),
                   window=700, norm_std=0.1, seed=24)
    else:
        cfg = _cfg("window-gemma2", arch, 2, 256, 4, 2, 512, 512, 1200, 10000.0, _types(*([N.Q8_0] * 8)),
                   head_dim=128, emb_type=N.BF16, window=700, attn_softcap=50.0, final_softcap=30.0,
                   norm_std=0.1, seed=25)
    desc = desc_of(cfg)
    tensors = {e[0]: (e, synth_bytes(cfg, e)) for e in tensor_plan(cfg)}
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 3, desc.vocab, 1100)
    try:
        if chunk:
            F.set_prefill_chunk(kv, chunk)
        fwd.prefill(prompt, 0, kv)
        _oracle_prefill(orc, prompt)
        assert kv.current_length == 1100
        assert O.normwise_rel_err(fwd.logits, orc.logits()) <= TOL
        kvdim = desc.n_kv_heads * desc.head_dim
        for l in range(desc.n_layers):
            k, v = kv.get_keys(l), kv.get_values(l)
            kr, vr = orc.kv(l, 0), orc.kv(l, 1)
            assert O.normwise_rel_err(k, kr) <= TOL and O.normwise_rel_err(v, vr) <= TOL
            for pos in (0, 511, 512, 699, 700, 701, 1023, 1024, 1099):
                row = slice(pos * kvdim, (pos + 1) * kvdim)
                assert O.normwise_rel_err(k[row], kr[row]) <= TOL, (l, pos)
                assert O.normwise_rel_err(v[row], vr[row]) <= TOL, (l, pos)
        toks = fwd.decode_greedy(int(prompt[-1]), 1100, 6, kv)
        assert list(toks) == _oracle_continue(orc, prompt[-1], 1100, 6)
    finally:
        orc.close()
        kv.close()
        m.close()


def test_batched_prefill_llama3_8b_shape(ctx):
    """Full Llama-3-8B shapes (Q4_K + Q6_K, tile-interleaved weights), two layers, a 24-token
    prompt: logits, K/V and the next greedy tokens against the oracle."""
    cfg, desc, tensors = synthetic("llama3-8b-q4km", n_layers=2)
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m, 64)
    fwd = F.HipForwardPass(m)
    orc = O.OracleModel(desc, tensors, 64)
    prompt = F.synth_tokens(cfg["seed"], 4, desc.vocab, 24)
    try:
        fwd.prefill(prompt, 0, kv)
        _oracle_prefill(orc, prompt)
        err = O.normwise_rel_err(fwd.logits, orc.logits())
        print(f"logits normwise rel err {err:.2e}")
        assert err <= TOL
        for l in range(desc.n_layers):
            assert O.normwise_rel_err(kv.get_keys(l), orc.kv(l, 0)) <= TOL
            assert O.normwise_rel_err(kv.get_values(l), orc.kv(l, 1)) <= TOL
        toks = fwd.decode_greedy(int(prompt[-1]), 24, 3, kv)
        assert list(toks) == _oracle_continue(orc, prompt[-1], 24, 3)
    finally:
        orc.close()
        kv.close()
        m.close()


def test_prefill_argument_contract(ctx):
    """Out-of-range tokens and a prompt beyond the cache fail before anything runs; a prompt that
    does not continue the cache takes the per-token path with the Forward checks."""
    cfg, desc, tensors = synthetic("test-llama")
    m = device_model(ctx, desc, tensors)
    kv = F.HipKvCache(m, 16)
    fwd = F.HipForwardPass(m)
    try:
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.prefill(np.array([1, desc.vocab, 2], dtype=np.int32), 0, kv)
        assert kv.current_length == 0
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.prefill(np.arange(17, dtype=np.int32), 0, kv)
        assert kv.current_length == 0
        fwd.prefill(np.arange(16, dtype=np.int32), 0, kv)
        assert kv.current_length == 16
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.prefill(np.array([1, 2], dtype=np.int32), 16, kv)  # cache full
    finally:
        kv.close()
        m.close()
