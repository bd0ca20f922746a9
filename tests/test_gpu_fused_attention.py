"""The decode layer's q/k/v projection and attention in one launch (fllm_seq_set_fused_attention)
against the three-launch path (q/k/v; attention chunks; merge) and the oracle.

ComputeAttention (LlamaForwardPass.cs:158-211, Qwen2ForwardPass.cs:62-103,
Gemma2ForwardPass.cs:126-185) with the q/k/v projections before it (LlamaForwardPass.cs:99-110).
The fused launch reads the step's q and the K/V row it wrote from other workgroups of the same
grid; every other number is computed the same way as in the three launches, and the merge of at
most 32 chunks is the one-wave merge's arithmetic, so the two paths agree bit for bit (logits and
K/V cache). The oracle bounds both at the parity bar.

Shapes: the q/k/v + attention shapes of Llama-3-8B, Qwen2-7B and Gemma-2-9B at a small FFN and
vocabulary (test-*-qkva, three layers: the first layer's input is the embedding row, so the fused
kernels run on the later ones for Llama and Qwen2 and on all of them for Gemma-2). Cases: a batched
prefill then decode steps whose new row falls at the end and at the start of a 32-position chunk;
a Forward at an earlier position (the new row outside the attended range); a full cache (eviction,
the new row at the kept length); the device greedy loop (graph replay).
"""
import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import oracle_bind as O
from fixtures import synthetic, upload

pytestmark = pytest.mark.gpu
TOL = 1e-3
NAMES = ["test-llama-qkva", "test-qwen2-qkva", "test-gemma2-qkva"]


def say(msg):
    import sys
    print(msg, file=sys.stderr, flush=True)


def launched_fused(kv, fwd, tok, pos):
    """Names of the launches of one profiled Forward (eager)."""
    F.set_profile(kv, True)
    F.profile_reset(kv)
    fwd.forward(tok, pos, kv)
    names = F.profile_launches(kv)
    F.set_profile(kv, False)
    return names


@pytest.mark.parametrize("name", NAMES)
def test_fused_equals_three_launches_and_oracle(ctx, name):
    cfg, desc, tensors = synthetic(name)
    m = F.Model(ctx, desc)
    upload(m, tensors)
    O.lib.orc_set_threads(8)
    orc = O.OracleModel(desc, tensors, desc.max_ctx)
    kva = F.HipKvCache(m, desc.max_ctx)
    kvb = F.HipKvCache(m, desc.max_ctx)
    F.set_fused_attention(kvb, False)
    fa, fb = F.HipForwardPass(m), F.HipForwardPass(m)
    try:
        prompt = F.synth_tokens(cfg["seed"], 2, desc.vocab, 150)
        say(f"{name}: prefill of {prompt.size - 1} tokens, fused and three-launch")
        fa.prefill(prompt[:-1], 0, kva)
        fb.prefill(prompt[:-1], 0, kvb)
        for p in range(prompt.size - 1):
            assert orc.forward(int(prompt[p]), p) == 0
        nxt, pos, worst = int(prompt[-1]), prompt.size - 1, 0.0
        # positions 149 .. 168: the new row at the end (159) and the start (160) of a 32-position chunk
        for step in range(20):
            if step == 0:
                # one launch per layer whose input is a table (Llama, Qwen2: all but the first) or a
                # vector the prologue normalizes (Gemma-2: all)
                names = launched_fused(kva, fa, nxt, pos)
                want = desc.n_layers if name == "test-gemma2-qkva" else desc.n_layers - 1
                assert names.count("qkv_attention") == want, names
            else:
                fa.forward(nxt, pos, kva)
            fb.forward(nxt, pos, kvb)
            assert orc.forward(nxt, pos) == 0
            la, lb, lo = fa.logits, fb.logits, orc.logits()
            assert np.array_equal(la, lb), f"step {step}: fused and three-launch logits differ " \
                                           f"({O.normwise_rel_err(la, lb):.2e})"
            worst = max(worst, O.normwise_rel_err(la, lo))
            nxt = int(np.argmax(lo))
            pos += 1
        for l in range(desc.n_layers):
            assert np.array_equal(kva.get_keys(l), kvb.get_keys(l)) and np.array_equal(kva.get_values(l), kvb.get_values(l))
            assert O.normwise_rel_err(kva.get_keys(l), orc.kv(l, 0)) <= TOL
            assert O.normwise_rel_err(kva.get_values(l), orc.kv(l, 1)) <= TOL
        say(f"{name}: fused == three-launch on 20 steps; worst logits error against the oracle {worst:.2e}")
        assert worst <= TOL
        # a Forward at an earlier position: the new row (at the current length) is outside the
        # attended range [.., pos]
        back = pos - 40
        fa.forward(7, back, kva)
        fb.forward(7, back, kvb)
        assert orc.forward(7, back) == 0
        assert np.array_equal(fa.logits, fb.logits)
        assert O.normwise_rel_err(fa.logits, orc.logits()) <= TOL
        # the device greedy loop from both
        ta = fa.decode_greedy(11, pos + 1, 12, kva)
        tb = fb.decode_greedy(11, pos + 1, 12, kvb)
        assert list(ta) == list(tb)
        assert np.array_equal(fa.logits, fb.logits)
    finally:
        O.lib.orc_set_threads(1)
        orc.close()
        kva.close()
        kvb.close()
        m.close()


def test_fused_full_cache_eviction(ctx):
    """A Forward on a full cache evicts the oldest half (KvCache.cs:82-85), so the new row goes to the
    kept length, not to the position: both paths and the oracle agree."""
    cfg, desc, tensors = synthetic("test-llama-qkva")
    cap = 70
    m = F.Model(ctx, desc)
    upload(m, tensors)
    O.lib.orc_set_threads(8)
    orc = O.OracleModel(desc, tensors, cap)
    kva, kvb = F.HipKvCache(m, cap), F.HipKvCache(m, cap)
    F.set_fused_attention(kvb, False)
    fa, fb = F.HipForwardPass(m), F.HipForwardPass(m)
    try:
        toks = F.synth_tokens(cfg["seed"], 3, desc.vocab, cap)
        fa.prefill(toks, 0, kva)
        fb.prefill(toks, 0, kvb)
        for p in range(cap):
            assert orc.forward(int(toks[p]), p) == 0
        # full: keep 35 positions, the new row at slot 35, attention over positions [0, 30]
        for tok, pos in [(40, 30), (41, 36)]:
            fa.forward(tok, pos, kva)
            fb.forward(tok, pos, kvb)
            assert orc.forward(tok, pos) == 0
            assert np.array_equal(fa.logits, fb.logits)
            assert O.normwise_rel_err(fa.logits, orc.logits()) <= TOL
        assert kva.was_evicted and kva.current_length == kvb.current_length == 37
        for l in range(desc.n_layers):
            assert np.array_equal(kva.get_keys(l), kvb.get_keys(l))
    finally:
        O.lib.orc_set_threads(1)
        orc.close()
        kva.close()
        kvb.close()
        m.close()
