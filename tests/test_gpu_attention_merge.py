"""The decode attention with its chunk merge inside its own launch (fllm_seq_set_attention_merge(1);
the default for at most 4 query heads per kv head and 32 chunks) against the two-launch path (chunks,
then a merge kernel) and the oracle.

ComputeAttention (LlamaForwardPass.cs:158-211, Qwen2ForwardPass.cs:62-103,
Gemma2ForwardPass.cs:126-185). In the one-launch path each chunk writes its partial output, max and
sum with write-through stores and counts itself for its kv head; the chunk that completes the count
reads the others' partials from memory and merges them. Its merge is the one-wave merge's
arithmetic, so up to 32 chunks per kv head the two paths agree bit for bit (logits and K/V cache);
past 32 the two-launch path merges with the four-wave kernel in another order, and both are held to
the oracle.

Shapes: the decode layers' q/k/v + attention shapes of Llama-3-8B (head_dim 128, 4 query heads per kv
head), Qwen2-7B (128, 7) and Gemma-2-9B (256, 2, softcaps, window 64 on the even layers) at a small
FFN and vocabulary (test-*-qkva). Cases: a batched prefill, then decode steps across a chunk
boundary; a Forward at an earlier position; the device greedy loop (graph replay); a full cache
(eviction); and 69 chunks per kv head (2 kv heads, a 2200-position cache).
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


def launches_of_one_forward(kv, fwd, tok, pos):
    """Names of the launches of one profiled Forward (eager)."""
    F.set_profile(kv, True)
    F.profile_reset(kv)
    fwd.forward(tok, pos, kv)
    names = F.profile_launches(kv)
    F.set_profile(kv, False)
    return names


@pytest.mark.parametrize("name", NAMES)
def test_merge_in_launch_equals_two_launches_and_oracle(ctx, name):
    cfg, desc, tensors = synthetic(name)
    m = F.Model(ctx, desc)
    upload(m, tensors)
    O.lib.orc_set_threads(8)
    orc = O.OracleModel(desc, tensors, desc.max_ctx)
    kva = F.HipKvCache(m, desc.max_ctx)
    kvb = F.HipKvCache(m, desc.max_ctx)
    F.set_attention_merge(kva, True)
    F.set_attention_merge(kvb, False)
    fa, fb = F.HipForwardPass(m), F.HipForwardPass(m)
    try:
        prompt = F.synth_tokens(cfg["seed"], 2, desc.vocab, 150)
        say(f"{name}: prefill of {prompt.size - 1} tokens")
        fa.prefill(prompt[:-1], 0, kva)
        fb.prefill(prompt[:-1], 0, kvb)
        for p in range(prompt.size - 1):
            assert orc.forward(int(prompt[p]), p) == 0
        nxt, pos, worst = int(prompt[-1]), prompt.size - 1, 0.0
        # positions 149 .. 168: the new row at the end (159) and the start (160) of a 32-position chunk
        for step in range(20):
            if step == 0:
                names = launches_of_one_forward(kva, fa, nxt, pos)
                assert names.count("attention") == desc.n_layers and "attention_merge" not in names, names
            else:
                fa.forward(nxt, pos, kva)
            fb.forward(nxt, pos, kvb)
            assert orc.forward(nxt, pos) == 0
            la, lb, lo = fa.logits, fb.logits, orc.logits()
            assert np.array_equal(la, lb), f"step {step}: one- and two-launch logits differ " \
                                           f"({O.normwise_rel_err(la, lb):.2e})"
            worst = max(worst, O.normwise_rel_err(la, lo))
            nxt = int(np.argmax(lo))
            pos += 1
        for l in range(desc.n_layers):
            assert np.array_equal(kva.get_keys(l), kvb.get_keys(l)) and np.array_equal(kva.get_values(l), kvb.get_values(l))
        say(f"{name}: one launch == two launches on 20 steps; worst logits error against the oracle {worst:.2e}")
        assert worst <= TOL
        back = pos - 40  # a Forward at an earlier position
        fa.forward(7, back, kva)
        fb.forward(7, back, kvb)
        assert orc.forward(7, back) == 0
        assert np.array_equal(fa.logits, fb.logits)
        assert O.normwise_rel_err(fa.logits, orc.logits()) <= TOL
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


def test_merge_in_launch_full_cache_eviction(ctx):
    """A Forward on a full cache evicts the oldest half (KvCache.cs:82-85) first: both paths and the
    oracle agree."""
    cfg, desc, tensors = synthetic("test-llama-qkva")
    cap = 70
    m = F.Model(ctx, desc)
    upload(m, tensors)
    O.lib.orc_set_threads(8)
    orc = O.OracleModel(desc, tensors, cap)
    kva, kvb = F.HipKvCache(m, cap), F.HipKvCache(m, cap)
    F.set_attention_merge(kva, True)
    F.set_attention_merge(kvb, False)
    fa, fb = F.HipForwardPass(m), F.HipForwardPass(m)
    try:
        toks = F.synth_tokens(cfg["seed"], 3, desc.vocab, cap)
        fa.prefill(toks, 0, kva)
        fb.prefill(toks, 0, kvb)
        for p in range(cap):
            assert orc.forward(int(toks[p]), p) == 0
        for tok, pos in [(40, 30), (41, 36)]:
            fa.forward(tok, pos, kva)
            fb.forward(tok, pos, kvb)
            assert orc.forward(tok, pos) == 0
            assert np.array_equal(fa.logits, fb.logits)
            assert O.normwise_rel_err(fa.logits, orc.logits()) <= TOL
        assert kva.was_evicted and kva.current_length == kvb.current_length == 37
    finally:
        O.lib.orc_set_threads(1)
        orc.close()
        kva.close()
        kvb.close()
        m.close()


@pytest.mark.parametrize("name", ["test-llama", "test-gemma2-hd256"])
def test_merge_in_launch_many_chunks(ctx, name):
    """More than 64 chunks per kv head: 2 kv heads on 256 compute units make 128 the target, and a
    2200-position cache gives 69 chunks of 32 positions, so the one-launch merge reads its partials in
    three passes of 32 and weighs them from two of its lanes' (max, sum) slots; the two-launch path
    merges them with the four-wave kernel. Head dims 64 (Llama) and 256 (Gemma-2 softcaps, window 64
    on the even layer is below the cache: only the odd layer spans every chunk). Both paths against
    the oracle after a 2100-token prefill."""
    cfg, desc, tensors = synthetic(name)
    m = F.Model(ctx, desc)
    upload(m, tensors)
    O.lib.orc_set_threads(8)
    cap = 2200
    orc = O.OracleModel(desc, tensors, cap)
    kva, kvb = F.HipKvCache(m, cap), F.HipKvCache(m, cap)
    F.set_attention_merge(kva, True)
    F.set_attention_merge(kvb, False)
    fa, fb = F.HipForwardPass(m), F.HipForwardPass(m)
    try:
        toks = F.synth_tokens(cfg["seed"], 5, desc.vocab, 2100)
        say(f"{name}: prefill of {toks.size - 1} tokens into a {cap}-position cache")
        fa.prefill(toks[:-1], 0, kva)
        fb.prefill(toks[:-1], 0, kvb)
        for p in range(toks.size - 1):
            assert orc.forward(int(toks[p]), p) == 0
        nxt, pos, worst, diff = int(toks[-1]), toks.size - 1, 0.0, 0.0
        for step in range(6):
            fa.forward(nxt, pos, kva)
            fb.forward(nxt, pos, kvb)
            assert orc.forward(nxt, pos) == 0
            lo = orc.logits()
            worst = max(worst, O.normwise_rel_err(fa.logits, lo), O.normwise_rel_err(fb.logits, lo))
            diff = max(diff, O.normwise_rel_err(fa.logits, fb.logits))
            nxt = int(np.argmax(lo))
            pos += 1
        say(f"{name}: against the oracle {worst:.2e}; one launch against two {diff:.2e}")
        assert worst <= TOL and diff <= 1e-5
    finally:
        O.lib.orc_set_threads(1)
        orc.close()
        kva.close()
        kvb.close()
        m.close()


@pytest.mark.parametrize("name", NAMES)
def test_default_choice(ctx, name):
    """By default the merge runs inside the attention launch for at most 4 query heads per kv head and
    32 chunks (the Llama-3-8B and Gemma-2-9B groups), in a second launch for Qwen2-7B's 7."""
    cfg, desc, tensors = synthetic(name)
    m = F.Model(ctx, desc)
    upload(m, tensors)
    kv = F.HipKvCache(m, desc.max_ctx)
    fwd = F.HipForwardPass(m)
    try:
        names = launches_of_one_forward(kv, fwd, 3, 0)
        separate = desc.n_heads // desc.n_kv_heads > 4
        assert names.count("attention") == desc.n_layers
        assert names.count("attention_merge") == (desc.n_layers if separate else 0), names
    finally:
        kv.close()
        m.close()
