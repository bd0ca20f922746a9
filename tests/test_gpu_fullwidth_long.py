"""Full-width long-prompt parity of the Qwen2-7B and Gemma-2-9B shapes against the oracle's goldens
(tests/golden/make_full_width_long.py), at two decoder layers and the benchmark configurations' own
prompt lengths.

- Qwen2-7B (dim 3584, 28 / 4 heads x 128, FFN 18944, QKV bias, vocab 152064, Q5_K + Q6_K head;
  Qwen2ForwardPass.cs:62-103): the 2048-token prompt through fllm_prefill, then 16 decode steps fed the
  oracle's tokens. Every step's 64 largest oracle logits are checked on the device logits; the first
  and last steps' logits normwise; K/V rows at ten positions. Then SamplerPipeline(temperature 0.8,
  top-k 40, the golden seed; SamplerPipeline.cs:58-89, TemperatureSampler.cs:53-70) runs on the
  device over each step's golden logits and draws the oracle's 16 tokens. The 64 largest logits
  decide top-k 40 completely (the 40th is above the 64th), so they are written with every other entry
  far below them.
- Gemma-2-9B (dim 3584, 16 / 8 heads x 256, FFN 14336 GeGLU, softcaps 50 / 30, window 4096 on layer
  0, Q8_0 + BF16 embedding; Gemma2ForwardPass.cs:86-87, 126-185): the 6144-token prompt through
  fllm_prefill (one 4096-token pass and one of 2047), then 8 steps fed the oracle's tokens, each
  step's logits normwise and K/V rows on both sides of the window edge. The seeded model's final
  logits sit on the softcap's plateau (top-1 about 29.99999, top-1/top-2 gaps of 0 to 8e-6, below
  float32 accumulation noise), so its greedy tokens are ties: the logits carry the check.
"""
import os
import sys

import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import oracle_bind as O
from fixtures import synthetic, upload

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 1e-3
TIGHT = 5e-5  # regression bar, far inside the parity bar


def say(msg):
    print(msg, file=sys.stderr, flush=True)


def build(ctx, name):
    cfg, desc, tensors = synthetic(name, n_layers=2)
    m = F.Model(ctx, desc)
    upload(m, tensors)
    return cfg, desc, m


def check_kv(kv, g, desc):
    pos = g["kv_positions"]
    worst = 0.0
    for l in range(desc.n_layers):
        K = kv.get_keys(l).reshape(kv.current_length, -1)[pos]
        V = kv.get_values(l).reshape(kv.current_length, -1)[pos]
        for j, p in enumerate(pos):
            ek = O.normwise_rel_err(K[j], g["keys"][l][j])
            ev = O.normwise_rel_err(V[j], g["values"][l][j])
            worst = max(worst, ek, ev)
            assert ek <= TOL and ev <= TOL, f"layer {l} position {p}: K {ek:.2e} V {ev:.2e}"
    return worst


def test_qwen2_7b_prompt2048_full_width(ctx):
    g = np.load(os.path.join(HERE, "golden", "qwen2_7b_2l_prompt2048.npz"))
    cfg, desc, m = build(ctx, "qwen2-7b-q5k")
    prompt, toks = g["prompt"], [int(t) for t in g["tokens"]]
    assert np.array_equal(prompt, F.synth_tokens(cfg["seed"], 0, desc.vocab, prompt.size))
    P, S = prompt.size, len(toks)
    kv = F.HipKvCache(m, P + S + 8)
    fwd = F.HipForwardPass(m)
    try:
        say(f"qwen2-7b at 2 layers: prefill of {P - 1} tokens")
        fwd.prefill(prompt[:-1], 0, kv)
        nxt, worst_top, worst_gap = int(prompt[-1]), 0.0, 0.0
        for step in range(S):
            fwd.forward(nxt, P - 1 + step, kv)
            lg = fwd.logits
            if step == 0:
                e_first = O.normwise_rel_err(lg, g["logits_first"])
            if step == S - 1:
                e_last = O.normwise_rel_err(lg, g["logits_last"])
            ids, vals = g["top_ids"][step], g["top_val"][step]
            top_abs = float(np.max(np.abs(lg[ids] - vals)))
            worst_top = max(worst_top, top_abs / float(np.max(np.abs(vals))))
            worst_gap = max(worst_gap, top_abs / float(g["gap"][step]))
            nxt = toks[step]  # the oracle's draw
        e_kv = check_kv(kv, g, desc)
        say(f"logits: first {e_first:.2e}, last {e_last:.2e}, top-64 {worst_top:.2e} (at most {worst_gap:.2e} of the "
            f"top-1/top-2 gap); K/V rows {e_kv:.2e}")
        assert e_first <= TIGHT and e_last <= TIGHT and worst_top <= TIGHT and worst_gap < 0.1
        # the device sampler over the golden logits draws the oracle's tokens
        temp, k, seed = float(g["temperature"]), int(g["top_k"]), int(g["seed"])
        sampler = F.SamplerPipeline(temp, k, 1.0, seed)
        try:
            for step in range(S):
                vals = g["top_val"][step]
                assert vals[k - 1] > vals[-1]  # no tie of the k-th largest beyond the stored 64
                full = np.full(desc.vocab, -1e30, dtype=np.float32)
                full[g["top_ids"][step]] = vals
                fwd.write_logits(full, kv)
                assert sampler.sample(kv) == toks[step], f"sampled token at step {step}"
        finally:
            sampler.close()
    finally:
        kv.close()
        m.close()


def test_gemma2_9b_prompt6144_full_width(ctx):
    g = np.load(os.path.join(HERE, "golden", "gemma2_9b_2l_prompt6144.npz"))
    cfg, desc, m = build(ctx, "gemma2-9b-q8")
    prompt, toks = g["prompt"], [int(t) for t in g["tokens"]]
    assert np.array_equal(prompt, F.synth_tokens(cfg["seed"], 0, desc.vocab, prompt.size))
    P, S = prompt.size, len(toks)
    kv = F.HipKvCache(m, P + S + 8)
    fwd = F.HipForwardPass(m)
    try:
        say(f"gemma2-9b at 2 layers: prefill of {P - 1} tokens")
        fwd.prefill(prompt[:-1], 0, kv)
        nxt, worst = int(prompt[-1]), 0.0
        for step in range(S):
            fwd.forward(nxt, P - 1 + step, kv)
            lg = fwd.logits
            if step == 0:
                worst = max(worst, O.normwise_rel_err(lg, g["logits_first"]))
            if step == S - 1:
                worst = max(worst, O.normwise_rel_err(lg, g["logits_last"]))
            ids, vals = g["top_ids"][step], g["top_val"][step]
            worst = max(worst, float(np.max(np.abs(lg[ids] - vals))) / float(np.max(np.abs(vals))))
            nxt = toks[step]
        e_kv = check_kv(kv, g, desc)
        say(f"logits worst {worst:.2e}; K/V rows {e_kv:.2e}")
        assert worst <= TIGHT
    finally:
        kv.close()
        m.close()
