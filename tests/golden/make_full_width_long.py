"""Writes the full-width long-prompt goldens of the Qwen2-7B and Gemma-2-9B shapes at two layers.

Both run the reference's loop protocol (LlamaLanguageModel.cs:131-166: one Forward per prompt
token, then decode) on the oracle, row-parallel (bit-identical to one thread), with the real
widths of the benchmark configurations and two decoder layers:

qwen2  -> tests/golden/qwen2_7b_2l_prompt2048.npz
    qwen2-7b-q5k at 2 layers (dim 3584, 28 query / 4 kv heads x 128, FFN 18944, QKV bias, vocab
    152064, RoPE base 1e6; Q5_K projections, Q6_K LM head), the 2048-token prompt
    synth_tokens(seed, 0, vocab, 2048): Forward on prompt[0..2046], then 16 decode steps from
    prompt[2047] at position 2047, each step's token drawn by SamplerPipeline with temperature 0.8,
    top-k 40 and XoshiroRandom(SEED) (SamplerPipeline.cs:58-89, TemperatureSampler.cs:53-70,
    Qwen2ForwardPass.cs:62-103).
gemma2 -> tests/golden/gemma2_9b_2l_prompt6144.npz
    gemma2-9b-q8 at 2 layers (dim 3584, 16 query / 8 kv heads x 256, FFN 14336 GeGLU, vocab 256000,
    softcaps 50 / 30, window 4096 on layer 0; Q8_0 weights, BF16 embedding), the 6144-token prompt
    synth_tokens(seed, 0, vocab, 6144): Forward on prompt[0..6142], then 8 greedy steps from
    prompt[6143] at position 6143 (Gemma2ForwardPass.cs:86-87, 126-185).

Stored in each:
  prompt             int32[P]
  tokens             int32[S]         the decode steps' tokens (drawn / greedy)
  top_ids, top_val   int32/float32[S, 64]  the 64 largest logits of every step, in descending order
                     (ties by index): they decide top-k 40 sampling completely
  gap                float32[S]       top-1 minus top-2 logit of every step
  logits_first/last  float32[V]       all logits of the first and the last step
  kv_positions       int32[K]         positions of the stored K/V rows
  keys, values       float32[2, K, kv_dim]  K/V rows of both layers at those positions, after the run
  seed, temperature, top_k (qwen2)    the sampler's settings

    python tests/golden/make_full_width_long.py qwen2|gemma2 [--threads 8]

Runtime on 8 cores: about 3 minutes (qwen2), 10 minutes (gemma2); host memory about 7 and 10 GB.
"""
import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "tests")]

import dotnetfoundryllm_amd as F  # noqa: E402
import oracle_bind as O  # noqa: E402
from fixtures import synthetic  # noqa: E402

TOP = 64
RUNS = {
    "qwen2": dict(config="qwen2-7b-q5k", prompt=2048, steps=16, sample=(0.8, 40, 0x5EED),
                  kv_positions=[0, 1, 2, 1023, 1024, 2045, 2046, 2047, 2050, 2062],
                  out="qwen2_7b_2l_prompt2048.npz"),
    # layer 0 at position p attends [p - 4095, p]: rows on both sides of the edge of the last steps'
    # windows (2047..2055) and of the prefill's
    "gemma2": dict(config="gemma2-9b-q8", prompt=6144, steps=8, sample=None,
                   kv_positions=[0, 1, 2, 2046, 2047, 2048, 2049, 2055, 2056, 4094, 4095, 4096, 4097, 6142, 6143,
                                 6150],
                   out="gemma2_9b_2l_prompt6144.npz"),
}


def log(msg):
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("run", choices=sorted(RUNS))
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    args = ap.parse_args()
    run = RUNS[args.run]
    O.lib.orc_set_threads(args.threads)
    t0 = time.time()
    cfg, desc, tensors = synthetic(run["config"], n_layers=2)
    P, S = run["prompt"], run["steps"]
    orc = O.OracleModel(desc, tensors, P + S + 8)
    del tensors
    log(f"{run['config']} at 2 layers built in {time.time() - t0:.0f} s")
    V = desc.vocab
    prompt = F.synth_tokens(cfg["seed"], 0, V, P)
    t0 = time.time()
    for pos in range(P - 1):
        if orc.forward(int(prompt[pos]), pos):
            raise RuntimeError(f"forward at {pos}")
        if pos % 512 == 0:
            log(f"prompt position {pos} ({(time.time() - t0) / (pos + 1) * 1e3:.0f} ms per Forward)")
    rng = O.Xoshiro(run["sample"][2]) if run["sample"] else None
    tokens, gaps, top_ids, top_val = [], [], [], []
    first = last = None
    nxt = int(prompt[-1])
    for step in range(S):
        if orc.forward(nxt, P - 1 + step):
            raise RuntimeError(f"decode step {step}")
        lg = orc.logits()
        order = np.argsort(-lg, kind="stable")[:TOP]
        if rng is not None:
            temp, k, _ = run["sample"]
            nxt = O.sampler_pipeline(lg, temp, k, rng)
        else:
            nxt = int(O.lib.orc_argmax(O.fp(lg), V))
            assert nxt == int(order[0])
        tokens.append(nxt)
        gaps.append(float(lg[order[0]] - lg[order[1]]))
        top_ids.append(order.astype(np.int32))
        top_val.append(lg[order])
        if step == 0:
            first = lg
        last = lg
        log(f"step {step}: token {nxt}, gap {gaps[-1]:.4g}")
    n = O.lib.orc_fwd_length(orc.f)
    pos = np.array(run["kv_positions"], np.int32)
    assert pos.max() < n
    keys = np.stack([orc.kv(l, 0).reshape(n, -1)[pos] for l in range(desc.n_layers)])
    values = np.stack([orc.kv(l, 1).reshape(n, -1)[pos] for l in range(desc.n_layers)])
    extra = {}
    if run["sample"]:
        extra = dict(temperature=np.float32(run["sample"][0]), top_k=np.int32(run["sample"][1]),
                     seed=np.uint64(run["sample"][2]))
    out = os.path.join(HERE, run["out"])
    np.savez_compressed(out, prompt=prompt.astype(np.int32), tokens=np.array(tokens, np.int32),
                        gap=np.array(gaps, np.float32), top_ids=np.stack(top_ids),
                        top_val=np.stack(top_val).astype(np.float32), logits_first=first.astype(np.float32),
                        logits_last=last.astype(np.float32), kv_positions=pos, keys=keys.astype(np.float32),
                        values=values.astype(np.float32), **extra)
    log(f"wrote {out} in {time.time() - t0:.0f} s: tokens {tokens}")
    orc.close()


if __name__ == "__main__":
    main()
