"""Writes tests/golden/gemma2_long_window.npz: the oracle's long-context run of the Gemma-2
attention shape (test-gemma2-long: 2 layers, hidden 512, head_dim 256, 16 query / 8 kv heads,
attention softcap 50, final softcap 30, window 4096 on layer 0, an 8192-position cache, Q8_0
weights, BF16 embedding).

Workload (LlamaLanguageModel.cs:131-166): the 6200-token prompt synth_tokens(seed, 0, 512, 6200),
Forward on prompt[0..6198] at positions 0..6198, then 8 greedy steps from prompt[6199].

Stored:
  prompt        int32[6200]
  tokens        int32[8]            greedy tokens
  logits        float32[8, 512]     logits of every decode step
  kv_positions  int32[P]            positions of the stored K/V rows, around the window edge
  keys, values  float32[2, P, 2048] K/V rows of both layers at those positions (after the 8 steps)

The oracle runs row-parallel (bit-identical to one thread): about a minute on 8 cores.

    python tests/golden/make_gemma2_long.py [--threads 8]
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

PROMPT, STEPS = 6200, 8
# both sides of the window edge: layer 0 at position p attends [p - 4095, p]
KV_POSITIONS = [0, 1, 2, 2103, 2104, 2105, 4094, 4095, 4096, 4097, 6000, 6198, 6199, 6206]
OUT = os.path.join(HERE, "gemma2_long_window.npz")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    args = ap.parse_args()
    O.lib.orc_set_threads(args.threads)
    cfg, desc, tensors = synthetic("test-gemma2-long")
    prompt = F.synth_tokens(cfg["seed"], 0, desc.vocab, PROMPT)
    orc = O.OracleModel(desc, tensors, desc.max_ctx)
    t0 = time.time()
    for pos in range(PROMPT - 1):
        if orc.forward(int(prompt[pos]), pos):
            raise RuntimeError(f"forward at {pos}")
        if pos % 1000 == 0:
            print(f"position {pos}: {time.time() - t0:.0f} s", flush=True)
    nxt, toks, logits = int(prompt[-1]), [], []
    for step in range(STEPS):
        if orc.forward(nxt, PROMPT - 1 + step):
            raise RuntimeError(f"decode step {step}")
        lg = orc.logits()
        logits.append(lg)
        nxt = int(O.lib.orc_argmax(O.fp(lg), lg.size))
        toks.append(nxt)
    n = O.lib.orc_fwd_length(orc.f)
    pos = np.array(KV_POSITIONS, np.int32)
    keys = np.stack([orc.kv(l, 0).reshape(n, -1)[pos] for l in range(desc.n_layers)])
    values = np.stack([orc.kv(l, 1).reshape(n, -1)[pos] for l in range(desc.n_layers)])
    np.savez_compressed(OUT, prompt=prompt.astype(np.int32), tokens=np.array(toks, np.int32),
                        logits=np.stack(logits).astype(np.float32), kv_positions=pos,
                        keys=keys.astype(np.float32), values=values.astype(np.float32))
    srt = np.sort(np.stack(logits), axis=1)
    print(f"wrote {OUT} in {time.time() - t0:.0f} s: tokens {toks}; gaps {(srt[:, -1] - srt[:, -2]).tolist()}")
    orc.close()


if __name__ == "__main__":
    main()
