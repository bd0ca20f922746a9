"""Decode benchmark: Llama-3-8B-shaped Q4_K/Q6_K model at batch 1 on one MI355X.

Workload: random-init weights of the Llama-3-8B shape (dim 4096, 32 layers, 32/8 heads x 128,
FFN 14336, vocab 128256; Q4_K for q/k/o/gate/up, Q6_K for v/down/output) generated from a
seed, a 512-token random prompt prefilled token by token, then greedy decode at batch 1.
A "step" is one decode token: the forward pass and the greedy argmax. The timed steps run as a
device-side loop (each step's argmax is the next step's input token on the device, one graph
launch per step, the tokens are read back after the last step); the same tokens come out of the
host loop (forward + argmax + 4-byte read-back per token), whose rate is reported beside it.

Prints one JSON line with the decode throughput, a roofline entry for the dominant kernel
(algorithmic bytes per launch / mean launch time from HIP events in a profiled pass of the
same decode steps) and a CPU baseline (the oracle's reference-order F32 forward pass on a
bounded sample, one thread). Progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(cfg_name, ctx_positions=8):
    """The oracle (reference-order restatement, F32 weights dequantized at load, one thread) on a
    bounded sample of the same workload: one decoder layer of the model shape and 1/16 of the
    LM-head rows, timed separately and scaled to a whole token."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np

    import oracle_bind as O
    from dotnetfoundryllm_amd.configs import CONFIGS, desc_of, synth_bytes, tensor_plan

    cfg = dict(CONFIGS[cfg_name])
    full_layers = cfg["n_layers"]
    cfg["n_layers"] = 1
    tensors = {e[0]: (e, synth_bytes(cfg, e)) for e in tensor_plan(cfg)}
    desc = desc_of(cfg)
    t0 = time.time()
    m = O.OracleModel(desc, tensors, 64)
    load_s = time.time() - t0
    del tensors
    head_rows = desc.vocab // 16
    try:
        m.limit(1, 0)
        for p in range(2):
            m.forward(11 + p, p)
        t = time.perf_counter()
        for p in range(2, 2 + ctx_positions):
            m.forward(11 + p, p)
        t_layer = (time.perf_counter() - t) / ctx_positions
        m.reset()
        m.limit(1, head_rows)
        for p in range(2):
            m.forward(11 + p, p)
        t = time.perf_counter()
        for p in range(2, 2 + ctx_positions):
            m.forward(11 + p, p)
        t_mixed = (time.perf_counter() - t) / ctx_positions
    finally:
        m.close()
    t_head = max(t_mixed - t_layer, 0.0) * (desc.vocab / head_rows)
    t_token = full_layers * t_layer + t_head
    return {
        "value": round(1.0 / t_token, 4),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle F32 forward (weights dequantized at load, reference operation order), one thread: "
                   f"1 decoder layer x {full_layers} ({t_layer * 1e3:.1f} ms) + {head_rows}/{desc.vocab} LM-head "
                   f"rows scaled x16 ({t_head * 1e3:.1f} ms), {ctx_positions} positions each; load {load_s:.1f} s"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode tokens before the timed ones")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--config", default="llama3-8b-q4km")
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--host-steps", type=int, default=32, help="steps of the host-driven loop timed after the device loop")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the decode path runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)

    import dotnetfoundryllm_amd as F
    from dotnetfoundryllm_amd.configs import CONFIGS, build_model, weight_bytes_per_token

    cfg = CONFIGS[args.config]
    layer_bytes, head_bytes = weight_bytes_per_token(cfg)
    tok_bytes = layer_bytes + head_bytes
    ctx = F.Context(0)
    n_cu, hbm = ctx.device_info()
    log(f"device: {n_cu} CUs, {hbm / 2**30:.0f} GiB; building {cfg['name']} ({tok_bytes / 1e9:.3f} GB of weights)")
    t = time.time()
    model, _ = build_model(ctx, cfg)
    log(f"weights generated and uploaded in {time.time() - t:.1f} s")
    max_seq = min(cfg["max_ctx"], args.prompt + args.warmup + args.steps + args.host_steps + args.profile_steps + 8)
    kv = F.HipKvCache(model, max_seq)
    if args.no_graph:
        F.set_graph(kv, False)
    fwd = F.HipForwardPass(model)
    prompt = F.synth_tokens(cfg["seed"], 0, cfg["vocab"], args.prompt)

    # prefill: Forward on prompt[0..n-2] (LlamaLanguageModel.cs:133-137)
    t = time.perf_counter()
    fwd.prefill(prompt[:-1], 0, kv)
    ctx.sync()
    F._check(F.N.dev.fllm_seq_sync(kv.h))
    prefill_s = time.perf_counter() - t
    pos = args.prompt - 1
    log(f"prefill {args.prompt - 1} tokens in {prefill_s:.2f} s")

    nxt = int(prompt[-1])
    warm = fwd.decode_greedy(nxt, pos, args.warmup, kv) if args.warmup else []
    pos += args.warmup
    nxt = int(warm[-1]) if len(warm) else nxt
    log(f"warmup {args.warmup} steps done; timing {args.steps} decode steps")

    F._check(F.N.dev.fllm_seq_sync(kv.h))
    t0 = time.perf_counter()
    toks = fwd.decode_greedy(nxt, pos, args.steps, kv)  # returns after the last token is on the host
    elapsed = time.perf_counter() - t0
    pos += args.steps
    nxt = int(toks[-1])
    tok_s = args.steps / elapsed
    log(f"decode (device loop): {tok_s:.1f} tok/s ({elapsed / args.steps * 1e3:.3f} ms/token)")

    # the same decode driven from the host, one token read-back per step
    host_steps = min(args.host_steps, args.steps)
    t0 = time.perf_counter()
    for _ in range(host_steps):
        fwd.forward(nxt, pos, kv)
        nxt = fwd.sample_greedy()
        pos += 1
    host_tok_s = host_steps / (time.perf_counter() - t0) if host_steps else None
    if host_tok_s:
        log(f"decode (host loop): {host_tok_s:.1f} tok/s")

    # profiled pass of the same decode steps: HIP events around every launch
    F.set_profile(kv, True)
    for _ in range(args.profile_steps):
        fwd.forward(nxt, pos, kv)
        nxt = fwd.sample_greedy()
        pos += 1
    F.set_profile(kv, False)
    ents = F.profile_entries(kv)
    total_ms = sum(e["ms"] for e in ents) / args.profile_steps
    ents.sort(key=lambda e: -e["ms"])
    for e in ents:
        log(f"  {e['name']:<18} {e['launches'] // args.profile_steps:4d}/step  {e['ms'] / args.profile_steps:8.3f} ms/step  "
            f"{e['bytes'] / e['ms'] / 1e6 if e['ms'] else 0:8.1f} GB/s")
    dom = ents[0]
    avg_ms = dom["ms"] / dom["launches"]
    bytes_launch = dom["bytes"] / dom["launches"]
    achieved = bytes_launch / (avg_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "kernel": dom["name"], "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "bytes_per_launch": int(bytes_launch), "avg_launch_us": round(avg_ms * 1e3, 2)}

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, one thread, bounded sample) ...")
        cpu = cpu_baseline(args.config)
        log(f"cpu baseline: {cpu['value']} tok/s")

    out = {
        "metric": "decode tok/s @bs1 (Llama-3-8B-shape Q4_K); GEMV HBM GB/s as % of peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{cfg['name']}: {args.prompt}-token random prompt prefilled token by token, then greedy "
                        f"decode at batch 1 (positions {args.prompt - 1 + args.warmup}..{args.prompt - 2 + args.warmup + args.steps}), "
                        "device-side greedy loop",
            "weights": "Q4_K (q,k,o,gate,up) + Q6_K (v,down,output), seeded random blocks",
            "weight_bytes_per_token": tok_bytes,
            "graph": not args.no_graph,
        },
        "roofline": roofline,
        "decode_step_hbm_frac": round(tok_s * tok_bytes / (HBM_PEAK_GBS * 1e9), 4),
        "prefill_tok_s": round((args.prompt - 1) / prefill_s, 2),
        "host_loop_tok_s": round(host_tok_s, 2) if host_tok_s else None,
        "profiled_step_ms": round(total_ms, 4),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    kv.close()
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
