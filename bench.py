"""Decode benchmark: Llama-3-8B-shaped Q4_K/Q6_K model at batch 1 on one MI355X.

Workload: random-init weights of the Llama-3-8B shape (dim 4096, 32 layers, 32/8 heads x 128,
FFN 14336, vocab 128256; Q4_K for q/k/o/gate/up, Q6_K for v/down/output) generated from a
seed, a 512-token random prompt prefilled in one batched pass (fllm_prefill), then greedy decode
at batch 1.
A "step" is one decode token: the forward pass and the greedy argmax. The timed steps run as a
device-side loop (each step's argmax is the next step's input token on the device, one graph
launch per step, the tokens are read back after the last step); the same tokens come out of the
host loop (forward + argmax + 4-byte read-back per token), whose rate is reported beside it.

Prints one JSON line with the decode throughput, a roofline entry for the dominant kernel and a
CPU baseline (the oracle's reference-order F32 forward pass on a bounded sample, one thread).
Progress goes to stderr.

Roofline: the dominant kernel is the one with the largest share of a profiled decode step (HIP
events around every launch). Its achieved bandwidth is its algorithmic bytes per launch (the weight
blocks it streams plus its activation reads and writes) over its mean duration. When rocprofv3 is
on PATH, the duration and the HBM traffic come from short child runs of this script under the
profiler at the timed run's context (the same prompt prefilled into a cache of the same capacity,
then eager decode steps): kernel trace; FETCH_SIZE; WRITE_SIZE, each scaled by what it reads for a
device copy of known size in the same child; and the read requests by size with the DRAM-side
32-byte read and write units, which show where that scale comes from. Without the profiler the
duration is the HIP-event mean (which includes the launch) and the traffic is null.

The second half of the metric, the isolated GEMV sweep (Q4_K, Q8_0, Q6_K at 4096x4096, 14336x4096 and
4096x14336, dotnetfoundryllm_amd.gemv_bench), goes into "gemv_sweep": algorithmic GB/s per launch
over at least 1 GiB of distinct copies, and the counted traffic per launch of the tile layout.
"""
import argparse
import csv
import ctypes
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(cfg_name, first, steps=20, head_tokens=10):
    """The oracle (reference-order restatement, F32 weights dequantized at load, one thread) on a
    bounded sample of the same workload at the timed decode context: one decoder layer of the model
    shape, its cache filled to position `first` (untimed, with the row-parallel threads, whose
    results are bit-identical to one thread), then `steps` Forward calls at positions first..
    timed on one thread and scaled by the layer count (the layers share one shape); and the whole
    LM head (every row) timed on one thread over `head_tokens` calls."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_bind as O
    from dotnetfoundryllm_amd.configs import CONFIGS, desc_of, synth_bytes, tensor_plan

    cfg = dict(CONFIGS[cfg_name])
    full_layers = cfg["n_layers"]
    cfg["n_layers"] = 1
    tensors = {e[0]: (e, synth_bytes(cfg, e)) for e in tensor_plan(cfg)}
    desc = desc_of(cfg)
    t0 = time.time()
    m = O.OracleModel(desc, tensors, first + steps + 8)
    load_s = time.time() - t0
    del tensors
    fill_threads = max(1, min(16, len(os.sched_getaffinity(0))))
    try:
        m.limit(1, 0)
        O.lib.orc_set_threads(fill_threads)
        t0 = time.time()
        for p in range(first):
            m.forward(11 + p % 1000, p)
        fill_s = time.time() - t0
        O.lib.orc_set_threads(1)
        t = time.perf_counter()
        for p in range(first, first + steps):
            m.forward(11 + p % 1000, p)
        t_layer = (time.perf_counter() - t) / steps
        m.limit(0, desc.vocab)  # embedding row, final norm and every LM-head row
        m.forward(7, 0)
        t = time.perf_counter()
        for k in range(head_tokens):
            m.forward(7 + k, 0)
        t_head = (time.perf_counter() - t) / head_tokens
    finally:
        O.lib.orc_set_threads(1)
        m.close()
    t_token = full_layers * t_layer + t_head
    # the reference prefills with one Forward per prompt token (LlamaLanguageModel.cs:133-137): its
    # prefill rate is the per-token rate over the prompt's positions (0..510 for the 511-token
    # prefill, against the decode positions sampled here; attention is a few percent of a token at
    # these lengths)
    return {
        "value": round(1.0 / t_token, 4),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "prefill_tok_s": round(1.0 / t_token, 4),
        "cpu_model": host_cpu_model(),
        "nproc": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "sample": (f"oracle F32 forward (weights dequantized at load, reference operation order), one thread, at "
                   f"the timed decode context: 1 decoder layer at positions {first}-{first + steps - 1} "
                   f"({t_layer * 1e3:.1f} ms per position, x {full_layers} layers) + the whole LM head "
                   f"({desc.vocab} rows, {t_head * 1e3:.1f} ms, {head_tokens} calls); the cache filled to "
                   f"position {first} untimed on {fill_threads} threads ({fill_s:.1f} s); load {load_s:.1f} s. "
                   f"Prefill = the same per-token Forward, as the reference prefills"),
    }


def host_cpu_model():
    """/proc/cpuinfo's model name with its family / model / stepping, clock and cache lines."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if not line.strip():
                break  # the first processor's block
            k, _, v = line.partition(":")
            fields[k.strip()] = v.strip()
    except OSError:
        return None
    name = fields.get("model name")
    if not name:
        return None
    extra = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping", "cpu MHz", "cache size") if k in fields]
    return f"{name} ({', '.join(extra)})" if extra else name


COPY_BYTES = 256 << 20  # calibration copy of the traffic counters


def device_copy_calibration():
    """A plain device-to-device copy of COPY_BYTES (the HIP runtime's copy kernel): what the traffic
    counters read for it calibrates them."""
    hip = ctypes.CDLL("libamdhip64.so")
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    if hip.hipMalloc(ctypes.byref(a), ctypes.c_size_t(COPY_BYTES)) or hip.hipMalloc(ctypes.byref(b), ctypes.c_size_t(COPY_BYTES)):
        raise RuntimeError("hipMalloc failed")
    hip.hipMemset(a, 1, ctypes.c_size_t(COPY_BYTES))
    for _ in range(3):
        hip.hipMemcpy(b, a, ctypes.c_size_t(COPY_BYTES), 3)  # hipMemcpyDeviceToDevice
    hip.hipDeviceSynchronize()
    hip.hipFree(a)
    hip.hipFree(b)


def timed_capacity(args, cfg):
    """KV capacity of the timed run (it sets the attention's chunking, so the profiled children use
    it too)."""
    return min(cfg["max_ctx"], args.prompt + args.warmup + args.steps + args.host_steps + args.profile_steps + 8)


def child_profile(args):
    """The workload profiled by the roofline child runs, at the timed run's context: the same
    prompt through the batched prefill into a cache of the same capacity, the warmup's decode steps,
    then eager decode steps with per-launch events (so the launch names come out in order) and the
    calibration copy."""
    import dotnetfoundryllm_amd as F
    from dotnetfoundryllm_amd.configs import CONFIGS, build_model

    cfg = CONFIGS[args.config]
    ctx = F.Context(0)
    model, _ = build_model(ctx, cfg)
    kv = F.HipKvCache(model, timed_capacity(args, cfg))
    if args.attention_merge != "auto":
        F.set_attention_merge(kv, args.attention_merge == "in")
    fwd = F.HipForwardPass(model)
    prompt = F.synth_tokens(cfg["seed"], 0, cfg["vocab"], args.prompt)
    fwd.prefill(prompt[:-1], 0, kv)
    nxt, pos = int(prompt[-1]), args.prompt - 1
    if args.warmup:
        nxt = int(fwd.decode_greedy(nxt, pos, args.warmup, kv)[-1])
        pos += args.warmup
    F.set_graph(kv, False)
    F.set_profile(kv, True)
    for _ in range(args.profile_steps):
        fwd.forward(nxt, pos, kv)
        nxt = fwd.sample_greedy()
        pos += 1
    F.set_profile(kv, False)
    ctx.sync()
    print(json.dumps({"launch_names": F.profile_launches(kv)}), flush=True)
    device_copy_calibration()
    kv.close()
    model.close()
    ctx.close()


def child_gemv(args):
    """The isolated-GEMV sweep's matrices under the traffic counters: for each type and shape,
    GEMV_COPIES distinct copies regrouped by fllm_gemv_pack, one fllm_gemv_ex launch on each (tile
    layout), then the calibration copy."""
    import numpy as np

    import dotnetfoundryllm_amd as F
    from dotnetfoundryllm_amd import gemv_bench as G
    from dotnetfoundryllm_amd._native import type_bytes

    ctx = F.Context(0)
    rng = np.random.default_rng(7)
    for t, tname in G.TYPES:
        p0, p1 = G.weight_range(t)
        for rows, cols in G.SHAPES:
            x = rng.standard_normal(cols).astype(np.float32)
            xb, yb = F.DeviceBuffer(ctx, x.nbytes), F.DeviceBuffer(ctx, rows * 4)
            xb.write(x)
            tiles = []
            for c in range(GEMV_COPIES):
                raw = F.synth_tensor(t, 0x5EED01, 1000 * rows + c, rows * cols, 0, p0, p1)
                b = F.DeviceBuffer(ctx, raw.nbytes)
                b.write(raw)
                tb = F.DeviceBuffer(ctx, raw.nbytes)
                F.gemv_pack(ctx, t, b, rows, cols, tb)
                b.close()
                tiles.append(tb)
            for tb in tiles:
                F.gemv(ctx, t, tb, rows, cols, xb, yb, layout=F.LAYOUT_TILES)
            ctx.sync()
            for b in tiles + [xb, yb]:
                b.close()
    device_copy_calibration()
    ctx.close()


GEMV_COPIES = 3


def gemv_report(args):
    """The second headline metric: the isolated GEMV sweep (Q4_K, Q8_0, Q6_K at 4096x4096, 14336x4096,
    4096x14336; dotnetfoundryllm_amd.gemv_bench) as algorithmic GB/s and fraction of 8 TB/s, with each
    tile-layout launch's HBM traffic from FETCH_SIZE + WRITE_SIZE (calibrated like the roofline's) when
    rocprofv3 is present."""
    from dotnetfoundryllm_amd import gemv_bench as G
    rows = G.run(iters=100, out=log)
    sweep = [{"type": tn, "rows": r, "cols": c, "layout": lay, "bytes": nb, "us_per_launch": round(us, 2),
              "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)} for tn, r, c, lay, nb, n, us, gbs in rows]
    if args.no_rocprof or not shutil.which("rocprofv3"):
        return sweep
    tmp = tempfile.mkdtemp(prefix="fllm_gemv_")
    try:
        traffic = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            order = pmc_dispatches(rocprof_child(args, counter, tmp, child="--child-gemv"), counter)
            factor = copy_factor(order)
            gemv = [v for n, v in order if "k_gemv" in n]
            cases = [(tn, r, c) for _, tn in G.TYPES for r, c in G.SHAPES]
            if len(gemv) != len(cases) * GEMV_COPIES:
                raise RuntimeError(f"{counter}: {len(gemv)} GEMV dispatches, expected {len(cases) * GEMV_COPIES}")
            for i, case in enumerate(cases):
                vals = gemv[i * GEMV_COPIES:(i + 1) * GEMV_COPIES]
                traffic[case] = traffic.get(case, 0.0) + sum(vals) / len(vals) * 1024.0 * factor
        for e in sweep:
            tr = traffic.get((e["type"], e["rows"], e["cols"]))
            if e["layout"] == "tiles" and tr is not None:
                e["traffic"] = int(tr)
                e["traffic_ratio"] = round(tr / e["bytes"], 3)
    except Exception as e:
        log(f"gemv sweep: traffic counters failed ({e})")
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return sweep


def child_args(args):
    return ["--config", args.config, "--profile-steps", str(args.profile_steps), "--prompt", str(args.prompt),
            "--warmup", str(args.warmup), "--steps", str(args.steps), "--host-steps", str(args.host_steps)] + \
        ["--attention-merge", args.attention_merge]


def rocprof_child(args, mode, tmp, child="--child-profile"):
    """Runs a child workload of this script under rocprofv3 (mode "trace": kernel trace; otherwise
    the space-separated counters of one --pmc pass); returns the rows of its CSV output."""
    out = os.path.join(tmp, mode.replace(" ", "+"))
    cmd = ["rocprofv3"]
    if mode == "trace":
        cmd += ["--kernel-trace"]
    else:
        cmd += ["--pmc", *mode.split()]
    cmd += ["--output-format", "csv", "-d", out, "-o", "run", "--",
            sys.executable, os.path.abspath(__file__), child, *child_args(args)]
    env = dict(os.environ, TMPDIR=tmp)
    log(f"  rocprofv3 {'--kernel-trace' if mode == 'trace' else '--pmc ' + mode} ({child})")
    r = subprocess.run(cmd, cwd=tmp, env=env, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=150)
    files = glob.glob(os.path.join(out, "**", "*kernel_trace.csv" if mode == "trace" else "*counter_collection.csv"),
                      recursive=True)
    if not files:
        raise RuntimeError(f"rocprofv3 {mode}: no output (rc {r.returncode}): {r.stderr[-400:]}")
    return list(csv.DictReader(open(files[0])))


def kernel_key(row):
    return (row["Kernel_Name"].split("(")[0], row.get("Grid_Size", row.get("Grid_Size_X", "")))


def pmc_dispatches(rows, counter):
    """[(kernel name, value)] of one counter per dispatch, in dispatch (= launch) order."""
    per = {}
    for r in rows:
        if r["Counter_Name"] != counter:
            continue
        d = int(r["Dispatch_Id"])
        name = r["Kernel_Name"]
        per[d] = (name, per.get(d, (name, 0.0))[1] + float(r["Counter_Value"]))
    return [per[d] for d in sorted(per)]


def copy_factor(order):
    """Bytes per counted KiB from the calibration copy, which reads and writes COPY_BYTES."""
    copy = [v for n, v in order if "copyBuffer" in n]
    if not copy:
        raise RuntimeError("missing calibration copy dispatch")
    return COPY_BYTES / (max(copy) * 1024.0)


# Read requests by size (TCC_EA0_RDREQ_{32B,64B,128B}) and the DRAM-side 32-byte read / write units: the
# per-size picture behind FETCH_SIZE, whose gfx950 formula counts a request as 128 bytes only when
# TCC_BUBBLE counts it (at most 4 TCC counters per pass)
SIZE_PASSES = (("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum"),
               ("TCC_BUBBLE_sum", "TCC_EA0_RDREQ_DRAM_32B_sum", "TCC_EA0_WRREQ_WRITE_DRAM_32B_sum"))


def profiler_roofline(args, bytes_per_launch, dom_name, steps_launches):
    """Mean duration and HBM traffic of the dominant launch from rocprofv3 child runs. The dominant
    launch is identified by position: the profiled steps' launches in order are the HIP-event
    names, so the kernel (and grid) at the positions named dom_name is the dominant one."""
    tmp = tempfile.mkdtemp(prefix="fllm_roofline_")
    n_prof = len(steps_launches)

    def dominant(order, what):
        # the dominant launch by position among the profiled launches, as for the durations (one
        # kernel can serve several launches of a step with the same grid: e.g. o and gate/up)
        fl = [(n, v) for n, v in order if "fllm::" in n and "k_set_params" not in n]
        if len(fl) < n_prof:
            raise RuntimeError(f"{what}: fewer dispatches than the profiled launches")
        dom = [v for (n, v), nm in zip(fl[-n_prof:], steps_launches) if nm == dom_name]
        if not dom:
            raise RuntimeError(f"{what}: no dominant-kernel dispatches")
        return sum(dom) / len(dom)

    try:
        trace = rocprof_child(args, "trace", tmp)
        trace.sort(key=lambda r: int(r["Start_Timestamp"]))
        # the profiled launches (one kernel each, names in order) are the child's last fllm kernels
        # (the step-parameter write at the start of each forward is not a profiled launch)
        mine = [r for r in trace if "fllm::" in r["Kernel_Name"] and "k_set_params" not in r["Kernel_Name"]]
        if n_prof == 0 or len(mine) < n_prof:
            raise RuntimeError("kernel trace shorter than the profiled launches")
        prof = mine[-n_prof:]
        keys = {kernel_key(r) for r, nm in zip(prof, steps_launches) if nm == dom_name}
        durs = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r, nm in zip(prof, steps_launches) if nm == dom_name]
        avg_us = sum(durs) / len(durs) / 1e3
        res = {"avg_launch_us": round(avg_us, 2), "duration_source": "rocprofv3 kernel trace",
               "kernel_symbol": sorted(k[0] for k in keys)[0] if keys else None}
        traffic = 0.0
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            order = pmc_dispatches(rocprof_child(args, counter, tmp), counter)
            factor = copy_factor(order)
            kib = dominant(order, counter)
            res[counter.lower() + "_kib_raw"] = round(kib, 1)
            res[counter.lower() + "_copy_factor"] = round(factor, 4)
            traffic += kib * 1024.0 * factor
        res["traffic"] = int(traffic)
        try:
            sizes = {}
            for group in SIZE_PASSES:
                rows = rocprof_child(args, " ".join(group), tmp)
                for counter in group:
                    sizes[counter] = round(dominant(pmc_dispatches(rows, counter), counter), 1)
            res["read_requests_per_launch"] = sizes
            res["dram_traffic_from_32b_units"] = int(32 * (sizes["TCC_EA0_RDREQ_DRAM_32B_sum"] +
                                                          sizes["TCC_EA0_WRREQ_WRITE_DRAM_32B_sum"]))
        except Exception as e:  # the cross-check is optional
            log(f"roofline: request-size counters failed ({e})")
        return res
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak
Q8_0_TYPE, Q4_K_TYPE, Q5_K_TYPE = 8, 12, 13


def prefill_report(cfg, n, seconds, stages=None):
    """Arithmetic rate of the batched prefill over the wall time of the whole prefill call (norms,
    element-wise steps and the last token's LM head included, so every fraction is a lower bound).
    `tflops`: the reference's own arithmetic, 2 flop per weight per token plus the causal attention's
    4 * heads * head_dim flop per (query, key) pair. The projections run on the fp16 matrix cores:
    a Q4_K or Q5_K matrix takes two fp16 products per weight (exact integer weights against the
    activations' hi and lo halves) plus one min-term product per 256-element block (1/8 of a
    product), a Q8_0 one two (its int8 codes against the hi and lo halves), any other three (Q6_K:
    exact integer hi / lo weights; other types: hi / lo splits of both operands); `gemm` is those
    fp16 products' rate against the fp16 peak. Attention runs on the f32 matrix cores, one product
    per flop, except at head_dim 128 and 256, where it takes three fp16 products per flop (hi / lo
    splits of both operands, the lo lo product dropped) against the fp16 peak."""
    H, L, F = cfg["hidden"], cfg["n_layers"], cfg["ffn"]
    hd = cfg["head_dim"]
    qdim, kvdim = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd
    ty = cfg["types"]
    weights = L * (qdim * H + 2 * kvdim * H + H * qdim + 3 * F * H)
    # (query, key) pairs per layer: causal, and inside the sliding window on the layers that have one
    # (every Mistral layer, Gemma-2's even layers)
    pairs = n * (n + 1) // 2
    win = cfg.get("window", 0)
    if 0 < win < n:
        pairs_w = win * (win + 1) // 2 + (n - win) * win
        n_win = L if cfg["arch"] == 1 else (L + 1) // 2 if cfg["arch"] == 3 else 0
    else:
        pairs_w, n_win = pairs, 0
    attn = 4.0 * cfg["n_heads"] * hd * (pairs * (L - n_win) + pairs_w * n_win)
    flops = 2.0 * n * weights + attn
    launches = [((qdim * H, ty["q"]), (kvdim * H, ty["k"]), (kvdim * H, ty["v"])), ((H * qdim, ty["o"]),),
                ((F * H, ty["gate"]), (F * H, ty["up"])), ((H * F, ty["down"]),)]
    def products(t):
        return 2.125 if t in (Q4_K_TYPE, Q5_K_TYPE) else 2.0 if t == Q8_0_TYPE else 3.0

    fp16 = sum(products(t) * w for g in launches for w, t in g)
    fp16_tf = 2.0 * n * L * fp16 / seconds / 1e12
    tf = flops / seconds / 1e12
    out = {"tokens": n, "tok_s": round(n / seconds, 2), "tflops": round(tf, 2),
           "gemm": {"dtype": "fp16", "mfma_tflops": round(fp16_tf, 2), "mfma_peak_tflops": FP16_MFMA_PEAK_TFLOPS,
                    "mfma_frac": round(fp16_tf / FP16_MFMA_PEAK_TFLOPS, 4)}}
    if stages:
        # each stage's own device time (events around its launches in a second, profiled prefill)
        gemm_of = {"pf_qkv": launches[0], "pf_o": launches[1], "pf_gate_up": launches[2], "pf_down": launches[3]}
        table = {}
        for name, st in sorted(stages.items(), key=lambda kv: -kv[1]["ms"]):
            row = {"launches": st["launches"], "ms": round(st["ms"], 3)}
            if name in gemm_of:
                g = gemm_of[name]
                issued = sum(products(t) * w for w, t in g)
                mf = 2.0 * n * L * issued / (st["ms"] * 1e-3) / 1e12
                row.update(dtype="fp16", products=round(issued / sum(w for w, _ in g), 3), mfma_tflops=round(mf, 1),
                           mfma_frac=round(mf / FP16_MFMA_PEAK_TFLOPS, 4))
            elif name == "pf_attention" and hd in (128, 256):
                mf = 3.0 * attn / (st["ms"] * 1e-3) / 1e12
                row.update(dtype="fp16", products=3.0, mfma_tflops=round(mf, 1),
                           mfma_frac=round(mf / FP16_MFMA_PEAK_TFLOPS, 4))
            elif name == "pf_attention":
                mf = attn / (st["ms"] * 1e-3) / 1e12
                row.update(dtype="f32", mfma_tflops=round(mf, 1), mfma_frac=round(mf / FP32_MFMA_PEAK_TFLOPS, 4))
            table[name] = row
        out["stages"] = table
    return out


def sampling_report(F, fwd, kv, cfg, seed, reps=50):
    """Wall time per call of the sampling stages on the last step's logits (each call returns its
    token on the host): the device paths of SamplerPipeline (top-k candidates + host walk; the
    nucleus on the device), the device repetition penalty over 256 ids, and the host pipeline over
    a vocab-sized logits copy for comparison."""
    import numpy as np
    saved = fwd.logits
    ids = np.arange(0, 256 * 97, 97, dtype=np.int32) % cfg["vocab"]
    out = {}

    def timed(name, fn):
        fwd.write_logits(saved)
        fn()  # first call: one-time costs
        t = 0.0
        for _ in range(reps):
            fwd.write_logits(saved)
            t0 = time.perf_counter()
            fn()
            t += time.perf_counter() - t0
        out[name] = round(t / reps * 1e6, 1)

    sp_k = F.SamplerPipeline(0.8, 40, 1.0, seed)
    sp_p = F.SamplerPipeline(0.8, 0, 0.9, seed)
    sp_h = F.SamplerPipeline(0.8, 0, 0.9, seed)
    try:
        timed("top_k40_T0.8_device", lambda: sp_k.sample(kv))
        timed("top_p0.9_T0.8_device", lambda: sp_p.sample(kv))
        timed("repetition_penalty_256_ids_device", lambda: fwd.penalize(ids, 1.1))
        timed("top_p0.9_T0.8_host_with_logits_copy", lambda: sp_h.sample_host(fwd.logits))
    finally:
        sp_k.close()
        sp_p.close()
        sp_h.close()
    fwd.write_logits(saved)
    return out


def upload_report(F, ctx, load, probe_bytes=1 << 30):
    """Host-to-device rate of the weight upload (fllm_model_upload: raw GGUF blocks from host memory,
    large tensors through the pinned staging ring) against one direct pageable copy of 1 GiB
    (fllm_buf_write), and the time finalize takes to regroup the matrices on the device."""
    import numpy as np
    src = np.random.default_rng(1).integers(0, 255, probe_bytes, dtype=np.uint8)
    buf = F.DeviceBuffer(ctx, probe_bytes)
    try:
        buf.write(src)  # first touch
        t = time.perf_counter()
        buf.write(src)
        direct = probe_bytes / (time.perf_counter() - t) / 1e9
    finally:
        buf.close()
    return {"bytes": load["upload_bytes"], "seconds": round(load["upload_s"], 3),
            "GB_s": round(load["upload_bytes"] / load["upload_s"] / 1e9, 2),
            "direct_pageable_copy_GB_s": round(direct, 2), "finalize_s": round(load["finalize_s"], 3)}


def gguf_load_report(F, ctx, cfg, model):
    """GgufModelLoader's path at full size: the model's seeded tensors written as a GGUF file, its
    page cache dropped, then fllmh_load_gguf (mapped file, large tensors through the pinned staging
    pair, finalize) timed cold (disk reads and page faults included) and again warm (page faults of a
    cached file); 8 greedy tokens from the loaded model against the in-memory one."""
    from dotnetfoundryllm_amd.gguf import drop_page_cache, write_synthetic_gguf
    path = os.path.join(tempfile.gettempdir(), f"fllm_bench_{os.getpid()}.gguf")
    try:
        t = time.perf_counter()
        write_synthetic_gguf(path, cfg)
        write_s = time.perf_counter() - t
        size = os.path.getsize(path)
        drop_page_cache(path)
        out = {"file_bytes": size, "write_s": round(write_s, 2)}
        prompt = F.synth_tokens(cfg["seed"], 9, cfg["vocab"], 16)
        ref_kv = F.HipKvCache(model, 64)
        ref = list(F.HipForwardPass(model).decode_greedy(int(prompt[0]), 0, 8, ref_kv))
        ref_kv.close()
        for mode in ("cold", "warm"):
            t = time.perf_counter()
            m, _ = F.GgufModelLoader.load(ctx, path)
            s_ = time.perf_counter() - t
            out[f"{mode}_s"] = round(s_, 3)
            out[f"{mode}_GB_s"] = round(size / s_ / 1e9, 2)
            kv = F.HipKvCache(m, 64)
            toks = list(F.HipForwardPass(m).decode_greedy(int(prompt[0]), 0, 8, kv))
            kv.close()
            m.close()
            out[f"{mode}_greedy_tokens_match"] = toks == ref
        return out
    finally:
        if os.path.exists(path):
            os.remove(path)


def weights_text(cfg):
    """'Q4_K (q,k,o,gate,up) + Q6_K (v,down,output), seeded random blocks' from the config's types."""
    from dotnetfoundryllm_amd._native import TYPE_NAMES
    groups = {}
    for slot in ("q", "k", "v", "o", "gate", "up", "down", "out"):
        groups.setdefault(cfg["types"][slot], []).append("output" if slot == "out" else slot)
    parts = [f"{TYPE_NAMES.get(t, t)} ({','.join(v)})" for t, v in groups.items()]
    emb = TYPE_NAMES.get(cfg.get("emb_type"), cfg.get("emb_type"))
    return " + ".join(parts) + f", {emb} embedding, seeded random blocks"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode tokens before the timed ones")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--config", default="llama3-8b-q4km")
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--host-steps", type=int, default=32, help="steps of the host-driven loop timed after the device loop")
    ap.add_argument("--temperature", type=float, default=0.0,
                    help="> 0: the timed decode samples with SamplerPipeline(temperature, top-k, top-p, seed) "
                         "from the host loop (one forward and one device sampling call per token)")
    ap.add_argument("--top-k", type=int, default=0)
    ap.add_argument("--top-p", type=float, default=1.0)
    ap.add_argument("--seed", type=int, default=0x5EED)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--attention-merge", choices=("auto", "in", "separate"), default="auto",
                    help="merge the decode attention's chunks inside the attention launch or in a second launch "
                         "(auto: the library's choice for the shape)")
    ap.add_argument("--no-rocprof", action="store_true", help="roofline from HIP events only (no profiler child runs)")
    ap.add_argument("--child-profile", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--child-gemv", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-gemv-sweep", action="store_true", help="skip the isolated GEMV sweep")
    ap.add_argument("--no-gguf-load", action="store_true", help="skip the GGUF file-to-device measurement")
    args = ap.parse_args()
    if args.child_profile:
        child_profile(args)
        return
    if args.child_gemv:
        child_gemv(args)
        return
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
    load = {}
    model, _ = build_model(ctx, cfg, stats=load)
    log(f"weights generated and uploaded in {time.time() - t:.1f} s")
    load_report = upload_report(F, ctx, load)
    log(f"upload: {load_report}")
    max_seq = timed_capacity(args, cfg)
    kv = F.HipKvCache(model, max_seq)
    if args.no_graph:
        F.set_graph(kv, False)
    if args.attention_merge != "auto":
        F.set_attention_merge(kv, args.attention_merge == "in")
    fwd = F.HipForwardPass(model)
    prompt = F.synth_tokens(cfg["seed"], 0, cfg["vocab"], args.prompt)

    # prefill: Forward on prompt[0..n-2] (LlamaLanguageModel.cs:133-137). A first pass pays the
    # one-time costs (scratch allocation, kernel loading); the timed pass starts from an empty cache.
    fwd.prefill(prompt[:-1], 0, kv)
    F._check(F.N.dev.fllm_seq_sync(kv.h))
    kv.clear()
    t = time.perf_counter()
    fwd.prefill(prompt[:-1], 0, kv)
    ctx.sync()
    F._check(F.N.dev.fllm_seq_sync(kv.h))
    prefill_s = time.perf_counter() - t
    pos = args.prompt - 1
    log(f"prefill {args.prompt - 1} tokens in {prefill_s:.2f} s")
    # the same prefill once more with each stage's launches timed by events; the cache ends as the
    # timed prefill left it
    kv.clear()
    F.set_profile(kv, True)
    fwd.prefill(prompt[:-1], 0, kv)
    F.set_profile(kv, False)
    prefill_stages = {e["name"]: e for e in F.profile_entries(kv)}
    F.profile_reset(kv)

    nxt = int(prompt[-1])
    sampled = args.temperature > 0.0
    if sampled:
        # LlamaLanguageModel's loop with SamplerPipeline(T, k, p, seed): Forward, then the sampler on
        # the device logits (top-k candidates or the nucleus on the device), one token read back
        sampler = F.SamplerPipeline(args.temperature, args.top_k, args.top_p, args.seed)

        def run_steps(n, nxt, pos):
            out = []
            for _ in range(n):
                fwd.forward(nxt, pos, kv)
                nxt = sampler.sample(kv)
                pos += 1
                out.append(nxt)
            return out

        warm = run_steps(args.warmup, nxt, pos)
    else:
        warm = fwd.decode_greedy(nxt, pos, args.warmup, kv) if args.warmup else []
    pos += args.warmup
    nxt = int(warm[-1]) if len(warm) else nxt
    log(f"warmup {args.warmup} steps done; timing {args.steps} decode steps")

    F._check(F.N.dev.fllm_seq_sync(kv.h))
    t0 = time.perf_counter()
    if sampled:
        toks = run_steps(args.steps, nxt, pos)
    else:
        toks = fwd.decode_greedy(nxt, pos, args.steps, kv)  # returns after the last token is on the host
    elapsed = time.perf_counter() - t0
    pos += args.steps
    nxt = int(toks[-1])
    tok_s = args.steps / elapsed
    mode = (f"host loop, SamplerPipeline(T={args.temperature}, top-k={args.top_k}, top-p={args.top_p}, "
            f"seed={args.seed})" if sampled else "device-side greedy loop")
    log(f"decode ({mode}): {tok_s:.1f} tok/s ({elapsed / args.steps * 1e3:.3f} ms/token)")
    if sampled:
        sampler.close()

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
    roofline = {"bound": "hbm", "kernel": dom["name"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "traffic": None,
                "bytes_per_launch": int(bytes_launch), "avg_launch_us": round(avg_ms * 1e3, 2),
                "duration_source": "HIP events around each launch (eager profiled steps)"}
    if not args.no_rocprof and shutil.which("rocprofv3"):
        log("roofline: rocprofv3 child runs (kernel trace, FETCH_SIZE, WRITE_SIZE) ...")
        try:
            names = json.loads(subprocess.run([sys.executable, os.path.abspath(__file__), "--child-profile",
                                               *child_args(args)],
                                              stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True,
                                              timeout=240).stdout.strip().splitlines()[-1])["launch_names"]
            roofline.update(profiler_roofline(args, bytes_launch, dom["name"], names))
            roofline["event_avg_launch_us"] = round(avg_ms * 1e3, 2)
        except Exception as e:  # the profiler is optional: keep the event timing
            log(f"roofline: profiler runs failed ({e}); using HIP-event durations")
    achieved = bytes_launch / (roofline["avg_launch_us"] * 1e-6) / 1e9
    roofline["achieved"] = round(achieved, 1)
    roofline["frac"] = round(achieved / HBM_PEAK_GBS, 4)

    sweep = None
    if not args.no_gemv_sweep:
        log("isolated GEMV sweep (Q4_K, Q8_0, Q6_K) ...")
        sweep = gemv_report(args)

    sampling = sampling_report(F, fwd, kv, cfg, args.seed)

    gguf_load = None
    if not args.no_gguf_load:
        log("GGUF file load (write, drop the page cache, fllmh_load_gguf cold and warm) ...")
        try:
            gguf_load = gguf_load_report(F, ctx, cfg, model)
            log(f"GGUF load: {gguf_load}")
        except Exception as e:
            log(f"GGUF load failed: {e}")
    log(f"sampling per call (us): {sampling}")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, one thread, bounded sample) ...")
        # 20 positions centred on the timed range's mean position
        t0, t1 = args.prompt - 1 + args.warmup, args.prompt - 2 + args.warmup + args.steps
        cpu = cpu_baseline(args.config, first=max(0, (t0 + t1) // 2 - 10))
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
            "workload": f"{cfg['name']}: {args.prompt}-token random prompt, batched prefill, then "
                        f"{'sampled' if sampled else 'greedy'} decode at batch 1 (positions "
                        f"{args.prompt - 1 + args.warmup}..{args.prompt - 2 + args.warmup + args.steps}), {mode}",
            "weights": weights_text(cfg),
            "weight_bytes_per_token": tok_bytes,
            "graph": not args.no_graph,
        },
        "roofline": roofline,
        "decode_step_hbm_frac": round(tok_s * tok_bytes / (HBM_PEAK_GBS * 1e9), 4),
        "prefill_tok_s": round((args.prompt - 1) / prefill_s, 2),
        "prefill": prefill_report(cfg, args.prompt - 1, prefill_s, prefill_stages),
        "host_loop_tok_s": round(host_tok_s, 2) if host_tok_s else None,
        "profiled_step_ms": round(total_ms, 4),
        "sampling_us_per_call": sampling,
        "weight_upload": load_report,
        "gemv_sweep": sweep,
        "gguf_file_load": gguf_load,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    kv.close()
    model.close()
    ctx.close()


if __name__ == "__main__":
    main()
