"""Model shapes and synthetic-weight recipes for the decode workloads.

Named configurations:
  tiny-llama-q4k   dim 512, 8 layers, 8/2 heads, FFN 1408, vocab 32000, all linear weights Q4_K
  llama3-8b-q4km   dim 4096, 32 layers, 32/8 heads, FFN 14336, vocab 128256, Q4_K + Q6_K (v, down, output)
  qwen2-7b-q5k     dim 3584, 28 layers, 28/4 heads, FFN 18944, vocab 152064, Q5_K + Q6_K output, q/k/v bias
  gemma2-9b-q8     dim 3584, 42 layers, 16/8 heads x 256, FFN 14336 GeGLU, vocab 256000, Q8_0, BF16 embedding
plus small test shapes for every architecture and tensor type. Quantized blocks are drawn
from the seed directly (nibbles uniform, 6-bit scales/mins uniform, f16 scales uniform in a
range); embeddings and biases are N(0, 0.02) floats; norm weights are 1.0 (test shapes use
N(1, 0.1) so a dropped norm weight shows up).
"""
import math

import numpy as np

from . import _native as N
from ._native import BF16, F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, Q8_K

SLOT_NAMES = {
    N.SLOT_TOKEN_EMBD: "token_embd.weight", N.SLOT_OUTPUT_NORM: "output_norm.weight", N.SLOT_OUTPUT: "output.weight",
    N.SLOT_ATTN_NORM: "attn_norm.weight", N.SLOT_ATTN_Q: "attn_q.weight", N.SLOT_ATTN_K: "attn_k.weight",
    N.SLOT_ATTN_V: "attn_v.weight", N.SLOT_ATTN_OUTPUT: "attn_output.weight", N.SLOT_ATTN_Q_BIAS: "attn_q.bias",
    N.SLOT_ATTN_K_BIAS: "attn_k.bias", N.SLOT_ATTN_V_BIAS: "attn_v.bias",
    N.SLOT_POST_ATTN_NORM: "post_attn_norm.weight", N.SLOT_FFN_NORM: "ffn_norm.weight",
    N.SLOT_FFN_GATE: "ffn_gate.weight", N.SLOT_FFN_UP: "ffn_up.weight", N.SLOT_FFN_DOWN: "ffn_down.weight",
    N.SLOT_POST_FFN_NORM: "post_ffn_norm.weight",
}
ARCH_NAMES = {N.ARCH_LLAMA: "llama", N.ARCH_MISTRAL: "mistral", N.ARCH_QWEN2: "qwen2", N.ARCH_GEMMA2: "gemma2"}

# scale ranges of the quantized blocks
KQ_RANGE = (1e-3, 4e-3)     # Q4_K/Q5_K d and dmin, Q6_K d
Q8_RANGE = (1e-3, 1e-2)     # Q8_0 d
NO_WINDOW = 0x7FFFFFFF


def _cfg(name, arch, layers, hidden, heads, kv_heads, ffn, vocab, max_ctx, rope_base, types, head_dim=None,
         emb_type=F32, window=NO_WINDOW, attn_softcap=0.0, final_softcap=0.0, tied=False, norm_std=0.0, seed=0,
         rope_scaled=0, rope_scale=1.0):
    hd = head_dim or hidden // heads
    return dict(name=name, arch=arch, n_layers=layers, hidden=hidden, n_heads=heads, n_kv_heads=kv_heads, ffn=ffn,
                vocab=vocab, max_ctx=max_ctx, rope_base=rope_base, head_dim=hd, types=types, emb_type=emb_type,
                window=window, attn_softcap=attn_softcap, final_softcap=final_softcap, tied=tied,
                norm_std=norm_std, seed=seed, rope_scaled=rope_scaled, rope_scale=rope_scale)


def _types(q, k, v, o, gate, up, down, out):
    return dict(q=q, k=k, v=v, o=o, gate=gate, up=up, down=down, out=out)


CONFIGS = {
    "tiny-llama-q4k": _cfg("tiny-llama-q4k", N.ARCH_LLAMA, 8, 512, 8, 2, 1408, 32000, 512, 10000.0,
                           _types(*([Q4_K] * 8)), seed=0x5EED00),
    "llama3-8b-q4km": _cfg("llama3-8b-q4km", N.ARCH_LLAMA, 32, 4096, 32, 8, 14336, 128256, 4096, 500000.0,
                           _types(Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K, Q6_K), seed=0x5EED02),
    "qwen2-7b-q5k": _cfg("qwen2-7b-q5k", N.ARCH_QWEN2, 28, 3584, 28, 4, 18944, 152064, 4096, 1000000.0,
                         _types(*([Q5_K] * 7), Q6_K), seed=0x5EED03),
    "gemma2-9b-q8": _cfg("gemma2-9b-q8", N.ARCH_GEMMA2, 42, 3584, 16, 8, 14336, 256000, 8192, 10000.0,
                         _types(*([Q8_0] * 8)), head_dim=256, emb_type=BF16, window=4096, attn_softcap=50.0,
                         final_softcap=30.0, seed=0x5EED04),
    # the same with the LM head tied to the BF16 token embedding (no output.weight in the file)
    "gemma2-9b-q8-tied": _cfg("gemma2-9b-q8-tied", N.ARCH_GEMMA2, 42, 3584, 16, 8, 14336, 256000, 8192, 10000.0,
                              _types(*([Q8_0] * 8)), head_dim=256, emb_type=BF16, window=4096, attn_softcap=50.0,
                              final_softcap=30.0, tied=True, seed=0x5EED04),
    # ---- small shapes for parity tests (every architecture and tensor type) ----
    "test-llama": _cfg("test-llama", N.ARCH_LLAMA, 2, 256, 4, 2, 512, 512, 128, 10000.0,
                       _types(Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K, Q6_K), norm_std=0.1, seed=11),
    "test-llama-straddle": _cfg("test-llama-straddle", N.ARCH_LLAMA, 2, 256, 4, 1, 352, 512, 64, 10000.0,
                                _types(*([Q4_K] * 8)), norm_std=0.1, seed=12, rope_scaled=1, rope_scale=2.0),
    "test-mistral": _cfg("test-mistral", N.ARCH_MISTRAL, 2, 256, 4, 2, 512, 512, 64, 10000.0,
                         _types(*([Q8_0] * 8)), window=7, norm_std=0.1, seed=13),
    "test-qwen2": _cfg("test-qwen2", N.ARCH_QWEN2, 2, 256, 4, 2, 512, 512, 64, 1000000.0,
                       _types(*([Q5_K] * 7), Q6_K), norm_std=0.1, seed=14),
    "test-gemma2": _cfg("test-gemma2", N.ARCH_GEMMA2, 3, 256, 4, 2, 512, 512, 64, 10000.0,
                        _types(*([Q8_0] * 8)), head_dim=128, emb_type=BF16, window=6, attn_softcap=50.0,
                        final_softcap=30.0, tied=True, norm_std=0.1, seed=15),
    "test-gemma2-hd256": _cfg("test-gemma2-hd256", N.ARCH_GEMMA2, 2, 256, 4, 2, 512, 512, 64, 10000.0,
                              _types(*([Q8_0] * 8)), head_dim=256, emb_type=BF16, window=6, attn_softcap=50.0,
                              final_softcap=30.0, tied=True, norm_std=0.1, seed=17),
    "test-mixed": _cfg("test-mixed", N.ARCH_LLAMA, 2, 256, 4, 2, 512, 512, 64, 10000.0,
                       _types(Q4_0, Q8_K, F16, BF16, F32, Q4_0, Q5_K, F16), emb_type=F16, norm_std=0.1, seed=16),
    # the Qwen2-7B vocabulary (152064 = 37.1 sampler segments of 4096) on one narrow layer
    "test-qwen2-v152k": _cfg("test-qwen2-v152k", N.ARCH_QWEN2, 1, 256, 4, 2, 512, 152064, 64, 1000000.0,
                             _types(*([Q5_K] * 7), Q6_K), norm_std=0.1, seed=19),
    # Gemma-2-9B attention at a narrow width: head_dim 256, 16 query / 8 kv heads, softcaps 50 / 30,
    # window 4096 on the even layer, an 8192-position cache
    "test-gemma2-long": _cfg("test-gemma2-long", N.ARCH_GEMMA2, 2, 512, 16, 8, 1024, 512, 8192, 10000.0,
                             _types(*([Q8_0] * 8)), head_dim=256, emb_type=BF16, window=4096, attn_softcap=50.0,
                             final_softcap=30.0, norm_std=0.1, seed=20),
    # FFN 16640 = 65 chunks of 256: down's rows split into 9 waves of 8 chunks, the last one with 1
    # chunk of the row and 7 past it
    "test-ragged": _cfg("test-ragged", N.ARCH_LLAMA, 2, 256, 4, 2, 16640, 512, 64, 10000.0,
                        _types(Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K, Q6_K), norm_std=0.1, seed=18),
    # the decode layers' q/k/v + attention shapes of the three full-size models at a small FFN and
    # vocabulary (the attention's head groups and widths at full size): Llama-3-8B (dim 4096, 32 / 8 heads x 128,
    # Q4_K q/k, Q6_K v), Qwen2-7B (dim 3584 = 14 chunks, 28 / 4 heads x 128, Q5_K, QKV bias),
    # Gemma-2-9B (dim 3584, 16 / 8 heads x 256, Q8_0, softcaps, window 64 on the even layers)
    "test-llama-qkva": _cfg("test-llama-qkva", N.ARCH_LLAMA, 3, 4096, 32, 8, 1024, 512, 320, 500000.0,
                            _types(Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K, Q6_K), norm_std=0.1, seed=22),
    "test-qwen2-qkva": _cfg("test-qwen2-qkva", N.ARCH_QWEN2, 3, 3584, 28, 4, 1024, 512, 320, 1000000.0,
                            _types(*([Q5_K] * 7), Q6_K), norm_std=0.1, seed=23),
    "test-gemma2-qkva": _cfg("test-gemma2-qkva", N.ARCH_GEMMA2, 3, 3584, 16, 8, 1024, 512, 320, 10000.0,
                             _types(*([Q8_0] * 8)), head_dim=256, emb_type=BF16, window=64, attn_softcap=50.0,
                             final_softcap=30.0, norm_std=0.1, seed=24),
    # FFN rows past the prefill's fused-split limit (20480) and past the matrix-core GEMV's splits
    "test-wide-ffn": _cfg("test-wide-ffn", N.ARCH_LLAMA, 2, 256, 4, 2, 20992, 512, 64, 10000.0,
                          _types(Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K, Q6_K), norm_std=0.1, seed=19),
}


def desc_of(cfg):
    d = N.ModelDesc()
    d.arch = cfg["arch"]
    d.n_layers = cfg["n_layers"]
    d.hidden = cfg["hidden"]
    d.ffn = cfg["ffn"]
    d.n_heads = cfg["n_heads"]
    d.n_kv_heads = cfg["n_kv_heads"]
    d.head_dim = cfg["head_dim"]
    d.vocab = cfg["vocab"]
    d.max_ctx = cfg["max_ctx"]
    d.rope_base = cfg["rope_base"]
    d.rope_scale = cfg["rope_scale"]
    d.rope_scaled = cfg["rope_scaled"]
    gemma = cfg["arch"] == N.ARCH_GEMMA2
    d.norm_eps = 1e-6 if gemma else 1e-5
    d.attn_scale = float(np.float32(1.0) / np.sqrt(np.float32(cfg["head_dim"])))
    d.attn_softcap = cfg["attn_softcap"]
    d.final_softcap = cfg["final_softcap"]
    d.sliding_window = cfg["window"]
    return d


def tensor_plan(cfg):
    """[(gguf_name, slot, layer, type, rows, cols, (dist, p0, p1), tensor_id)] for every tensor."""
    h, f, V = cfg["hidden"], cfg["ffn"], cfg["vocab"]
    q = cfg["n_heads"] * cfg["head_dim"]
    kv = cfg["n_kv_heads"] * cfg["head_dim"]
    t = cfg["types"]
    nstd = cfg["norm_std"]
    norm_dist = (0, 1.0, nstd) if nstd > 0 else (1, 1.0, 0.0)

    def wdist(tt):
        if tt == Q8_0:
            return (0,) + Q8_RANGE
        if tt in (Q4_K, Q5_K, Q6_K, Q4_0, Q8_K):
            return (0,) + KQ_RANGE
        return (0, 0.0, 0.02)

    plan = [("token_embd.weight", N.SLOT_TOKEN_EMBD, 0, cfg["emb_type"], V, h, (0, 0.0, 0.02))]
    plan.append(("output_norm.weight", N.SLOT_OUTPUT_NORM, 0, F32, 1, h, norm_dist))
    if not cfg["tied"]:
        plan.append(("output.weight", N.SLOT_OUTPUT, 0, t["out"], V, h, wdist(t["out"])))
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        layer = [
            ("attn_norm.weight", N.SLOT_ATTN_NORM, F32, 1, h, norm_dist),
            ("attn_q.weight", N.SLOT_ATTN_Q, t["q"], q, h, wdist(t["q"])),
            ("attn_k.weight", N.SLOT_ATTN_K, t["k"], kv, h, wdist(t["k"])),
            ("attn_v.weight", N.SLOT_ATTN_V, t["v"], kv, h, wdist(t["v"])),
            ("attn_output.weight", N.SLOT_ATTN_OUTPUT, t["o"], h, q, wdist(t["o"])),
            ("ffn_norm.weight", N.SLOT_FFN_NORM, F32, 1, h, norm_dist),
            ("ffn_gate.weight", N.SLOT_FFN_GATE, t["gate"], f, h, wdist(t["gate"])),
            ("ffn_up.weight", N.SLOT_FFN_UP, t["up"], f, h, wdist(t["up"])),
            ("ffn_down.weight", N.SLOT_FFN_DOWN, t["down"], h, f, wdist(t["down"])),
        ]
        if cfg["arch"] == N.ARCH_QWEN2:
            layer += [("attn_q.bias", N.SLOT_ATTN_Q_BIAS, F32, 1, q, (0, 0.0, 0.02)),
                      ("attn_k.bias", N.SLOT_ATTN_K_BIAS, F32, 1, kv, (0, 0.0, 0.02)),
                      ("attn_v.bias", N.SLOT_ATTN_V_BIAS, F32, 1, kv, (0, 0.0, 0.02))]
        if cfg["arch"] == N.ARCH_GEMMA2:
            layer += [("post_attn_norm.weight", N.SLOT_POST_ATTN_NORM, F32, 1, h, norm_dist),
                      ("post_ffn_norm.weight", N.SLOT_POST_FFN_NORM, F32, 1, h, norm_dist)]
        for name, slot, tt, rows, cols, dist in layer:
            plan.append((b + name, slot, l, tt, rows, cols, dist))
    return [(n, s, l, tt, r, c, dist, s * 10000 + l) for (n, s, l, tt, r, c, dist) in plan]


def synth_bytes(cfg, entry, threads=0):
    from . import synth_tensor
    name, slot, layer, tt, rows, cols, (dist, p0, p1), tid = entry
    return synth_tensor(tt, cfg["seed"], tid, rows * cols, dist, p0, p1, threads)


def weight_bytes_per_token(cfg):
    """Bytes of every linear weight read by one decode step, as stored (layers, LM head)."""
    from ._native import type_bytes
    layers = head = 0
    for (name, slot, layer, tt, rows, cols, dist, tid) in tensor_plan(cfg):
        if slot in (N.SLOT_ATTN_Q, N.SLOT_ATTN_K, N.SLOT_ATTN_V, N.SLOT_ATTN_OUTPUT, N.SLOT_FFN_GATE,
                    N.SLOT_FFN_UP, N.SLOT_FFN_DOWN):
            layers += type_bytes(tt, rows * cols) if tt not in (F32, F16, BF16) else rows * cols * (4 if tt == F32 else 2)
    out_t = cfg["types"]["out"] if not cfg["tied"] else cfg["emb_type"]
    n = cfg["vocab"] * cfg["hidden"]
    head = type_bytes(out_t, n) if out_t not in (F32, F16, BF16) else n * (4 if out_t == F32 else 2)
    return layers, head


def build_model(ctx, cfg, keep_bytes=False, threads=0, n_layers=None, stats=None):
    """Generate every tensor of cfg from its seed and upload it; returns (Model, {name: bytes}).
    With a dict as stats, adds the bytes uploaded and the seconds spent in the upload calls."""
    import time
    from . import Model
    c = dict(cfg)
    if n_layers is not None:
        c["n_layers"] = n_layers
    m = Model(ctx, desc_of(c))
    kept = {}
    up_s, up_b = 0.0, 0
    for entry in tensor_plan(c):
        data = synth_bytes(c, entry, threads)
        t = time.perf_counter()
        m.upload(entry[1], entry[2], entry[3], data)
        up_s += time.perf_counter() - t
        up_b += len(data)
        if keep_bytes:
            kept[entry[0]] = (entry, data)
        del data
    t = time.perf_counter()
    m.finalize()
    if stats is not None:
        stats.update(upload_s=up_s, upload_bytes=up_b, finalize_s=time.perf_counter() - t)
    return m, kept


def attn_scale(cfg):
    return float(np.float32(1.0) / np.float32(math.sqrt(cfg["head_dim"])))
