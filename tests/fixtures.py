"""Shared model fixtures for the parity tests.

reference_fixture(arch): the deterministic F32 models of the reference's forward-pass tests
(tests/DotNetFoundryLLM.Architectures.Tests/{Qwen2,Mistral,Gemma2}ForwardPassTests.cs:
2 layers, hidden 8, FFN 8, 2/2 heads, vocab 16, weights ((i % 7) - 3) * scale with the
per-tensor scale schedule of those files), as (ModelDesc, {name: (plan entry, bytes)}).
"""
import numpy as np

import dotnetfoundryllm_amd._native as N
from dotnetfoundryllm_amd.configs import CONFIGS, desc_of, synth_bytes, tensor_plan

REF_TOKENS = [(1, 0), (2, 1), (3, 2)]  # the fixtures' Forward(token, position) calls


def _make_array(n, scale):
    i = np.arange(n)
    return (((i % 7) - 3) * np.float32(scale)).astype(np.float32)


def _jagged(layer, scale):
    return np.float32(scale + layer * np.float32(0.01))


def reference_fixture(arch):
    d = N.ModelDesc()
    d.arch = arch
    d.n_layers, d.hidden, d.ffn, d.n_heads, d.n_kv_heads = 2, 8, 8, 2, 2
    d.head_dim, d.vocab, d.max_ctx = 4, 16, 8
    d.rope_base, d.rope_scale, d.rope_scaled = 10000.0, 1.0, 0
    d.norm_eps = 1e-5
    d.attn_scale = float(np.float32(1.0) / np.sqrt(np.float32(4)))
    d.attn_softcap = d.final_softcap = 0.0
    d.sliding_window = 0x7FFFFFFF
    if arch == N.ARCH_MISTRAL:
        d.sliding_window = 2
    if arch == N.ARCH_GEMMA2:
        d.sliding_window, d.attn_softcap, d.final_softcap, d.attn_scale, d.norm_eps = 2, 4.0, 6.0, 0.5, 1e-6
    h, f, q, kv, V = 8, 8, 8, 8, 16
    per_layer = [("attn_norm.weight", N.SLOT_ATTN_NORM, h, 0.02)]
    if arch == N.ARCH_GEMMA2:
        per_layer += [("post_attn_norm.weight", N.SLOT_POST_ATTN_NORM, h, 0.025)]
    per_layer += [("attn_q.weight", N.SLOT_ATTN_Q, q * h, 0.03), ("attn_k.weight", N.SLOT_ATTN_K, kv * h, 0.04),
                  ("attn_v.weight", N.SLOT_ATTN_V, kv * h, 0.05), ("attn_output.weight", N.SLOT_ATTN_OUTPUT, h * q, 0.06)]
    if arch == N.ARCH_QWEN2:
        per_layer += [("attn_q.bias", N.SLOT_ATTN_Q_BIAS, q, 0.015), ("attn_k.bias", N.SLOT_ATTN_K_BIAS, kv, 0.016),
                      ("attn_v.bias", N.SLOT_ATTN_V_BIAS, kv, 0.017)]
    per_layer += [("ffn_norm.weight", N.SLOT_FFN_NORM, h, 0.07)]
    if arch == N.ARCH_GEMMA2:
        per_layer += [("post_ffn_norm.weight", N.SLOT_POST_FFN_NORM, h, 0.075)]
    per_layer += [("ffn_gate.weight", N.SLOT_FFN_GATE, f * h, 0.08), ("ffn_up.weight", N.SLOT_FFN_UP, f * h, 0.09),
                  ("ffn_down.weight", N.SLOT_FFN_DOWN, h * f, 0.10)]
    tensors = {}

    def put(name, slot, layer, arr):
        entry = (name, slot, layer, N.F32, 1, arr.size, (1, 0.0, 0.0), slot * 10000 + layer)
        tensors[name] = (entry, arr.view(np.uint8).copy())

    put("token_embd.weight", N.SLOT_TOKEN_EMBD, 0, _make_array(V * h, 0.01))
    for l in range(2):
        for name, slot, n, sc in per_layer:
            put(f"blk.{l}.{name}", slot, l, _make_array(n, _jagged(l, sc)))
    put("output_norm.weight", N.SLOT_OUTPUT_NORM, 0, _make_array(h, 0.11))
    put("output.weight", N.SLOT_OUTPUT, 0, _make_array(V * h, 0.12))
    return d, tensors


def synthetic(cfg_name, n_layers=None):
    cfg = dict(CONFIGS[cfg_name])
    if n_layers is not None:
        cfg["n_layers"] = n_layers
    tensors = {}
    for entry in tensor_plan(cfg):
        tensors[entry[0]] = (entry, synth_bytes(cfg, entry))
    return cfg, desc_of(cfg), tensors


def upload(model, tensors):
    for name, (entry, data) in tensors.items():
        model.upload(entry[1], entry[2], entry[3], data)
    model.finalize()


def f32_of(tensors, name):
    entry, data = tensors[name]
    import oracle_bind as O
    rc, out = O.dequantize(entry[3], data, entry[4] * entry[5])
    assert rc == 0
    return out
