"""ctypes binding of the CPU oracle (oracle/build/liboracle.so) — the checker for the parity
tests. Only tests/, the smoke check and bench.py's cpu_baseline leg use it."""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "build", "liboracle.so")


def _ensure_built():
    if not os.path.exists(LIB):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, stdout=subprocess.DEVNULL)


_ensure_built()
lib = C.CDLL(LIB)

P, I32, I64, U64, F32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float
PF = C.POINTER(C.c_float)


class OrcDesc(C.Structure):
    _fields_ = [("arch", I32), ("n_layers", I32), ("hidden", I32), ("ffn", I32), ("n_heads", I32),
                ("n_kv_heads", I32), ("head_dim", I32), ("vocab", I32), ("max_ctx", I32), ("rope_base", F32),
                ("rope_scale", F32), ("rope_scaled", I32), ("norm_eps", F32), ("attn_scale", F32),
                ("attn_softcap", F32), ("final_softcap", F32), ("sliding_window", I32)]


class OrcXoshiro(C.Structure):
    _fields_ = [("s0", U64), ("s1", U64), ("s2", U64), ("s3", U64)]


_sigs = {
    "orc_set_threads": (C.c_int, [C.c_int]),
    "orc_get_threads": (C.c_int, []),
    "orc_half_to_float": (F32, [C.c_uint16]),
    "orc_bf16_to_float": (F32, [C.c_uint16]),
    "orc_dequantize": (C.c_int, [C.c_int, P, I64, PF, I64]),
    "orc_element_count": (C.c_int, [C.c_int, I64, C.POINTER(I64)]),
    "orc_decode_kscale_min": (None, [P, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "orc_dot": (F32, [PF, PF, I64]),
    "orc_linear": (None, [PF, PF, PF, I64, I64]),
    "orc_rmsnorm": (C.c_int, [PF, PF, PF, I64, F32]),
    "orc_gemma_rmsnorm": (None, [PF, PF, PF, I64]),
    "orc_silu": (None, [PF, I64]),
    "orc_gelu": (None, [PF, I64]),
    "orc_softcap": (None, [PF, I64, F32]),
    "orc_softmax": (None, [PF, I64]),
    "orc_rope_inv_freqs": (None, [F32, C.c_int, PF]),
    "orc_apply_rope": (None, [PF, F32, PF, C.c_int]),
    "orc_argmax": (I64, [PF, I64]),
    "orc_xoshiro_init": (None, [C.POINTER(OrcXoshiro), U64]),
    "orc_xoshiro_next": (U64, [C.POINTER(OrcXoshiro)]),
    "orc_xoshiro_next_float": (F32, [C.POINTER(OrcXoshiro)]),
    "orc_topk_threshold": (F32, [PF, I64, C.c_int]),
    "orc_apply_topk": (None, [PF, I64, C.c_int]),
    "orc_sample_from_probs": (I64, [PF, I64, C.POINTER(OrcXoshiro)]),
    "orc_sampler_pipeline": (I64, [PF, I64, F32, C.c_int, C.POINTER(OrcXoshiro)]),
    "orc_sampler_pipeline_p": (I64, [PF, I64, F32, C.c_int, F32, C.POINTER(OrcXoshiro)]),
    "orc_apply_top_p": (None, [PF, I64, F32]),
    "orc_repetition_penalty": (None, [PF, I64, C.POINTER(C.c_int32), I64, F32]),
    "orc_model_create": (P, [C.POINTER(OrcDesc)]),
    "orc_model_destroy": (None, [P]),
    "orc_model_set": (C.c_int, [P, C.c_int, C.c_int, C.c_int, P, I64]),
    "orc_model_finalize": (C.c_int, [P]),
    "orc_fwd_create": (P, [P, I32]),
    "orc_fwd_destroy": (None, [P]),
    "orc_fwd_reset": (None, [P]),
    "orc_forward": (C.c_int, [P, I32, I32]),
    "orc_logits": (PF, [P]),
    "orc_fwd_hidden": (C.c_int, [P, C.c_int, PF, I64]),
    "orc_fwd_kv": (C.c_int, [P, C.c_int, C.c_int, PF, I64]),
    "orc_fwd_length": (I32, [P]),
    "orc_fwd_limit": (None, [P, C.c_int, C.c_int]),
}
for _n, (_r, _a) in _sigs.items():
    _f = getattr(lib, _n)
    _f.restype = _r
    _f.argtypes = _a


def fp(a):
    return a.ctypes.data_as(PF)


def dequantize(tensor_type, raw, n=None):
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray)
                               else raw.view(np.uint8).reshape(-1))
    if n is None:
        cnt = I64()
        rc = lib.orc_element_count(tensor_type, raw.nbytes, C.byref(cnt))
        if rc:
            return rc, None
        n = cnt.value
    out = np.zeros(max(n, 1), dtype=np.float32)
    rc = lib.orc_dequantize(tensor_type, raw.ctypes.data_as(P), raw.nbytes, fp(out), n)
    return rc, out[:n]


def linear(W, x):
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(W.shape[0], dtype=np.float32)
    lib.orc_linear(fp(x), fp(W), fp(y), W.shape[0], W.shape[1])
    return y


class Xoshiro:
    def __init__(self, seed):
        self.s = OrcXoshiro()
        lib.orc_xoshiro_init(C.byref(self.s), seed)

    def next(self):
        return lib.orc_xoshiro_next(C.byref(self.s))

    def next_float(self):
        return lib.orc_xoshiro_next_float(C.byref(self.s))


def sampler_pipeline(logits, temperature, top_k, rng):
    a = np.ascontiguousarray(logits, dtype=np.float32).copy()
    return int(lib.orc_sampler_pipeline(fp(a), a.size, temperature, top_k, C.byref(rng.s)))


def sampler_pipeline_p(logits, temperature, top_k, top_p, rng):
    a = np.ascontiguousarray(logits, dtype=np.float32).copy()
    return int(lib.orc_sampler_pipeline_p(fp(a), a.size, temperature, top_k, top_p, C.byref(rng.s)))


def apply_top_p(probs, p):
    a = np.ascontiguousarray(probs, dtype=np.float32).copy()
    lib.orc_apply_top_p(fp(a), a.size, p)
    return a


def repetition_penalty(logits, ids, penalty):
    a = np.ascontiguousarray(logits, dtype=np.float32).copy()
    i = np.ascontiguousarray(ids, dtype=np.int32)
    lib.orc_repetition_penalty(fp(a), a.size, i.ctypes.data_as(C.POINTER(C.c_int32)), i.size, penalty)
    return a


def desc_from(d):
    o = OrcDesc()
    for name, _ in OrcDesc._fields_:
        setattr(o, name, getattr(d, name))
    return o


class OracleModel:
    """The reference forward pass on F32 weights dequantized at load (GgufModelLoader.LoadTensor)."""

    def __init__(self, desc, tensors, max_seq=0):
        self.desc = desc
        self._d = desc_from(desc)
        self.m = lib.orc_model_create(C.byref(self._d))
        for name, (entry, data) in tensors.items():
            _, slot, layer, tt, rows, cols, dist, tid = entry
            data = np.ascontiguousarray(data)
            rc = lib.orc_model_set(self.m, slot, layer, tt, data.ctypes.data_as(P), data.nbytes)
            if rc:
                raise RuntimeError(f"oracle rejected {name}: {rc}")
        rc = lib.orc_model_finalize(self.m)
        if rc:
            raise RuntimeError(f"oracle finalize: {rc}")
        self.f = lib.orc_fwd_create(self.m, max_seq)

    def forward(self, token, position):
        return lib.orc_forward(self.f, token, position)

    def logits(self):
        p = lib.orc_logits(self.f)
        return np.ctypeslib.as_array(p, shape=(self.desc.vocab,)).copy()

    def hidden(self, layer):
        out = np.zeros(self.desc.hidden, dtype=np.float32)
        rc = lib.orc_fwd_hidden(self.f, layer, fp(out), out.size)
        assert rc == 0
        return out

    def kv(self, layer, kind):
        n = lib.orc_fwd_length(self.f) * self.desc.n_kv_heads * self.desc.head_dim
        out = np.zeros(max(n, 1), dtype=np.float32)
        rc = lib.orc_fwd_kv(self.f, layer, kind, fp(out), out.size)
        assert rc == 0
        return out[:n]

    def reset(self):
        lib.orc_fwd_reset(self.f)

    def limit(self, n_layers, head_rows):
        lib.orc_fwd_limit(self.f, n_layers, head_rows)

    def close(self):
        if self.f:
            lib.orc_fwd_destroy(self.f)
            self.f = None
        if self.m:
            lib.orc_model_destroy(self.m)
            self.m = None


def normwise_rel_err(a, b):
    """max|a-b| / max|b|, the parity measure for hidden states and logits."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / (den if den > 0 else 1.0))
