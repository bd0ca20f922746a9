"""dotnetfoundryllm_amd — MI355X (gfx950) decode path of DotNetFoundryLLM behind a C ABI.

Python surface over libfllm_hip.so / libfllm_host.so, shaped like the reference's managed
interfaces so tests read like the reference's own:
  Dequantizer.dequantize / element_count   (Dequantizer.cs:466-504)
  HipForwardPass.forward(token_id, position, kv) / .logits   (IForwardPass.cs:11-14)
  HipKvCache: append order, current_length, get_keys/get_values, clear   (Interfaces.cs:73-92)
  SamplerPipeline(temperature, top_k, top_p, seed).sample(...)  (SamplerPipeline.cs:14-89)
  XoshiroRandom(seed)                                             (XoshiroRandom.cs)
  GgufModelLoader.load(path)                                      (GgufModelLoader.cs:42-85)
  LlamaLanguageModel.generate(prompt_ids, ...)                    (LlamaLanguageModel.cs:100-331)
Errors raise the exception class named after the .NET exception the reference throws.
"""
import ctypes as C

import numpy as np

from . import _native as N
from ._native import (ARCH_GEMMA2, ARCH_LLAMA, ARCH_MISTRAL, ARCH_QWEN2, BF16, F16, F32, Q4_0, Q4_K, Q5_K,
                      Q6_K, Q8_0, Q8_K, ModelDesc, type_bytes)


class FoundryError(Exception):
    code = None


class ArgumentOutOfRangeException(FoundryError, IndexError):
    code = N.E_ARG_RANGE


class ArgumentException(FoundryError, ValueError):
    code = N.E_ARG


class InvalidOperationException(FoundryError, RuntimeError):
    code = N.E_INVALID_OP


class NotSupportedException(FoundryError, NotImplementedError):
    code = N.E_NOT_SUPPORTED


class ObjectDisposedException(FoundryError, RuntimeError):
    code = N.E_DISPOSED


class ModelLoadException(FoundryError, RuntimeError):
    code = N.E_MODEL_LOAD


class DeviceError(FoundryError, RuntimeError):
    code = N.E_DEVICE


class ArgumentNullException(FoundryError, ValueError):
    code = N.E_NULL


class OutOfMemoryException(FoundryError, MemoryError):
    code = N.E_OOM


_BY_CODE = {c.code: c for c in (ArgumentOutOfRangeException, ArgumentException, InvalidOperationException,
                                NotSupportedException, ObjectDisposedException, ModelLoadException, DeviceError,
                                ArgumentNullException, OutOfMemoryException)}


def _check(rc, host=False):
    if rc == N.OK:
        return
    msg = (N.host.fllmh_last_error() if host else N.dev.fllm_last_error()) or b""
    raise _BY_CODE.get(rc, FoundryError)(msg.decode(errors="replace"))


def _hcheck(rc):
    _check(rc, host=True)


def _fptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _iptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


# ----------------------------------------------------------------------------------------
class Context:
    """One device: default stream and utility scratch (fllm_ctx)."""

    def __init__(self, device=0):
        h = C.c_void_p()
        _check(N.dev.fllm_ctx_create(device, C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            N.dev.fllm_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def sync(self):
        _check(N.dev.fllm_ctx_sync(self.h))

    def device_info(self):
        n = C.c_int32()
        m = C.c_int64()
        _check(N.dev.fllm_ctx_device_info(self.h, C.byref(n), C.byref(m)))
        return n.value, m.value


class Dequantizer:
    """Dequantizer.Dequantize / ElementCount on the device (bit-exact)."""

    @staticmethod
    def element_count(tensor_type, byte_length):
        out = C.c_int64()
        _check(N.dev.fllm_element_count(tensor_type, byte_length, C.byref(out)))
        return out.value

    @staticmethod
    def dequantize(ctx, tensor_type, src, dst_len=None):
        src = np.ascontiguousarray(np.frombuffer(bytes(src), dtype=np.uint8) if not isinstance(src, np.ndarray)
                                   else src.view(np.uint8).reshape(-1))
        n = dst_len
        if n is None:
            bb, be = N.BLOCK.get(tensor_type, (1, 1))
            n = src.nbytes // bb * be
        dst = np.zeros(max(n, 1), dtype=np.float32)
        _check(N.dev.fllm_dequantize(ctx.h, tensor_type, src.ctypes.data_as(C.c_void_p), src.nbytes, _fptr(dst), n))
        return dst[:n]


class DeviceBuffer:
    def __init__(self, ctx, nbytes):
        h = C.c_void_p()
        _check(N.dev.fllm_buf_create(ctx.h, nbytes, C.byref(h)))
        self.h, self.n, self.ctx = h, nbytes, ctx

    def write(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        _check(N.dev.fllm_buf_write(self.h, offset, arr.ctypes.data_as(C.c_void_p), arr.nbytes))

    def read(self, nbytes, dtype=np.float32, offset=0):
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype=dtype)
        _check(N.dev.fllm_buf_read(self.h, offset, out.ctypes.data_as(C.c_void_p), out.nbytes))
        return out

    def close(self):
        if self.h:
            N.dev.fllm_buf_destroy(self.h)
            self.h = None


LAYOUT_GGUF, LAYOUT_TILES = 0, 1  # fllm_layout


def gemv(ctx, tensor_type, w_buf, rows, cols, x_buf, y_buf, w_offset=0, layout=LAYOUT_GGUF):
    """LinearProjection on device buffers (enqueued on the context stream); layout
    LAYOUT_TILES reads a matrix written by gemv_pack."""
    if layout == LAYOUT_GGUF:
        _check(N.dev.fllm_gemv(ctx.h, tensor_type, w_buf.h, w_offset, rows, cols, x_buf.h, y_buf.h))
    else:
        _check(N.dev.fllm_gemv_ex(ctx.h, tensor_type, w_buf.h, w_offset, rows, cols, x_buf.h, y_buf.h, layout))


def gemv_pack(ctx, tensor_type, src_buf, rows, cols, dst_buf, src_offset=0):
    """Regroups a GGUF matrix into the tile-interleaved layout of the matrix-core GEMV."""
    _check(N.dev.fllm_gemv_pack(ctx.h, tensor_type, src_buf.h, src_offset, rows, cols, dst_buf.h))


def gemv_time(ctx, tensor_type, w_bufs, rows, cols, x_buf, y_buf, iters, layout=None):
    """Mean microseconds per launch over `iters` launches cycling through w_bufs: with layout
    None, one HIP event pair per launch (fllm_gemv_time, GGUF rows); with a layout, one pair around
    all launches back to back (fllm_gemv_time_ex)."""
    arr = (C.c_void_p * len(w_bufs))(*[b.h.value for b in w_bufs])
    out = C.c_double()
    if layout is None:
        _check(N.dev.fllm_gemv_time(ctx.h, tensor_type, C.cast(arr, C.POINTER(C.c_void_p)), len(w_bufs), rows, cols,
                                    x_buf.h, y_buf.h, iters, C.byref(out)))
    else:
        _check(N.dev.fllm_gemv_time_ex(ctx.h, tensor_type, C.cast(arr, C.POINTER(C.c_void_p)), len(w_bufs), rows,
                                       cols, x_buf.h, y_buf.h, iters, layout, C.byref(out)))
    return out.value


# ----------------------------------------------------------------------------------------
class Model:
    """Device-resident weights in GGUF block layout (LlamaWeights / Qwen2Weights / Gemma2Weights)."""

    def __init__(self, ctx, desc, handle=None):
        self.ctx = ctx
        self.desc = desc
        if handle is None:
            h = C.c_void_p()
            _check(N.dev.fllm_model_create(ctx.h, C.byref(desc), C.byref(h)))
            self.h = h
        else:
            self.h = handle

    def upload(self, slot, layer, tensor_type, data):
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        _check(N.dev.fllm_model_upload(self.h, slot, layer, tensor_type, data.ctypes.data_as(C.c_void_p),
                                       data.nbytes))

    def finalize(self):
        _check(N.dev.fllm_model_finalize(self.h))

    def weight_bytes(self):
        a, b = C.c_uint64(), C.c_uint64()
        _check(N.dev.fllm_model_weight_bytes(self.h, C.byref(a), C.byref(b)))
        return a.value, b.value

    def close(self):
        if self.h:
            N.dev.fllm_model_destroy(self.h)
            self.h = None


class HipKvCache:
    """IKvCache over the device KV cache of one sequence (fllm_seq): MaxSequenceLength,
    CurrentLength, Append, GetKeys / GetValues, Clear, WasEvicted, Dispose (KvCache.cs:14-174)."""

    def __init__(self, model, max_sequence_length=0):
        if max_sequence_length < 0:
            raise ArgumentOutOfRangeException("maxSequenceLength")
        h = C.c_void_p()
        _check(N.dev.fllm_seq_create(model.h, max_sequence_length, C.byref(h)))
        self.h = h
        self.model = model
        self.kv_dim = model.desc.n_kv_heads * model.desc.head_dim

    def _handle(self):
        # ObjectDisposedException.ThrowIf(_disposed, this) (KvCache.cs:61,102,121,140)
        if not self.h:
            raise ObjectDisposedException("KvCache")
        return self.h

    @property
    def max_sequence_length(self):
        v = C.c_int32()
        _check(N.dev.fllm_seq_capacity(self._handle(), C.byref(v)))
        return v.value

    @property
    def current_length(self):
        v = C.c_int32()
        _check(N.dev.fllm_seq_length(self._handle(), C.byref(v)))
        return v.value

    @property
    def was_evicted(self):
        v = C.c_int32()
        _check(N.dev.fllm_kv_was_evicted(self._handle(), C.byref(v)))
        return bool(v.value)

    def append(self, layer, key_slice, value_slice):
        """KvCache.Append(layer, keySlice, valueSlice) (KvCache.cs:59-97)."""
        h = self._handle()
        k = np.ascontiguousarray(key_slice, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(value_slice, dtype=np.float32).reshape(-1)
        _check(N.dev.fllm_kv_append(h, int(layer), _fptr(k), k.size, _fptr(v), v.size))

    def get_keys(self, layer):
        return self._kv(layer, 0)

    def get_values(self, layer):
        return self._kv(layer, 1)

    def _kv(self, layer, kind):
        h = self._handle()
        n_pos = C.c_int32()
        _check(N.dev.fllm_kv_length(h, int(layer), C.byref(n_pos)))
        n = n_pos.value * self.kv_dim
        out = np.zeros(max(n, 1), dtype=np.float32)
        _check(N.dev.fllm_kv_read(h, int(layer), kind, _fptr(out), out.size))
        return out[:n]

    def clear(self):
        _check(N.dev.fllm_seq_reset(self._handle()))

    def dispose(self):
        if self.h:
            N.dev.fllm_seq_destroy(self.h)
            self.h = None

    close = dispose

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.dispose()


class HipForwardPass:
    """IForwardPass on the device: forward(token_id, position, kv) then .logits."""

    def __init__(self, model):
        self.model = model
        self._kv = None

    def forward(self, token_id, position, kv):
        if kv is None:
            raise ArgumentNullException("kvCache")
        if not isinstance(kv, HipKvCache):
            # the device forward pass appends to and attends over a device-resident cache only
            raise ArgumentException("kvCache must be a HipKvCache created from this model")
        _check(N.dev.fllm_forward(kv._handle(), int(token_id), int(position)))
        self._kv = kv

    def prefill(self, tokens, pos0, kv):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        _check(N.dev.fllm_prefill(kv.h, _iptr(t), len(t), pos0))
        self._kv = kv

    def decode_greedy(self, token_id, position, n_steps, kv):
        """n greedy decode steps from token_id at position, each step's token fed to the next on
        the device; returns the n generated tokens."""
        if kv is None:
            raise ArgumentNullException("kvCache")
        out = np.zeros(max(int(n_steps), 1), dtype=np.int32)
        _check(N.dev.fllm_decode_greedy(kv.h, int(token_id), int(position), int(n_steps), _iptr(out)))
        self._kv = kv
        return out[: int(n_steps)]

    @property
    def logits(self):
        # before the first Forward: zeros, as LlamaForwardPass's fresh _logits (LlamaForwardPass.cs:38)
        if self._kv is None:
            return np.zeros(self.model.desc.vocab, dtype=np.float32)
        out = np.empty(self.model.desc.vocab, dtype=np.float32)
        _check(N.dev.fllm_logits_copy(self._kv.h, _fptr(out), out.size))
        return out

    def write_logits(self, values, kv=None):
        kv = kv or self._kv
        a = np.ascontiguousarray(values, dtype=np.float32)
        _check(N.dev.fllm_logits_write(kv.h, _fptr(a), a.size))
        self._kv = kv

    def sample_greedy(self):
        v = C.c_int32()
        _check(N.dev.fllm_sample_greedy(self._kv.h, C.byref(v)))
        return v.value

    def sample_topk(self, inv_temp, k, cap=4096):
        ids = np.zeros(cap, dtype=np.int32)
        vals = np.zeros(cap, dtype=np.float32)
        n = C.c_int32()
        _check(N.dev.fllm_sample_topk(self._kv.h, inv_temp, k, _iptr(ids), _fptr(vals), cap, C.byref(n)))
        return ids[: n.value], vals[: n.value]

    def penalize(self, ids, penalty):
        """LlamaLanguageModel.ApplyRepetitionPenalty over `ids` on the device logits."""
        a = np.ascontiguousarray(ids, dtype=np.int32)
        _check(N.dev.fllm_logits_penalize(self._kv.h, _iptr(a), a.size, penalty))

    def sample_nucleus(self, inv_temp, top_p, u):
        """SamplerPipeline stages 1, 3, 4, 5 (no top-k) on the device with the draw's u."""
        v = C.c_int32()
        _check(N.dev.fllm_sample_nucleus(self._kv.h, inv_temp, top_p, u, C.byref(v)))
        return v.value

    def probs(self):
        out = np.empty(self.model.desc.vocab, dtype=np.float32)
        _check(N.dev.fllm_probs_copy(self._kv.h, _fptr(out), out.size))
        return out

    def hidden(self, layer):
        out = np.empty(self.model.desc.hidden, dtype=np.float32)
        _check(N.dev.fllm_debug_hidden(self._kv.h, layer, _fptr(out), out.size))
        return out


def set_graph(kv, enable):
    _check(N.dev.fllm_seq_set_graph(kv.h, 1 if enable else 0))


def set_debug(kv, enable):
    _check(N.dev.fllm_seq_set_debug(kv.h, 1 if enable else 0))


def set_prefill_chunk(kv, tokens):
    """Tokens per pass of the batched prefill (for the sequence's later prefills)."""
    _check(N.dev.fllm_seq_set_prefill_chunk(kv.h, int(tokens)))


def set_attention_merge(kv, in_launch):
    """Decode attention chunks merged inside the attention launch or by a second launch (the default
    is chosen per shape: inside when a kv head has at most 4 query heads and 32 chunks)."""
    _check(N.dev.fllm_seq_set_attention_merge(kv.h, 1 if in_launch else 0))


def set_profile(kv, enable):
    _check(N.dev.fllm_seq_set_profile(kv.h, 1 if enable else 0))


def profile_entries(kv):
    n = C.c_int32()
    _check(N.dev.fllm_seq_profile_count(kv.h, C.byref(n)))
    out = []
    for i in range(n.value):
        name = C.create_string_buffer(64)
        l, ms, b = C.c_int64(), C.c_double(), C.c_double()
        _check(N.dev.fllm_seq_profile_entry(kv.h, i, name, 64, C.byref(l), C.byref(ms), C.byref(b)))
        out.append({"name": name.value.decode(), "launches": l.value, "ms": ms.value, "bytes": b.value})
    return out


def profile_reset(kv):
    _check(N.dev.fllm_seq_profile_reset(kv.h))


def profile_launches(kv):
    """Names of the profiled launches in launch order (one kernel each) since the last reset."""
    out = []
    name = C.create_string_buffer(64)
    i = 0
    while N.dev.fllm_seq_profile_launch(kv.h, i, name, 64) == 0:
        out.append(name.value.decode())
        i += 1
    return out


# ----------------------------------------------------------------------------------------
class XoshiroRandom:
    def __init__(self, seed=0):
        self.s = N.Xoshiro()
        N.host.fllmh_xoshiro_init(C.byref(self.s), seed)

    def next_uint64(self):
        return N.host.fllmh_xoshiro_next(C.byref(self.s))

    def next_float(self):
        return N.host.fllmh_xoshiro_next_float(C.byref(self.s))


class SamplerPipeline:
    """SamplerPipeline(temperature, topK, topP, seed) over the device sampler."""

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, seed=0):
        h = C.c_void_p()
        _hcheck(N.host.fllmh_sampler_create(temperature, top_k, top_p, seed, C.byref(h)))
        self.h = h

    def sample(self, kv):
        v = C.c_int32()
        _hcheck(N.host.fllmh_sampler_sample(self.h, kv.h, C.byref(v)))
        return v.value

    def sample_host(self, logits):
        a = np.ascontiguousarray(logits, dtype=np.float32).copy()
        v = C.c_int32()
        _hcheck(N.host.fllmh_sampler_sample_host(self.h, _fptr(a), a.size, C.byref(v)))
        return v.value

    def close(self):
        if self.h:
            N.host.fllmh_sampler_destroy(self.h)
            self.h = None


class LlamaLanguageModel:
    """Token loop of LlamaLanguageModel.GenerateAsync over already-tokenized ids."""

    def __init__(self, model, kv, bos_token_id=1, eos_token_id=2):
        self.model, self.kv = model, kv
        self.bos, self.eos = bos_token_id, eos_token_id

    def generate(self, prompt_ids, max_tokens, sampler, stop_at_eos=True, repetition_penalty=1.0):
        p = np.ascontiguousarray(prompt_ids, dtype=np.int32)
        out = np.zeros(max(max_tokens, 1), dtype=np.int32)
        st = N.GenerateStats()
        _hcheck(N.host.fllmh_generate(self.kv.h, _iptr(p), len(p), max_tokens, sampler.h,
                                      self.eos if stop_at_eos else -1, self.bos, repetition_penalty,
                                      _iptr(out), C.byref(st)))
        return out[: st.completion_tokens].copy(), st


class GgufModelLoader:
    """GgufModelLoader.LoadAsync: parse GGUF, upload raw tensor bytes to the device."""

    @staticmethod
    def read_info(path):
        info = N.ModelInfo()
        _hcheck(N.host.fllmh_read_gguf_info(str(path).encode(), C.byref(info)))
        return info

    @staticmethod
    def load(ctx, path):
        info = N.ModelInfo()
        h = C.c_void_p()
        _hcheck(N.host.fllmh_load_gguf(ctx.h, str(path).encode(), C.byref(h), C.byref(info)))
        m = Model(ctx, info.desc, handle=h)
        return m, info


def synth_tensor(tensor_type, seed, tensor_id, n_elems, dist=0, p0=0.0, p1=1.0, threads=0):
    """Seeded synthetic tensor bytes in GGUF block layout (fllmh_synth_tensor)."""
    if tensor_type in (F32, F16, BF16):
        nbytes = n_elems * (4 if tensor_type == F32 else 2)
    else:
        nbytes = type_bytes(tensor_type, n_elems)
    out = np.empty(nbytes, dtype=np.uint8)
    _hcheck(N.host.fllmh_synth_tensor(tensor_type, seed, tensor_id, n_elems, dist, p0, p1,
                                      out.ctypes.data_as(C.c_void_p), nbytes, threads))
    return out


def synth_tokens(seed, stream, vocab, n):
    out = np.zeros(max(n, 1), dtype=np.int32)
    _hcheck(N.host.fllmh_synth_tokens(seed, stream, vocab, _iptr(out), n))
    return out[:n]
