"""ctypes bindings of libfllm_hip.so (include/fllm.h) and libfllm_host.so (include/fllm_host.h).

The libraries are built in-tree by dotnetfoundryllm_amd.build; importing this module loads
them and fails loudly when they are missing (there is no fallback implementation).
"""
import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
DEVICE_LIB = os.path.join(PKG, "libfllm_hip.so")
HOST_LIB = os.path.join(PKG, "libfllm_host.so")

# status codes (include/fllm.h enum fllm_status)
OK = 0
E_ARG_RANGE = -1
E_ARG = -2
E_INVALID_OP = -3
E_NOT_SUPPORTED = -4
E_DISPOSED = -5
E_MODEL_LOAD = -6
E_DEVICE = -7
E_NULL = -8
E_OOM = -9

# tensor types (GgufTensorType ids)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 15, 30
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K",
              Q6_K: "Q6_K", Q8_K: "Q8_K", BF16: "BF16"}
# (block bytes, block elements)
BLOCK = {F32: (4, 1), F16: (2, 1), BF16: (2, 1), Q4_0: (18, 32), Q8_0: (34, 32), Q4_K: (144, 256),
         Q5_K: (176, 256), Q6_K: (210, 256), Q8_K: (292, 256)}

ARCH_LLAMA, ARCH_MISTRAL, ARCH_QWEN2, ARCH_GEMMA2 = 0, 1, 2, 3

# limits of fllm_dequantize_noalloc (FLLM_NOALLOC_MAX_BYTES / FLLM_NOALLOC_MAX_ELEMS)
NOALLOC_MAX_BYTES = 2 << 20
NOALLOC_MAX_ELEMS = 2 << 20

SLOT_TOKEN_EMBD, SLOT_OUTPUT_NORM, SLOT_OUTPUT = 0, 1, 2
SLOT_ATTN_NORM, SLOT_ATTN_Q, SLOT_ATTN_K, SLOT_ATTN_V, SLOT_ATTN_OUTPUT = 10, 11, 12, 13, 14
SLOT_ATTN_Q_BIAS, SLOT_ATTN_K_BIAS, SLOT_ATTN_V_BIAS, SLOT_POST_ATTN_NORM = 15, 16, 17, 18
SLOT_FFN_NORM, SLOT_FFN_GATE, SLOT_FFN_UP, SLOT_FFN_DOWN, SLOT_POST_FFN_NORM = 19, 20, 21, 22, 23


def type_bytes(t, n):
    bb, be = BLOCK[t]
    if n % be:
        raise ValueError(f"{n} elements is not a whole number of {TYPE_NAMES[t]} blocks")
    return n // be * bb


class ModelDesc(C.Structure):
    _fields_ = [
        ("arch", C.c_int32), ("n_layers", C.c_int32), ("hidden", C.c_int32), ("ffn", C.c_int32),
        ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("vocab", C.c_int32),
        ("max_ctx", C.c_int32), ("rope_base", C.c_float), ("rope_scale", C.c_float), ("rope_scaled", C.c_int32),
        ("norm_eps", C.c_float), ("attn_scale", C.c_float), ("attn_softcap", C.c_float),
        ("final_softcap", C.c_float), ("sliding_window", C.c_int32),
    ]


class ModelInfo(C.Structure):
    _fields_ = [("desc", ModelDesc), ("bos_token_id", C.c_int32), ("eos_token_id", C.c_int32),
                ("gguf_version", C.c_int32), ("n_tensors", C.c_int32), ("data_offset", C.c_uint64)]


class Xoshiro(C.Structure):
    _fields_ = [("s0", C.c_uint64), ("s1", C.c_uint64), ("s2", C.c_uint64), ("s3", C.c_uint64)]


class GenerateStats(C.Structure):
    _fields_ = [("prompt_tokens", C.c_int32), ("completion_tokens", C.c_int32), ("prefill_ms", C.c_double),
                ("decode_ms", C.c_double), ("tokens_per_second", C.c_double), ("finish_reason", C.c_int32)]


P = C.c_void_p
I32, I64, U64, F32_, F64 = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double
PI32, PI64, PU64, PF32, PF64 = (C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.POINTER(C.c_uint64),
                                C.POINTER(C.c_float), C.POINTER(C.c_double))
PP = C.POINTER(C.c_void_p)

DEVICE_SIGS = {
    "fllm_last_error": (C.c_char_p, []),
    "fllm_version": (I32, []),
    "fllm_ctx_create": (I32, [I32, PP]),
    "fllm_ctx_destroy": (I32, [P]),
    "fllm_ctx_sync": (I32, [P]),
    "fllm_ctx_device_info": (I32, [P, PI32, PI64]),
    "fllm_model_create": (I32, [P, C.POINTER(ModelDesc), PP]),
    "fllm_model_upload": (I32, [P, I32, I32, I32, P, U64]),
    "fllm_model_finalize": (I32, [P]),
    "fllm_model_destroy": (I32, [P]),
    "fllm_model_get_desc": (I32, [P, C.POINTER(ModelDesc)]),
    "fllm_model_weight_bytes": (I32, [P, PU64, PU64]),
    "fllm_seq_create": (I32, [P, I32, PP]),
    "fllm_seq_destroy": (I32, [P]),
    "fllm_seq_reset": (I32, [P]),
    "fllm_seq_length": (I32, [P, PI32]),
    "fllm_seq_capacity": (I32, [P, PI32]),
    "fllm_seq_get_model": (I32, [P, PP]),
    "fllm_seq_set_graph": (I32, [P, I32]),
    "fllm_seq_set_debug": (I32, [P, I32]),
    "fllm_seq_set_prefill_chunk": (I32, [P, I32]),
    "fllm_seq_set_attention_merge": (I32, [P, I32]),
    "fllm_forward": (I32, [P, I32, I32]),
    "fllm_prefill": (I32, [P, PI32, I32, I32]),
    "fllm_decode_greedy": (I32, [P, I32, I32, I32, PI32]),
    "fllm_seq_sync": (I32, [P]),
    "fllm_logits_copy": (I32, [P, PF32, I64]),
    "fllm_logits_write": (I32, [P, PF32, I64]),
    "fllm_sample_greedy": (I32, [P, PI32]),
    "fllm_sample_topk": (I32, [P, F32_, I32, PI32, PF32, I32, PI32]),
    "fllm_logits_penalize": (I32, [P, PI32, I32, F32_]),
    "fllm_sample_nucleus": (I32, [P, F32_, F32_, F32_, PI32]),
    "fllm_probs_copy": (I32, [P, PF32, I64]),
    "fllm_debug_hidden": (I32, [P, I32, PF32, I64]),
    "fllm_kv_read": (I32, [P, I32, I32, PF32, I64]),
    "fllm_kv_length": (I32, [P, I32, PI32]),
    "fllm_kv_append": (I32, [P, I32, PF32, I64, PF32, I64]),
    "fllm_kv_was_evicted": (I32, [P, PI32]),
    "fllm_dequantize": (I32, [P, I32, P, U64, PF32, I64]),
    "fllm_dequantize_noalloc": (I32, [P, I32, P, U64, PF32, I64]),
    "fllm_element_count": (I32, [I32, I64, PI64]),
    "fllm_buf_create": (I32, [P, U64, PP]),
    "fllm_buf_destroy": (I32, [P]),
    "fllm_buf_write": (I32, [P, U64, P, U64]),
    "fllm_buf_read": (I32, [P, U64, P, U64]),
    "fllm_gemv": (I32, [P, I32, P, U64, I64, I64, P, P]),
    "fllm_gemv_time": (I32, [P, I32, PP, I32, I64, I64, P, P, I32, PF64]),
    "fllm_gemv_pack": (I32, [P, I32, P, U64, I64, I64, P]),
    "fllm_gemv_ex": (I32, [P, I32, P, U64, I64, I64, P, P, I32]),
    "fllm_gemv_time_ex": (I32, [P, I32, PP, I32, I64, I64, P, P, I32, I32, PF64]),
    "fllm_seq_set_profile": (I32, [P, I32]),
    "fllm_seq_profile_count": (I32, [P, PI32]),
    "fllm_seq_profile_entry": (I32, [P, I32, C.c_char_p, I32, PI64, PF64, PF64]),
    "fllm_seq_profile_reset": (I32, [P]),
    "fllm_seq_profile_launch": (I32, [P, I32, C.c_char_p, I32]),
}

HOST_SIGS = {
    "fllmh_last_error": (C.c_char_p, []),
    "fllmh_synth_tensor": (I32, [I32, U64, U64, I64, I32, F32_, F32_, P, U64, I32]),
    "fllmh_synth_tokens": (I32, [U64, U64, I32, PI32, I32]),
    "fllmh_f32_to_f16": (C.c_uint16, [F32_]),
    "fllmh_f32_to_bf16": (C.c_uint16, [F32_]),
    "fllmh_load_gguf": (I32, [P, C.c_char_p, PP, C.POINTER(ModelInfo)]),
    "fllmh_read_gguf_info": (I32, [C.c_char_p, C.POINTER(ModelInfo)]),
    "fllmh_xoshiro_init": (None, [C.POINTER(Xoshiro), U64]),
    "fllmh_xoshiro_next": (U64, [C.POINTER(Xoshiro)]),
    "fllmh_xoshiro_next_float": (F32_, [C.POINTER(Xoshiro)]),
    "fllmh_sampler_create": (I32, [F32_, I32, F32_, U64, PP]),
    "fllmh_sampler_destroy": (I32, [P]),
    "fllmh_sampler_sample": (I32, [P, P, PI32]),
    "fllmh_sampler_sample_host": (I32, [P, PF32, I32, PI32]),
    "fllmh_generate": (I32, [P, PI32, I32, I32, P, I32, I32, F32_, PI32, C.POINTER(GenerateStats)]),
}


def _bind(lib, sigs):
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args


def _load():
    for path in (DEVICE_LIB, HOST_LIB):
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build the native libraries first "
                "(python -m dotnetfoundryllm_amd.build); there is no non-native fallback")
    dev = C.CDLL(DEVICE_LIB)
    host = C.CDLL(HOST_LIB)
    _bind(dev, DEVICE_SIGS)
    _bind(host, HOST_SIGS)
    return dev, host


dev, host = _load()


def exported_symbols():
    """Names declared in include/fllm.h and include/fllm_host.h that the loaded libraries export."""
    names = {}
    for lib, sigs in ((dev, DEVICE_SIGS), (host, HOST_SIGS)):
        for n in sigs:
            names[n] = hasattr(lib, n)
    return names
