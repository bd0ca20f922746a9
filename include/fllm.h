/*
 * fllm.h — C ABI of libfllm_hip.so, the MI355X (gfx950) decode path that replaces
 * DotNetFoundryLLM's per-token forward pass.
 *
 * The reference has no FFI layer: its hot path sits behind the C# interfaces
 *   IForwardPass  (src/DotNetFoundryLLM.Architectures/IForwardPass.cs:11-14)
 *   IKvCache      (src/DotNetFoundryLLM.Abstractions/Interfaces.cs:73-92)
 *   ISampler      (src/DotNetFoundryLLM.Abstractions/Interfaces.cs:66-70)
 * and the loader seam GgufModelLoader.LoadTensor
 *   (src/DotNetFoundryLLM.ModelFormats.Gguf/GgufModelLoader.cs:409-418).
 * A C# HipForwardPass : IForwardPass / HipKvCache : IKvCache binds the functions
 * below with [LibraryImport]; every signature uses plain pointers, sizes and
 * POD structs so that it is blittable.
 *
 * Conventions
 *  - Every function returns int32_t status: FLLM_OK (0) or a negative code that
 *    maps 1:1 onto the exception the reference throws for the same condition.
 *    fllm_last_error() returns a thread-local message for the last failure.
 *  - No C++ exception crosses this ABI.
 *  - Objects are single-threaded, like the reference's forward pass ("thread-unsafe
 *    by design", LlamaForwardPass.cs:29): one fllm_seq per request; a model's
 *    weights are immutable after finalize and may be shared by many seqs.
 *  - Host pointers are host memory; fllm_buf handles are device memory.
 */
#ifndef FLLM_H
#define FLLM_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLLM_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------------------
 * Status codes. Each negative code names the .NET exception it stands for.
 * ------------------------------------------------------------------------- */
enum fllm_status {
    FLLM_OK                = 0,
    FLLM_E_ARG_RANGE       = -1,  /* ArgumentOutOfRangeException (token id, layer, position) */
    FLLM_E_ARG             = -2,  /* ArgumentException (sizes / lengths) */
    FLLM_E_INVALID_OP      = -3,  /* InvalidOperationException (KV append order, missing tensor) */
    FLLM_E_NOT_SUPPORTED   = -4,  /* NotSupportedException (tensor type, architecture) */
    FLLM_E_DISPOSED        = -5,  /* ObjectDisposedException */
    FLLM_E_MODEL_LOAD      = -6,  /* ModelLoadException */
    FLLM_E_DEVICE          = -7,  /* HIP runtime error (no reference counterpart) */
    FLLM_E_NULL            = -8,  /* ArgumentNullException */
    FLLM_E_OOM             = -9   /* device allocation failed (OutOfMemoryException) */
};

/* GGML tensor type ids, as GgufTensorType (src/DotNetFoundryLLM.ModelFormats.Gguf/GgufTensorType.cs). */
enum fllm_type {
    FLLM_TYPE_F32  = 0,
    FLLM_TYPE_F16  = 1,
    FLLM_TYPE_Q4_0 = 2,
    FLLM_TYPE_Q8_0 = 8,
    FLLM_TYPE_Q4_K = 12,
    FLLM_TYPE_Q5_K = 13,
    FLLM_TYPE_Q6_K = 14,
    FLLM_TYPE_Q8_K = 15,
    FLLM_TYPE_BF16 = 30
};

/* Architectures accepted by GgufModelLoader.Build (GgufModelLoader.cs:89-102). */
enum fllm_arch {
    FLLM_ARCH_LLAMA   = 0,   /* LlamaForwardPass.cs */
    FLLM_ARCH_MISTRAL = 1,   /* MistralForwardPass.cs: window on every layer */
    FLLM_ARCH_QWEN2   = 2,   /* Qwen2ForwardPass.cs: q/k/v bias */
    FLLM_ARCH_GEMMA2  = 3    /* Gemma2ForwardPass.cs: (1+w) norms, post-norms, GELU, softcaps */
};

/* Tensor slots, named after the GGUF tensor names the loader reads
 * (GgufModelLoader.cs:336-372 LoadWeights, :518-552 LoadGemma2Weights, :554-591 LoadQwen2Weights). */
enum fllm_slot {
    FLLM_SLOT_TOKEN_EMBD     = 0,   /* token_embd.weight              [vocab x hidden] */
    FLLM_SLOT_OUTPUT_NORM    = 1,   /* output_norm.weight             [hidden] */
    FLLM_SLOT_OUTPUT         = 2,   /* output.weight (optional: tied) [vocab x hidden] */
    FLLM_SLOT_ATTN_NORM      = 10,  /* blk.{i}.attn_norm.weight       [hidden] */
    FLLM_SLOT_ATTN_Q         = 11,  /* blk.{i}.attn_q.weight          [q_dim x hidden] */
    FLLM_SLOT_ATTN_K         = 12,  /* blk.{i}.attn_k.weight          [kv_dim x hidden] */
    FLLM_SLOT_ATTN_V         = 13,  /* blk.{i}.attn_v.weight          [kv_dim x hidden] */
    FLLM_SLOT_ATTN_OUTPUT    = 14,  /* blk.{i}.attn_output.weight     [hidden x q_dim] */
    FLLM_SLOT_ATTN_Q_BIAS    = 15,  /* blk.{i}.attn_q.bias (Qwen2)    [q_dim] */
    FLLM_SLOT_ATTN_K_BIAS    = 16,  /* blk.{i}.attn_k.bias (Qwen2)    [kv_dim] */
    FLLM_SLOT_ATTN_V_BIAS    = 17,  /* blk.{i}.attn_v.bias (Qwen2)    [kv_dim] */
    FLLM_SLOT_POST_ATTN_NORM = 18,  /* blk.{i}.post_attn_norm.weight (Gemma2) [hidden] */
    FLLM_SLOT_FFN_NORM       = 19,  /* blk.{i}.ffn_norm.weight        [hidden] */
    FLLM_SLOT_FFN_GATE       = 20,  /* blk.{i}.ffn_gate.weight        [ffn x hidden] */
    FLLM_SLOT_FFN_UP         = 21,  /* blk.{i}.ffn_up.weight          [ffn x hidden] */
    FLLM_SLOT_FFN_DOWN       = 22,  /* blk.{i}.ffn_down.weight        [hidden x ffn] */
    FLLM_SLOT_POST_FFN_NORM  = 23   /* blk.{i}.post_ffn_norm.weight (Gemma2) [hidden] */
};

/* Model description: the fields of LlamaConfig (LlamaConfig.cs:6-65), MistralConfig
 * (MistralConfig.cs) and Gemma2Config (Gemma2Config.cs:6-72) that the forward pass reads.
 * The C# side fills it from the config object the loader built (GgufModelLoader.cs:308-334,
 * :213-241), so every quirk of that mapping (eps not read from GGUF, raw
 * query_pre_attn_scalar, head_dim override) stays on the managed side. */
typedef struct fllm_model_desc {
    int32_t arch;              /* enum fllm_arch */
    int32_t n_layers;          /* LayerCount */
    int32_t hidden;            /* HiddenSize */
    int32_t ffn;               /* IntermediateSize */
    int32_t n_heads;           /* NumHeads */
    int32_t n_kv_heads;        /* NumKvHeads */
    int32_t head_dim;          /* HeadDim (hidden/heads, or Gemma2 key_length override) */
    int32_t vocab;             /* VocabSize */
    int32_t max_ctx;           /* MaxContextLength (KV capacity default) */
    float   rope_base;         /* RopeBaseFreq */
    float   rope_scale;        /* RopeScalingFactor */
    int32_t rope_scaled;       /* 1 when RopeScalingType is "linear" or "yarn" (LlamaForwardPass.cs:150-152) */
    float   norm_eps;          /* 1e-5 for RmsNorm (TensorOperations.cs:42); Gemma2 uses 1e-6 (:93) */
    float   attn_scale;        /* 1/sqrt(head_dim); Gemma2: QueryPreAttnScalar (Gemma2ForwardPass.cs:132) */
    float   attn_softcap;      /* Gemma2 AttnLogitSoftcap, 0 = off */
    float   final_softcap;     /* Gemma2 FinalLogitSoftcap, 0 = off */
    int32_t sliding_window;    /* SlidingWindowSize; INT32_MAX = none */
} fllm_model_desc;

typedef struct fllm_ctx   fllm_ctx;    /* device, default stream, utility scratch */
typedef struct fllm_model fllm_model;  /* device-resident weights in GGUF block layout */
typedef struct fllm_seq   fllm_seq;    /* one request: device KV cache, scratch, stream */
typedef struct fllm_buf   fllm_buf;    /* raw device buffer (microbenchmarks, tests) */

/* ---- errors / version -------------------------------------------------- */
FLLM_API const char* fllm_last_error(void);
FLLM_API int32_t     fllm_version(void);

/* ---- context ------------------------------------------------------------ */
FLLM_API int32_t fllm_ctx_create(int32_t device, fllm_ctx** out);
FLLM_API int32_t fllm_ctx_destroy(fllm_ctx* ctx);
FLLM_API int32_t fllm_ctx_sync(fllm_ctx* ctx);
/* Number of compute units of the context's device (for launch sizing reports). */
FLLM_API int32_t fllm_ctx_device_info(fllm_ctx* ctx, int32_t* n_cu, int64_t* hbm_bytes);

/* ---- model (replaces LlamaWeights/Qwen2Weights/Gemma2Weights + LoadTensor) ---- */
FLLM_API int32_t fllm_model_create(fllm_ctx* ctx, const fllm_model_desc* desc, fllm_model** out);
/* Copies raw GGUF tensor bytes (GgufFile.GetTensorBytes, GgufFile.cs:76-97) to device memory,
 * kept in their quantized block layout. The element count is implied by the slot and the
 * config, as LoadTensor's expectedElements (GgufModelLoader.cs:409-418); nbytes must be the
 * exact byte size of that many elements of `type`. Returns after the copy, so the caller may
 * reuse `bytes` (the mmap path reuses one scratch array, GgufFile.cs:94-96).
 * layer is ignored for the model-level slots. Norm and bias tensors of any supported type
 * are dequantized on the device to F32 at upload. */
FLLM_API int32_t fllm_model_upload(fllm_model* m, int32_t slot, int32_t layer, int32_t type,
                                   const void* bytes, uint64_t nbytes);
/* Checks that every required slot is present; ties output.weight to token_embd.weight when
 * absent (GgufModelLoader.cs:365-366); builds the RoPE inverse-frequency table. Q4_K / Q6_K
 * matrices whose decode launches run on the matrix cores are regrouped on the device by 16-row
 * tile (the same blocks, permuted; one temporary copy of a matrix at a time). */
FLLM_API int32_t fllm_model_finalize(fllm_model* m);
/* LlamaWeights.Dispose (LlamaWeights.cs:93-107): marks the model disposed. Forward, prefill and
 * decode on a sequence of a disposed model return FLLM_E_DISPOSED before anything runs
 * (LlamaForwardPass.cs:87, LlamaWeights.cs:138-139), as do upload, finalize and seq_create while
 * the handle is still valid. The device memory is released at once when no sequence of the model
 * is alive, otherwise when the last one is destroyed (sequences keep using the weights until
 * then, so destroy never frees memory a sequence still reads). Repeated calls are harmless while a
 * sequence of the model is alive; once destroy has released the model (no sequence left) the
 * handle is invalid and must not be passed again. */
FLLM_API int32_t fllm_model_destroy(fllm_model* m);
/* The description the model was created with. */
FLLM_API int32_t fllm_model_get_desc(fllm_model* m, fllm_model_desc* out);
/* Device bytes held by the model's weights (as uploaded) and the LM head alone. */
FLLM_API int32_t fllm_model_weight_bytes(fllm_model* m, uint64_t* layer_bytes, uint64_t* head_bytes);

/* ---- sequence (replaces KvCache + the per-request forward scratch) ------ */
/* max_seq: KV capacity in positions (KvCache(layerCount, maxContextLength, kvDim),
 * LlamaLanguageModel.cs:129); 0 = desc.max_ctx. */
FLLM_API int32_t fllm_seq_create(fllm_model* m, int32_t max_seq, fllm_seq** out);
FLLM_API int32_t fllm_seq_destroy(fllm_seq* s);
FLLM_API int32_t fllm_seq_reset(fllm_seq* s);                         /* KvCache.Clear (also clears WasEvicted) */
FLLM_API int32_t fllm_seq_length(fllm_seq* s, int32_t* len);          /* KvCache.CurrentLength */
FLLM_API int32_t fllm_seq_capacity(fllm_seq* s, int32_t* cap);        /* KvCache.MaxSequenceLength */
FLLM_API int32_t fllm_seq_get_model(fllm_seq* s, fllm_model** out);
/* 1 = replay the decode step from a captured HIP graph (default), 0 = launch kernels one by one. */
FLLM_API int32_t fllm_seq_set_graph(fllm_seq* s, int32_t enable);
/* Tokens per pass of the batched prefill through the layers (default 4096, capped at the
 * capacity): each pass's projections are GEMMs over that many rows and its attention a grid over
 * them, so long prompts fill the GPU. A tuning knob with no counterpart in the reference (whose
 * prefill is one Forward per token). Applies to later prefills; the sequence's prefill scratch
 * holds rows for the longest pass seen so far (the prompt rounded up to 256, at most one pass) and
 * grows when a prefill needs more. tokens < 1 returns FLLM_E_ARG_RANGE. */
FLLM_API int32_t fllm_seq_set_prefill_chunk(fllm_seq* s, int32_t tokens);
/* 1 = keep the residual stream after every layer for fllm_debug_hidden (parity hook). */
FLLM_API int32_t fllm_seq_set_debug(fllm_seq* s, int32_t enable);
/* 1 = the decode attention merges its position chunks inside its own launch (the last chunk of each
 * kv head to finish merges them); 0 = a second launch merges them. The default is 1 when a kv head
 * has at most 4 query heads and 32 chunks (Llama-3-8B, Gemma-2-9B), else 0 (Qwen2-7B's 7 heads).
 * Results agree (bit for bit up to 32 chunks per kv head, to float32 rounding beyond). A tuning knob
 * with no counterpart in the reference. */
FLLM_API int32_t fllm_seq_set_attention_merge(fllm_seq* s, int32_t in_launch);

/* IForwardPass.Forward(tokenId, position, kv): one decode step. Appends K/V at the current
 * length, attends over positions [window_start, position], leaves logits on the device.
 * A full cache first evicts its oldest half, as KvCache.Append does for layer 0
 * (KvCache.cs:82-85, 152-173); the RoPE position stays `position`.
 * Errors, in the reference's order:
 *  - disposed model -> FLLM_E_DISPOSED (LlamaForwardPass.cs:87);
 *  - token outside [0,vocab) -> FLLM_E_ARG_RANGE (LlamaForwardPass.cs:89-93);
 *  - a cache part-way through a position's layers (fllm_kv_append) -> FLLM_E_INVALID_OP
 *    (KvCache.cs:69-74);
 *  - position > current length (after any eviction) -> FLLM_E_ARG_RANGE: the reference has then
 *    appended layer 0 and its attention Slice throws (LlamaForwardPass.cs:186-188), leaving the
 *    cache expecting layer 1; the same state is kept here (layer 0's row at that slot is zeros),
 *    so later Forward calls fail with FLLM_E_INVALID_OP until fllm_seq_reset. */
FLLM_API int32_t fllm_forward(fllm_seq* s, int32_t token, int32_t position);
/* n consecutive Forward calls for tokens[0..n) at positions pos0.. (prefill loop,
 * LlamaLanguageModel.cs:133-137), with their results: the K/V rows of every position, the last
 * position's logits and greedy token. When pos0 is the cache's current length (a prompt) and debug
 * capture is off, the tokens go through each layer together in chunks (fllm_seq_set_prefill_chunk;
 * fp16 matrix-core GEMMs over the chunk, causal attention over the cache); otherwise, and for n = 1,
 * it is n fllm_forward calls. On both paths the token ids and the cache capacity are checked before
 * anything runs: a prompt that would overflow the cache (current length + n > capacity) returns
 * FLLM_E_ARG_RANGE with the cache unchanged (no eviction), unlike a lone fllm_forward at a full
 * cache, which evicts the oldest half first as KvCache.Append does (KvCache.cs:82-85). */
FLLM_API int32_t fllm_prefill(fllm_seq* s, const int32_t* tokens, int32_t n, int32_t pos0);
/* The greedy part of LlamaLanguageModel.GenerateAsync's decode loop (LlamaLanguageModel.cs:162-293
 * with SamplerPipeline Temperature == 0, SamplerPipeline.cs:61-64, no EOS stop): n_steps Forward
 * calls starting with `token` at `position`, each step's argmax fed to the next step on the device
 * (no host round trip per token). out_tokens receives the n_steps greedy tokens; the logits of the
 * last step stay on the device. Same argument contract as fllm_forward; the KV cache must have
 * room for n_steps positions (FLLM_E_ARG_RANGE otherwise). */
FLLM_API int32_t fllm_decode_greedy(fllm_seq* s, int32_t token, int32_t position, int32_t n_steps,
                                    int32_t* out_tokens);
/* Waits for the sequence's stream. */
FLLM_API int32_t fllm_seq_sync(fllm_seq* s);

/* IForwardPass.Logits: copies the last step's logits (vocab floats) to host memory. */
FLLM_API int32_t fllm_logits_copy(fllm_seq* s, float* dst, int64_t n);
/* Overwrites the device logits with n == vocab host floats, e.g. after the host applied
 * LlamaLanguageModel.ApplyRepetitionPenalty (LlamaLanguageModel.cs:183-186, 357-373) to a copy,
 * so the device sampler runs on the penalised values. */
FLLM_API int32_t fllm_logits_write(fllm_seq* s, const float* src, int64_t n);
/* SamplerPipeline with Temperature == 0 (SamplerPipeline.cs:61-64): device argmax over the
 * logits, first index of the maximum (TensorOperations.ArgMax, TensorOperations.cs:187-195). */
FLLM_API int32_t fllm_sample_greedy(fllm_seq* s, int32_t* out_token);
/* Top-k candidate selection of SamplerPipeline.Sample stages 1-2 (SamplerPipeline.cs:67-74,
 * TopKSampler.ApplyTopK TopKSampler.cs:42-71): scales the logits by inv_temp in place
 * (when inv_temp != 1), finds the k-th largest scaled value and returns every index whose
 * scaled logit is >= that threshold (ties kept, -0 and +0 equal as in float comparison), in
 * ascending index order, with the scaled values. cap is the capacity of ids/vals; FLLM_E_ARG if
 * more than cap survive. A grid of 4096-entry segments samples, counts and gathers the
 * candidates; one workgroup selects among them (or over the whole vocabulary when the sample
 * misses). inv_temp must be finite and >= 0 (FLLM_E_ARG_RANGE otherwise); vocabularies above
 * 262144 -> FLLM_E_NOT_SUPPORTED. */
FLLM_API int32_t fllm_sample_topk(fllm_seq* s, float inv_temp, int32_t k,
                                  int32_t* ids, float* vals, int32_t cap, int32_t* n_out);
/* LlamaLanguageModel.ApplyRepetitionPenalty (LlamaLanguageModel.cs:183-186, 357-373) on the device
 * logits: for every id of ids[0..n_ids) in order, l > 0 ? l / penalty : l * penalty, an id listed
 * k times is penalised k times, ids outside [0, vocab) are skipped. Bit-identical to the host loop.
 * penalty <= 0 -> FLLM_E_ARG_RANGE (RepetitionPenaltySampler.cs:27-28); penalty == 1 changes
 * nothing. Replaces the vocab-sized logits round trip of fllm_logits_copy + fllm_logits_write. */
FLLM_API int32_t fllm_logits_penalize(fllm_seq* s, const int32_t* ids, int32_t n_ids, float penalty);
/* SamplerPipeline.Sample (SamplerPipeline.cs:58-89) with topK disabled, on the device: scales the
 * logits by inv_temp in place (stage 1), softmax (stage 3), nucleus of top_p (stage 4,
 * TopPSampler.ApplyTopP TopPSampler.cs:60-110; top_p == 1 keeps everything, equal probabilities at
 * the edge are taken in ascending index order), and draws the first index whose running
 * probability exceeds u (stage 5, TemperatureSampler.SampleFromProbabilities
 * TemperatureSampler.cs:53-70), u being the pipeline's XoshiroRandom.NextFloat() for this draw.
 * Running sums are exact fixed-point where the reference sums f32 in order: the token can differ
 * from the reference only when u or top_p falls within f32 rounding of a boundary.
 * Errors: top_p outside (0,1], u outside [0,1), inv_temp not finite or negative -> FLLM_E_ARG_RANGE
 * (inv_temp 0, an infinite temperature, makes every logit 0: the draw is uniform);
 * vocabularies above 262144 -> FLLM_E_NOT_SUPPORTED (one workgroup). */
FLLM_API int32_t fllm_sample_nucleus(fllm_seq* s, float inv_temp, float top_p, float u, int32_t* out_token);
/* The distribution fllm_sample_nucleus drew from (vocab floats: the renormalised nucleus, zeros
 * elsewhere); a parity hook. */
FLLM_API int32_t fllm_probs_copy(fllm_seq* s, float* dst, int64_t n);

/* ---- parity hooks -------------------------------------------------------- */
/* Residual stream x after layer `layer` of the last step (requires fllm_seq_set_debug(1)
 * before that step); layer == n_layers gives the final-normed vector fed to the LM head. */
FLLM_API int32_t fllm_debug_hidden(fllm_seq* s, int32_t layer, float* dst, int64_t n);
/* KvCache.GetKeys / GetValues (KvCache.cs:100-135): kind 0 = keys, 1 = values.
 * Copies effective_length * kv_dim floats, effective_length being the current length plus one
 * for the layers already appended at the position being filled (KvCache.cs:109-115).
 * Layer outside [0, n_layers) -> FLLM_E_ARG_RANGE; n too small -> FLLM_E_ARG. */
FLLM_API int32_t fllm_kv_read(fllm_seq* s, int32_t layer, int32_t kind, float* dst, int64_t n);
/* KvCache.Append (KvCache.cs:59-97) for a caller that fills the device cache itself (a C# forward
 * pass over HipKvCache): copies kv_dim host floats of keys and of values to the slot at the current
 * length of `layer`. Layers go in order 0..n_layers-1 for each position; the last one advances the
 * length. A full cache first evicts its oldest half (KvCache.cs:82-85, 152-173) and sets
 * WasEvicted. Errors, in the reference's order: layer outside [0, n_layers) -> FLLM_E_ARG_RANGE;
 * layer out of order -> FLLM_E_INVALID_OP; n_keys or n_values != kv_dim -> FLLM_E_ARG. */
FLLM_API int32_t fllm_kv_append(fllm_seq* s, int32_t layer, const float* keys, int64_t n_keys,
                                const float* values, int64_t n_values);
/* Positions GetKeys / GetValues of `layer` hold (the effective length above: the span length over
 * kv_dim, KvCache.cs:109-115). Layer outside [0, n_layers) -> FLLM_E_ARG_RANGE. */
FLLM_API int32_t fllm_kv_length(fllm_seq* s, int32_t layer, int32_t* out);
/* KvCache.WasEvicted (KvCache.cs:56): 1 once an eviction happened since creation or the last reset. */
FLLM_API int32_t fllm_kv_was_evicted(fllm_seq* s, int32_t* out);

/* ---- kernels exposed for verification and microbenchmarks ------------------ */
/* Dequantizer.Dequantize(type, src, dst) (Dequantizer.cs:488-504) on the device:
 * host src (nbytes) -> host dst (n floats), bit-exact. Same error contract:
 * unsupported type -> FLLM_E_NOT_SUPPORTED; nbytes not a multiple of the block size or
 * dst too small -> FLLM_E_ARG. */
FLLM_API int32_t fllm_dequantize(fllm_ctx* ctx, int32_t type, const void* src, uint64_t nbytes,
                                 float* dst, int64_t n);
/* fllm_dequantize without any device allocation, for callers that cannot allocate (harnesses that
 * forbid it, tight serving loops). No counterpart in the reference. The source blocks and the
 * floats are staged through a fixed scratch array in device memory that the library holds per
 * device for the life of the process (FLLM_NOALLOC_MAX_BYTES source bytes and FLLM_NOALLOC_MAX_ELEMS
 * floats); larger calls return FLLM_E_ARG. Same results and error contract as fllm_dequantize
 * otherwise. Every call on one device uses the same array; the call is synchronous and holds a
 * per-device lock on it throughout, so calls from several threads or contexts on one device run
 * one after the other. */
#define FLLM_NOALLOC_MAX_BYTES (2u << 20)
#define FLLM_NOALLOC_MAX_ELEMS (2u << 20)
FLLM_API int32_t fllm_dequantize_noalloc(fllm_ctx* ctx, int32_t type, const void* src, uint64_t nbytes,
                                         float* dst, int64_t n);
/* Dequantizer.ElementCount (Dequantizer.cs:466-479). */
FLLM_API int32_t fllm_element_count(int32_t type, int64_t nbytes, int64_t* out);

/* Device buffers. */
FLLM_API int32_t fllm_buf_create(fllm_ctx* ctx, uint64_t nbytes, fllm_buf** out);
FLLM_API int32_t fllm_buf_destroy(fllm_buf* b);
FLLM_API int32_t fllm_buf_write(fllm_buf* b, uint64_t offset, const void* src, uint64_t n);
FLLM_API int32_t fllm_buf_read(fllm_buf* b, uint64_t offset, void* dst, uint64_t n);

/* LinearProjection (LlamaForwardPass.cs:237-260): y[i] = sum_j W[i,j] x[j] for a
 * rows x cols matrix of `type` stored at w+w_offset (GGUF layout, rows may straddle blocks),
 * x (cols floats) and y (rows floats) in device buffers. Enqueued on the context stream. */
FLLM_API int32_t fllm_gemv(fllm_ctx* ctx, int32_t type, fllm_buf* w, uint64_t w_offset,
                           int64_t rows, int64_t cols, fllm_buf* x, fllm_buf* y);
/* Times `iters` fused dequant-GEMV launches cycling through n_w weight buffers (a working
 * set larger than the 256 MB Infinity Cache keeps every launch an HBM read), with HIP
 * events on the context stream. Returns the mean launch duration in microseconds. */
FLLM_API int32_t fllm_gemv_time(fllm_ctx* ctx, int32_t type, fllm_buf* const* w, int32_t n_w,
                                int64_t rows, int64_t cols, fllm_buf* x, fllm_buf* y,
                                int32_t iters, double* avg_us);

/* Weight layouts of the GEMV entry points: GGUF rows as uploaded, or the matrix-core layout
 * that fllm_model_finalize gives model weights (16-row tiles interleaved per 256-column chunk). */
enum fllm_layout {
    FLLM_LAYOUT_GGUF = 0,
    FLLM_LAYOUT_TILES = 1
};
/* Regroups a rows x cols matrix of `type` (GGUF layout at src + src_offset) into
 * FLLM_LAYOUT_TILES at dst (the same number of bytes; every byte kept), for a caller that
 * multiplies one matrix many times. FLLM_E_NOT_SUPPORTED where the layout does not apply (types
 * other than Q4_K, Q5_K, Q6_K, Q8_0; rows not a multiple of 16; cols not a multiple of 256).
 * No counterpart in the reference, whose weights are F32 after load (GgufModelLoader.cs:409-418);
 * it is the standalone form of the regrouping fllm_model_finalize does. */
FLLM_API int32_t fllm_gemv_pack(fllm_ctx* ctx, int32_t type, fllm_buf* src, uint64_t src_offset,
                                int64_t rows, int64_t cols, fllm_buf* dst);
/* fllm_gemv for a matrix in `layout` (FLLM_LAYOUT_TILES: as written by fllm_gemv_pack, at
 * offset 0). LinearProjection (LlamaForwardPass.cs:237-260). */
FLLM_API int32_t fllm_gemv_ex(fllm_ctx* ctx, int32_t type, fllm_buf* w, uint64_t w_offset,
                              int64_t rows, int64_t cols, fllm_buf* x, fllm_buf* y, int32_t layout);
/* Times `iters` launches back to back cycling through n_w weight buffers in `layout`: the mean
 * time per launch between one HIP event pair around all of them (launch gaps included). */
FLLM_API int32_t fllm_gemv_time_ex(fllm_ctx* ctx, int32_t type, fllm_buf* const* w, int32_t n_w,
                                   int64_t rows, int64_t cols, fllm_buf* x, fllm_buf* y,
                                   int32_t iters, int32_t layout, double* avg_us);

/* ---- per-kernel timing of the decode step ----------------------------------- */
/* When enabled, fllm_forward launches kernels one by one (no graph) with a HIP event pair
 * around every launch on the sequence's stream, and aggregates per kernel name the number of
 * launches, the summed device time and the summed algorithmic bytes (weights, activations
 * and KV read + written, as stored). fllm_seq_profile_entry enumerates the aggregates. */
FLLM_API int32_t fllm_seq_set_profile(fllm_seq* s, int32_t enable);
FLLM_API int32_t fllm_seq_profile_count(fllm_seq* s, int32_t* n);
FLLM_API int32_t fllm_seq_profile_entry(fllm_seq* s, int32_t i, char* name, int32_t name_cap,
                                        int64_t* launches, double* total_ms, double* total_bytes);
FLLM_API int32_t fllm_seq_profile_reset(fllm_seq* s);
/* Name of profiled launch i (0-based, in launch order since the last reset; one kernel each). */
FLLM_API int32_t fllm_seq_profile_launch(fllm_seq* s, int32_t i, char* name, int32_t name_cap);

#ifdef __cplusplus
}
#endif
#endif /* FLLM_H */
