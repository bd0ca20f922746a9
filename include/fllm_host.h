/*
 * fllm_host.h — host side above the C ABI (libfllm_host.so).
 *
 * The reference's host code is C#; no .NET SDK is available to this build, so the managed
 * side is restated in C++ over include/fllm.h, keeping the reference's names, argument
 * meaning and error behaviour:
 *   - GgufReader / GgufModelLoader (src/DotNetFoundryLLM.ModelFormats.Gguf/GgufReader.cs,
 *     GgufModelLoader.cs): parse GGUF v2/v3, build the config from metadata, hand raw tensor
 *     bytes to fllm_model_upload instead of dequantizing them to F32 (LoadTensor :397-406).
 *   - XoshiroRandom (src/DotNetFoundryLLM.Core/XoshiroRandom.cs) and SamplerPipeline
 *     (src/DotNetFoundryLLM.Sampling/SamplerPipeline.cs) over the device argmax / top-k.
 *   - LlamaLanguageModel.GenerateAsync's token loop
 *     (src/DotNetFoundryLLM.Inference/LlamaLanguageModel.cs:100-331).
 *   - a seeded synthetic tensor generator that writes GGUF block bytes (test/benchmark data).
 * Status codes are those of fllm.h.
 */
#ifndef FLLM_HOST_H
#define FLLM_HOST_H

#include "fllm.h"

#ifdef __cplusplus
extern "C" {
#endif

FLLM_API const char* fllmh_last_error(void);

/* ---- synthetic tensors ----------------------------------------------------------
 * Fills dst (exactly the GGUF byte size of n elements of `type`) from a counter-based
 * generator: SplitMix64 over (seed, tensor_id, block index), so any block can be produced
 * independently and in parallel. Distributions:
 *   F32/F16/BF16: dist 0 = normal(p0 mean, p1 std), 1 = constant p0, 2 = uniform[p0, p1)
 *   Q4_K / Q5_K : d, dmin = f16(U[p0,p1)); 6-bit scales and mins U{0..63}; qs (and Q5_K qh) uniform bytes
 *   Q6_K        : ql, qh uniform bytes; scales int8 U{0..63}; d = f16(U[p0,p1))
 *   Q8_0        : qs int8 U{-127..127}; d = f16(U[p0,p1))
 *   Q4_0        : nibbles uniform; d = f16(U[p0,p1))
 *   Q8_K        : qs int8 U{-127..127}; d = f32 U[p0,p1)
 * threads <= 0 uses the hardware concurrency, at most 16. */
FLLM_API int32_t fllmh_synth_tensor(int32_t type, uint64_t seed, uint64_t tensor_id, int64_t n_elems,
                                    int32_t dist, float p0, float p1, void* dst, uint64_t dst_bytes,
                                    int32_t threads);
/* Uniform token ids in [0, vocab) from (seed, stream). */
FLLM_API int32_t fllmh_synth_tokens(uint64_t seed, uint64_t stream, int32_t vocab, int32_t* dst, int32_t n);
FLLM_API uint16_t fllmh_f32_to_f16(float f);   /* round to nearest even */
FLLM_API uint16_t fllmh_f32_to_bf16(float f);  /* round to nearest even */

/* ---- GGUF loader (GgufModelLoader.LoadAsync -> device upload) ------------------------ */
typedef struct fllmh_model_info {
    fllm_model_desc desc;
    int32_t bos_token_id;   /* tokenizer.ggml.bos_token_id, default 1 */
    int32_t eos_token_id;   /* tokenizer.ggml.eos_token_id, default 2 */
    int32_t gguf_version;
    int32_t n_tensors;
    uint64_t data_offset;   /* aligned start of tensor data */
} fllmh_model_info;
/* Reads the GGUF file at `path`, builds the model description from its metadata exactly as
 * GgufModelLoader.Build* does, uploads every tensor's raw bytes and finalizes the model.
 * Errors: FLLM_E_MODEL_LOAD (unreadable / not GGUF / bad version), FLLM_E_NOT_SUPPORTED
 * (architecture, tensor type), FLLM_E_INVALID_OP (required tensor missing). */
FLLM_API int32_t fllmh_load_gguf(fllm_ctx* ctx, const char* path, fllm_model** model, fllmh_model_info* info);
/* Parses only the header + metadata + tensor infos (no device work). */
FLLM_API int32_t fllmh_read_gguf_info(const char* path, fllmh_model_info* info);

/* ---- XoshiroRandom --------------------------------------------------------------- */
typedef struct fllmh_xoshiro { uint64_t s0, s1, s2, s3; } fllmh_xoshiro;
FLLM_API void     fllmh_xoshiro_init(fllmh_xoshiro* r, uint64_t seed);
FLLM_API uint64_t fllmh_xoshiro_next(fllmh_xoshiro* r);
FLLM_API float    fllmh_xoshiro_next_float(fllmh_xoshiro* r);

/* ---- SamplerPipeline over the device sampler --------------------------------------- */
typedef struct fllmh_sampler fllmh_sampler;
/* temperature >= 0, top_p in (0,1]; seed 0 seeds from the clock as the reference does
 * (SamplerPipeline.cs:14-23). Errors: FLLM_E_ARG_RANGE for invalid temperature / top_p. */
FLLM_API int32_t fllmh_sampler_create(float temperature, int32_t top_k, float top_p, uint64_t seed, fllmh_sampler** out);
FLLM_API int32_t fllmh_sampler_destroy(fllmh_sampler* s);
/* Samples from the sequence's current logits: greedy -> device argmax (fllm_sample_greedy);
 * top-k -> device candidates (fllm_sample_topk) + host softmax / top-p / CDF walk over them;
 * otherwise temperature, softmax, top-p and the draw on the device (fllm_sample_nucleus, u from
 * this sampler's generator). No vocab-sized copy on any path. */
FLLM_API int32_t fllmh_sampler_sample(fllmh_sampler* s, fllm_seq* seq, int32_t* out_token);
/* The same pipeline over host logits (modified in place), for parity tests. */
FLLM_API int32_t fllmh_sampler_sample_host(fllmh_sampler* s, float* logits, int32_t n, int32_t* out_token);

/* ---- token loop ------------------------------------------------------------------- */
typedef struct fllmh_generate_stats {
    int32_t prompt_tokens;
    int32_t completion_tokens;
    double prefill_ms;
    double decode_ms;
    double tokens_per_second;  /* completion / decode seconds (LlamaLanguageModel.cs:302-304) */
    int32_t finish_reason;     /* 0 = length, 1 = stop (EOS) */
} fllmh_generate_stats;
/* LlamaLanguageModel.GenerateAsync over already-tokenized ids: clears the KV cache,
 * runs the Forward calls of prompt[0..n-2] at positions 0.. as one batched fllm_prefill, then
 * decodes from prompt[n-1] for up to max_tokens steps, sampling each step and stopping at
 * eos_token_id (eos < 0 disables). repetition_penalty != 1 applies
 * LlamaLanguageModel.ApplyRepetitionPenalty over the generated ids on the device logits
 * (fllm_logits_penalize) before sampling; penalty <= 0 -> FLLM_E_ARG_RANGE. */
FLLM_API int32_t fllmh_generate(fllm_seq* seq, const int32_t* prompt, int32_t n_prompt, int32_t max_tokens,
                                fllmh_sampler* sampler, int32_t eos_token_id, int32_t bos_token_id,
                                float repetition_penalty, int32_t* out_tokens, fllmh_generate_stats* stats);

#ifdef __cplusplus
}
#endif
#endif
