/*
 * oracle.h — CPU restatement of DotNetFoundryLLM's decode path, in plain C.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the smoke check and
 * bench.py's cpu_baseline leg load it to produce expected values and a CPU timing.
 * The product (libfllm_hip.so and the host library) never links, loads or calls it.
 *
 * Every function follows a reference file:line, cited at its definition in oracle.c.
 * Return codes use the same numbering as include/fllm.h (0 ok, -1 ArgumentOutOfRange,
 * -2 Argument, -3 InvalidOperation, -4 NotSupported).
 */
#ifndef FLLM_ORACLE_H
#define FLLM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Row-parallel mode: n threads (1 = the reference's single thread, the default). Rows of a
 * projection, heads of an attention and blocks of a dequantization are split over them; every
 * output element is computed exactly as with one thread. Returns the thread count in effect. */
int orc_set_threads(int n);
int orc_get_threads(void);

/* scalar conversions */
float orc_half_to_float(uint16_t h);
float orc_bf16_to_float(uint16_t b);

/* Dequantizer */
int orc_dequantize(int type, const uint8_t* src, int64_t nbytes, float* dst, int64_t n);
int orc_element_count(int type, int64_t nbytes, int64_t* out);
void orc_decode_kscale_min(const uint8_t* packed12, int g, int* scale, int* min);

/* TensorOperations */
float orc_dot(const float* a, const float* b, int64_t n);
void  orc_linear(const float* x, const float* W, float* y, int64_t rows, int64_t cols);
int   orc_rmsnorm(const float* x, const float* w, float* dst, int64_t n, float eps);
void  orc_gemma_rmsnorm(const float* x, const float* w, float* dst, int64_t n);
void  orc_silu(float* x, int64_t n);
void  orc_gelu(float* x, int64_t n);
void  orc_softcap(float* x, int64_t n, float cap);
void  orc_softmax(float* x, int64_t n);
void  orc_rope_inv_freqs(float base, int head_dim, float* inv);
void  orc_apply_rope(float* x, float pos, const float* inv, int half);
int64_t orc_argmax(const float* x, int64_t n);

/* Sampling + RNG */
typedef struct { uint64_t s0, s1, s2, s3; } orc_xoshiro;
void     orc_xoshiro_init(orc_xoshiro* r, uint64_t seed);
uint64_t orc_xoshiro_next(orc_xoshiro* r);
float    orc_xoshiro_next_float(orc_xoshiro* r);
float    orc_topk_threshold(const float* logits, int64_t n, int k);
void     orc_apply_topk(float* logits, int64_t n, int k);
int64_t  orc_sample_from_probs(const float* probs, int64_t n, orc_xoshiro* r);
/* SamplerPipeline.Sample with topP == 1 (greedy when temperature == 0). Modifies logits. */
int64_t  orc_sampler_pipeline(float* logits, int64_t n, float temperature, int top_k, orc_xoshiro* r);
/* SamplerPipeline.Sample with every stage, top-p included. Modifies logits. */
int64_t  orc_sampler_pipeline_p(float* logits, int64_t n, float temperature, int top_k, float top_p, orc_xoshiro* r);
/* TopPSampler.ApplyTopP on probabilities (in place). */
void     orc_apply_top_p(float* probs, int64_t n, float p);
/* LlamaLanguageModel.ApplyRepetitionPenalty (in place). */
void     orc_repetition_penalty(float* logits, int64_t n, const int32_t* ids, int64_t n_ids, float penalty);

/* Model + forward pass */
typedef struct orc_desc {
    int32_t arch, n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, max_ctx;
    float rope_base, rope_scale;
    int32_t rope_scaled;
    float norm_eps, attn_scale, attn_softcap, final_softcap;
    int32_t sliding_window;
} orc_desc;

typedef struct orc_model orc_model;
typedef struct orc_fwd orc_fwd;

orc_model* orc_model_create(const orc_desc* d);
void       orc_model_destroy(orc_model* m);
/* LoadTensor: dequantize raw bytes into a new F32 array of the expected element count. */
int        orc_model_set(orc_model* m, int slot, int layer, int type, const uint8_t* bytes, int64_t nbytes);
int        orc_model_finalize(orc_model* m);

orc_fwd*   orc_fwd_create(orc_model* m, int32_t max_seq);
void       orc_fwd_destroy(orc_fwd* f);
void       orc_fwd_reset(orc_fwd* f);
int        orc_forward(orc_fwd* f, int32_t token, int32_t position);
const float* orc_logits(orc_fwd* f);
/* residual stream after layer l (l == n_layers: final normed vector); needs keep_hidden */
int        orc_fwd_hidden(orc_fwd* f, int layer, float* dst, int64_t n);
int        orc_fwd_kv(orc_fwd* f, int layer, int kind, float* dst, int64_t n);
int32_t    orc_fwd_length(orc_fwd* f);
/* only run layers [0, n) and skip the LM head when head == 0 (timing samples) */
void       orc_fwd_limit(orc_fwd* f, int n_layers, int head_rows);

#ifdef __cplusplus
}
#endif
#endif
