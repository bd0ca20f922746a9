// kernels.hpp — launch wrappers for the gfx950 kernels (host-callable, defined in kernels.hip).
#pragma once

#include "common.hpp"

namespace fllm {

// Device-side step parameters, written by a one-thread kernel before each step so that one
// captured graph serves every step.
struct StepParams {
    int token;    // token fed to this step (the LM-head epilogue stores the greedy token here)
    int pos;      // RoPE position and last attended index
    int cur_len;  // KV slot written by this step
    int argmax;   // result of the greedy sampler
    int nstep;    // decode steps completed since the parameters were last set
    int pad[3];
};

// A weight matrix in GGUF block layout: row r covers elements [r*cols, (r+1)*cols) of the
// flat element stream, so rows may start inside a block.
struct WMat {
    const uint8_t* w;
    int type;
    int64_t rows;
    int64_t cols;
};

hipError_t launch_dequant(int type, const uint8_t* src, int64_t nelem, float* dst, hipStream_t st);

// y = W x (+ residual when non-null; residual may alias y).
hipError_t launch_gemv(const WMat& m, const float* xf, float* y, const float* residual, int n_cu, hipStream_t st);
// y = W x for a matrix in the tile-interleaved layout (launch_pack_tiles): matrix-core variant only
hipError_t launch_gemv_tiles(const WMat& m, const float* xf, float* y, int n_cu, hipStream_t st);

hipError_t launch_set_params(StepParams* p, int token, int pos, int cur_len, hipStream_t st);
hipError_t launch_embed(const uint8_t* emb, int type, int hidden, const StepParams* p, float* x,
                        hipStream_t st);
// norm_kind 0: (x*rms)*w with eps; 1: Gemma (x*rms)*(1+w), eps 1e-6.
hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, int norm_kind, float* xn, hipStream_t st);
hipError_t launch_qkv_post(float* q, float* k, float* v, const float* bq, const float* bk, const float* bv,
                           const float2* rope, int n_heads, int n_kv, int head_dim, float* kcache,
                           float* vcache, const StepParams* p, hipStream_t st);
hipError_t launch_attention(const float* q, const float* kcache, const float* vcache, int n_heads, int n_kv,
                            int head_dim, int window, float scale, float softcap, int nsplit,
                            float* part_o, float* part_ml, float* out, const StepParams* p, hipStream_t st);
// h = act(g) * u, act 0 = SiLU, 1 = GELU(tanh).
hipError_t launch_act(const float* g, const float* u, int n, int act, float* h, hipStream_t st);
// x += GemmaRmsNorm(t, w)
// x_out = x_in + GemmaRmsNorm(t, w) (x_out may be x_in)
hipError_t launch_postnorm_add(const float* t, const float* w, int n, const float* x_in, float* x_out, hipStream_t st);
hipError_t launch_softcap(float* x, int64_t n, float cap, hipStream_t st);
// argmax into p->argmax; with tokens_out also tokens_out[p->nstep] = argmax and the step advance
// (token = argmax, pos + 1, cur_len + 1, nstep + 1).
hipError_t launch_argmax(const float* x, int64_t n, StepParams* p, int* tokens_out, int tokens_cap, hipStream_t st);
// reduce per-workgroup argmax keys of the fused LM head; advances the step as launch_argmax
hipError_t launch_argmax_keys(const unsigned long long* keys, int n, StepParams* p, int* tokens_out, int tokens_cap,
                              hipStream_t st);
// the first maximum of each 4096-entry segment of x (n entries) as an argmax key (argmax_segments(n)
// slots), for launch_argmax_keys
int argmax_segments(int64_t n);
hipError_t launch_argmax_seg(const float* x, int64_t n, unsigned long long* keys, hipStream_t st);
// largest vocabulary of the one-workgroup samplers (launch_topk, launch_sample_nucleus)
constexpr int SAMPLE_MAX_VOCAB = 262144;
// Device scratch of the grid form of launch_topk: the sample's threshold key, per-segment counts
// (segments of 4096 entries), the candidates reaching the threshold in index order.
constexpr int TOPK_CMAX = 4096, TOPK_MAX_SEG = SAMPLE_MAX_VOCAB / 4096;
struct TopkScratch {
    uint32_t t;
    int nc;
    int wg_cnt[TOPK_MAX_SEG];
    float cand_v[TOPK_CMAX];
    int cand_i[TOPK_CMAX];
};
// sc may be null (one-workgroup form only)
hipError_t launch_topk(float* x, int64_t n, float inv_temp, int k, int cap, int* ids, float* vals, int* count,
                       TopkScratch* sc, hipStream_t st);
// LlamaLanguageModel.ApplyRepetitionPenalty on device logits; counts: n zeroed ints, left zeroed.
hipError_t launch_rep_penalty(float* x, int n, const int* ids, int n_ids, float penalty, int* counts,
                              hipStream_t st);
// Device scratch of launch_sample_nucleus: the edge's mass histograms (zero between calls) and the
// per-segment results of its passes (segments of 4096 entries).
constexpr int NUC_MAX_SEG = SAMPLE_MAX_VOCAB / 4096;
struct NucleusScratch {
    unsigned long long hist[4][256];
    float seg_max[NUC_MAX_SEG];
    float seg_sum[NUC_MAX_SEG];
    float seg_kept[NUC_MAX_SEG];
    unsigned long long seg_mass[NUC_MAX_SEG];
    int seg_tie[NUC_MAX_SEG];
    int seg_last[NUC_MAX_SEG];
};
// SamplerPipeline stages 1, 3, 4, 5 (temperature, softmax, top-p, draw with u) over x; pr: n floats
// of scratch (left holding the final distribution); the token goes to *out_token. sc: zeroed once
// at allocation.
hipError_t launch_sample_nucleus(float* x, int n, float inv_temp, float top_p, float u, float* pr, int* out_token,
                                 NucleusScratch* sc, hipStream_t st);
hipError_t launch_copy_hidden(const float* x, int n, float* dst, hipStream_t st);

}  // namespace fllm
