// kernels.hpp — launch wrappers for the gfx950 kernels (host-callable, defined in kernels.hip).
#pragma once

#include "common.hpp"

namespace fllm {

// Activation vector prepared for the int8 dot-product GEMVs: for every group of 32 elements,
// 24 dwords of signed-byte digits (three base-256 digits of x * 2^16 / s, in the even/odd
// element order of the 4-bit formats) and {s, sum32, sum16a, sum16b}.
struct XQ {
    uint4* parts;   // [groups][6] uint4
    float4* stats;  // [groups]
};

// Device-side step parameters, written by a one-thread kernel before each step so that one
// captured graph serves every step.
struct StepParams {
    int token;
    int pos;      // RoPE position and last attended index
    int cur_len;  // KV slot written by this step
    int argmax;   // result of the greedy sampler
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
hipError_t launch_gemv(const WMat& m, const float* xf, const XQ& xq, float* y, const float* residual,
                       hipStream_t st);
// Quantize a float vector (n % 32 == 0) into the XQ layout.
hipError_t launch_quantize(const float* x, int64_t n, XQ xq, hipStream_t st);

hipError_t launch_set_params(StepParams* p, int token, int pos, int cur_len, hipStream_t st);
hipError_t launch_embed(const uint8_t* emb, int type, int hidden, const StepParams* p, float* x,
                        hipStream_t st);
// norm_kind 0: (x*rms)*w with eps; 1: Gemma (x*rms)*(1+w), eps 1e-6.
hipError_t launch_rmsnorm_q(const float* x, const float* w, int n, float eps, int norm_kind, float* xn,
                            XQ xq, hipStream_t st);
hipError_t launch_qkv_post(float* q, float* k, float* v, const float* bq, const float* bk, const float* bv,
                           const float2* rope, int n_heads, int n_kv, int head_dim, float* kcache,
                           float* vcache, const StepParams* p, hipStream_t st);
hipError_t launch_attention(const float* q, const float* kcache, const float* vcache, int n_heads, int n_kv,
                            int head_dim, int window, float scale, float softcap, int nsplit,
                            float* part_o, float* part_ml, float* out, XQ out_q, const StepParams* p,
                            hipStream_t st);
// h = act(g) * u, act 0 = SiLU, 1 = GELU(tanh); also quantizes h.
hipError_t launch_act(const float* g, const float* u, int n, int act, float* h, XQ hq, hipStream_t st);
// x += GemmaRmsNorm(t, w)
hipError_t launch_postnorm_add(const float* t, const float* w, int n, float* x, hipStream_t st);
hipError_t launch_softcap(float* x, int64_t n, float cap, hipStream_t st);
hipError_t launch_argmax(const float* x, int64_t n, StepParams* p, hipStream_t st);
hipError_t launch_topk(float* x, int64_t n, float inv_temp, int k, int cap, int* ids, float* vals, int* count,
                       hipStream_t st);
hipError_t launch_copy_hidden(const float* x, int n, float* dst, hipStream_t st);

}  // namespace fllm
