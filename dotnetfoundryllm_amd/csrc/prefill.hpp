// prefill.hpp — launch interface of the batched prefill kernels (prefill.hip): the prompt's
// tokens pass through each layer together, the projections as fp16 matrix-core GEMMs on 22-bit
// operand splits.
#pragma once

#include "kernels.hpp"

namespace fllm {

// Y[t][n] (+)= sum_k X[t][k] W[n][k] for t < T, n < N on the fp16 matrix cores, for up to three
// matrices that share X (one launch: q, k, v or gate, up). X: f32 rows of stride ldx, read by the
// kernels as the fp16 planes launch_pf_split wrote (xh, required); each W in its stored layout
// (LAYOUT_TILES Q4_K / Q5_K / Q6_K / Q8_0, or GGUF rows of any supported type), decoded exactly in
// the kernel; all segments of a launch are tile-interleaved or none is. K is a multiple of 32.
struct PfSeg {
    const uint8_t* w;
    int type, layout;
    int N;
    float* y;   // [T][ldy], column 0 = weight row 0
    int ldy;
    int tiles;  // set by launch_pf_gemm: 128-row column tiles of the segment
    int wexp;   // fp16 matrix cores: the weights enter scaled by 2^-wexp (launch_pf_wmax gives it)
};
struct PfGemm {
    const float* x;
    int ldx;
    int K;
    int T;
    int add;  // 1: y += X W^T (residual add), 0: y = X W^T
    int nseg;
    PfSeg seg[3];
    // optional scratch of part_cap floats: a launch whose grid is at most two waves of resident
    // workgroups may split K over grid.z (nsplit parts of kpart whole 256-element blocks, the last
    // one possibly shorter, set by launch_pf_gemm) when its segments fill one buffer's rows side by
    // side; part 0 writes y, part z > 0 its own [T][ldy] slice of part, and a reduction adds the
    // slices into y in order (or the caller's next kernel does: see launch_pf_gemm's pending)
    float* part;
    size_t part_cap;
    int nsplit, kpart;
    // X as written by launch_pf_split (two fp16 planes of row stride ldh, each token row scaled by a
    // power of two, then the group-sum planes) and xs[t], the factor that undoes that scale
    const _Float16* xh;
    int ldh;
    const float* xs;
};
// With pending non-null, a K-split launch leaves its parts z > 0 in a.part and sets *pending to their
// number (0 when unsplit) instead of adding them: the next kernel that reads y adds them first, in
// order (launch_pf_split_norm, launch_pf_qkv_post, launch_pf_postnorm_add), or launch_pf_split_add does.
hipError_t launch_pf_gemm(PfGemm a, int n_cu, hipStream_t st, int* pending = nullptr);
// y[i] += part[0][i] + ... + part[nsp - 1][i] (in that order), slices of n floats
hipError_t launch_pf_split_add(float* y, const float* part, int nsp, int64_t n, hipStream_t st);
// The fp16 operand of a GEMM input: each row t of X [T][K] (stride ldx) scaled by 2^e_t, so that its
// largest magnitude lies in [2^14, 2^15), and written as hi = fp16(x 2^e_t) (plane 0) and
// lo = fp16(x 2^e_t - hi) (plane 1, at xh + T * ldh), 22 significant bits together; xs[t] = 2^-e_t.
// After the two planes: the hi and lo halves of each 32-element group's sum of the scaled values
// (xh + 2 T ldh: T rows of K / 32, then the lo plane), for the Q4_K form's min term. xh holds
// 2 T (ldh + K / 32) halves.
hipError_t launch_pf_split(const float* x, int ldx, int T, int K, _Float16* xh, int ldh, float* xs, hipStream_t st);
// launch_pf_split of a row computed on the way, never written: RmsNorm / GemmaRmsNorm (kind 1) of
// every row of x [T][K] (launch_pf_norm's arithmetic), or act(gate) * up of every row of gu [T][2 ffn]
// (launch_pf_act's). For K up to 20480 (pf_split_src_ok); larger rows: hipErrorNotSupported.
// The norm form first adds nsp pending K-split slices of part ([T][K] each) into x, written back.
bool pf_split_src_ok(int K);
hipError_t launch_pf_split_norm(float* x, int T, int K, const float* w, float eps, int kind, _Float16* xh,
                                int ldh, float* xs, hipStream_t st, const float* part = nullptr, int nsp = 0);
hipError_t launch_pf_split_act(const float* gu, int T, int ffn, int act, _Float16* xh, int ldh, float* xs,
                               hipStream_t st);
// *out = max(*out, bits of the largest |w| over the n elements of a weight matrix in GGUF row layout)
// (out holds a non-negative float's bits; zero it first). pf_wexp turns it into the exponent that
// brings the matrix's largest magnitude into [2^14, 2^15) for the fp16 split.
hipError_t launch_pf_wmax(int type, const uint8_t* w, int64_t n, unsigned* out, hipStream_t st);
int pf_wexp(unsigned max_bits);

// X[t] = embedding row tokens[t] (exact dequantization of any supported type)
hipError_t launch_pf_embed(const int* tokens, int T, const uint8_t* emb, int type, int H, float* x, hipStream_t st);
// RmsNorm / GemmaRmsNorm (kind 1) of every row of X [T][n] into xn (row stride ldx)
hipError_t launch_pf_norm(const float* x, int T, int n, const float* w, float eps, int kind, float* xn, int ldx,
                          hipStream_t st);
// h = act(gate) * up per row of gu [T][2 ffn] (gate columns, then up columns), row stride ldx
hipError_t launch_pf_act(const float* gu, int T, int ffn, int act, float* h, int ldx, hipStream_t st);
// rows of qkv [T][ldq] = (q | k | v): bias, RoPE at position pos0 + t on q and k, q written back,
// k and v stored in cache slot pos0 + t of this layer's K / V cache; nsp pending K-split slices of
// part ([T][ldq] each) are added to every value first, in order
hipError_t launch_pf_qkv_post(float* qkv, int ldq, int T, int pos0, const float* bq, const float* bk, const float* bv,
                              const float2* rope, int nh, int nkv, int hd, float* kc, float* vc, hipStream_t st,
                              const float* part = nullptr, int nsp = 0);
// x[t] += GemmaRmsNorm(tmp[t], w) for every row (n a multiple of 4); nsp pending K-split slices of
// part ([T][n] each) are added to tmp first, in order
hipError_t launch_pf_postnorm_add(float* tmp, int T, int n, const float* w, float* x, hipStream_t st,
                                  const float* part = nullptr, int nsp = 0);

// Causal attention of T query rows (positions pos0 + t) over this layer's cache, which already
// holds the T new rows: out[t][h*hd + d].
struct PfAttn {
    const float* q;  // [T][ldq], head h at h * hd
    int ldq;
    const float* kc;
    const float* vc;
    float* out;      // [T][nh * hd]
    int T, pos0;
    int nh, nkv, hd, kvdim;
    int window;      // attend to the last `window` positions (INT32_MAX = all)
    float scale, softcap;
    // optional scratch of part_cap floats for the halves of split key ranges (launch_pf_attn splits
    // the longer query blocks when all halves then fit the resident workgroup slots of n_cu CUs)
    float* part;
    size_t part_cap;
    int n_cu;
    int split;  // set by launch_pf_attn
    // head_dim 256 (required there): the fp16 planes of the cached K / V, nblk blocks of 32
    // positions per KV head (pf_kv_planes_halves halves), and their exponents (2 ints per block)
    _Float16* kvh;
    int* kvs;
    int nblk;
};
// halves of the K / V planes launch_pf_attn needs for head_dim hd over nkv heads and max_seq positions
// (0 when it needs none)
size_t pf_kv_planes_halves(int hd, int nkv, int max_seq);
hipError_t launch_pf_attn(const PfAttn& a, hipStream_t st);

}  // namespace fllm
