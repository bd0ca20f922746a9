// gemv.hpp — launch interface of the fused dequant-GEMV kernel (gemv.hip).
#pragma once

#include "kernels.hpp"

namespace fllm {

// input of the projection
// XIN_TAB: the matrix-core variant's activation table, written by the producer's epilogue
// XIN_POST (matrix-core variant only): x + GemmaRmsNorm(x2, post_w) is the new residual (stored to
// x_out by workgroup 0), then normalized as XIN_NORM: a Gemma-2 post-norm folded into its consumer
enum { XIN_F32 = 0, XIN_NORM = 1, XIN_EMBED_NORM = 2, XIN_TAB = 3, XIN_POST = 4 };
// epilogue of a segment
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_Q = 2, EPI_K = 3, EPI_V = 4, EPI_LOGITS = 5 };

// weight layout of a matrix
// LAYOUT_ROWS: GGUF rows, row r = elements [r*cols, (r+1)*cols) of the block stream.
// LAYOUT_TILES: the same blocks regrouped by 16-row tile (launch_pack_tiles), read only by the
// matrix-core variant.
enum { LAYOUT_ROWS = 0, LAYOUT_TILES = 1 };

// One matrix of a fused launch. The segment owns workgroups [wg_begin, next segment's wg_begin).
struct GemvSeg {
    const uint8_t* w;      // weight blocks in `layout`
    int layout;
    int type;
    int rows;
    int wg_begin;
    int epi;
    float* out;            // EPI_STORE / EPI_RESID / EPI_Q / EPI_LOGITS destination
    const float* bias;     // optional (Qwen2 q/k/v bias)
    const float* resid;    // EPI_RESID: out[r] = resid[r] + W x (may alias out)
};

struct GemvArgs {
    GemvSeg seg[3];
    int nseg;
    int G;                 // groups of 32 columns per row
    int S;                 // groups per wave slice
    int rpw;               // rows per workgroup (multiple of 8)
    int glu;               // 1: seg[0] = gate, seg[1] = up, seg[0].out = act(gate x) * (up x)
    int act;               // 0 SiLU, 1 GELU (tanh form)
    int mfma;              // set by gemv_plan: 1 = matrix-core variant
    int nunits;            // matrix-core variant: 16-row units of the launch (seg[i].wg_begin = first unit)
    int nw;                // matrix-core variant: waves per workgroup
    int mix_unit, mix_wg;  // matrix-core variant with Q4_K then Q6_K segments: first Q6_K unit and workgroup (0: one type)
    // input
    int xin;
    const float* x;        // XIN_F32 / XIN_NORM input vector (XIN_POST: the residual)
    float* x_out;          // XIN_EMBED_NORM: the embedding row is also stored here (workgroup 0);
                           // XIN_POST: the new residual (workgroup 0; not x: others still read it)
    const float* norm_w;   // XIN_NORM / XIN_EMBED_NORM
    float eps;
    int norm_kind;         // 0: (x*rms)*w, 1: (x*rms)*(1+w)
    const uint8_t* emb;
    int emb_type;
    const StepParams* params;
    const void* xtab;      // XIN_TAB: activation table of the input
    const float* xssq;     // XIN_TAB with RMSNorm: per-16-element sums of squares of the raw input
    // matrix-core EPI_RESID / GLU producers: activation table of the output for the next launch
    void* tab_out;         // table of out * tab_w (RESID) or of h (GLU); nullptr: none
    float* ssq_out;        // RESID: per-16-row sums of squares of out
    const float* tab_w;    // RESID: the consumer's RMSNorm weight
    int tab_kind;          // 0: w, 1: 1 + w
    // RoPE + KV store
    const float2* rope;
    int hd;
    float* kc;             // this layer's K cache [pos][kvdim]
    float* vc;             // this layer's V cache
    int kvdim;
    // logits
    float softcap;
    unsigned long long* wg_keys;  // per workgroup: (order key of its largest logit << 32) | ~index
    // XIN_POST
    const float* x2;       // the output whose post-norm is added to x
    const float* post_w;   // the post-norm weight (1 + w)
    int chunks_per_wave;   // matrix-core variant: chunks per wave (nw * chunks_per_wave = chunks per row)
};

bool gemv_fusable_type(int t);
bool gemv_fusable_cols(int64_t cols);
// Fills G, S, rpw and the segments' wg_begin (or the MFMA variant's units); returns the grid
// size. The MFMA variant is chosen only when every segment has the same weight type.
int gemv_plan(GemvArgs& a, int64_t cols, int n_cu, int rows_per_wg, int* block_threads, size_t* lds_bytes);
// true when gemv_plan picks the matrix-core variant for this launch (only those launches read or
// write activation tables)
bool gemv_uses_mfma(const GemvArgs& a, int64_t cols);
// bytes of the activation table of a vector of `cols` elements
size_t gemv_tab_bytes(int64_t cols);
// true when a Q4_K / Q6_K matrix of this shape can be stored as LAYOUT_TILES (rows a multiple of 16,
// whole 256-element chunks per row, a matrix-core wave split of the row)
bool gemv_tiles_shape_ok(int type, int64_t rows, int64_t cols);
// regroup a GGUF-row matrix (src) into LAYOUT_TILES (dst, same byte count); a byte permutation
hipError_t launch_pack_tiles(int type, const uint8_t* src, uint8_t* dst, int64_t rows, int64_t cols, hipStream_t st);
hipError_t launch_gemv_fused(const GemvArgs& a, int grid, int block_threads, size_t lds, hipStream_t st);

}  // namespace fllm
