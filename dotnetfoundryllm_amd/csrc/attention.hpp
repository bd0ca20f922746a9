// attention.hpp — launch interface of the split-K decode attention kernel (attention.hip).
#pragma once

#include "kernels.hpp"

namespace fllm {

constexpr int ATTN_GROUP_MAX = 8;     // query heads per kv head handled by the fast kernel
constexpr int ATTN_MAX_CHUNKS = 256;  // position chunks per kv head (chunks hold at most 256 positions)

struct AttnArgs {
    const float* q;        // [nh][hd]
    const float* kc;       // this layer's K cache [pos][kvdim]
    const float* vc;       // this layer's V cache
    int nh, nkv, hd, kvdim;
    int window;            // attend to the last `window` positions (INT32_MAX = all)
    float scale, softcap;  // softcap 0 = off
    int nc;                // chunks per kv head (grid.y)
    float* part_o;         // [nh][nc][hd]
    float* part_ml;        // [nh][nc][2]
    float* out;            // [nh][hd]
    const StepParams* params;
    void* tab_out;         // optional: activation table of out (nh * hd elements, a multiple of 256)
};

// The attended positions [ws, pos] of a step split into nchunks chunks of ch positions (ch =
// ceil(len / nc) rounded up to 32; the last chunk may be shorter): the split of the attention
// kernel and of every reader of its partials.
struct AttnRange { int ws, ch, nchunks; };
__host__ __device__ __forceinline__ AttnRange attn_range(int pos, int window, int nc) {
    const int seq = pos + 1;
    int ws = seq - window;
    if (ws < 0) ws = 0;
    const int alen = seq - ws;
    int ch = (alen + nc - 1) / nc;
    ch = (ch + 31) / 32 * 32;
    return AttnRange{ws, ch, (alen + ch - 1) / ch};
}

// Counters of the attention launch that merges its own chunks: one per kv head, on its own 128-byte
// line (word kvh * ATTN_CNT_STRIDE), zero between launches (each launch's merging chunks clear them).
constexpr int ATTN_CNT_STRIDE = 32;
__host__ __device__ __forceinline__ int attn_cnt_words(int nkv) { return nkv * ATTN_CNT_STRIDE; }

bool attn_fast_supported(int head_dim, int group, int max_seq);
int attn_chunks(int n_kv, int max_seq, int n_cu);
size_t attn_lds_bytes(int head_dim, int group, int nc, int max_seq);
// the two kernels of the decode attention: per-chunk partials, then the merge over chunks
hipError_t launch_attn_partial(const AttnArgs& a, size_t lds, hipStream_t st);
hipError_t launch_attn_merge(const AttnArgs& a, hipStream_t st);
// the decode attention as one launch: the chunks' partials, and the last chunk of each kv head to
// finish merges them (cnt: attn_cnt_words(nkv) counters, zero before the launch, zero after it)
hipError_t launch_attn_merged(const AttnArgs& a, size_t lds, unsigned* cnt, hipStream_t st);
hipError_t launch_attn_decode(const AttnArgs& a, size_t lds, hipStream_t st);

}  // namespace fllm
