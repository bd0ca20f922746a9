// attention.hip — decode attention over the device KV cache (gfx950).
//
// ComputeAttention (LlamaForwardPass.cs:158-211; Mistral window MistralForwardPass.cs:121-175;
// Gemma2 scale, score softcap and window Gemma2ForwardPass.cs:126-185): for every query head,
// scores s_t = Dot(q, k_t) * scale over t in [window_start, position], optional tanh softcap,
// Softmax, out = sum_t p_t v_t.
//
// Split-K ("flash decoding") layout, device code in attn_body.hpp: workgroup (kv head, chunk)
// takes a contiguous chunk of the attended range for the whole query group of that kv head and
// writes its unnormalised partial output with the chunk's max and sum; a second kernel merges the
// chunks of every head. The q/k/v launch can also run both steps in its own grid
// (launch_qkv_attention, gemv.hip).
#include "attention.hpp"
#include "actab.hpp"
#include "attn_body.hpp"

#include <math.h>

namespace fllm {

template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_decode(const AttnArgs a) {
    extern __shared__ float sh[];
    attn_chunk<HD, G, false>(a, (int)blockIdx.x, (int)blockIdx.y, sh);
}

// the same chunks, merged by the last chunk of each kv head to finish (attn_chunk_and_merge)
template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_decode_merged(const AttnArgs a, unsigned* cnt) {
    attn_chunk_and_merge<HD, G>(a, cnt + blockIdx.x * ATTN_CNT_STRIDE, (int)blockIdx.x, (int)blockIdx.y);
}

// The head's part of the activation table of out, for the output projection: lanes 4k .. 4k + 3
// hold the 16 elements of half k (res: one float4 each, HD / 4 lanes in all). Called by all 64
// lanes of the workgroup.
template <int HD>
__device__ __forceinline__ void merge_emit_table(const AttnArgs& a, int h, int lane, const float4 res) {
    __shared__ __attribute__((aligned(16))) uint8_t stg[HD / 16][3][16];
    const bool live = lane < HD / 4;
    const float4 v = res;
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    float sum = (v.x + v.y) + (v.z + v.w);
#pragma unroll
    for (int o = 1; o < 4; o <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o));
        sum += __shfl_xor(sum, o);
    }
    float sc, qinv;
    half_scale(amax, sc, qinv);
    const int hl = lane >> 2, by = lane & 3;  // element 4 by + j of half hl, j = component
    if (live) {
        const float c4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int b2, b1, b0;
            digits3(quant_x(c4[j], qinv), b2, b1, b0);
            stg[hl][0][4 * j + by] = (uint8_t)b2;
            stg[hl][1][4 * j + by] = (uint8_t)b1;
            stg[hl][2][4 * j + by] = (uint8_t)b0;
        }
    }
    __syncthreads();
    const int n = a.nh * HD;
    uint4* tab = (uint4*)a.tab_out;
    if (lane < (HD / 16) * 3) {
        const int k = lane / 3, d = lane % 3;
        int entry0, byte, stat, half;
        tab_pos(h * HD + 16 * k, n, entry0, byte, stat, half);
        tab[entry0 + d] = *(const uint4*)&stg[k][d][0];
    }
    if (live && by == 0) {
        int entry0, byte, stat, half;
        tab_pos(h * HD + 16 * hl, n, entry0, byte, stat, half);
        float* st = (float*)(tab + stat);
        st[half] = sc;
        st[2 + half] = sum;
    }
}

// Merge for at most NCM chunks: every load that does not depend on the step (the chunks' (m, l) and
// this lane's slices of their outputs for all nc chunk slots) goes out at the start, beside the
// read of the step's position; the weights reach the lanes by readlane.
template <int HD, int NCM>
__global__ __launch_bounds__(64) void k_attn_merge_fast(const AttnArgs a) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const float2 ml = *(const float2*)(a.part_ml + ((int64_t)h * a.nc + (lane < a.nc ? lane : a.nc - 1)) * 2);
    const float* po = a.part_o + (int64_t)h * a.nc * HD + (lane < HD / 4 ? lane : 0) * 4;
    // unconditional loads (slots past nc re-read the last one) so that all of them are in flight
    float4 p[NCM];
#pragma unroll
    for (int k = 0; k < NCM; k++) p[k] = *(const float4*)(po + (int64_t)(k < a.nc ? k : a.nc - 1) * HD);
    const int nchunks = attn_range(a.params->pos, a.window, a.nc).nchunks;
    const bool valid = lane < nchunks;
    const float M = wave_max(valid ? ml.x : -INFINITY);
    const float w = valid ? expf(ml.x - M) : 0.0f;
    const float L = wave_sum(valid ? ml.y * w : 0.0f);
    // slots from nchunks on hold no partial of this step (possibly never-written memory): skipped,
    // not weighted by zero
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < NCM; k++) {
        const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), k));
        const bool use = k < nchunks;
        o.x = use ? fmaf(p[k].x, wk, o.x) : o.x;
        o.y = use ? fmaf(p[k].y, wk, o.y) : o.y;
        o.z = use ? fmaf(p[k].z, wk, o.z) : o.z;
        o.w = use ? fmaf(p[k].w, wk, o.w) : o.w;
    }
    const float inv = 1.0f / L;
    const float4 res = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    if (lane < HD / 4) *(float4*)(a.out + (int64_t)h * HD + lane * 4) = res;
    if (a.tab_out) merge_emit_table<HD>(a, h, lane, res);
}

// out[h] = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M) over the chunks of head h, for more chunks
// than the one-wave merge holds (up to 256). Four waves per head: thread t holds chunk t's (m, l);
// the chunk outputs are read as NS = 4 * 64 / (HD / 4) streams (HD / 4 lanes per chunk slice), each
// lane loading its stream's slices of NB chunks at once, beside the (m, l) and step reads, so the
// launch waits about one memory round trip. The streams' sums are added in stream order in LDS.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge_wide(const AttnArgs a) {
    constexpr int LPC = HD / 4;   // lanes per chunk slice
    constexpr int S = 64 / LPC;   // chunk streams per wave
    constexpr int NS = 4 * S;     // chunk streams per workgroup
    constexpr int NB = 16;        // chunks per stream in flight
    __shared__ float wts[ATTN_MAX_CHUNKS];
    __shared__ float red[8];
    __shared__ float4 ored[NS][LPC];
    const int h = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int stream = wave * S + lane / LPC, d4 = lane % LPC;
    const int nc = a.nc;
    const float2 ml = *(const float2*)(a.part_ml + ((int64_t)h * nc + (t < nc ? t : nc - 1)) * 2);
    const float* po = a.part_o + (int64_t)h * nc * HD + d4 * 4;
    // unconditional loads (chunk indices clamped) so that all of them are in flight at once
    float4 p[NB];
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const int k = stream + u * NS;
        p[u] = *(const float4*)(po + (int64_t)(k < nc ? k : nc - 1) * HD);
    }
    const int nchunks = attn_range(a.params->pos, a.window, nc).nchunks;
    // slots from nchunks on hold no partial of this step (possibly never-written memory): skipped,
    // not weighted by zero
    const bool valid = t < nchunks;
    float m = wave_max(valid ? ml.x : -INFINITY);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float w = valid ? expf(ml.x - M) : 0.0f;
    wts[t] = w;
    const float lw = wave_sum(valid ? ml.y * w : 0.0f);
    if (lane == 0) red[4 + wave] = lw;
    __syncthreads();
    const float L = (red[4] + red[5]) + (red[6] + red[7]);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const int k = stream + u * NS;
        if (k < nchunks) {
            const float wk = wts[k];
            o.x = fmaf(p[u].x, wk, o.x);
            o.y = fmaf(p[u].y, wk, o.y);
            o.z = fmaf(p[u].z, wk, o.z);
            o.w = fmaf(p[u].w, wk, o.w);
        }
    }
    for (int k0 = NB * NS; k0 < nchunks; k0 += NB * NS) {  // more chunks than one pass holds
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int k = k0 + stream + u * NS;
            p[u] = *(const float4*)(po + (int64_t)(k < nc ? k : nc - 1) * HD);
        }
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int k = k0 + stream + u * NS;
            if (k < nchunks) {
                const float wk = wts[k];
                o.x = fmaf(p[u].x, wk, o.x);
                o.y = fmaf(p[u].y, wk, o.y);
                o.z = fmaf(p[u].z, wk, o.z);
                o.w = fmaf(p[u].w, wk, o.w);
            }
        }
    }
    ored[stream][d4] = o;
    __syncthreads();
    float4 res = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < LPC) {
        float4 acc = ored[0][t];
#pragma unroll
        for (int sidx = 1; sidx < NS; sidx++) {
            const float4 v = ored[sidx][t];
            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
        }
        const float inv = 1.0f / L;
        res = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        *(float4*)(a.out + (int64_t)h * HD + t * 4) = res;
    }
    // (threads from 64 on take no part in the table but reach its barrier)
    if (a.tab_out) merge_emit_table<HD>(a, h, t, res);
}

bool attn_fast_supported(int head_dim, int group, int max_seq) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && group >= 1 && group <= ATTN_GROUP_MAX &&
           max_seq <= 256 * ATTN_MAX_CHUNKS;
}

int attn_chunks(int n_kv, int max_seq, int n_cu) {
    // about one workgroup per CU at long context (twice as many, which puts two on some CUs,
    // measured 3% slower for Qwen2-7B at 2k positions), chunks of at most 256 positions, and at
    // most 256 chunks (the merge's limit)
    int target = (n_cu + n_kv - 1) / n_kv;
    if (target > ATTN_MAX_CHUNKS) target = ATTN_MAX_CHUNKS;
    int by_min = (max_seq + 31) / 32;
    int by_max = (max_seq + 255) / 256;
    int nc = target < by_min ? target : by_min;
    if (nc < by_max) nc = by_max;
    if (nc < 1) nc = 1;
    return nc;
}

size_t attn_lds_bytes(int head_dim, int group, int nc, int max_seq) {
    int ch_max = (max_seq + nc - 1) / nc;
    ch_max = (ch_max + 31) / 32 * 32;
    // scores, the partial sums of the 4 waves' row slots (4 * 256 / head_dim slots of head_dim), m and l
    (void)head_dim;
    return sizeof(float) * ((size_t)group * ch_max + 1024 * (size_t)group + 2 * (size_t)group);
}

template <int HD>
static void attn_decode_g(const AttnArgs& a, dim3 grid, size_t lds, hipStream_t st) {
    switch (a.nh / a.nkv) {
        case 1: k_attn_decode<HD, 1><<<grid, 256, lds, st>>>(a); break;
        case 2: k_attn_decode<HD, 2><<<grid, 256, lds, st>>>(a); break;
        case 3: k_attn_decode<HD, 3><<<grid, 256, lds, st>>>(a); break;
        case 4: k_attn_decode<HD, 4><<<grid, 256, lds, st>>>(a); break;
        case 5: k_attn_decode<HD, 5><<<grid, 256, lds, st>>>(a); break;
        case 6: k_attn_decode<HD, 6><<<grid, 256, lds, st>>>(a); break;
        case 7: k_attn_decode<HD, 7><<<grid, 256, lds, st>>>(a); break;
        default: k_attn_decode<HD, 8><<<grid, 256, lds, st>>>(a); break;
    }
}

hipError_t launch_attn_partial(const AttnArgs& a, size_t lds, hipStream_t st) {
    dim3 grid(a.nkv, a.nc);
    const int g = a.nh / a.nkv;
    if (g < 1 || g > ATTN_GROUP_MAX || g * a.nkv != a.nh) return hipErrorInvalidValue;
    switch (a.hd) {
        case 64: attn_decode_g<64>(a, grid, lds, st); break;
        case 128: attn_decode_g<128>(a, grid, lds, st); break;
        default: attn_decode_g<256>(a, grid, lds, st); break;
    }
    return hipGetLastError();
}

hipError_t launch_attn_merge(const AttnArgs& a, hipStream_t st) {
    if (a.nc <= 32) {
        switch (a.hd) {
            case 64: k_attn_merge_fast<64, 32><<<a.nh, 64, 0, st>>>(a); break;
            case 128: k_attn_merge_fast<128, 32><<<a.nh, 64, 0, st>>>(a); break;
            default: k_attn_merge_fast<256, 32><<<a.nh, 64, 0, st>>>(a); break;
        }
        return hipGetLastError();
    }
    if (a.nc > ATTN_MAX_CHUNKS) return hipErrorInvalidValue;
    switch (a.hd) {
        case 64: k_attn_merge_wide<64><<<a.nh, 256, 0, st>>>(a); break;
        case 128: k_attn_merge_wide<128><<<a.nh, 256, 0, st>>>(a); break;
        default: k_attn_merge_wide<256><<<a.nh, 256, 0, st>>>(a); break;
    }
    return hipGetLastError();
}

template <int HD>
static void attn_merged_g(const AttnArgs& a, dim3 grid, size_t lds, unsigned* cnt, hipStream_t st) {
    switch (a.nh / a.nkv) {
        case 1: k_attn_decode_merged<HD, 1><<<grid, 256, lds, st>>>(a, cnt); break;
        case 2: k_attn_decode_merged<HD, 2><<<grid, 256, lds, st>>>(a, cnt); break;
        case 3: k_attn_decode_merged<HD, 3><<<grid, 256, lds, st>>>(a, cnt); break;
        case 4: k_attn_decode_merged<HD, 4><<<grid, 256, lds, st>>>(a, cnt); break;
        case 5: k_attn_decode_merged<HD, 5><<<grid, 256, lds, st>>>(a, cnt); break;
        case 6: k_attn_decode_merged<HD, 6><<<grid, 256, lds, st>>>(a, cnt); break;
        case 7: k_attn_decode_merged<HD, 7><<<grid, 256, lds, st>>>(a, cnt); break;
        default: k_attn_decode_merged<HD, 8><<<grid, 256, lds, st>>>(a, cnt); break;
    }
}

hipError_t launch_attn_merged(const AttnArgs& a, size_t lds, unsigned* cnt, hipStream_t st) {
    dim3 grid(a.nkv, a.nc);
    const int g = a.nh / a.nkv;
    if (g < 1 || g > ATTN_GROUP_MAX || g * a.nkv != a.nh || cnt == nullptr || a.nc > ATTN_MAX_CHUNKS)
        return hipErrorInvalidValue;
    // the merging chunk's staging of the output table: one wave's share per head of the group
    const size_t need = lds > (size_t)4 * (a.hd / 16) * 48 ? lds : (size_t)4 * (a.hd / 16) * 48;
    switch (a.hd) {
        case 64: attn_merged_g<64>(a, grid, need, cnt, st); break;
        case 128: attn_merged_g<128>(a, grid, need, cnt, st); break;
        default: attn_merged_g<256>(a, grid, need, cnt, st); break;
    }
    return hipGetLastError();
}

hipError_t launch_attn_decode(const AttnArgs& a, size_t lds, hipStream_t st) {
    hipError_t e = launch_attn_partial(a, lds, st);
    return e != hipSuccess ? e : launch_attn_merge(a, st);
}

}  // namespace fllm
