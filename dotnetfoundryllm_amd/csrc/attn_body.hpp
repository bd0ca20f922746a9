// attn_body.hpp — device code of the split-K decode attention (ComputeAttention,
// LlamaForwardPass.cs:158-211; Mistral window MistralForwardPass.cs:121-175; Gemma2 scale, score
// softcap and window Gemma2ForwardPass.cs:126-185) for the kernels of attention.hip.
//
// One workgroup of 256 threads takes a contiguous chunk of the attended range for the whole query
// group of a kv head, so each K/V row is read from HBM once per group. Lanes split a K/V row into
// float4 slices (hd/4 lanes per row, 64/(hd/4) rows per wave load, fully coalesced); q for the group
// stays in registers. Each workgroup writes its unnormalised partial output with the chunk's max
// and sum; the merge combines the chunks of every head.
//
// In-launch merge (WT): the chunks write their partials with write-through stores (agent-scope
// relaxed atomics: global stores with sc1), wait until those stores are acknowledged, then count
// themselves on a per-kv-head counter with a relaxed agent-scope atomic; the chunk whose count
// completes the kv head reads the others' partials with sc1 loads, which are served from memory
// rather than from a non-coherent L2 of another XCD, and merges them. No L2 write-back or invalidate
// (release / acquire fences) is needed: on this multi-XCD part those cost several microseconds per
// handoff, against about one for the write-through path.
#pragma once

#include "attention.hpp"
#include "actab.hpp"

#include <math.h>

namespace fllm {

// Cross-lane reductions with DPP row operations (VALU, no LDS round trip). dpp<CTRL, ROWS>(old, v):
// v moved by the DPP control CTRL in the rows of mask ROWS, old elsewhere.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, false));
}
enum { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140, DPP_BCAST15 = 0x142,
       DPP_BCAST31 = 0x143 };

// sum over each group of N lanes (16, 32 or 64); the total is in the group's last lane
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp<DPP_XOR1>(0.0f, v);
    v += dpp<DPP_XOR2>(0.0f, v);
    v += dpp<DPP_HALF_MIRROR>(0.0f, v);
    v += dpp<DPP_MIRROR>(0.0f, v);  // every lane: its 16-lane row
    if (N >= 32) v += dpp<DPP_BCAST15, 0xA>(0.0f, v);  // rows 1, 3: rows 0 + 1, 2 + 3
    if (N >= 64) v += dpp<DPP_BCAST31, 0xC>(0.0f, v);  // rows 2, 3: adds rows 0 + 1 (row 3 = all)
    return v;
}
// maximum over the wave, in every lane
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<DPP_XOR1>(v, v));
    v = fmaxf(v, dpp<DPP_XOR2>(v, v));
    v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v, v));
    v = fmaxf(v, dpp<DPP_MIRROR>(v, v));
    v = fmaxf(v, dpp<DPP_BCAST15, 0xA>(v, v));
    v = fmaxf(v, dpp<DPP_BCAST31, 0xC>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(group_sum<64>(v)), 63));
}

// ---- write-through access for in-launch handoffs ------------------------------------------
// buffer resource over n bytes at p (raw buffer, gfx9 word 3); loads past n return zeros
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wt_rsrc(const void* p, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)n, 0x00020000);
}
constexpr int CPOL_SC1 = 16;  // cache policy bit: agent-scope coherent (served from memory, write-through)
typedef float wt_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_wt4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const wt_f4 v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, CPOL_SC1);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float2 ld_wt2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, CPOL_SC1);
    return make_float2(v.x, v.y);
}
__device__ __forceinline__ void st_wt(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_wt_u(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// every store this thread issued has been acknowledged (the write-through data is in memory)
__device__ __forceinline__ void wt_complete() { __builtin_amdgcn_s_waitcnt(0); }

// dot of q with the K row slice kr for every head of the group, reduced over the row's lanes; the
// row's last lane stores the raw dot of row t (scale and softcap come in the softmax pass, one score
// per lane, rather than here with one lane of the wave active)
template <int HD, int G>
__device__ __forceinline__ void attn_scores(const float4* qv, const float4& kr, int t, int len, int dl, float* sc,
                                            int ch) {
    constexpr int LPR = HD / 4;
#pragma unroll
    for (int h = 0; h < G; h++) {
        float s = qv[h].x * kr.x;
        s = fmaf(qv[h].y, kr.y, s);
        s = fmaf(qv[h].z, kr.z, s);
        s = fmaf(qv[h].w, kr.w, s);
        s = group_sum<LPR>(s);
        if (dl == LPR - 1 && t < len) sc[h * ch + t] = s;
    }
}

// acc[h] += p_t v_t for the rows of the group's heads
template <int G>
__device__ __forceinline__ void attn_pv(float4* acc, const float4& vr, int t, int len, const float* sc, int ch) {
    if (t >= len) return;
#pragma unroll
    for (int h = 0; h < G; h++) {
        const float p = sc[h * ch + t];
        acc[h].x = fmaf(p, vr.x, acc[h].x);
        acc[h].y = fmaf(p, vr.y, acc[h].y);
        acc[h].z = fmaf(p, vr.z, acc[h].z);
        acc[h].w = fmaf(p, vr.w, acc[h].w);
    }
}

// K / V cache rows, read once per step: non-temporal, so that they do not displace the weights'
// neighbours in L2 (activation tables, epilogue operands, code)
typedef float kv_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 kv_ld(const float* p) {
    const kv_f4 v = __builtin_nontemporal_load((const kv_f4*)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// this lane's NP = 4 rows of the block at b0 (row indices clamped to the chunk) as one register
// vector (a vector rather than an array of float4 keeps it out of scratch memory across the loops)
typedef float kv_blk __attribute__((ext_vector_type(16)));
__device__ __forceinline__ float4 kv_row(const kv_blk& v, int u) {
    return make_float4(v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]);
}
__device__ __forceinline__ void kv_set(kv_blk& v, int u, const float4 t) {
    v[4 * u] = t.x; v[4 * u + 1] = t.y; v[4 * u + 2] = t.z; v[4 * u + 3] = t.w;
}

template <int RPP>
__device__ __forceinline__ kv_blk kv_ld_blk(const float* base, int b0, int r0, int len, int kvdim) {
    kv_blk v;
#pragma unroll
    for (int u = 0; u < 4; u++) kv_set(v, u, kv_ld(base + (int64_t)min(b0 + r0 + u * RPP, len - 1) * kvdim));
    return v;
}

// G = query heads per kv head. Rows of the chunk go in blocks of BLK = 4 rows per lane; the K and V
// rows of the first two blocks are loaded together up front (row indices clamped to the chunk, so
// every load is unconditional and all are in flight at once); later blocks (long chunks) stream
// through a ring of two blocks loaded ahead of the one in use, K's during the first blocks' scores,
// V's during the softmax. WT: the partials go out with write-through stores (read by the merging
// chunk of the same launch). Returns the step's chunk count, 0 when chunk c is past the attended
// range (the whole workgroup returns together).
template <int HD, int G, bool WT>
__device__ __forceinline__ int attn_chunk(const AttnArgs& a, const int kvh, const int c, float* sh) {
    constexpr int LPR = HD / 4;    // lanes per K/V row
    constexpr int RPL = 64 / LPR;  // rows per wave load
    constexpr int RPP = 4 * RPL;   // rows per load of the 4 waves
    constexpr int NP = 4;          // rows per lane per block
    constexpr int BLK = NP * RPP;  // rows per block
    const int h0 = kvh * G;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sub = lane / LPR, dl = lane % LPR;
    const int r0 = wave * RPL + sub;  // this lane's rows in a block: r0 + u * RPP

    // q slice of every head of the group (independent of the position)
    float4 qv[G];
#pragma unroll
    for (int h = 0; h < G; h++) qv[h] = *(const float4*)(a.q + (int64_t)(h0 + h) * HD + dl * 4);

    const int seq = a.params->pos + 1;
    const AttnRange rg = attn_range(a.params->pos, a.window, a.nc);
    const int ws = rg.ws, ch = rg.ch, nchunks = rg.nchunks;
    if (c >= nchunks) return 0;
    const int t0 = ws + c * ch;
    const int len = min(ch, seq - t0);

    float* sc = sh;                                   // [G][ch] scores, then weights
    float* red = sh + G * ch;                         // [4 waves * RPL row slots][G][HD] = 1024 G floats
    float* ml = red + 4 * RPL * G * HD;               // [G][2]

    const float* kbase = a.kc + (int64_t)t0 * a.kvdim + (int64_t)kvh * HD + dl * 4;
    const float* vbase = a.vc + (int64_t)t0 * a.kvdim + (int64_t)kvh * HD + dl * 4;
    const float inv_cap = a.softcap > 0.0f ? 1.0f / a.softcap : 0.0f;
    // ---- K and V rows of blocks 0 and 1 (block 1 only when the chunk reaches it) ---------------
    const bool blk1 = BLK < len;
    float4 kA[NP], kB[NP], vA[NP], vB[NP];
#pragma unroll
    for (int u = 0; u < NP; u++) kA[u] = kv_ld(kbase + (int64_t)min(r0 + u * RPP, len - 1) * a.kvdim);
    if (blk1) {
#pragma unroll
        for (int u = 0; u < NP; u++) kB[u] = kv_ld(kbase + (int64_t)min(BLK + r0 + u * RPP, len - 1) * a.kvdim);
    }
#pragma unroll
    for (int u = 0; u < NP; u++) vA[u] = kv_ld(vbase + (int64_t)min(r0 + u * RPP, len - 1) * a.kvdim);
    if (blk1) {
#pragma unroll
        for (int u = 0; u < NP; u++) vB[u] = kv_ld(vbase + (int64_t)min(BLK + r0 + u * RPP, len - 1) * a.kvdim);
    }

    static_assert(NP == 4, "kv_blk holds 4 rows");
    // K of blocks 2 .. 2 + KR - 1 (then the next KR, ...). Past the chunk the rows clamp to its last
    // one (re-read from cache; blocks wholly past it are not scored), so every load of the ring is
    // unconditional and they complete in the order issued: a block waits only for its own loads.
    constexpr int KR = 2;  // blocks in flight (4 measured slower for head_dim 256 at 6k positions)
    kv_blk kn[KR];  // (read only when the ring was loaded: the loops run only when 2 BLK < len)
    const bool ring = 2 * BLK < len;
    if (ring) {
#pragma unroll
        for (int j = 0; j < KR; j++) kn[j] = kv_ld_blk<RPP>(kbase, (2 + j) * BLK, r0, len, a.kvdim);
    }

    // ---- scores ---------------------------------------------------------------------------------
#pragma unroll
    for (int u = 0; u < NP; u++) attn_scores<HD, G>(qv, kA[u], r0 + u * RPP, len, dl, sc, ch);
    if (blk1) {
#pragma unroll
        for (int u = 0; u < NP; u++) attn_scores<HD, G>(qv, kB[u], BLK + r0 + u * RPP, len, dl, sc, ch);
    }
    for (int b0 = 2 * BLK; b0 < len; b0 += KR * BLK) {
#pragma unroll
        for (int j = 0; j < KR; j++) {
            if (b0 + j * BLK < len) {
#pragma unroll
                for (int u = 0; u < NP; u++)
                    attn_scores<HD, G>(qv, kv_row(kn[j], u), b0 + j * BLK + r0 + u * RPP, len, dl, sc, ch);
            }
            kn[j] = kv_ld_blk<RPP>(kbase, b0 + (j + KR) * BLK, r0, len, a.kvdim);
        }
    }
    kv_blk vn[KR];  // V of blocks 2 .. 2 + KR - 1, in flight during the softmax
    if (ring) {
#pragma unroll
        for (int j = 0; j < KR; j++) vn[j] = kv_ld_blk<RPP>(vbase, (2 + j) * BLK, r0, len, a.kvdim);
    }
    __syncthreads();

    // ---- softmax pieces per head: scores (scale, softcap), max, exp(s - max), sum ------------
    for (int h = wave; h < G; h += 4) {
        float m = -INFINITY;
        for (int t = lane; t < len; t += 64) {
            float v = sc[h * ch + t] * a.scale;
            if (a.softcap > 0.0f) v = tanhf(v * inv_cap) * a.softcap;
            sc[h * ch + t] = v;
            m = fmaxf(m, v);
        }
        m = wave_max(m);
        float l = 0.0f;
        for (int t = lane; t < len; t += 64) {
            float e = expf(sc[h * ch + t] - m);
            sc[h * ch + t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) { ml[2 * h] = m; ml[2 * h + 1] = l; }
    }
    __syncthreads();

    // ---- weighted sum of V ------------------------------------------------------------------
    float4 acc[G];
#pragma unroll
    for (int h = 0; h < G; h++) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < NP; u++) attn_pv<G>(acc, vA[u], r0 + u * RPP, len, sc, ch);
    if (blk1) {
#pragma unroll
        for (int u = 0; u < NP; u++) attn_pv<G>(acc, vB[u], BLK + r0 + u * RPP, len, sc, ch);
    }
    for (int b0 = 2 * BLK; b0 < len; b0 += KR * BLK) {
#pragma unroll
        for (int j = 0; j < KR; j++) {
            if (b0 + j * BLK < len) {
#pragma unroll
                for (int u = 0; u < NP; u++) attn_pv<G>(acc, kv_row(vn[j], u), b0 + j * BLK + r0 + u * RPP, len, sc, ch);
            }
            vn[j] = kv_ld_blk<RPP>(vbase, b0 + (j + KR) * BLK, r0, len, a.kvdim);
        }
    }
    // every (wave, row slot) leaves its partial sums in LDS; 4 * RPL slots are then summed
#pragma unroll
    for (int h = 0; h < G; h++) *(float4*)(red + (((wave * RPL + sub) * G + h) * HD) + dl * 4) = acc[h];
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * HD; idx += blockDim.x) {
        float o = 0.0f;
#pragma unroll
        for (int sl = 0; sl < 4 * RPL; sl++) o += red[sl * G * HD + idx];
        int h = idx / HD, d = idx % HD;
        float* po = a.part_o + ((int64_t)(h0 + h) * a.nc + c) * HD + d;
        if constexpr (WT) st_wt(po, o);
        else *po = o;
    }
    for (int h = threadIdx.x; h < G; h += blockDim.x) {
        float* pm = a.part_ml + ((int64_t)(h0 + h) * a.nc + c) * 2;
        if constexpr (WT) {
            st_wt(pm, ml[2 * h]);
            st_wt(pm + 1, ml[2 * h + 1]);
        } else {
            pm[0] = ml[2 * h];
            pm[1] = ml[2 * h + 1];
        }
    }
    return nchunks;
}

// The head's part of the activation table of out, for the output projection, from one wave: lanes
// 4k .. 4k + 3 hold the 16 elements of half k (res: one float4 each, HD / 4 lanes in all). stg: this
// wave's staging area in LDS (HD / 16 * 48 bytes). Called by all 64 lanes of the wave.
template <int HD>
__device__ __forceinline__ void merge_emit_table_wave(const AttnArgs& a, int h, int lane, const float4 res,
                                                      uint8_t* stg) {
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
            stg[(hl * 3 + 0) * 16 + 4 * j + by] = (uint8_t)b2;
            stg[(hl * 3 + 1) * 16 + 4 * j + by] = (uint8_t)b1;
            stg[(hl * 3 + 2) * 16 + 4 * j + by] = (uint8_t)b0;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int n = a.nh * HD;
    uint4* tab = (uint4*)a.tab_out;
    if (lane < (HD / 16) * 3) {
        const int k = lane / 3, d = lane % 3;
        int entry0, byte, stat, half;
        tab_pos(h * HD + 16 * k, n, entry0, byte, stat, half);
        tab[entry0 + d] = *(const uint4*)&stg[(k * 3 + d) * 16];
    }
    if (live && by == 0) {
        int entry0, byte, stat, half;
        tab_pos(h * HD + 16 * hl, n, entry0, byte, stat, half);
        float* st = (float*)(tab + stat);
        st[half] = sc;
        st[2 + half] = sum;
    }
}

// out[h] = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M) over the nchunks chunks of head h, by one
// wave, reading the partials other workgroups of this launch wrote (write-through loads). Up to 256
// chunks: (m, l) of chunks lane + 64 i in registers; the chunk outputs NCM at a time, the first NCM
// loaded together with the (m, l) so that a merge of up to NCM chunks waits one memory round trip.
// With at most 64 chunks the arithmetic is the one-wave merge's (k_attn_merge_fast): the same
// weights and the same order of the sums.
template <int HD>
__device__ __forceinline__ float4 merge_head_wave(const AttnArgs& a, int h, int nchunks, int lane) {
    constexpr int NCM = 32;
    const __amdgpu_buffer_rsrc_t pr = wt_rsrc(a.part_o, (uint32_t)((size_t)a.nh * a.nc * HD * 4));
    const __amdgpu_buffer_rsrc_t mr = wt_rsrc(a.part_ml, (uint32_t)((size_t)a.nh * a.nc * 8));
    const uint32_t lo = (uint32_t)(((h * a.nc) * HD + (lane < HD / 4 ? lane : 0) * 4) * 4);
    // (only the slots of existing chunks are read: each load goes to memory, and one workgroup
    // pulls the whole head group's partials)
    float4 p[NCM];
#pragma unroll
    for (int k = 0; k < NCM; k++)
        if (k < nchunks) p[k] = ld_wt4(pr, lo + (uint32_t)(k * HD * 4));
    float2 mlv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int k = lane + 64 * i;
        mlv[i] = make_float2(-INFINITY, 0.0f);
        if (64 * i < nchunks) mlv[i] = ld_wt2(mr, (uint32_t)(((h * a.nc) + (k < nchunks ? k : nchunks - 1)) * 8));
    }
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (lane + 64 * i < nchunks) M = fmaxf(M, mlv[i].x);
    M = wave_max(M);
    float w[4], lw = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const bool valid = lane + 64 * i < nchunks;
        w[i] = valid ? expf(mlv[i].x - M) : 0.0f;
        lw += valid ? mlv[i].y * w[i] : 0.0f;
    }
    const float L = wave_sum(lw);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = 0; k0 < nchunks; k0 += NCM) {
        if (k0 > 0) {
#pragma unroll
            for (int k = 0; k < NCM; k++)
                if (k0 + k < nchunks) p[k] = ld_wt4(pr, lo + (uint32_t)((k0 + k) * HD * 4));
        }
#pragma unroll
        for (int k = 0; k < NCM; k++) {
            const int kk = k0 + k;
            if (kk < nchunks) {
                const int src = kk & 63, i = kk >> 6;
                const float wi = i == 0 ? w[0] : i == 1 ? w[1] : i == 2 ? w[2] : w[3];
                const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wi), src));
                o.x = fmaf(p[k].x, wk, o.x);
                o.y = fmaf(p[k].y, wk, o.y);
                o.z = fmaf(p[k].z, wk, o.z);
                o.w = fmaf(p[k].w, wk, o.w);
            }
        }
    }
    const float inv = 1.0f / L;
    return make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
}

// The attention kernel with its own merge, workgroup (kv head kvh, chunk c): the chunk's partials
// (write-through), then the chunk that completes the kv head's count merges the head group's chunks
// (one wave per head), writes out and the output projection's table, and clears the counter for the
// next launch. cnt: this kv head's counter, zero before the launch.
template <int HD, int G>
__device__ __forceinline__ void attn_chunk_and_merge(const AttnArgs& a, unsigned* cnt, int kvh, int c) {
    extern __shared__ __attribute__((aligned(16))) float sh_attn[];
    __shared__ __attribute__((aligned(16))) int s_last[4];
    const int nchunks = attn_chunk<HD, G, true>(a, kvh, c, sh_attn);
    if (nchunks == 0) return;
    wt_complete();
    __syncthreads();
    if (threadIdx.x == 0)
        s_last[0] = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(nchunks - 1);
    __syncthreads();
    if (!s_last[0]) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint8_t* stg = (uint8_t*)sh_attn + wave * (HD / 16) * 48;  // (the chunk's LDS is free again)
    for (int hb = 0; hb < G; hb += 4) {
        const int hh = hb + wave;
        if (hh < G) {
            const int h = kvh * G + hh;
            const float4 res = merge_head_wave<HD>(a, h, nchunks, lane);
            if (lane < HD / 4) *(float4*)(a.out + (int64_t)h * HD + lane * 4) = res;
            if (a.tab_out) merge_emit_table_wave<HD>(a, h, lane, res, stg);
        }
    }
    if (threadIdx.x == 0) st_wt_u(cnt, 0u);
}

}  // namespace fllm
