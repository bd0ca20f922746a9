// prefill.hip — batched prefill kernels (gfx950).
//
// The reference's prefill is n consecutive Forward calls (LlamaLanguageModel.cs:133-137). Here the
// n prompt tokens go through each layer together: every projection is one GEMM over the tokens,
// Y[t][n] = sum_k X[t][k] W[n][k] (LinearProjection, LlamaForwardPass.cs:237-260, for all rows at
// once), and the element-wise steps of the layer run over all rows.
//
// GEMM numerics: fp16 matrix cores (v_mfma_f32_16x16x32_f16, exact fp16 products summed in f32) on
// operands of 22 significant bits. launch_pf_split scales each token row of X by a power of two so
// that its largest magnitude lies in [2^14, 2^15) and writes hi = fp16(x) and lo = fp16(x - hi); the
// epilogues undo the scale exactly. The weights enter in one of four forms:
//  - Q4_K (pf_gemm_tile_q4k): sc q, an integer below 2048, exact in fp16; two products per weight,
//    each 256-element block's sum scaled by its d in f32 and its min term one more product;
//  - Q6_K (pf_gemm_tile_q6k): sc q as exact hi / lo fp16 integers; three products, d per block;
//  - tile-interleaved Q8_0 (pf_gemm_tile_h): the int8 code q, exact in fp16; two products per
//    weight, each 32-element block's sum scaled by its d in f32;
//  - the other types (pf_gemm_tile_h): dequantized exactly (the Dequantizer arithmetic), scaled by
//    a per-matrix power of two (pf_wexp) and split hi / lo; hi_x hi_w + hi_x lo_w + lo_x hi_w,
//    within 2^-21 of the f32 product.
#include "prefill.hpp"
#include "deq.hpp"
#include "gemv.hpp"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

namespace fllm {

typedef float pf_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float pf_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float pf_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
// sum over a 256-thread workgroup (called once per kernel by every thread)
__device__ __forceinline__ float pf_block_sum(float v, float* red) {
    v = pf_wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
// LDS written by lanes of a wave, then read by other lanes of the same wave
__device__ __forceinline__ void pf_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- exact dequantization of 32 weights [k0, k0 + 32) of row r (k0 a multiple of 32) -----------
// load() fetches the raw bytes of the group (issued a K step ahead), deq() decodes them.
template <int WT> struct PfW;

// LAYOUT_TILES Q4_K (DequantizeQ4_K, Dequantizer.cs:251-294): group g of the row's block kb is the
// 16 qs bytes of lane 16 (g & 3) + n in the region's first (g < 4) or second KiB; the row's header
// (d, dmin, 12 scale bytes) sits at 2048 + 16 n.
template <> struct PfW<FLLM_TYPE_Q4_K> {
    struct Raw { uint4 qs, hdr; };
    __device__ static void load(Raw& w4, const uint8_t* __restrict__ w, int K, int r, int k0) {
        const int NB = K >> 8, kb = k0 >> 8, g = (k0 >> 5) & 7, n = r & 15;
        const uint8_t* reg = w + ((size_t)(r >> 4) * NB + kb) * (16 * 144);
        w4.qs = *(const uint4*)(reg + (g < 4 ? 0 : 1024) + 16 * (16 * (g & 3) + n));
        w4.hdr = *(const uint4*)(reg + 2048 + 16 * n);
    }
    // byte idx of the 16-byte header
    __device__ static uint32_t hbyte(const uint4& h, int idx) {
        // selects of values, not of lvalues: a select of the fields' addresses keeps the header in
        // scratch memory
        const uint32_t x = h.x, y = h.y, z = h.z, w4 = h.w;
        const uint32_t w = idx < 8 ? (idx < 4 ? x : y) : (idx < 12 ? z : w4);
        return (w >> (8 * (idx & 3))) & 0xFFu;
    }
    // DecodeKScaleMin (Dequantizer.cs:506-521) on scale bytes 4..15 of the header
    __device__ static void scale_min(const uint4& h, int g, int& sc, int& mn) {
        if (g < 4) {
            sc = (int)(hbyte(h, 4 + g) & 63u);
            mn = (int)(hbyte(h, 8 + g) & 63u);
        } else {
            const uint32_t b = hbyte(h, 8 + g), lo = hbyte(h, g), hi = hbyte(h, 4 + g);
            sc = (int)((b & 15u) | ((lo >> 6) << 4));
            mn = (int)((b >> 4) | ((hi >> 6) << 4));
        }
    }
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v, float s = 1.0f) {
        const int g = (k0 >> 5) & 7;
        const float d = half_exact(w4.hdr.x & 0xFFFFu), dmin = half_exact(w4.hdr.x >> 16);
        // DecodeKScaleMin (Dequantizer.cs:506-521) on scale bytes 4..15 of the header
        int sc, mn;
        if (g < 4) {
            sc = (int)(hbyte(w4.hdr, 4 + g) & 63u);
            mn = (int)(hbyte(w4.hdr, 8 + g) & 63u);
        } else {
            const uint32_t b = hbyte(w4.hdr, 8 + g), lo = hbyte(w4.hdr, g), hi = hbyte(w4.hdr, 4 + g);
            sc = (int)((b & 15u) | ((lo >> 6) << 4));
            mn = (int)((b >> 4) | ((hi >> 6) << 4));
        }
        // a power-of-two scale s commutes with the roundings: (dg s) q - mg s = s (dg q - mg) exactly
        const float dg = d * (float)sc * s;
        const float mg = dmin * (float)mn * s;
        const uint32_t wd[4] = {w4.qs.x, w4.qs.y, w4.qs.z, w4.qs.w};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const int at = q4t_pos(i >> 1);  // the tile layout's position of group byte i / 2
            const uint32_t byte = (wd[at >> 2] >> (8 * (at & 3))) & 0xFFu;
            const int q = (i & 1) ? (int)(byte >> 4) : (int)(byte & 15u);
            v[i] = dg * (float)q - mg;
        }
    }
};

// LAYOUT_TILES Q6_K (DequantizeQ6_K, Dequantizer.cs:378-417): lane L = 16 (g & 3) + n holds ql of
// group g (16 bytes, first or second KiB), qh of group g (8 bytes at 2048 + 16 L, +8 for g >= 4),
// the group's two scales (bytes 0-1 or 2-3 of the dword at 3072 + 4 L); d at 3328 + 2 n.
template <> struct PfW<FLLM_TYPE_Q6_K> {
    struct Raw { uint4 ql; uint2 qh; uint32_t s4, d; };
    __device__ static void load(Raw& w4, const uint8_t* __restrict__ w, int K, int r, int k0) {
        const int NB = K >> 8, kb = k0 >> 8, g = (k0 >> 5) & 7, n = r & 15, L = 16 * (g & 3) + n;
        const uint8_t* reg = w + ((size_t)(r >> 4) * NB + kb) * (16 * 210);
        w4.ql = *(const uint4*)(reg + (g < 4 ? 0 : 1024) + 16 * L);
        w4.qh = *(const uint2*)(reg + 2048 + 16 * L + (g < 4 ? 0 : 8));
        w4.s4 = *(const uint32_t*)(reg + 3072 + 4 * L);
        w4.d = *(const uint16_t*)(reg + 3328 + 2 * n);
    }
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v, float s = 1.0f) {
        const int g = (k0 >> 5) & 7;
        const uint32_t sc2 = g < 4 ? (w4.s4 & 0xFFFFu) : (w4.s4 >> 16);
        const float d = half_exact(w4.d) * s;
        const uint32_t l4[4] = {w4.ql.x, w4.ql.y, w4.ql.z, w4.ql.w}, h2[2] = {w4.qh.x, w4.qh.y};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t lb = (l4[i >> 3] >> (8 * ((i >> 1) & 3))) & 0xFFu;
            const int low = (i & 1) ? (int)(lb >> 4) : (int)(lb & 15u);
            const uint32_t hb = (h2[i >> 4] >> (8 * ((i >> 2) & 3))) & 0xFFu;
            const int high = (int)((hb >> (2 * (i & 3))) & 3u);
            const int q = ((high << 4) | low) - 32;
            const int scale = (int)(int8_t)((sc2 >> (8 * (i >> 4))) & 0xFFu);
            v[i] = d * (float)scale * (float)q;
        }
    }
};

// LAYOUT_TILES Q8_0: block g & 3 (+4) of the row's chunk; its 32 int8 as two 16-byte pieces in
// element order 4 by + j at byte 4 j + by; d of blocks q and q + 4 in one dword at 4096 + 16 n + 4 q
template <> struct PfW<FLLM_TYPE_Q8_0> {
    struct Raw { uint4 h0, h1; uint32_t d; };
    __device__ static void load(Raw& w4, const uint8_t* __restrict__ w, int K, int r, int k0) {
        const int NB = K >> 8, kb = k0 >> 8, g = (k0 >> 5) & 7, n = r & 15, q = g & 3, L = 16 * q + n;
        const uint8_t* reg = w + ((size_t)(r >> 4) * NB + kb) * (16 * 272);
        const uint8_t* base = reg + (g < 4 ? 0 : 2048) + 16 * L;
        w4.h0 = *(const uint4*)base;
        w4.h1 = *(const uint4*)(base + 1024);
        w4.d = *(const uint32_t*)(reg + 4096 + 16 * n + 4 * q);
    }
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v, float s = 1.0f) {
        const int g = (k0 >> 5) & 7;
        const float d = half_exact(g < 4 ? (w4.d & 0xFFFFu) : (w4.d >> 16)) * s;
        const uint32_t hw[8] = {w4.h0.x, w4.h0.y, w4.h0.z, w4.h0.w, w4.h1.x, w4.h1.y, w4.h1.z, w4.h1.w};
#pragma unroll
        for (int e = 0; e < 32; e++) {
            const int h = e >> 4, ee = e & 15, j = ee & 3, by = ee >> 2;  // byte 4 j + by of half h
            v[e] = (float)(int8_t)((hw[4 * h + j] >> (8 * by)) & 0xFFu) * d;
        }
    }
};

// LAYOUT_TILES Q5_K: low nibbles as Q4_K, the group's regrouped high bits (bit 8 by + 4 h + j =
// element 16 h + 4 by + j) in the dword at 2048 + 8 L (+4 for g >= 4), header at 2560 + 16 n
template <> struct PfW<FLLM_TYPE_Q5_K> {
    struct Raw { uint4 qs, hdr; uint32_t h; };
    __device__ static void load(Raw& w4, const uint8_t* __restrict__ w, int K, int r, int k0) {
        const int NB = K >> 8, kb = k0 >> 8, g = (k0 >> 5) & 7, n = r & 15, L = 16 * (g & 3) + n;
        const uint8_t* reg = w + ((size_t)(r >> 4) * NB + kb) * (16 * 176);
        w4.qs = *(const uint4*)(reg + (g < 4 ? 0 : 1024) + 16 * L);
        w4.h = *(const uint32_t*)(reg + 2048 + 8 * L + (g < 4 ? 0 : 4));
        w4.hdr = *(const uint4*)(reg + 2560 + 16 * n);
    }
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v, float s = 1.0f) {
        const int g = (k0 >> 5) & 7;
        const float d = half_exact(w4.hdr.x & 0xFFFFu), dmin = half_exact(w4.hdr.x >> 16);
        int sc, mn;
        if (g < 4) {
            sc = (int)(PfW<FLLM_TYPE_Q4_K>::hbyte(w4.hdr, 4 + g) & 63u);
            mn = (int)(PfW<FLLM_TYPE_Q4_K>::hbyte(w4.hdr, 8 + g) & 63u);
        } else {
            const uint32_t b = PfW<FLLM_TYPE_Q4_K>::hbyte(w4.hdr, 8 + g), lo = PfW<FLLM_TYPE_Q4_K>::hbyte(w4.hdr, g),
                           hi = PfW<FLLM_TYPE_Q4_K>::hbyte(w4.hdr, 4 + g);
            sc = (int)((b & 15u) | ((lo >> 6) << 4));
            mn = (int)((b >> 4) | ((hi >> 6) << 4));
        }
        // a power-of-two scale s commutes with the roundings: (dg s) q - mg s = s (dg q - mg) exactly
        const float dg = d * (float)sc * s;
        const float mg = dmin * (float)mn * s;
        const uint32_t wd[4] = {w4.qs.x, w4.qs.y, w4.qs.z, w4.qs.w};
#pragma unroll
        for (int e = 0; e < 32; e++) {
            const uint32_t byte = (wd[e >> 3] >> (8 * ((e >> 1) & 3))) & 0xFFu;
            const int lo = (e & 1) ? (int)(byte >> 4) : (int)(byte & 15u);
            const int hi = (int)((w4.h >> (8 * ((e >> 2) & 3) + 4 * (e >> 4) + (e & 3))) & 1u);
            v[e] = dg * (float)((hi << 4) | lo) - mg;
        }
    }
};

// GGUF rows: elements e0 = r * K + k0 .. e0 + 31 of the flat block stream (K % 32 == 0, so the
// group lies in one block of every format), decoded from memory when staged. PF_ROWS + type: one
// decoder per format with the block header read once per group; PfW<-1> is element-wise for the
// remaining types.
constexpr int PF_ROWS = 100;

template <> struct PfW<-1> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int type, int K, int r, int k0, float* v, float s = 1.0f) {
        const int64_t e0 = (int64_t)r * K + k0;
        for (int i = 0; i < 32; i++) v[i] = deq_elem(type, w, e0 + i) * s;
    }
};

// Q8_0 (Dequantizer.cs:203-231): (sbyte)q * d, one 34-byte block per group
template <> struct PfW<PF_ROWS + FLLM_TYPE_Q8_0> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const uint8_t* p = w + (((int64_t)r * K + k0) >> 5) * 34;
        const float d = half_exact(deq_ld_u16(p)) * s;
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = (float)(int8_t)p[2 + i] * d;
    }
};

// Q4_0 (Dequantizer.cs:155-185): (nibble - 8) * d, low nibbles are elements 0..15
template <> struct PfW<PF_ROWS + FLLM_TYPE_Q4_0> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const uint8_t* p = w + (((int64_t)r * K + k0) >> 5) * 18;
        const float d = half_exact(deq_ld_u16(p)) * s;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t b = p[2 + j];
            v[j] = (float)((int)(b & 15u) - 8) * d;
            v[16 + j] = (float)((int)(b >> 4) - 8) * d;
        }
    }
};

// Q4_K (Dequantizer.cs:251-294) in GGUF rows
template <> struct PfW<PF_ROWS + FLLM_TYPE_Q4_K> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const int64_t e0 = (int64_t)r * K + k0;
        const uint8_t* p = w + (e0 >> 8) * 144;
        const int g = (int)((e0 & 255) >> 5);
        const float d = half_exact(deq_ld_u16(p)), dmin = half_exact(deq_ld_u16(p + 2));
        int sc, mn;
        kscale_min(p + 4, g, sc, mn);
        // a power-of-two scale s commutes with the roundings: (dg s) q - mg s = s (dg q - mg) exactly
        const float dg = d * (float)sc * s;
        const float mg = dmin * (float)mn * s;
        const uint8_t* qs = p + 16 + 16 * g;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t b = qs[j];
            v[2 * j] = dg * (float)(int)(b & 15u) - mg;
            v[2 * j + 1] = dg * (float)(int)(b >> 4) - mg;
        }
    }
};

// Q5_K (Dequantizer.cs:316-368): low nibble from qs, bit 4 from qh[t >> 3] bit (t & 7)
template <> struct PfW<PF_ROWS + FLLM_TYPE_Q5_K> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const int64_t e0 = (int64_t)r * K + k0;
        const uint8_t* p = w + (e0 >> 8) * 176;
        const int t0 = (int)(e0 & 255), g = t0 >> 5;
        const float d = half_exact(deq_ld_u16(p)), dmin = half_exact(deq_ld_u16(p + 2));
        int sc, mn;
        kscale_min(p + 4, g, sc, mn);
        // a power-of-two scale s commutes with the roundings: (dg s) q - mg s = s (dg q - mg) exactly
        const float dg = d * (float)sc * s;
        const float mg = dmin * (float)mn * s;
        const uint32_t qh = deq_ld_u32(p + 16 + (t0 >> 3));  // bits of elements t0 .. t0 + 31
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t b = p[48 + (t0 >> 1) + j];
            const int lo0 = (int)(b & 15u), lo1 = (int)(b >> 4);
            const int hi0 = (int)((qh >> (2 * j)) & 1u), hi1 = (int)((qh >> (2 * j + 1)) & 1u);
            v[2 * j] = dg * (float)((hi0 << 4) | lo0) - mg;
            v[2 * j + 1] = dg * (float)((hi1 << 4) | lo1) - mg;
        }
    }
};

// Q6_K (Dequantizer.cs:378-417) in GGUF rows
template <> struct PfW<PF_ROWS + FLLM_TYPE_Q6_K> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const int64_t e0 = (int64_t)r * K + k0;
        const uint8_t* p = w + (e0 >> 8) * 210;
        const int i0 = (int)(e0 & 255);
        const float d = half_exact(deq_ld_u16(p + 208)) * s;
        const uint32_t qh = deq_ld_u32(p + 128 + (i0 >> 2));
        const uint32_t qh2 = deq_ld_u32(p + 128 + (i0 >> 2) + 4);
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const int i = i0 + j;
            const uint32_t lb = p[i >> 1];
            const int low = (j & 1) ? (int)(lb >> 4) : (int)(lb & 15u);
            const uint32_t hw = j < 16 ? qh : qh2;
            const int high = (int)((hw >> (2 * (j & 15))) & 3u);
            const int q = ((high << 4) | low) - 32;
            const int scale = (int)(int8_t)p[192 + (i >> 4)];
            v[j] = d * (float)scale * (float)q;
        }
    }
};

// F16 / BF16 / F32 rows: exact widening (Dequantizer.cs:68-137)
template <> struct PfW<PF_ROWS + FLLM_TYPE_F32> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const uint8_t* p = w + ((int64_t)r * K + k0) * 4;
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = bits_f32(deq_ld_u32(p + 4 * i)) * s;
    }
};
template <> struct PfW<PF_ROWS + FLLM_TYPE_F16> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const uint8_t* p = w + ((int64_t)r * K + k0) * 2;
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = half_exact(deq_ld_u16(p + 2 * i)) * s;
    }
};
template <> struct PfW<PF_ROWS + FLLM_TYPE_BF16> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v, float s = 1.0f) {
        const uint8_t* p = w + ((int64_t)r * K + k0) * 2;
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = bf16_exact(deq_ld_u16(p + 2 * i)) * s;
    }
};

// ---- GEMM ---------------------------------------------------------------------------------------
// Workgroup tile: BM tokens (64 in every launch) x 128 weight rows, 4 waves in a 2 x 2 arrangement, each
// (BM / 2) x 64 (BM / 32 x 4 MFMA tiles of 16 x 16). Per K step of 64 the workgroup stages X and the
// decoded weights into LDS.
constexpr int PF_BN = 128, PF_BK = 64;

// workgroup (x, y): column tile x of the launch's segments, token tile y
__device__ __forceinline__ int pf_seg_of(const PfGemm& a, int& bx) {
    int si = 0;
    while (si + 1 < a.nseg && bx >= a.seg[si].tiles) {
        bx -= a.seg[si].tiles;
        si++;
    }
    return si;
}

// ---- fp16 form ----------------------------------------------------------------------------------
// LDS rows of PF_BK halves plus 32 bytes; X and W as [plane][row][k] with plane 0 = hi, 1 = lo.
// A 128-bit LDS read on gfx950 is served for lanes 0-31 and 32-63 apart, over 128 banks of 4 bytes:
// an operand read (16 rows x two 16-byte columns per half-wave) is conflict-free when the row
// stride is 40 dwords (the 16 rows' 32-byte spans tile the 128 banks); at 36 dwords, rows r and
// r + 7 share banks and every such read took two passes.
constexpr int PF_LDH = PF_BK + 16;
typedef _Float16 pf_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 pf_hv2 __attribute__((ext_vector_type(2)));

template <int BM>
static constexpr size_t pf_gemm_lds_h() {
    return sizeof(_Float16) * 2 * (size_t)(BM + PF_BN) * PF_LDH;
}

// hi / lo halves of 8 scaled values, two at a time with the packed round-toward-zero conversion:
// hi keeps 11 bits of each value, lo the remainder (exact in f32) to 11 bits
typedef __fp16 pf_h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void pf_split8(const float* v, uint4& hi, uint4& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const pf_h2 hh = __builtin_amdgcn_cvt_pkrtz(v[2 * u], v[2 * u + 1]);
        const pf_h2 ll = __builtin_amdgcn_cvt_pkrtz(v[2 * u] - (float)hh[0], v[2 * u + 1] - (float)hh[1]);
        h[u] = __builtin_bit_cast(uint32_t, hh);
        l[u] = __builtin_bit_cast(uint32_t, ll);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// Same tile as pf_gemm_tile: BM tokens x 128 weight rows, 4 waves of (BM / 2) x 64, K steps of 64.
// MFMA 16x16x32 f16: lane l supplies row (l & 15) of the A (tokens) and B (weight rows) tiles with
// k = 8 (l >> 4) .. + 7 of a 32-wide slice, one 16-byte LDS read per operand and plane; D lane l holds
// rows 4 (l >> 4) .. + 3 of column l & 15.
template <int WT, int BM>
__device__ __forceinline__ void pf_gemm_tile_h(const PfGemm& a, const PfSeg& sg, int n0, int t0, _Float16* sx,
                                               _Float16* sw) {
    constexpr int WM = BM / 2;   // tokens per wave
    constexpr int TI = WM / 16;  // MFMA tiles along the tokens
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    pf_f32x4 acc[TI][4];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // X: per K step BM rows x 64 halves x 2 planes = BM * 16 pieces of 8 halves; piece c = tid + 256 i
    // is plane c / (8 BM), row (c % (8 BM)) / 8, halves 8 (c % 8) .. + 7. W: group wgrp of row wrow
    constexpr int XP = BM * 16 / 256;
    const size_t plane = (size_t)a.T * a.ldh;
    const int wrow = tid & (PF_BN - 1), wgrp = tid / PF_BN, wr = n0 + wrow;
    const bool wlive = wr < sg.N;
    const float wsc = ldexpf(1.0f, -sg.wexp);
    using Raw = typename PfW<WT>::Raw;
    uint4 xr[XP];
    Raw wraw;
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XP; i++) {
            const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM), row = rem >> 3, t = t0 + row;
            const int k = k0 + (rem & 7) * 8;
            xr[i] = (t < a.T && k < a.K) ? *(const uint4*)(a.xh + pl * plane + (size_t)t * a.ldh + k)
                                         : make_uint4(0u, 0u, 0u, 0u);
        }
        if (wlive && k0 + 32 * wgrp < a.K) PfW<WT>::load(wraw, sg.w, a.K, wr, k0 + 32 * wgrp);
    };
    const int kb = (int)blockIdx.z * a.kpart, ke = kb + a.kpart < a.K ? kb + a.kpart : a.K;
    fetch(kb);
    for (int k0 = kb; k0 < ke; k0 += PF_BK) {
        __syncthreads();  // the previous step's operands have been read
#pragma unroll
        for (int i = 0; i < XP; i++) {
            const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM);
            *(uint4*)(sx + ((size_t)pl * BM + (rem >> 3)) * PF_LDH + (rem & 7) * 8) = xr[i];
        }
        if constexpr (WT == FLLM_TYPE_Q8_0) {
            // exact-integer form: the int8 code q as an fp16 integer (its byte as 0x64 80 ^ byte =
            // 1024 + 128 + q, minus 1152) in the weight plane, and the block's d' = d 2^-wexp (f32,
            // exact) beside it; the products sum x hi q + x lo q per 32-element block and the block
            // sum is added times d' in f32. Element 16 hh + 4 by + j is byte by of dword j of half hh,
            // so a pair (e, e + 1) takes byte by of dwords j and j + 1.
            const int k = k0 + 32 * wgrp;
            uint32_t qv[16];
            float dq = 0.0f;
            if (wlive && k < a.K) {
                const int g = (k >> 5) & 7;
                dq = half_exact(g < 4 ? (wraw.d & 0xFFFFu) : (wraw.d >> 16)) * wsc;
                const pf_hv2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
                const uint32_t wd[8] = {wraw.h0.x, wraw.h0.y, wraw.h0.z, wraw.h0.w, wraw.h1.x, wraw.h1.y, wraw.h1.z, wraw.h1.w};
#pragma unroll
                for (int pr = 0; pr < 16; pr++) {
                    const int e = 2 * pr, hh = e >> 4, by = (e & 15) >> 2, j = e & 3;
                    const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + by) << 16) | (uint32_t)by;
                    const uint32_t p = __builtin_amdgcn_perm(wd[4 * hh + j + 1], wd[4 * hh + j], sel) ^ 0x64806480u;
                    qv[pr] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(pf_hv2, p) + off);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) qv[i] = 0u;
            }
            _Float16* d0 = sw + (size_t)wrow * PF_LDH + 32 * wgrp;
#pragma unroll
            for (int i = 0; i < 4; i++)
                *(uint4*)(d0 + 8 * i) = make_uint4(qv[4 * i], qv[4 * i + 1], qv[4 * i + 2], qv[4 * i + 3]);
            // the block scales in the second weight plane, which this form leaves free
            ((float*)(sw + (size_t)PF_BN * PF_LDH))[wgrp * PF_BN + wrow] = dq;
        } else {
            float v[32];
            const int k = k0 + 32 * wgrp;
            if (wlive && k < a.K) {
                PfW<WT>::deq(wraw, sg.w, sg.type, a.K, wr, k, v, wsc);
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) v[i] = 0.0f;
            }
            _Float16* d0 = sw + (size_t)wrow * PF_LDH + 32 * wgrp;
            _Float16* d1 = d0 + (size_t)PF_BN * PF_LDH;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint4 hi, lo;
                pf_split8(v + 8 * i, hi, lo);
                *(uint4*)(d0 + 8 * i) = hi;
                *(uint4*)(d1 + 8 * i) = lo;
            }
        }
        // the next step's global loads fly while this step multiplies
        if (k0 + PF_BK < ke) fetch(k0 + PF_BK);
        __syncthreads();
        if constexpr (WT == FLLM_TYPE_Q8_0) {
            const float* sdq = (const float*)(sw + (size_t)PF_BN * PF_LDH);
#pragma unroll
            for (int kk = 0; kk < PF_BK; kk += 32) {
                const int ko = kk + 8 * (lane >> 4);
                pf_h8 ah[TI], al[TI], bq[4];
                float dj[4];
#pragma unroll
                for (int i = 0; i < TI; i++) {
                    const _Float16* p = sx + (size_t)(WM * wm + 16 * i + (lane & 15)) * PF_LDH + ko;
                    ah[i] = *(const pf_h8*)p;
                    al[i] = *(const pf_h8*)(p + (size_t)BM * PF_LDH);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int r = 64 * wn + 16 * j + (lane & 15);
                    bq[j] = *(const pf_h8*)(sw + (size_t)r * PF_LDH + ko);
                    dj[j] = sdq[(kk >> 5) * PF_BN + r];
                }
                // the block's sum (x lo q, then x hi q) over all tiles in turn, then its d' times it
                pf_f32x4 bs[TI][4];
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        bs[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bq[j], pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) bs[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bq[j], bs[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[i][j][e] = fmaf(dj[j], bs[i][j][e], acc[i][j][e]);
            }
        } else {
#pragma unroll
        for (int kk = 0; kk < PF_BK; kk += 32) {
            const int ko = kk + 8 * (lane >> 4);
            pf_h8 ah[TI], al[TI], bh[4], bl[4];
#pragma unroll
            for (int i = 0; i < TI; i++) {
                const _Float16* p = sx + (size_t)(WM * wm + 16 * i + (lane & 15)) * PF_LDH + ko;
                ah[i] = *(const pf_h8*)p;
                al[i] = *(const pf_h8*)(p + (size_t)BM * PF_LDH);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const _Float16* p = sw + (size_t)(64 * wn + 16 * j + (lane & 15)) * PF_LDH + ko;
                bh[j] = *(const pf_h8*)p;
                bl[j] = *(const pf_h8*)(p + (size_t)PF_BN * PF_LDH);
            }
            // the three products go over all tiles in turn, so consecutive MFMAs write different
            // accumulators
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
        }
        }
    }
    const float wun = ldexpf(1.0f, sg.wexp);
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = t0 + WM * wm + 16 * i + 4 * (lane >> 4) + e;
            if (t >= a.T) continue;
            const float f = a.xs[t] * wun;  // undoes both scales: exact
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = n0 + 64 * wn + 16 * j + (lane & 15);
                if (n >= sg.N) continue;
                const float r = acc[i][j][e] * f;
                if (blockIdx.z == 0) {
                    float* p = sg.y + (size_t)t * sg.ldy + n;
                    *p = a.add ? *p + r : r;
                } else {
                    const size_t col = (size_t)(sg.y - a.seg[0].y);
                    a.part[(size_t)(blockIdx.z - 1) * a.T * sg.ldy + (size_t)t * sg.ldy + col + n] = r;
                }
            }
        }
}

// ---- fp16 form, Q4_K -------------------------------------------------------------------------
// A Q4_K weight is dg q - mg with dg = d sc_g, mg = dmin m_g (Dequantizer.cs:251-294), so
//   sum_i w_i x_i = d sum_(g in block) sum_(i in g) (sc_g q_i) x_i - sum_g (dmin m_g) X_g,
// X_g the sum of group g's x. sc_g q_i <= 945 is an integer, exact in fp16: the weights need no split
// and a product is two MFMAs (x hi and x lo against the same weights). Every 256-element block's sum
// is scaled by its d in f32; the min term of a block is one more MFMA whose K slice packs, per row,
// (v_g hi, v_g lo, v_g hi) for v_g = -dmin m_g against, per token, (X_g hi, X_g hi, X_g lo), the
// three products of the two splits, added to the same accumulator. The group sums are stored times
// 2^-6 (to stay in fp16's range) and v_g taken times 2^6, so their products are unchanged.
// LDS row stride (halves) of a block's min-term slice: its three used 16-byte chunks (the fourth
// of the MFMA's K slice is zero and is not stored: the lanes that would read it take zeros)
constexpr int PF_LDV = 24;

template <int BM>
static constexpr size_t pf_gemm_lds_k() {
    return sizeof(_Float16) * ((size_t)(2 * BM + PF_BN) * PF_LDH + (size_t)(BM + PF_BN) * PF_LDV) + sizeof(float) * PF_BN;
}

// sc q_i for the 8 elements of one qs dword (bytes b = 0..3: element 2 b the low nibble, 2 b + 1 the
// high one), as 4 dwords of fp16 pairs: 1024 + q by setting the fp16 pattern 0x6400 | q, minus 1024,
// times sc, all exact
__device__ __forceinline__ void pf_q4_pairs(uint32_t x, pf_hv2 sc2, uint32_t* out) {
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    // (1024 + q) sc - 1024 sc in one fma: exact, the result sc q being an integer below 2048
    const pf_hv2 nb = sc2 * pf_hv2{(_Float16)-1024.0f, (_Float16)-1024.0f};
#pragma unroll
    for (int b = 0; b < 4; b++) {
        // bytes: low nibble of byte b, 0, high nibble of byte b, 0
        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
        const uint32_t p = __builtin_amdgcn_perm(hi, lo, sel) | 0x64006400u;
        const pf_hv2 v = __builtin_elementwise_fma(__builtin_bit_cast(pf_hv2, p), sc2, nb);
        out[b] = __builtin_bit_cast(uint32_t, v);
    }
}

// Q5_K: the same for 5-bit codes (sc q <= 63 * 31 < 2048, still exact). The group's regrouped
// high-bit dword h holds element 16 hf + 4 by + j at bit 8 by + 4 hf + j: the pair (2 b, 2 b + 1)
// of qs dword u has its high bits at bits p, p + 1 of the half (u & 1) of h, p = 8 (b >> 1) +
// 4 (u >> 1) + 2 (b & 1) < 15. With z = h16 | h16 << 15 for that 16-bit half, (z >> p) puts them at
// bits 0 and 16.
template <int U>
__device__ __forceinline__ void pf_q5_pairs(uint32_t x, uint32_t z, pf_hv2 sc2, uint32_t* out) {
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    const pf_hv2 nb = sc2 * pf_hv2{(_Float16)-1024.0f, (_Float16)-1024.0f};
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
        const int pos = 8 * (b >> 1) + 4 * (U >> 1) + 2 * (b & 1);
        const uint32_t t = (pos >= 4 ? (z >> (pos - 4)) : (z << (4 - pos))) & 0x00100010u;
        const uint32_t p = __builtin_amdgcn_perm(hi, lo, sel) | t | 0x64006400u;
        const pf_hv2 v = __builtin_elementwise_fma(__builtin_bit_cast(pf_hv2, p), sc2, nb);
        out[b] = __builtin_bit_cast(uint32_t, v);
    }
}

// WT: FLLM_TYPE_Q4_K or FLLM_TYPE_Q5_K (same header, scales and block structure)
template <int BM, int WT = FLLM_TYPE_Q4_K>
__device__ __forceinline__ void pf_gemm_tile_q4k(const PfGemm& a, const PfSeg& sg, int n0, int t0, _Float16* lds) {
    constexpr int WM = BM / 2, TI = WM / 16;
    _Float16* sx = lds;                                    // [2][BM][PF_LDH]
    _Float16* sw = sx + (size_t)2 * BM * PF_LDH;           // [PF_BN][PF_LDH]
    _Float16* sav = sw + (size_t)PF_BN * PF_LDH;           // [BM][PF_LDV]
    _Float16* swv = sav + (size_t)BM * PF_LDV;             // [PF_BN][PF_LDV]
    float* sd = (float*)(swv + (size_t)PF_BN * PF_LDV);    // [PF_BN]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    pf_f32x4 acc[TI][4], blk[TI][4];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = blk[i][j] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    constexpr int XP = BM * 16 / 256;
    const size_t plane = (size_t)a.T * a.ldh;
    const int G = a.K / 32;
    const _Float16* xg = a.xh + 2 * plane;  // group sums: hi plane, then lo plane
    const size_t gplane = (size_t)a.T * G;
    const int wrow = tid & (PF_BN - 1), wgrp = tid / PF_BN, wr = n0 + wrow;
    const bool wlive = wr < sg.N;
    // block-start extras: token row (tid >> 1) of the min-term slice, its hi (tid even) or lo group sums
    const int vt = tid >> 1, vhl = tid & 1;
    using Raw = typename PfW<WT>::Raw;
    uint4 xr[XP], xv = make_uint4(0u, 0u, 0u, 0u);
    Raw wraw;
    // a tile of BM whole token rows (uniform over the workgroup) loads without the row test
    const bool full = t0 + BM <= a.T;
    auto fetch = [&](int k0) {
        if (full) {
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM);
                xr[i] = *(const uint4*)(a.xh + pl * plane + (size_t)(t0 + (rem >> 3)) * a.ldh + k0 + (rem & 7) * 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM), t = t0 + (rem >> 3);
                xr[i] = t < a.T ? *(const uint4*)(a.xh + pl * plane + (size_t)t * a.ldh + k0 + (rem & 7) * 8)
                                : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        if ((k0 & 255) == 0 && vt < BM) {
            const int t = t0 + vt;
            xv = t < a.T ? *(const uint4*)(xg + vhl * gplane + (size_t)t * G + (k0 >> 5)) : make_uint4(0u, 0u, 0u, 0u);
        }
        if (wlive) PfW<WT>::load(wraw, sg.w, a.K, wr, k0 + 32 * wgrp);
    };
    // whole 256-element blocks (K and the split parts are multiples of 256): four K steps per block,
    // the block's end straight-line after them, so the accumulators stay in place across steps
    const int kb = (int)blockIdx.z * a.kpart, ke = kb + a.kpart < a.K ? kb + a.kpart : a.K;
    fetch(kb);
    for (int kblk = kb; kblk < ke; kblk += 256) {
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int k0 = kblk + st * PF_BK;
            __syncthreads();  // the previous step's operands have been read
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM);
                *(uint4*)(sx + ((size_t)pl * BM + (rem >> 3)) * PF_LDH + (rem & 7) * 8) = xr[i];
            }
            const int g = 2 * st + wgrp;
            {
                uint32_t out[16];
                if (wlive) {
                    int sc, mn;
                    PfW<FLLM_TYPE_Q4_K>::scale_min(wraw.hdr, g, sc, mn);
                    const _Float16 sch = (_Float16)(float)sc;
                    const pf_hv2 sc2 = {sch, sch};
                    if constexpr (WT == FLLM_TYPE_Q5_K) {
                        const uint32_t h0 = wraw.h & 0xFFFFu, h1 = wraw.h >> 16;
                        const uint32_t z0 = h0 | (h0 << 15), z1 = h1 | (h1 << 15);
                        pf_q5_pairs<0>(wraw.qs.x, z0, sc2, out);
                        pf_q5_pairs<1>(wraw.qs.y, z1, sc2, out + 4);
                        pf_q5_pairs<2>(wraw.qs.z, z0, sc2, out + 8);
                        pf_q5_pairs<3>(wraw.qs.w, z1, sc2, out + 12);
                    } else {
                        // the tile layout's dwords of a half: its bytes 0, 2, 4, 6 and 1, 3, 5, 7
                        // (element pairs 0, 2, 4, 6 and 1, 3, 5, 7 of the half)
                        uint32_t ev[4], od[4];
#pragma unroll
                        for (int hf = 0; hf < 2; hf++) {
                            pf_q4_pairs(hf ? wraw.qs.z : wraw.qs.x, sc2, ev);
                            pf_q4_pairs(hf ? wraw.qs.w : wraw.qs.y, sc2, od);
#pragma unroll
                            for (int b = 0; b < 4; b++) {
                                out[8 * hf + 2 * b] = ev[b];
                                out[8 * hf + 2 * b + 1] = od[b];
                            }
                        }
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++) out[i] = 0u;
                }
                uint4* dst = (uint4*)(sw + (size_t)wrow * PF_LDH + 32 * wgrp);
#pragma unroll
                for (int i = 0; i < 4; i++) dst[i] = make_uint4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
            }
            if (st == 0) {
                // the block's d and min-term slice of this row (v_g = -dmin m_g, exact in f32, split)
                if (wgrp == 0) {
                    const float d = wlive ? half_exact(wraw.hdr.x & 0xFFFFu) : 0.0f;
                    const float dmin = wlive ? half_exact(wraw.hdr.x >> 16) : 0.0f;
                    sd[wrow] = d;
                    uint32_t vh[4], vl[4];
#pragma unroll
                    for (int gg = 0; gg < 8; gg += 2) {
                        int sc0, mn0, sc1, mn1;
                        PfW<FLLM_TYPE_Q4_K>::scale_min(wraw.hdr, gg, sc0, mn0);
                        PfW<FLLM_TYPE_Q4_K>::scale_min(wraw.hdr, gg + 1, sc1, mn1);
                        const float v0 = wlive ? -(dmin * (float)mn0) * 64.0f : 0.0f;
                        const float v1 = wlive ? -(dmin * (float)mn1) * 64.0f : 0.0f;
                        const pf_h2 h = __builtin_amdgcn_cvt_pkrtz(v0, v1);
                        const pf_h2 l = __builtin_amdgcn_cvt_pkrtz(v0 - (float)h[0], v1 - (float)h[1]);
                        vh[gg >> 1] = __builtin_bit_cast(uint32_t, h);
                        vl[gg >> 1] = __builtin_bit_cast(uint32_t, l);
                    }
                    uint4* dv = (uint4*)(swv + (size_t)wrow * PF_LDV);
                    dv[0] = make_uint4(vh[0], vh[1], vh[2], vh[3]);
                    dv[1] = make_uint4(vl[0], vl[1], vl[2], vl[3]);
                    dv[2] = dv[0];
                }
                // tokens: (X hi, X hi, X lo, 0) against (v hi, v lo, v hi, 0)
                if (vt < BM) {
                    uint4* av = (uint4*)(sav + (size_t)vt * PF_LDV);
                    if (vhl == 0) {
                        av[0] = xv;
                        av[1] = xv;
                    } else {
                        av[2] = xv;
                    }
                }
            }
            if (k0 + PF_BK < ke) fetch(k0 + PF_BK);
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < PF_BK; kk += 32) {
                const int ko = kk + 8 * (lane >> 4);
                pf_h8 ah[TI], al[TI], bw[4];
#pragma unroll
                for (int i = 0; i < TI; i++) {
                    const _Float16* p = sx + (size_t)(WM * wm + 16 * i + (lane & 15)) * PF_LDH + ko;
                    ah[i] = *(const pf_h8*)p;
                    al[i] = *(const pf_h8*)(p + (size_t)BM * PF_LDH);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) bw[j] = *(const pf_h8*)(sw + (size_t)(64 * wn + 16 * j + (lane & 15)) * PF_LDH + ko);
                // the block's first product starts its sum from zero
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            al[i], bw[j], (st == 0 && kk == 0) ? pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f} : blk[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bw[j], blk[i][j], 0, 0, 0);
            }
        }
        // the block's d times its sum, and its min term (sd / sav / swv were written at the block's
        // first step and are rewritten only after the next block's first barrier)
        const int ko = 8 * (lane >> 4);
        const bool kz = (lane >> 4) == 3;  // the slice's fourth chunk: zeros
        const pf_h8 z8 = {};
        pf_h8 av[TI], bv[4];
#pragma unroll
        for (int i = 0; i < TI; i++)
            av[i] = kz ? z8 : *(const pf_h8*)(sav + (size_t)(WM * wm + 16 * i + (lane & 15)) * PF_LDV + (kz ? 0 : ko));
#pragma unroll
        for (int j = 0; j < 4; j++)
            bv[j] = kz ? z8 : *(const pf_h8*)(swv + (size_t)(64 * wn + 16 * j + (lane & 15)) * PF_LDV + (kz ? 0 : ko));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float d = sd[64 * wn + 16 * j + (lane & 15)];
#pragma unroll
            for (int i = 0; i < TI; i++) {
#pragma unroll
                for (int e = 0; e < 4; e++) acc[i][j][e] = fmaf(d, blk[i][j][e], acc[i][j][e]);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = t0 + WM * wm + 16 * i + 4 * (lane >> 4) + e;
            if (t >= a.T) continue;
            const float f = a.xs[t];  // undoes the activations' scale: exact
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = n0 + 64 * wn + 16 * j + (lane & 15);
                if (n >= sg.N) continue;
                const float r = acc[i][j][e] * f;
                if (blockIdx.z == 0) {
                    float* p = sg.y + (size_t)t * sg.ldy + n;
                    *p = a.add ? *p + r : r;
                } else {
                    const size_t col = (size_t)(sg.y - a.seg[0].y);
                    a.part[(size_t)(blockIdx.z - 1) * a.T * sg.ldy + (size_t)t * sg.ldy + col + n] = r;
                }
            }
        }
}

// ---- fp16 form, Q6_K --------------------------------------------------------------------------
// A Q6_K weight is d (sc q) with q = v - 32 (v the 6-bit code) and sc the int8 scale of its 16
// elements (Dequantizer.cs:378-417). I = sc q is an integer of magnitude at most 4096: hi = fp16(I)
// (exact up to 2048, even integers above) and lo = I - hi (0 or +-1) hold it exactly. A block's sum
// is x hi * I hi + x lo * I hi + x hi * I lo (the dropped x lo * I lo is below 2^-22 of a product),
// accumulated apart and added times the block's d in f32 at its end. The weights need no matrix
// scale: the epilogue only undoes the activations' power of two.
template <int BM>
static constexpr size_t pf_gemm_lds_q6() {
    return sizeof(_Float16) * (size_t)(2 * BM + 2 * PF_BN) * PF_LDH + sizeof(float) * PF_BN;
}

// the 8 elements of ql dword x (element 2 b: low nibble of byte b, 2 b + 1: high nibble) with their
// high bits (element j: bits 2 j, 2 j + 1 of h16), scale pair sc2: hi and lo halves of sc q as 4
// fp16 pairs each. A pair's code v goes into fp16 1024 + v (nibble at bits 0-3, high bits at 4-5 of
// each half, pattern 0x6400), minus 1056 gives q exactly.
__device__ __forceinline__ void pf_q6_pairs(uint32_t x, uint32_t h16, pf_hv2 sc2, uint32_t* hi, uint32_t* lo) {
    const uint32_t nl = x & 0x0F0F0F0Fu, nh = (x >> 4) & 0x0F0F0F0Fu;
    // y >> 4 b: bits 0-1 the high bits of element 2 b, bits 16-17 those of element 2 b + 1
    const uint32_t y = h16 | (h16 << 14);
    const pf_hv2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
        const uint32_t t = (b == 0 ? (y << 4) : (y >> (4 * b - 4))) & 0x00300030u;
        const uint32_t p = __builtin_amdgcn_perm(nh, nl, sel) | t | 0x64006400u;
        const pf_hv2 q = __builtin_bit_cast(pf_hv2, p) + off;
        const pf_hv2 vh = q * sc2;
        const pf_hv2 vl = __builtin_elementwise_fma(q, sc2, -vh);
        hi[b] = __builtin_bit_cast(uint32_t, vh);
        lo[b] = __builtin_bit_cast(uint32_t, vl);
    }
}

// Same tile and step structure as pf_gemm_tile_q4k (whole 256-element blocks, four K steps each);
// the weights go into LDS as hi / lo planes.
template <int BM>
__device__ __forceinline__ void pf_gemm_tile_q6k(const PfGemm& a, const PfSeg& sg, int n0, int t0, _Float16* lds) {
    constexpr int WM = BM / 2, TI = WM / 16;
    _Float16* sx = lds;                                    // [2][BM][PF_LDH]
    _Float16* sw = sx + (size_t)2 * BM * PF_LDH;           // [2][PF_BN][PF_LDH]
    float* sd = (float*)(sw + (size_t)2 * PF_BN * PF_LDH);  // [PF_BN]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    pf_f32x4 acc[TI][4], blk[TI][4];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = blk[i][j] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    constexpr int XP = BM * 16 / 256;
    const size_t plane = (size_t)a.T * a.ldh;
    const int wrow = tid & (PF_BN - 1), wgrp = tid / PF_BN, wr = n0 + wrow;
    const bool wlive = wr < sg.N;
    using Raw = typename PfW<FLLM_TYPE_Q6_K>::Raw;
    uint4 xr[XP];
    Raw wraw;
    const bool full = t0 + BM <= a.T;
    auto fetch = [&](int k0) {
        if (full) {
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM);
                xr[i] = *(const uint4*)(a.xh + pl * plane + (size_t)(t0 + (rem >> 3)) * a.ldh + k0 + (rem & 7) * 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM), t = t0 + (rem >> 3);
                xr[i] = t < a.T ? *(const uint4*)(a.xh + pl * plane + (size_t)t * a.ldh + k0 + (rem & 7) * 8)
                                : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        if (wlive) PfW<FLLM_TYPE_Q6_K>::load(wraw, sg.w, a.K, wr, k0 + 32 * wgrp);
    };
    const int kb = (int)blockIdx.z * a.kpart, ke = kb + a.kpart < a.K ? kb + a.kpart : a.K;
    fetch(kb);
    for (int kblk = kb; kblk < ke; kblk += 256) {
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int k0 = kblk + st * PF_BK;
            __syncthreads();  // the previous step's operands have been read
#pragma unroll
            for (int i = 0; i < XP; i++) {
                const int c = tid + 256 * i, pl = c / (8 * BM), rem = c % (8 * BM);
                *(uint4*)(sx + ((size_t)pl * BM + (rem >> 3)) * PF_LDH + (rem & 7) * 8) = xr[i];
            }
            const int g = 2 * st + wgrp;
            {
                uint32_t hv[16], lv[16];
                if (wlive) {
                    const uint32_t sc = g < 4 ? (wraw.s4 & 0xFFFFu) : (wraw.s4 >> 16);
                    const pf_hv2 sa = {(_Float16)(float)(int)(int8_t)(sc & 0xFFu), (_Float16)(float)(int)(int8_t)(sc & 0xFFu)};
                    const pf_hv2 sb = {(_Float16)(float)(int)(int8_t)(sc >> 8), (_Float16)(float)(int)(int8_t)(sc >> 8)};
                    pf_q6_pairs(wraw.ql.x, wraw.qh.x & 0xFFFFu, sa, hv, lv);
                    pf_q6_pairs(wraw.ql.y, wraw.qh.x >> 16, sa, hv + 4, lv + 4);
                    pf_q6_pairs(wraw.ql.z, wraw.qh.y & 0xFFFFu, sb, hv + 8, lv + 8);
                    pf_q6_pairs(wraw.ql.w, wraw.qh.y >> 16, sb, hv + 12, lv + 12);
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++) hv[i] = lv[i] = 0u;
                }
                uint4* dh = (uint4*)(sw + (size_t)wrow * PF_LDH + 32 * wgrp);
                uint4* dl = (uint4*)(sw + (size_t)(PF_BN + wrow) * PF_LDH + 32 * wgrp);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    dh[i] = make_uint4(hv[4 * i], hv[4 * i + 1], hv[4 * i + 2], hv[4 * i + 3]);
                    dl[i] = make_uint4(lv[4 * i], lv[4 * i + 1], lv[4 * i + 2], lv[4 * i + 3]);
                }
            }
            if (st == 0 && wgrp == 0) sd[wrow] = wlive ? half_exact(wraw.d & 0xFFFFu) : 0.0f;
            if (k0 + PF_BK < ke) fetch(k0 + PF_BK);
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < PF_BK; kk += 32) {
                const int ko = kk + 8 * (lane >> 4);
                pf_h8 ah[TI], al[TI], bh[4], bl[4];
#pragma unroll
                for (int i = 0; i < TI; i++) {
                    const _Float16* p = sx + (size_t)(WM * wm + 16 * i + (lane & 15)) * PF_LDH + ko;
                    ah[i] = *(const pf_h8*)p;
                    al[i] = *(const pf_h8*)(p + (size_t)BM * PF_LDH);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const _Float16* p = sw + (size_t)(64 * wn + 16 * j + (lane & 15)) * PF_LDH + ko;
                    bh[j] = *(const pf_h8*)p;
                    bl[j] = *(const pf_h8*)(p + (size_t)PF_BN * PF_LDH);
                }
                // the block's first product starts its sum from zero
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            al[i], bh[j], (st == 0 && kk == 0) ? pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f} : blk[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl[j], blk[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) blk[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh[j], blk[i][j], 0, 0, 0);
            }
        }
        // the block's d times its sum (sd was written at the block's first step and is rewritten only
        // after the next block's first barrier)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float d = sd[64 * wn + 16 * j + (lane & 15)];
#pragma unroll
            for (int i = 0; i < TI; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[i][j][e] = fmaf(d, blk[i][j][e], acc[i][j][e]);
        }
    }
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int t = t0 + WM * wm + 16 * i + 4 * (lane >> 4) + e;
            if (t >= a.T) continue;
            const float f = a.xs[t];  // undoes the activations' scale: exact
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = n0 + 64 * wn + 16 * j + (lane & 15);
                if (n >= sg.N) continue;
                const float r = acc[i][j][e] * f;
                if (blockIdx.z == 0) {
                    float* p = sg.y + (size_t)t * sg.ldy + n;
                    *p = a.add ? *p + r : r;
                } else {
                    const size_t col = (size_t)(sg.y - a.seg[0].y);
                    a.part[(size_t)(blockIdx.z - 1) * a.T * sg.ldy + (size_t)t * sg.ldy + col + n] = r;
                }
            }
        }
}

// launches whose segments are all tile-interleaved Q6_K
template <int BM>
__global__ __launch_bounds__(256) void k_pf_gemm_q6k(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_ld6[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    pf_gemm_tile_q6k<BM>(a, a.seg[si], bx * PF_BN, blockIdx.y * BM, pf_ld6);
}

// launches of tile-interleaved Q4_K and Q6_K segments (q, k in Q4_K, v in Q6_K): each workgroup
// takes its segment's form
template <int BM>
__global__ __launch_bounds__(256) void k_pf_gemm_q46(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_ld46[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    const PfSeg& sg = a.seg[si];
    if (sg.type == FLLM_TYPE_Q6_K)
        pf_gemm_tile_q6k<BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_ld46);
    else
        pf_gemm_tile_q4k<BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_ld46);
}

template <int BM>
__global__ __launch_bounds__(256) void k_pf_gemm_tiles_h(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_ldh[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    const PfSeg& sg = a.seg[si];
    _Float16* sw = pf_ldh + (size_t)2 * BM * PF_LDH;
    if (sg.type == FLLM_TYPE_Q6_K)
        pf_gemm_tile_h<FLLM_TYPE_Q6_K, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_ldh, sw);
    else if (sg.type == FLLM_TYPE_Q8_0)
        pf_gemm_tile_h<FLLM_TYPE_Q8_0, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_ldh, sw);
    else if (sg.type == FLLM_TYPE_Q5_K)
        pf_gemm_tile_h<FLLM_TYPE_Q5_K, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_ldh, sw);
    else
        pf_gemm_tile_h<FLLM_TYPE_Q4_K, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_ldh, sw);
}

// launches whose segments are all tile-interleaved Q8_0: the exact-integer Q8_0 form uses one weight
// plane plus the block scales (pf_gemm_lds_q8 bytes instead of pf_gemm_lds_h), so three workgroups
// share a CU
template <int BM>
static constexpr size_t pf_gemm_lds_q8() {
    return sizeof(_Float16) * (size_t)(2 * BM + PF_BN) * PF_LDH + sizeof(float) * 2 * PF_BN;
}
template <int BM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_pf_gemm_q8t(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_ld8[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    pf_gemm_tile_h<FLLM_TYPE_Q8_0, BM>(a, a.seg[si], bx * PF_BN, blockIdx.y * BM, pf_ld8, pf_ld8 + (size_t)2 * BM * PF_LDH);
}

// launches whose segments are all tile-interleaved Q5_K
template <int BM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BM == 64 ? 3 : 1))) void k_pf_gemm_q5k(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_ld5[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    pf_gemm_tile_q4k<BM, FLLM_TYPE_Q5_K>(a, a.seg[si], bx * PF_BN, blockIdx.y * BM, pf_ld5);
}

// launches whose segments are all tile-interleaved Q4_K
template <int BM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BM == 64 ? 3 : 1))) void k_pf_gemm_q4k(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_ldk[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    pf_gemm_tile_q4k<BM>(a, a.seg[si], bx * PF_BN, blockIdx.y * BM, pf_ldk);
}

template <int BM, int RT>
__global__ __launch_bounds__(256) void k_pf_gemm_rows_h(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) _Float16 pf_ldh[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    pf_gemm_tile_h<RT, BM>(a, a.seg[si], bx * PF_BN, blockIdx.y * BM, pf_ldh, pf_ldh + (size_t)2 * BM * PF_LDH);
}

// row t of X: the power of two bringing its largest magnitude into [2^14, 2^15), then the hi / lo
// halves of the scaled values (K a multiple of 32, ldx and ldh multiples of 4), and the hi / lo halves
// of every 32-element group's sum of the scaled values (planes of K / 32 per row after the two value
// planes: hi at 2 T ldh + t K / 32, lo T K / 32 further)
__global__ __launch_bounds__(256) void k_pf_split(const float* __restrict__ x, int ldx, int K, _Float16* __restrict__ xh,
                                                  int ldh, size_t plane, float* __restrict__ xs, int T) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    const float4* xr = (const float4*)(x + (size_t)t * ldx);
    float m = 0.0f;
    for (int i = threadIdx.x; i < K / 4; i += 256) {
        const float4 v = xr[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    m = pf_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (m > 0.0f && m <= 3.0e38f) {
        int ex;
        (void)frexpf(m, &ex);  // m in [2^(ex-1), 2^ex)
        e = 15 - ex;
        e = e < -120 ? -120 : (e > 120 ? 120 : e);
    }
    const float sc = ldexpf(1.0f, e);
    _Float16* h = xh + (size_t)t * ldh;
    for (int i = threadIdx.x; i < K / 4; i += 256) {
        const float4 v = xr[i];
        const float c[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            hi[u] = (_Float16)c[u];
            lo[u] = (_Float16)(c[u] - (float)hi[u]);
        }
        *(uint2*)(h + 4 * i) = *(const uint2*)hi;
        *(uint2*)(h + plane + 4 * i) = *(const uint2*)lo;
    }
    // group sums: 8 lanes of 4 elements per 32-element group, summed in a fixed order
    const int G = K / 32;
    _Float16* gs = xh + 2 * plane + (size_t)t * G;
    const size_t gplane = (size_t)T * G;
    for (int g0 = 0; g0 < G; g0 += 32) {
        const int g = g0 + (threadIdx.x >> 3), sub = threadIdx.x & 7;
        float v = 0.0f;
        if (g < G) {
            const float4 q = xr[g * 8 + sub];
            v = ((q.x * sc + q.y * sc) + (q.z * sc + q.w * sc));
        }
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        v += __shfl_xor(v, 4);
        if (g < G && sub == 0) {
            // times 2^-6 (exact): 32 values of magnitude below 2^15 sum below 2^20, past fp16's range
            v *= 0.015625f;
            const _Float16 hi = (_Float16)v;
            gs[g] = hi;
            gs[gplane + g] = (_Float16)(v - (float)hi);
        }
    }
    if (threadIdx.x == 0) xs[t] = ldexpf(1.0f, -e);
}

hipError_t launch_pf_split(const float* x, int ldx, int T, int K, _Float16* xh, int ldh, float* xs, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    if (K % 32 != 0 || ldx % 4 != 0 || ldh % 8 != 0 || ldh < K) return hipErrorInvalidValue;
    k_pf_split<<<T, 256, 0, st>>>(x, ldx, K, xh, ldh, (size_t)T * ldh, xs, T);
    return hipGetLastError();
}

// The split of a row computed here rather than read: SRC 1, RmsNorm / GemmaRmsNorm (kind 1) of row
// t of x (row stride ldx, weights w), k_pf_norm's arithmetic per element; SRC 2, act(gate) * up of row
// t of gu (gate in columns [0, K), up in [K, 2 K) of a row of stride ldx), k_pf_act's. The row stays
// in registers (NPT float4 per thread: element 4 i .. 4 i + 3 with i = thread + 256 j), so the
// normalized or gated row is never written; the scale, planes and group sums are k_pf_split's.
// SRC 1 with nsp > 0: the row is x[t] + part[0][t] + ... + part[nsp - 1][t] (slices of pn floats,
// row stride ldx), k_pf_split_add's sum, written back to x before the norm.
template <int NPT, int SRC>
__global__ __launch_bounds__(256) void k_pf_split_src(float* __restrict__ x, int ldx, int K,
                                                      const float* __restrict__ w, float eps, int kind,
                                                      _Float16* __restrict__ xh, int ldh, size_t plane,
                                                      float* __restrict__ xs, int T, const float* __restrict__ part,
                                                      int nsp, size_t pn) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    float* xr = x + (size_t)t * ldx;
    const int K4 = K / 4;
    float4 v[NPT];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; j++) {
        const int i = threadIdx.x + 256 * j;
        float4 q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < K4) {
            if constexpr (SRC == 2) {
                const float4 g = ((const float4*)xr)[i], u = ((const float4*)(xr + K))[i];
                q = make_float4(act_fn(g.x, kind) * u.x, act_fn(g.y, kind) * u.y, act_fn(g.z, kind) * u.z,
                                act_fn(g.w, kind) * u.w);
            } else {
                q = ((const float4*)xr)[i];
                if (nsp > 0) {
                    for (int z = 0; z < nsp; z++) {
                        const float4 p = ((const float4*)(part + (size_t)z * pn + (size_t)t * ldx))[i];
                        q.x += p.x;
                        q.y += p.y;
                        q.z += p.z;
                        q.w += p.w;
                    }
                    ((float4*)xr)[i] = q;
                }
                ss = fmaf(q.x, q.x, ss);
                ss = fmaf(q.y, q.y, ss);
                ss = fmaf(q.z, q.z, ss);
                ss = fmaf(q.w, q.w, ss);
            }
        }
        v[j] = q;
    }
    if constexpr (SRC == 1) {
        const float tot = pf_block_sum(ss, red);
        const float rms = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
        for (int j = 0; j < NPT; j++) {
            const int i = threadIdx.x + 256 * j;
            if (i < K4) {
                const float4 w4 = ((const float4*)w)[i];
                const float t0 = v[j].x * rms, t1 = v[j].y * rms, t2 = v[j].z * rms, t3 = v[j].w * rms;
                v[j] = kind ? make_float4(t0 * (w4.x + 1.0f), t1 * (w4.y + 1.0f), t2 * (w4.z + 1.0f), t3 * (w4.w + 1.0f))
                            : make_float4(t0 * w4.x, t1 * w4.y, t2 * w4.z, t3 * w4.w);
            }
        }
        __syncthreads();  // red is reused below
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NPT; j++)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    m = pf_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (m > 0.0f && m <= 3.0e38f) {
        int ex;
        (void)frexpf(m, &ex);  // m in [2^(ex-1), 2^ex)
        e = 15 - ex;
        e = e < -120 ? -120 : (e > 120 ? 120 : e);
    }
    const float sc = ldexpf(1.0f, e);
    _Float16* h = xh + (size_t)t * ldh;
    const int G = K / 32;
    _Float16* gs = xh + 2 * plane + (size_t)t * G;
    const size_t gplane = (size_t)T * G;
#pragma unroll
    for (int j = 0; j < NPT; j++) {
        const int i = threadIdx.x + 256 * j;
        const float c[4] = {v[j].x * sc, v[j].y * sc, v[j].z * sc, v[j].w * sc};
        if (i < K4) {
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                hi[u] = (_Float16)c[u];
                lo[u] = (_Float16)(c[u] - (float)hi[u]);
            }
            *(uint2*)(h + 4 * i) = *(const uint2*)hi;
            *(uint2*)(h + plane + 4 * i) = *(const uint2*)lo;
        }
        // group i / 8: 8 lanes of 4 elements, summed in k_pf_split's order
        float gv = i < K4 ? ((c[0] + c[1]) + (c[2] + c[3])) : 0.0f;
        gv += __shfl_xor(gv, 1);
        gv += __shfl_xor(gv, 2);
        gv += __shfl_xor(gv, 4);
        if (i < K4 && (i & 7) == 0) {
            gv *= 0.015625f;  // times 2^-6 (exact), as k_pf_split
            const _Float16 ghi = (_Float16)gv;
            gs[i >> 3] = ghi;
            gs[gplane + (i >> 3)] = (_Float16)(gv - (float)ghi);
        }
    }
    if (threadIdx.x == 0) xs[t] = ldexpf(1.0f, -e);
}

template <int SRC>
static hipError_t pf_split_src(float* x, int ldx, int T, int K, const float* w, float eps, int kind,
                               _Float16* xh, int ldh, float* xs, hipStream_t st, const float* part = nullptr,
                               int nsp = 0) {
    if (T <= 0) return hipSuccess;
    if (K % 32 != 0 || ldx % 4 != 0 || ldh % 8 != 0 || ldh < K) return hipErrorInvalidValue;
    if (nsp < 0 || (nsp > 0 && (SRC != 1 || part == nullptr || (uintptr_t)part % 16 != 0))) return hipErrorInvalidValue;
    const int n4 = (K / 4 + 255) / 256;
    const size_t plane = (size_t)T * ldh, pn = (size_t)T * ldx;
    if (n4 <= 1) k_pf_split_src<1, SRC><<<T, 256, 0, st>>>(x, ldx, K, w, eps, kind, xh, ldh, plane, xs, T, part, nsp, pn);
    else if (n4 <= 2) k_pf_split_src<2, SRC><<<T, 256, 0, st>>>(x, ldx, K, w, eps, kind, xh, ldh, plane, xs, T, part, nsp, pn);
    else if (n4 <= 4) k_pf_split_src<4, SRC><<<T, 256, 0, st>>>(x, ldx, K, w, eps, kind, xh, ldh, plane, xs, T, part, nsp, pn);
    else if (n4 <= 8) k_pf_split_src<8, SRC><<<T, 256, 0, st>>>(x, ldx, K, w, eps, kind, xh, ldh, plane, xs, T, part, nsp, pn);
    else if (n4 <= 16) k_pf_split_src<16, SRC><<<T, 256, 0, st>>>(x, ldx, K, w, eps, kind, xh, ldh, plane, xs, T, part, nsp, pn);
    else if (n4 <= 20) k_pf_split_src<20, SRC><<<T, 256, 0, st>>>(x, ldx, K, w, eps, kind, xh, ldh, plane, xs, T, part, nsp, pn);
    else return hipErrorNotSupported;
    return hipGetLastError();
}

bool pf_split_src_ok(int K) { return K % 32 == 0 && (K / 4 + 255) / 256 <= 20; }

hipError_t launch_pf_split_norm(float* x, int T, int K, const float* w, float eps, int kind, _Float16* xh,
                                int ldh, float* xs, hipStream_t st, const float* part, int nsp) {
    return pf_split_src<1>(x, K, T, K, w, eps, kind, xh, ldh, xs, st, part, nsp);
}

hipError_t launch_pf_split_act(const float* gu, int T, int ffn, int act, _Float16* xh, int ldh, float* xs,
                               hipStream_t st) {
    // the gated form only reads gu
    return pf_split_src<2>(const_cast<float*>(gu), 2 * ffn, T, ffn, nullptr, 0.0f, act, xh, ldh, xs, st);
}

// largest |w| of a matrix (exact dequantization of every element), as float bits (non-negative floats
// order like their bits)
__global__ __launch_bounds__(256) void k_pf_wmax(int type, const uint8_t* __restrict__ w, int64_t n, unsigned* out) {
    __shared__ float red[4];
    float m = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float v = fabsf(deq_elem(type, w, i));
        m = v > m ? v : m;  // a NaN weight is skipped
    }
    m = pf_wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        if (m > 0.0f) atomicMax(out, __float_as_uint(m));
    }
}

hipError_t launch_pf_wmax(int type, const uint8_t* w, int64_t n, unsigned* out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_pf_wmax<<<(unsigned)blocks, 256, 0, st>>>(type, w, n, out);
    return hipGetLastError();
}

int pf_wexp(unsigned max_bits) {
    float m;
    memcpy(&m, &max_bits, 4);
    if (!(m > 0.0f) || !(m <= 3.0e38f)) return 0;  // zero or not finite: no scaling
    int ex;
    (void)frexpf(m, &ex);
    int e = ex - 15;  // m 2^-e in [2^14, 2^15)
    return e < -120 ? -120 : (e > 120 ? 120 : e);
}

typedef void (*PfGemmKernel)(const PfGemm);

// y[i] += part[0][i] + part[1][i] + ... (in that order) over n = T * ldy values
__global__ __launch_bounds__(256) void k_pf_split_add(float* __restrict__ y, const float* __restrict__ part, int nsp,
                                                      int64_t n) {
    // four floats per thread and step where n and the pointers allow (the parts are added in order
    // either way)
    const int64_t n4 = n % 4 == 0 && ((uintptr_t)y | (uintptr_t)part) % 16 == 0 ? n / 4 : 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
        float4 v = ((const float4*)y)[i];
        for (int z = 0; z < nsp; z++) {
            const float4 w = ((const float4*)(part + (int64_t)z * n))[i];
            v.x += w.x;
            v.y += w.y;
            v.z += w.z;
            v.w += w.w;
        }
        ((float4*)y)[i] = v;
    }
    for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = y[i];
        for (int z = 0; z < nsp; z++) v += part[(int64_t)z * n + i];
        y[i] = v;
    }
}


template <int BM>
static PfGemmKernel pf_rows_kernel_h(int type) {
    switch (type) {
        case FLLM_TYPE_Q8_0: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_Q8_0>;
        case FLLM_TYPE_Q4_0: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_Q4_0>;
        case FLLM_TYPE_Q4_K: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_Q4_K>;
        case FLLM_TYPE_Q5_K: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_Q5_K>;
        case FLLM_TYPE_Q6_K: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_Q6_K>;
        case FLLM_TYPE_F32: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_F32>;
        case FLLM_TYPE_F16: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_F16>;
        case FLLM_TYPE_BF16: return k_pf_gemm_rows_h<BM, PF_ROWS + FLLM_TYPE_BF16>;
        default: return k_pf_gemm_rows_h<BM, -1>;
    }
}

static hipError_t pf_lds_attr(const void* k, size_t bytes) {
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// resident workgroups of 256 threads per CU for a GEMM kernel at its LDS size (asked once per kernel)
static int pf_resident(PfGemmKernel k, size_t lds) {
    static std::mutex mu;
    static std::vector<std::pair<PfGemmKernel, int>> seen;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& e : seen)
        if (e.first == k) return e.second;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k, 256, lds) != hipSuccess) per_cu = 0;
    seen.emplace_back(k, per_cu);
    return per_cu;
}

hipError_t launch_pf_gemm(PfGemm a, int n_cu, hipStream_t st, int* pending) {
    if (pending) *pending = 0;
    if (a.T <= 0 || a.nseg <= 0) return hipSuccess;
    if (a.nseg > 3 || a.K <= 0 || a.K % 32 != 0 || a.ldx < a.K || a.ldx % 4 != 0) return hipErrorInvalidValue;
    const bool tiles = a.seg[0].layout == LAYOUT_TILES;
    int64_t col_tiles = 0;
    for (int i = 0; i < a.nseg; i++) {
        PfSeg& g = a.seg[i];
        if (g.N <= 0 || g.ldy < g.N || (g.layout == LAYOUT_TILES) != tiles) return hipErrorInvalidValue;
        if (!tiles && g.type != a.seg[0].type) return hipErrorInvalidValue;  // one decoder per row launch
        if (tiles && (a.K % 256 != 0 || g.N % 16 != 0 ||
                      (g.type != FLLM_TYPE_Q4_K && g.type != FLLM_TYPE_Q6_K && g.type != FLLM_TYPE_Q8_0 &&
                       g.type != FLLM_TYPE_Q5_K)))
            return hipErrorInvalidValue;
        g.tiles = (g.N + PF_BN - 1) / PF_BN;
        col_tiles += g.tiles;
    }
    // 64-token tiles at every length: two or three workgroups per CU against one for 128-token
    // tiles (at 288-352 registers), which ran 15-25% slower even on 4096-token chunks
    PfGemmKernel k;
    size_t lds;
    if (a.xh) {
        if (a.ldh < a.K || a.ldh % 8 != 0 || a.xs == nullptr) return hipErrorInvalidValue;
        bool all_q4k = tiles;
        for (int i = 0; i < a.nseg; i++) all_q4k = all_q4k && a.seg[i].type == FLLM_TYPE_Q4_K;
        bool all_q6k = tiles, all_q5k = tiles, q46 = tiles, all_q8 = tiles;
        for (int i = 0; i < a.nseg; i++) {
            all_q8 = all_q8 && a.seg[i].type == FLLM_TYPE_Q8_0;
            all_q6k = all_q6k && a.seg[i].type == FLLM_TYPE_Q6_K;
            all_q5k = all_q5k && a.seg[i].type == FLLM_TYPE_Q5_K;
            q46 = q46 && (a.seg[i].type == FLLM_TYPE_Q4_K || a.seg[i].type == FLLM_TYPE_Q6_K);
        }
        if (all_q4k) {
            k = k_pf_gemm_q4k<64>;
            lds = pf_gemm_lds_k<64>();
        } else if (all_q5k) {
            k = k_pf_gemm_q5k<64>;
            lds = pf_gemm_lds_k<64>();
        } else if (all_q6k) {
            k = k_pf_gemm_q6k<64>;
            lds = pf_gemm_lds_q6<64>();
        } else if (all_q8) {
            k = k_pf_gemm_q8t<64>;
            lds = pf_gemm_lds_q8<64>();
        } else if (q46) {
            k = k_pf_gemm_q46<64>;
            lds = std::max(pf_gemm_lds_k<64>(), pf_gemm_lds_q6<64>());
        } else {
            if (tiles) k = k_pf_gemm_tiles_h<64>;
            else k = pf_rows_kernel_h<64>(a.seg[0].type);
            lds = pf_gemm_lds_h<64>();
        }
    } else {
        return hipErrorInvalidValue;  // the fp16 planes are required
    }
    hipError_t e = pf_lds_attr((const void*)k, lds);
    if (e != hipSuccess) return e;
    constexpr int bm = 64;
    // K split: a launch whose segments fill the rows of one buffer side by side may run its K in
    // nsplit parts of whole 256-element blocks (part 0 into y, parts z > 0 into the scratch, then a
    // reduction in order). The choice minimises waves of resident workgroups x blocks per part
    // plus the reduction's bytes, in units of one block of one full wave: about 0.0118 us per
    // resident workgroup slot (a 64 x 128 tile's fp16 products at the forms' measured rate), the
    // reduction reading the parts and y and writing y at 4 TB/s. Llama-3-8B at 511 tokens: o 256
    // tiles in 3 parts on 768 slots, down 256 in 2 on 512, q/k/v 384 in 4; Qwen2-7B at 2047 tokens:
    // down 896 tiles in 4 on 768.
    int nsplit = 1, nbk = 0;
    if (a.part != nullptr && a.K % 256 == 0) {
        const int64_t base = col_tiles * ((a.T + bm - 1) / bm);
        bool side_by_side = true;
        int64_t off = 0;
        for (int i = 0; i < a.nseg; i++) {
            const PfSeg& g = a.seg[i];
            side_by_side = side_by_side && g.ldy == a.seg[0].ldy && g.y - a.seg[0].y == off;
            off += g.N;
        }
        side_by_side = side_by_side && off == a.seg[0].ldy;
        const int per_cu = side_by_side ? pf_resident(k, lds) : 0;
        if (per_cu > 0) {
            const int64_t slots = (int64_t)per_cu * (n_cu > 0 ? n_cu : 256);
            const int nb = a.K / 256;
            const double out_bytes = 4.0 * (double)a.T * (double)a.seg[0].ldy;
            const double unit_us = 0.0118 * (double)slots;  // one block of one full wave
            double best = 0.0;
            // grids of three or more waves unsplit (there the last wave's share is small and the
            // reduction's cost was not repaid: Gemma-2-9B's o at 4096 tokens ran 6% longer in 2 parts)
            const int nmax = (base + slots - 1) / slots <= 2 ? 4 : 1;
            for (int n = 1; n <= nmax && n <= nb; n++) {
                if (n > 1 && (size_t)(n - 1) * (size_t)a.T * (size_t)a.seg[0].ldy > a.part_cap) break;
                const int64_t waves = (base * n + slots - 1) / slots;
                const int bpp = (nb + n - 1) / n;
                if ((n - 1) * bpp >= nb) continue;  // every part holds at least one block
                const double cost = (double)waves * bpp + (n > 1 ? (n + 1) * out_bytes / 4.0e6 / unit_us : 0.0);
                if (n == 1 || cost < best) {
                    best = cost;
                    nsplit = n;
                    nbk = bpp;
                }
            }
        }
    }
    a.nsplit = nsplit;
    a.kpart = nsplit > 1 ? 256 * nbk : a.K;
    dim3 grid((unsigned)col_tiles, (unsigned)((a.T + bm - 1) / bm), (unsigned)nsplit);
    k<<<grid, 256, lds, st>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess || nsplit == 1) return e;
    if (pending) {
        *pending = nsplit - 1;
        return hipSuccess;
    }
    return launch_pf_split_add(a.seg[0].y, a.part, nsplit - 1, (int64_t)a.T * a.seg[0].ldy, st);
}

hipError_t launch_pf_split_add(float* y, const float* part, int nsp, int64_t n, hipStream_t st) {
    if (nsp <= 0 || n <= 0) return hipSuccess;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 2048) blocks = 2048;
    k_pf_split_add<<<blocks, 256, 0, st>>>(y, part, nsp, n);
    return hipGetLastError();
}

// ---- element-wise steps over the rows ----------------------------------------------------------
__global__ __launch_bounds__(256) void k_pf_embed(const int* __restrict__ tok, const uint8_t* __restrict__ emb, int type,
                                                  int H, float* __restrict__ x) {
    const int t = blockIdx.x;
    const int64_t base = (int64_t)tok[t] * H;
    for (int i = threadIdx.x; i < H; i += 256) x[(size_t)t * H + i] = deq_elem(type, emb, base + i);
}

hipError_t launch_pf_embed(const int* tokens, int T, const uint8_t* emb, int type, int H, float* x, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    k_pf_embed<<<T, 256, 0, st>>>(tokens, emb, type, H, x);
    return hipGetLastError();
}

// RmsNorm (TensorOperations.cs:42-54) / GemmaRmsNorm (:90-107) of row blockIdx.x
__global__ __launch_bounds__(256) void k_pf_norm(const float* __restrict__ x, int n, const float* __restrict__ w, float eps,
                                                 int kind, float* __restrict__ xn, int ldx) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    const float* xr = x + (size_t)t * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
    const float tot = pf_block_sum(ss, red);
    const float rms = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float tv = xr[i] * rms;
        xn[(size_t)t * ldx + i] = kind ? tv * (w[i] + 1.0f) : tv * w[i];
    }
}

hipError_t launch_pf_norm(const float* x, int T, int n, const float* w, float eps, int kind, float* xn, int ldx,
                          hipStream_t st) {
    if (T <= 0) return hipSuccess;
    k_pf_norm<<<T, 256, 0, st>>>(x, n, w, eps, kind, xn, ldx);
    return hipGetLastError();
}

// ComputeSiluFfn / ComputeGeluFfn gating (LlamaForwardPass.cs:217-232; Gemma2ForwardPass.cs:187-199)
__global__ __launch_bounds__(256) void k_pf_act(const float* __restrict__ gu, int ffn, int act, float* __restrict__ h,
                                                int ldx) {
    const int t = blockIdx.y;
    const float* row = gu + (size_t)t * 2 * ffn;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < ffn; i += gridDim.x * 256)
        h[(size_t)t * ldx + i] = act_fn(row[i], act) * row[ffn + i];
}

hipError_t launch_pf_act(const float* gu, int T, int ffn, int act, float* h, int ldx, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    dim3 grid((unsigned)((ffn + 255) / 256 < 64 ? (ffn + 255) / 256 : 64), (unsigned)T);
    k_pf_act<<<grid, 256, 0, st>>>(gu, ffn, act, h, ldx);
    return hipGetLastError();
}

// Qwen2 bias (Qwen2ForwardPass.cs:83-85), RoPE on interleaved pairs (TensorOperations.cs:250-260)
// at position pos0 + t, KvCache.Append into slot pos0 + t (KvCache.cs:86-89)
// (nsp pending K-split slices of part, pn floats apart, added to each value first: k_pf_split_add's sum)
__global__ __launch_bounds__(256) void k_pf_qkv_post(float* __restrict__ qkv, int ldq, int pos0,
                                                     const float* __restrict__ bq, const float* __restrict__ bk,
                                                     const float* __restrict__ bv, const float2* __restrict__ rope,
                                                     int nh, int nkv, int hd, float* __restrict__ kc,
                                                     float* __restrict__ vc, const float* __restrict__ part, int nsp,
                                                     size_t pn) {
    const int t = blockIdx.x, pos = pos0 + t, half = hd >> 1, qdim = nh * hd, kvdim = nkv * hd;
    float* row = qkv + (size_t)t * ldq;
    const float* prow = part + (size_t)t * ldq;
    // values c, c + 1 (c even; every row, slice and cache row starts at an even offset)
    auto val2 = [&](int c) {
        float2 v = *(const float2*)(row + c);
        for (int z = 0; z < nsp; z++) {
            const float2 p = *(const float2*)(prow + (size_t)z * pn + c);
            v.x += p.x;
            v.y += p.y;
        }
        return v;
    };
    const float2* rp = rope + (size_t)pos * half;
    const int npairs = (nh + nkv) * half;
    for (int idx = threadIdx.x; idx < npairs; idx += 256) {
        const bool isq = idx < nh * half;
        const int li = isq ? idx : idx - nh * half;
        const int head = li / half, i = li % half, o = head * hd + 2 * i;
        const float2 xv = val2((isq ? 0 : qdim) + o);
        float x0 = xv.x, x1 = xv.y;
        const float* b = isq ? bq : bk;
        if (b) {
            const float2 bb = *(const float2*)(b + o);
            x0 = x0 + bb.x;
            x1 = x1 + bb.y;
        }
        const float2 cs = rp[i];
        const float2 y = make_float2(x0 * cs.x - x1 * cs.y, x0 * cs.y + x1 * cs.x);
        if (isq) *(float2*)(row + o) = y;
        else *(float2*)(kc + (size_t)pos * kvdim + o) = y;
    }
    for (int i = 2 * threadIdx.x; i < kvdim; i += 512) {
        float2 v = val2(qdim + kvdim + i);
        if (bv) {
            const float2 bb = *(const float2*)(bv + i);
            v.x = v.x + bb.x;
            v.y = v.y + bb.y;
        }
        *(float2*)(vc + (size_t)pos * kvdim + i) = v;
    }
}

hipError_t launch_pf_qkv_post(float* qkv, int ldq, int T, int pos0, const float* bq, const float* bk, const float* bv,
                              const float2* rope, int nh, int nkv, int hd, float* kc, float* vc, hipStream_t st,
                              const float* part, int nsp) {
    if (T <= 0) return hipSuccess;
    if (nsp < 0 || (nsp > 0 && part == nullptr)) return hipErrorInvalidValue;
    if (ldq % 2 != 0 || hd % 2 != 0) return hipErrorInvalidValue;  // pairs of floats at even offsets
    k_pf_qkv_post<<<T, 256, 0, st>>>(qkv, ldq, pos0, bq, bk, bv, rope, nh, nkv, hd, kc, vc, nsp > 0 ? part : qkv, nsp,
                                     (size_t)T * ldq);
    return hipGetLastError();
}

// Gemma2 post-norm: x += GemmaRmsNorm(tmp, w), eps 1e-6 (Gemma2ForwardPass.cs:90-96)
// (n a multiple of 4: float4 pieces; nsp pending K-split slices of part, pn floats apart, added to
// tmp's row first and written back, k_pf_split_add's sum)
__global__ __launch_bounds__(256) void k_pf_postnorm_add(float* __restrict__ tmp, int n, const float* __restrict__ w,
                                                         float* __restrict__ x, const float* __restrict__ part, int nsp,
                                                         size_t pn) {
    __shared__ float red[4];
    const int t = blockIdx.x, n4 = n / 4;
    float4* tr = (float4*)(tmp + (size_t)t * n);
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n4; i += 256) {
        float4 v = tr[i];
        if (nsp > 0) {
            for (int z = 0; z < nsp; z++) {
                const float4 p = ((const float4*)(part + (size_t)z * pn + (size_t)t * n))[i];
                v.x += p.x;
                v.y += p.y;
                v.z += p.z;
                v.w += p.w;
            }
            tr[i] = v;  // read back below by this same thread
        }
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    const float tot = pf_block_sum(ss, red);
    const float rms = 1.0f / sqrtf(tot / (float)n + 1e-6f);
    float4* xr = (float4*)(x + (size_t)t * n);
    for (int i = threadIdx.x; i < n4; i += 256) {
        const float4 v = tr[i], w4 = ((const float4*)w)[i];
        float4 o = xr[i];
        o.x = o.x + (v.x * rms) * (w4.x + 1.0f);
        o.y = o.y + (v.y * rms) * (w4.y + 1.0f);
        o.z = o.z + (v.z * rms) * (w4.z + 1.0f);
        o.w = o.w + (v.w * rms) * (w4.w + 1.0f);
        xr[i] = o;
    }
}

hipError_t launch_pf_postnorm_add(float* tmp, int T, int n, const float* w, float* x, hipStream_t st,
                                  const float* part, int nsp) {
    if (T <= 0) return hipSuccess;
    if (n % 4 != 0 || nsp < 0 || (nsp > 0 && part == nullptr)) return hipErrorInvalidValue;
    k_pf_postnorm_add<<<T, 256, 0, st>>>(tmp, n, w, x, nsp > 0 ? part : tmp, nsp, (size_t)T * n);
    return hipGetLastError();
}

// ---- causal attention over the cache (ComputeAttention, LlamaForwardPass.cs:158-211 and the
// Mistral / Qwen2 / Gemma2 variants) ----------------------------------------------------------------
// Workgroup = (query head, block of 64 consecutive queries, the last block first), wave w = queries
// 16 w .. + 15. Keys go in blocks of 64 rows (32 for head_dim 256) of the head's kv head, staged in
// LDS (K rows padded to HD + 8 floats, V rows to HD + 16); the next block's rows are loaded into registers while
// the current one multiplies. Per
// block a wave forms the transposed scores S^T = K Q^T on the f32 matrix cores
// (v_mfma_f32_16x16x4f32: lane l holds keys 16 t + 4 (l >> 4) + e of query l & 15), updates the running
// max / sum per query (online softmax), and adds O^T += V^T P^T with P^T straight from the score
// registers: a step's four keys are the four keys one lane holds, so V's rows are taken in that order.
// The order of the terms inside the dot products and sums is a permutation of the reference's; every
// product and sum is f32.
constexpr int PF_AQ = 64;
// key block: 64 positions, 32 for head_dim 256 (LDS for two workgroups per CU: 66.5 KB each)
template <int HD> struct PfAk {
    static constexpr int v = HD <= 128 ? 64 : 32;
    // head_dim up to 128: the next block's rows are prefetched into registers while the current one
    // multiplies (216 registers at 128). Head_dim 256 loads each block when it is staged instead:
    // the prefetch took it to 300 registers and one workgroup per CU; without it two workgroups
    // share a CU (at most 256 registers) and each one's products cover the other's loads
    static constexpr bool pre = HD <= 128;
};

// LDS row strides (floats) of the staged K and V rows. A half-wave reads K as 16 rows x two 16-byte
// columns (conflict-free over gfx950's 128 banks when the stride is 8 mod 16 dwords: the rows'
// 32-byte spans tile the banks) and V as two rows 4 apart x 64 dwords (conflict-free when 4 strides
// are 64 mod 128 dwords); HD + 4 had every K and V read take two passes.
template <int HD> struct PfAld {
    static constexpr int k = HD + 8, v = HD + 16;
};
template <int HD>
static constexpr size_t pf_attn_lds() {
    return sizeof(float) * (size_t)PfAk<HD>::v * (PfAld<HD>::k + PfAld<HD>::v);
}

template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PfAk<HD>::pre ? 1 : 2))) void k_pf_attn(const PfAttn a) {
    constexpr int LDK = PfAld<HD>::k, LDV = PfAld<HD>::v, NU = HD / 16, NT = HD / 16;
    constexpr int PF_AK = PfAk<HD>::v, KT = PF_AK / 16;  // key block and its 16-key MFMA tiles
    extern __shared__ float pa_lds[];
    float* sk = pa_lds;             // [PF_AK][LDK]
    float* sv = sk + PF_AK * LDK;   // [PF_AK][LDV]
    // query blocks from the last (the most keys under the causal mask) to the first, so that the
    // longest workgroups are dispatched first and the short ones fill in behind them. With a.split,
    // rows 2 i and 2 i + 1 of the grid are the first and second half of the key blocks of query
    // block nqb - 1 - i (every block but block 0, which stays whole in the last row): the halves
    // leave their unnormalised sums, max and sum in a.part for k_pf_attn_merge.
    const int nqb = (a.T + PF_AQ - 1) / PF_AQ;
    int qbi = nqb - 1 - (int)blockIdx.y, half = -1;
    if (a.split) {
        const int y = (int)blockIdx.y;
        qbi = y < 2 * (nqb - 1) ? nqb - 1 - (y >> 1) : 0;
        half = y < 2 * (nqb - 1) ? (y & 1) : -1;
    }
    const int h = blockIdx.x, qb = qbi * PF_AQ;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q16 = lane & 15, kq = lane >> 4;
    const int kvh = h / (a.nh / a.nkv);
    // this lane's query (the column it holds) and the wave's query range
    const int tq = qb + 16 * wave + q16, w0 = qb + 16 * wave;
    const bool qlive = tq < a.T, wlive = w0 < a.T;
    const int pos = a.pos0 + (qlive ? tq : a.T - 1);
    const int ws = pos + 1 - a.window > 0 ? pos + 1 - a.window : 0;
    const int wpos_hi = a.pos0 + (w0 + 15 < a.T ? w0 + 15 : a.T - 1);
    const int wws = a.pos0 + w0 + 1 - a.window > 0 ? a.pos0 + w0 + 1 - a.window : 0;
    // Q^T operand: dims 16 u + 4 (l >> 4) .. + 3 of the lane's query, one per MFMA step
    float4 qr[NU];
#pragma unroll
    for (int u = 0; u < NU; u++)
        qr[u] = qlive ? *(const float4*)(a.q + (size_t)tq * a.ldq + (size_t)h * HD + 16 * u + 4 * kq)
                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // keys of the workgroup: from the first query's window start to the last live query
    const int tl = (qb + PF_AQ < a.T ? qb + PF_AQ : a.T) - 1;
    int kend = a.pos0 + tl;
    int kstart = a.pos0 + qb + 1 - a.window > 0 ? a.pos0 + qb + 1 - a.window : 0;
    if (half >= 0) {
        // the first ceil(nk / 2) key blocks, or the rest (empty when the range is one block: the
        // half then leaves max -inf and sum 0)
        const int nk = (kend - kstart) / PF_AK + 1, kmid = kstart + ((nk + 1) / 2) * PF_AK;
        if (half == 0) kend = kmid - 1 < kend ? kmid - 1 : kend;
        else kstart = kmid;
    }
    const int kclamp = a.pos0 + tl;  // a valid cache row for the clamped loads of an empty half
    const float inv_cap = a.softcap > 0.0f ? 1.0f / a.softcap : 0.0f;
    float m = -INFINITY, l = 0.0f;
    // O^T tile d = 4 c + r (c = dt / 4, r = dt % 4) holds dims 64 c + 4 i + r, i = 0..15
    pf_f32x4 o[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) o[i] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // the next block's K / V rows are loaded into registers while this block multiplies
    // (PF_AK * HD / 4 float4 pieces of each, NPC per thread; vectors rather than arrays of float4,
    // which the compiler would keep in scratch memory)
    constexpr int NPC = PF_AK * (HD / 4) / 256;
    typedef float pf_fv __attribute__((ext_vector_type(4 * NPC)));
    pf_fv pk, pv;
    // piece c = thread + 256 i: key row c / (HD / 4), dims 4 (c % (HD / 4)) .. + 3
    const int jrow = threadIdx.x / (HD / 4), d4 = (threadIdx.x % (HD / 4)) * 4;
    if constexpr (PfAk<HD>::pre) {
#pragma unroll
        for (int i = 0; i < NPC; i++) {
            const int j = jrow + i * (256 / (HD / 4)), key = kstart + j < kend ? kstart + j : (kend < kstart ? kclamp : kend);
            const size_t off = (size_t)key * a.kvdim + (size_t)kvh * HD + d4;
            const float4 k4 = *(const float4*)(a.kc + off), v4 = *(const float4*)(a.vc + off);
            pk[4 * i] = k4.x; pk[4 * i + 1] = k4.y; pk[4 * i + 2] = k4.z; pk[4 * i + 3] = k4.w;
            pv[4 * i] = v4.x; pv[4 * i + 1] = v4.y; pv[4 * i + 2] = v4.z; pv[4 * i + 3] = v4.w;
        }
    }
    for (int kb = kstart; kb <= kend; kb += PF_AK) {
        __syncthreads();  // the previous block's rows have been read
        if constexpr (PfAk<HD>::pre) {
#pragma unroll
            for (int i = 0; i < NPC; i++) {
                const int j = jrow + i * (256 / (HD / 4));
                *(float4*)(sk + j * LDK + d4) = make_float4(pk[4 * i], pk[4 * i + 1], pk[4 * i + 2], pk[4 * i + 3]);
                *(float4*)(sv + j * LDV + d4) = make_float4(pv[4 * i], pv[4 * i + 1], pv[4 * i + 2], pv[4 * i + 3]);
            }
            if (kb + PF_AK <= kend) {
#pragma unroll
                for (int i = 0; i < NPC; i++) {
                    const int j = jrow + i * (256 / (HD / 4)), key = kb + PF_AK + j < kend ? kb + PF_AK + j : kend;
                    const size_t off = (size_t)key * a.kvdim + (size_t)kvh * HD + d4;
                    const float4 k4 = *(const float4*)(a.kc + off), v4 = *(const float4*)(a.vc + off);
                    pk[4 * i] = k4.x; pk[4 * i + 1] = k4.y; pk[4 * i + 2] = k4.z; pk[4 * i + 3] = k4.w;
                    pv[4 * i] = v4.x; pv[4 * i + 1] = v4.y; pv[4 * i + 2] = v4.z; pv[4 * i + 3] = v4.w;
                }
            }
        } else {
            // this block's rows, all loads issued before the stores
            float4 k4[NPC], v4[NPC];
#pragma unroll
            for (int i = 0; i < NPC; i++) {
                const int j = jrow + i * (256 / (HD / 4)), key = kb + j < kend ? kb + j : kend;
                const size_t off = (size_t)key * a.kvdim + (size_t)kvh * HD + d4;
                k4[i] = *(const float4*)(a.kc + off);
                v4[i] = *(const float4*)(a.vc + off);
            }
#pragma unroll
            for (int i = 0; i < NPC; i++) {
                const int j = jrow + i * (256 / (HD / 4));
                *(float4*)(sk + j * LDK + d4) = k4[i];
                *(float4*)(sv + j * LDV + d4) = v4[i];
            }
        }
        __syncthreads();
        if (!wlive || kb > wpos_hi || kb + PF_AK - 1 < wws) continue;  // no key of the block for the wave
        pf_f32x4 s[KT];
#pragma unroll
        for (int t = 0; t < KT; t++) s[t] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < NU; u++)
#pragma unroll
            for (int t = 0; t < KT; t++) {
                const float4 kr = *(const float4*)(sk + (16 * t + q16) * LDK + 16 * u + 4 * kq);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr.x, qr[u].x, s[t], 0, 0, 0);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr.y, qr[u].y, s[t], 0, 0, 0);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr.z, qr[u].z, s[t], 0, 0, 0);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr.w, qr[u].w, s[t], 0, 0, 0);
            }
        // scores of keys kb + 16 t + 4 (l >> 4) + e for query l & 15
        float bmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < KT; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int key = kb + 16 * t + 4 * kq + e;
                float x = s[t][e] * a.scale;
                if (a.softcap > 0.0f) x = tanhf(x * inv_cap) * a.softcap;
                x = (qlive && key >= ws && key <= pos) ? x : -INFINITY;
                s[t][e] = x;
                bmax = fmaxf(bmax, x);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float m_new = fmaxf(m, bmax);
        const float corr = m_new == -INFINITY ? 1.0f : expf(m - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < KT; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float p = s[t][e] == -INFINITY ? 0.0f : expf(s[t][e] - m_new);
                s[t][e] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        l = l * corr + psum;
        m = m_new;
#pragma unroll
        for (int i = 0; i < NT; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) o[i][e] *= corr;
#pragma unroll
        for (int t = 0; t < KT; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float* vr = sv + (16 * t + 4 * kq + e) * LDV + 4 * q16;
#pragma unroll
                for (int c = 0; c < HD / 64; c++) {
                    const float4 vv = *(const float4*)(vr + 64 * c);
                    o[4 * c + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, s[t][e], o[4 * c + 0], 0, 0, 0);
                    o[4 * c + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, s[t][e], o[4 * c + 1], 0, 0, 0);
                    o[4 * c + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, s[t][e], o[4 * c + 2], 0, 0, 0);
                    o[4 * c + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, s[t][e], o[4 * c + 3], 0, 0, 0);
                }
            }
    }
    if (qlive && half >= 0) {
        // the half's unnormalised sums (the layout below), then max and sum of the lane's query
        const size_t row = ((size_t)(h * nqb + qbi) * 2 + half) * PF_AQ + (tq - qb);
        float* orow = a.part + row * HD + 16 * kq;
#pragma unroll
        for (int c = 0; c < HD / 64; c++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                *(float4*)(orow + 64 * c + 4 * e) = make_float4(o[4 * c][e], o[4 * c + 1][e], o[4 * c + 2][e], o[4 * c + 3][e]);
        if (kq == 0) {
            float* ml = a.part + (size_t)a.nh * nqb * 2 * PF_AQ * HD + row * 2;
            ml[0] = m;
            ml[1] = l;
        }
    } else if (qlive) {
        // lane l holds dims 64 c + 16 (l >> 4) + 4 e + r (tile 4 c + r, row 4 (l >> 4) + e) of its query
        const float inv = 1.0f / l;
        float* orow = a.out + (size_t)tq * a.nh * HD + (size_t)h * HD + 16 * kq;
#pragma unroll
        for (int c = 0; c < HD / 64; c++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                *(float4*)(orow + 64 * c + 4 * e) = make_float4(o[4 * c][e] * inv, o[4 * c + 1][e] * inv,
                                                                o[4 * c + 2][e] * inv, o[4 * c + 3][e] * inv);
    }
}

// The two halves of the split query blocks (1 .. nqb - 1) of head blockIdx.x, query block
// blockIdx.y + 1 (its rows spread over gridDim.z workgroups):
// out = (o1 e^(m1 - M) + o2 e^(m2 - M)) / (l1 e^(m1 - M) + l2 e^(m2 - M)), M = max(m1, m2)
template <int HD, int QB>
__global__ __launch_bounds__(256) void k_pf_attn_merge(const PfAttn a) {
    const int nqb = (a.T + QB - 1) / QB, h = blockIdx.x, qbi = blockIdx.y + 1, qb = qbi * QB;
    const size_t r0 = ((size_t)(h * nqb + qbi) * 2) * QB;
    const float* ml = a.part + (size_t)a.nh * nqb * 2 * QB * HD;
    for (int idx = threadIdx.x + 256 * (int)blockIdx.z; idx < QB * HD / 4; idx += 256 * (int)gridDim.z) {
        const int ql = idx / (HD / 4), d4 = (idx % (HD / 4)) * 4, tq = qb + ql;
        if (tq >= a.T) continue;
        const size_t ra = r0 + ql, rb = r0 + QB + ql;
        const float m1 = ml[2 * ra], l1 = ml[2 * ra + 1], m2 = ml[2 * rb], l2 = ml[2 * rb + 1];
        const float M = fmaxf(m1, m2);
        const float w1 = m1 == -INFINITY ? 0.0f : expf(m1 - M), w2 = m2 == -INFINITY ? 0.0f : expf(m2 - M);
        const float inv = 1.0f / (l1 * w1 + l2 * w2);
        const float4 oa = *(const float4*)(a.part + ra * HD + d4), ob = *(const float4*)(a.part + rb * HD + d4);
        *(float4*)(a.out + (size_t)tq * a.nh * HD + (size_t)h * HD + d4) =
            make_float4((oa.x * w1 + ob.x * w2) * inv, (oa.y * w1 + ob.y * w2) * inv, (oa.z * w1 + ob.z * w2) * inv,
                        (oa.w * w1 + ob.w * w2) * inv);
    }
}

// ---- head_dim 256: attention on the fp16 matrix cores ---------------------------------------------
// The f32 products above bound the head_dim 256 kernel (v_mfma_f32_16x16x4f32 has 1/16 of the fp16
// rate). Here a pass first splits the layer's cached K and V rows into fp16 hi / lo planes, per KV
// head and block of PF_HK positions, each block scaled by its own power of two (its largest
// magnitude into [2^14, 2^15), as the GEMM inputs: 22 significant bits with the lo plane), and
// k_pf_attn_h forms S^T = K Q^T and O^T += V^T P^T with three v_mfma_f32_16x16x32_f16 products per
// tile (hi hi, lo hi, hi lo; the dropped lo lo term is below 2^-22 of a product). Q is split per
// query row in the kernel and P as p 2^14. Every sum is f32; exp, max, softcap and masks as above.
// A block's planes are the LDS image the kernel stages, so staging is one contiguous copy:
//   K hi [PF_HK keys][HD], K lo, V^T hi [HD][PF_HK], V^T lo, rows of 16-byte chunks (8 halves);
//   K row r keeps chunk c at c ^ 2 (r & 15) (head_dim 256: 32 chunks, a row spans the 128 banks) or
//   c ^ 2 ((r >> 1) & 7) (head_dim 128: two rows span them), V^T row d keeps chunk c at
//   c ^ 2 ((d >> 3) & 1), so the operand reads of a half-wave (16 rows x two chunks) cover gfx950's
//   128 banks once;
//   V^T row d lists keys in MFMA k order: position 8 g + 4 t + e holds key 16 t + 4 g + e, the order
//   in which lane (g = l >> 4) holds P^T in its score registers (keys 16 t + 4 g + e, t = 0, 1).
// kvs holds each block's two exponents (K, V).
constexpr int PF_HK = 32;
template <int HD> constexpr int pf_kvh_block() { return 4 * PF_HK * HD; }  // halves per (head, block)
// chunk c of K row r in its plane
template <int HD> __device__ __forceinline__ int pf_kchunk(int c, int r) {
    static_assert(HD == 128 || HD == 256, "head_dim 128 or 256");
    return HD == 256 ? c ^ (2 * (r & 15)) : c ^ (2 * ((r >> 1) & 7));
}

// exponent e with m 2^e in [2^14, 2^15) (0 for m = 0 or non-finite), clamped to [-60, 60]
__device__ __forceinline__ int pf_exp15(float m) {
    int e = 0;
    if (m > 0.0f && m <= 3.0e38f) {
        int ex;
        (void)frexpf(m, &ex);
        e = 15 - ex;
        e = e < -60 ? -60 : (e > 60 ? 60 : e);
    }
    return e;
}

// grid (blocks of the keys [0, nkeys), KV heads), 256 threads: block b of head h into its planes
// (keys from nkeys on as zeros)
template <int HD>
__global__ __launch_bounds__(256) void k_pf_kv_split(const float* __restrict__ kc, const float* __restrict__ vc,
                                                     int kvdim, int nkeys, int nblk, _Float16* __restrict__ kvh,
                                                     int* __restrict__ kvs) {
    static_assert(HD == 128 || HD == 256, "head_dim 128 or 256");
    __shared__ float sv[PF_HK * HD];
    __shared__ float red[8];
    const int b = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    constexpr int NF = PF_HK * HD / 4 / 256;  // float4 pieces of K per thread
    float4 kr[NF];
    float mk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int i = 0; i < NF; i++) {
        const int f = tid + 256 * i, r = f / (HD / 4), c4 = f % (HD / 4), key = b * PF_HK + r;
        float4 k4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), v4 = k4;
        if (key < nkeys) {
            const size_t off = (size_t)key * kvdim + (size_t)h * HD + 4 * c4;
            k4 = *(const float4*)(kc + off);
            v4 = *(const float4*)(vc + off);
        }
        kr[i] = k4;
        mk = fmaxf(mk, fmaxf(fmaxf(fabsf(k4.x), fabsf(k4.y)), fmaxf(fabsf(k4.z), fabsf(k4.w))));
        mv = fmaxf(mv, fmaxf(fmaxf(fabsf(v4.x), fabsf(v4.y)), fmaxf(fabsf(v4.z), fabsf(v4.w))));
        *(float4*)(sv + r * HD + 4 * c4) = v4;
    }
    mk = pf_wave_max(mk);
    mv = pf_wave_max(mv);
    if ((tid & 63) == 0) {
        red[tid >> 6] = mk;
        red[4 + (tid >> 6)] = mv;
    }
    __syncthreads();  // the maxima and the V rows in sv
    mk = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    mv = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
    const int ek = pf_exp15(mk), ev = pf_exp15(mv);
    const float fk = ldexpf(1.0f, ek), fv = ldexpf(1.0f, ev);
    _Float16* blk = kvh + ((size_t)h * nblk + b) * pf_kvh_block<HD>();
#pragma unroll
    for (int i = 0; i < NF; i++) {
        const int f = tid + 256 * i, r = f / (HD / 4), c4 = f % (HD / 4);
        const int off = r * HD + (pf_kchunk<HD>(c4 >> 1, r) << 3) + 4 * (c4 & 1);
        const float c[4] = {kr[i].x * fk, kr[i].y * fk, kr[i].z * fk, kr[i].w * fk};
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            hi[u] = (_Float16)c[u];
            lo[u] = (_Float16)(c[u] - (float)hi[u]);
        }
        *(uint2*)(blk + off) = *(const uint2*)hi;
        *(uint2*)(blk + PF_HK * HD + off) = *(const uint2*)lo;
    }
    // V^T row d: 256 / HD threads per row, each its share of the four chunks
    constexpr int TPR = 256 / HD, GPT = 4 / TPR;
    const int d = tid % HD, g0 = (tid / HD) * GPT;
    _Float16* vh = blk + 2 * PF_HK * HD + d * PF_HK;
#pragma unroll
    for (int g = g0; g < g0 + GPT; g++) {
        _Float16 hi[8], lo[8];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x = sv[(16 * t + 4 * g + e) * HD + d] * fv;
                hi[4 * t + e] = (_Float16)x;
                lo[4 * t + e] = (_Float16)(x - (float)hi[4 * t + e]);
            }
        const int gs = g ^ (2 * ((d >> 3) & 1));
        *(uint4*)(vh + 8 * gs) = *(const uint4*)hi;
        *(uint4*)(vh + HD * PF_HK + 8 * gs) = *(const uint4*)lo;
    }
    if (tid == 0) {
        kvs[2 * ((size_t)h * nblk + b)] = ek;
        kvs[2 * ((size_t)h * nblk + b) + 1] = ev;
    }
}

// k_pf_attn's grid of (head, query block) rows, halves included, over the planes of k_pf_kv_split;
// eight waves of 16 queries share each staged key block of PF_HK aligned positions, brought in by
// direct global -> LDS loads into two buffers, the next block's while the current one multiplies
// (against four waves staging each block through registers into one buffer: Gemma-2-9B over 6143
// tokens attention 59.5-60.1 -> 55.3-56.5 ms, one workgroup per CU; Qwen2-7B over 2047 tokens
// 7.0 -> 5.0 ms, two per CU). O^T accumulates in units of 2^-E, E = 14 + the V exponent of the last
// block added (a block of another exponent rescales it by the power of two with the max correction).
template <int HD> struct PfHq {
    static constexpr int nw = 8, q = 16 * nw, threads = 64 * nw;  // waves, queries, threads
};
template <int HD>
__global__ __launch_bounds__(PfHq<HD>::threads) __attribute__((amdgpu_waves_per_eu(HD == 256 ? 2 : 4))) void k_pf_attn_h(const PfAttn a) {
    static_assert(HD == 128 || HD == 256, "head_dim 128 or 256");
    constexpr int NS = HD / 32, NT = HD / 16, BLK = pf_kvh_block<HD>();
    constexpr int QB = PfHq<HD>::q, NTH = PfHq<HD>::threads, NPU = BLK / 8 / NTH;
    static_assert(BLK / 8 % NTH == 0, "whole 16-byte pieces per thread");
    extern __shared__ uint4 ph_lds[];  // two buffers of BLK halves
    const int nqb = (a.T + QB - 1) / QB;
    int qbi = nqb - 1 - (int)blockIdx.y, half = -1;
    if (a.split) {
        const int y = (int)blockIdx.y;
        qbi = y < 2 * (nqb - 1) ? nqb - 1 - (y >> 1) : 0;
        half = y < 2 * (nqb - 1) ? (y & 1) : -1;
    }
    const int h = blockIdx.x, qb = qbi * QB;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q16 = lane & 15, kq = lane >> 4;
    const int kvh = h / (a.nh / a.nkv);
    const int tq = qb + 16 * wave + q16, w0 = qb + 16 * wave;
    const bool qlive = tq < a.T, wlive = w0 < a.T;
    const int pos = a.pos0 + (qlive ? tq : a.T - 1);
    const int ws = pos + 1 - a.window > 0 ? pos + 1 - a.window : 0;
    const int wpos_hi = a.pos0 + (w0 + 15 < a.T ? w0 + 15 : a.T - 1);
    const int wws = a.pos0 + w0 + 1 - a.window > 0 ? a.pos0 + w0 + 1 - a.window : 0;
    // Q^T operand of step s: dims 32 s + 8 (l >> 4) .. + 7 of the lane's query, scaled by 2^eq
    pf_h8 qh[NS], ql[NS];
    int eq;
    {
        float4 qv[2 * NS];
        float qm = 0.0f;
#pragma unroll
        for (int st = 0; st < NS; st++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                qv[2 * st + u] = qlive ? *(const float4*)(a.q + (size_t)tq * a.ldq + (size_t)h * HD + 32 * st + 8 * kq + 4 * u)
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                const float4 x = qv[2 * st + u];
                qm = fmaxf(qm, fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
            }
        qm = fmaxf(qm, __shfl_xor(qm, 16));
        qm = fmaxf(qm, __shfl_xor(qm, 32));
        eq = pf_exp15(qm);
        const float fq = ldexpf(1.0f, eq);
#pragma unroll
        for (int st = 0; st < NS; st++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float4 x = qv[2 * st + u];
                const float c[4] = {x.x * fq, x.y * fq, x.z * fq, x.w * fq};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const _Float16 hi = (_Float16)c[e];
                    qh[st][4 * u + e] = hi;
                    ql[st][4 * u + e] = (_Float16)(c[e] - (float)hi);
                }
            }
    }
    const int tl = (qb + QB < a.T ? qb + QB : a.T) - 1;
    const int kend = a.pos0 + tl;
    const int kfirst = a.pos0 + qb + 1 - a.window > 0 ? a.pos0 + qb + 1 - a.window : 0;
    int b0 = kfirst / PF_HK, b1 = kend / PF_HK;  // key blocks b0 .. b1
    if (half >= 0) {
        // the first ceil(n / 2) blocks, or the rest (none when the range is one block: the half then
        // leaves max -inf and sum 0)
        const int bm = b0 + (b1 - b0 + 2) / 2;
        if (half == 0) b1 = bm - 1;
        else b0 = bm;
    }
    const float inv_cap = a.softcap > 0.0f ? 1.0f / a.softcap : 0.0f;
    float m = -INFINITY, l = 0.0f;
    int E = 0;
    pf_f32x4 o[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) o[i] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint4* hsrc = (const uint4*)(a.kvh + (size_t)kvh * a.nblk * BLK);
    const int* hexp = a.kvs + 2 * (size_t)kvh * a.nblk;
    // block b's planes into buffer u: 16 bytes per lane, lane l of a wave at the wave's base + 16 l,
    // which is the planes' own order
    auto stage = [&](int b, int u) {
        const uint4* src = hsrc + (size_t)b * (BLK / 8) + threadIdx.x;
        uint4* dst = ph_lds + u * (BLK / 8) + 64 * wave;
#pragma unroll
        for (int i = 0; i < NPU; i++)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + NTH * i),
                                             (__attribute__((address_space(3))) void*)(dst + NTH * i), 16, 0, 0);
    };
    if (b0 <= b1) stage(b0, 0);
    for (int b = b0; b <= b1; b++) {
        const int kb = b * PF_HK, u = (b - b0) & 1;
        // this thread's loads of block b have landed; after the barrier every thread's have, and
        // every wave has left block b - 1, whose buffer the next block's loads then overwrite
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (b < b1) stage(b + 1, u ^ 1);
        if (!wlive || kb > wpos_hi || kb + PF_HK - 1 < wws) continue;  // no key of the block for the wave
        const _Float16* skh = (const _Float16*)(ph_lds + u * (BLK / 8));
        const _Float16* skl = skh + PF_HK * HD;
        const _Float16* svh = skl + PF_HK * HD;
        const _Float16* svl = svh + HD * PF_HK;
        const int ek = hexp[2 * b], ev = hexp[2 * b + 1];
        pf_f32x4 s[2];
        s[0] = s[1] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < NS; st++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int off = (16 * t + q16) * HD + (pf_kchunk<HD>(4 * st + kq, 16 * t + q16) << 3);
                const pf_h8 kh = *(const pf_h8*)(skh + off), kl = *(const pf_h8*)(skl + off);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[st], s[t], 0, 0, 0);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[st], s[t], 0, 0, 0);
                s[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[st], s[t], 0, 0, 0);
            }
        // scores of keys kb + 16 t + 4 (l >> 4) + e for query l & 15
        const float sc = ldexpf(a.scale, -(eq + ek));
        float bmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int key = kb + 16 * t + 4 * kq + e;
                float x = s[t][e] * sc;
                if (a.softcap > 0.0f) x = tanhf(x * inv_cap) * a.softcap;
                x = (qlive && key >= ws && key <= pos) ? x : -INFINITY;
                s[t][e] = x;
                bmax = fmaxf(bmax, x);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float m_new = fmaxf(m, bmax);
        const float corr = m_new == -INFINITY ? 1.0f : expf(m - m_new);
        float psum = 0.0f;
        pf_h8 ph, pl;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float p = s[t][e] == -INFINITY ? 0.0f : expf(s[t][e] - m_new);
                psum += p;
                const float x = p * 16384.0f;
                const _Float16 hi = (_Float16)x;
                ph[4 * t + e] = hi;
                pl[4 * t + e] = (_Float16)(x - (float)hi);
            }
        psum += __shfl_xor(psum, 16);
        psum += __shfl_xor(psum, 32);
        l = l * corr + psum;
        m = m_new;
        // the sums so far into this block's units 2^-(14 + ev), with the max correction
        const int Eb = 14 + ev;
        const float f = ldexpf(corr, Eb - E);
        E = Eb;
#pragma unroll
        for (int i = 0; i < NT; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) o[i][e] *= f;
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int off = (16 * j + q16) * PF_HK + ((kq ^ ((q16 >> 2) & 2)) << 3);
            const pf_h8 vh = *(const pf_h8*)(svh + off), vl = *(const pf_h8*)(svl + off);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, o[j], 0, 0, 0);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, o[j], 0, 0, 0);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, o[j], 0, 0, 0);
        }
    }
    // lane l holds dims 16 j + 4 (l >> 4) + e of its query, in units of 2^-E
    const float un = ldexpf(1.0f, -E);
    if (qlive && half >= 0) {
        const size_t row = ((size_t)(h * nqb + qbi) * 2 + half) * QB + (tq - qb);
        float* orow = a.part + row * HD + 4 * kq;
#pragma unroll
        for (int j = 0; j < NT; j++)
            *(float4*)(orow + 16 * j) = make_float4(o[j][0] * un, o[j][1] * un, o[j][2] * un, o[j][3] * un);
        if (kq == 0) {
            float* ml = a.part + (size_t)a.nh * nqb * 2 * QB * HD + row * 2;
            ml[0] = m;
            ml[1] = l;
        }
    } else if (qlive) {
        const float inv = un / l;
        float* orow = a.out + (size_t)tq * a.nh * HD + (size_t)h * HD + 4 * kq;
#pragma unroll
        for (int j = 0; j < NT; j++)
            *(float4*)(orow + 16 * j) = make_float4(o[j][0] * inv, o[j][1] * inv, o[j][2] * inv, o[j][3] * inv);
    }
}

size_t pf_kv_planes_halves(int hd, int nkv, int max_seq) {
    if (hd != 128 && hd != 256) return 0;
    return (size_t)nkv * (size_t)((max_seq + PF_HK - 1) / PF_HK) * 4 * PF_HK * (size_t)hd;
}

template <int HD>
static hipError_t pf_attn_run(PfAttn a, hipStream_t st) {
    // head_dim 128 and 256: the planes of keys [0, pos0 + T), then the fp16 kernel (attention over
    // 2047 tokens of Qwen2-7B 10.2 -> 5.0 ms, over 511 of Llama-3-8B 1.48 -> 1.35 ms); head_dim 64:
    // the f32 kernel
    constexpr int PH = HD == 128 || HD == 256 ? HD : 256;  // the fp16 kernel's instance
    constexpr bool planes = HD == 128 || HD == 256;
    const void* kfn = planes ? (const void*)k_pf_attn_h<PH> : (const void*)k_pf_attn<HD>;
    const size_t lds = planes ? 2 * sizeof(_Float16) * (size_t)pf_kvh_block<PH>() : pf_attn_lds<HD>();
    const int qblk = planes ? PfHq<PH>::q : PF_AQ, nthr = planes ? PfHq<PH>::threads : 256;
    hipError_t e = pf_lds_attr(kfn, lds);
    if (e != hipSuccess) return e;
    if (planes) {
        const int nkeys = a.pos0 + a.T, nb = (nkeys + PF_HK - 1) / PF_HK;
        if (a.kvh == nullptr || a.kvs == nullptr || nb > a.nblk) return hipErrorInvalidValue;
        k_pf_kv_split<PH><<<dim3((unsigned)nb, (unsigned)a.nkv), 256, 0, st>>>(a.kc, a.vc, a.kvdim, nkeys, a.nblk, a.kvh,
                                                                                a.kvs);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const int nqb = (a.T + qblk - 1) / qblk;
    // split the key ranges of query blocks 1 .. nqb - 1 in two when every half and block 0 then run
    // at once on the resident slots and the scratch holds the halves (Llama-3-8B at 511 tokens:
    // 32 heads x 15 rows on 512 slots; the longest workgroup had 8 key blocks against 4.5 on average)
    a.split = 0;
    if (a.part != nullptr && nqb >= 2) {
        // resident workgroups per CU of the f32 and the fp16 kernel (each asked once)
        static std::atomic<int> resident[2] = {{-1}, {-1}};
        int per_cu = resident[planes].load(std::memory_order_relaxed);
        if (per_cu < 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kfn, nthr, lds) != hipSuccess)
                per_cu = 0;
            resident[planes].store(per_cu, std::memory_order_relaxed);
        }
        const int64_t items = (int64_t)a.nh * (2 * (nqb - 1) + 1);
        const size_t need = (size_t)a.nh * nqb * 2 * qblk * (HD + 2);
        if (per_cu > 0 && items <= (int64_t)per_cu * (a.n_cu > 0 ? a.n_cu : 256) && need <= a.part_cap) a.split = 1;
    }
    dim3 grid((unsigned)a.nh, (unsigned)(a.split ? 2 * (nqb - 1) + 1 : nqb));
    if (planes) k_pf_attn_h<PH><<<grid, nthr, lds, st>>>(a);
    else k_pf_attn<HD><<<grid, 256, lds, st>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess || !a.split) return e;
    // a block's rows over 4 workgroups (32 heads x 3 split blocks of 128 queries alone took 9.3 us)
    if (planes) k_pf_attn_merge<HD, PfHq<PH>::q><<<dim3((unsigned)a.nh, (unsigned)(nqb - 1), 4), 256, 0, st>>>(a);
    else k_pf_attn_merge<HD, PF_AQ><<<dim3((unsigned)a.nh, (unsigned)(nqb - 1), 2), 256, 0, st>>>(a);
    return hipGetLastError();
}

hipError_t launch_pf_attn(const PfAttn& a, hipStream_t st) {
    if (a.T <= 0) return hipSuccess;
    if (a.nkv <= 0 || a.nh % a.nkv != 0 || a.kvdim != a.nkv * a.hd) return hipErrorInvalidValue;
    switch (a.hd) {
        case 64: return pf_attn_run<64>(a, st);
        case 128: return pf_attn_run<128>(a, st);
        case 256: return pf_attn_run<256>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace fllm
