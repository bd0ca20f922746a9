// prefill.hip — batched prefill kernels (gfx950).
//
// The reference's prefill is n consecutive Forward calls (LlamaLanguageModel.cs:133-137). Here the
// n prompt tokens go through each layer together: every projection is one GEMM over the tokens,
// Y[t][n] = sum_k X[t][k] W[n][k] (LinearProjection, LlamaForwardPass.cs:237-260, for all rows at
// once), and the element-wise steps of the layer run over all rows.
//
// GEMM numerics. Weights are dequantized exactly (the Dequantizer arithmetic, as the device
// dequant kernels do) while they are staged into LDS, and multiplied with the f32 activations on the
// matrix cores in f32 (v_mfma_f32_16x16x4f32): the products of the reference's F32 path, summed in
// f32 in the matrix core's order.
#include "prefill.hpp"
#include "deq.hpp"
#include "gemv.hpp"

#include <math.h>

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
        const uint32_t w = idx < 8 ? (idx < 4 ? h.x : h.y) : (idx < 12 ? h.z : h.w);
        return (w >> (8 * (idx & 3))) & 0xFFu;
    }
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v) {
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
        const float dg = d * (float)sc;
        const float mg = dmin * (float)mn;
        const uint32_t wd[4] = {w4.qs.x, w4.qs.y, w4.qs.z, w4.qs.w};
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t byte = (wd[i >> 3] >> (8 * ((i >> 1) & 3))) & 0xFFu;
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
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v) {
        const int g = (k0 >> 5) & 7;
        const uint32_t sc2 = g < 4 ? (w4.s4 & 0xFFFFu) : (w4.s4 >> 16);
        const float d = half_exact(w4.d);
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
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v) {
        const int g = (k0 >> 5) & 7;
        const float d = half_exact(g < 4 ? (w4.d & 0xFFFFu) : (w4.d >> 16));
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
    __device__ static void deq(const Raw& w4, const uint8_t*, int, int, int, int k0, float* v) {
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
        const float dg = d * (float)sc;
        const float mg = dmin * (float)mn;
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
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int type, int K, int r, int k0, float* v) {
        const int64_t e0 = (int64_t)r * K + k0;
        for (int i = 0; i < 32; i++) v[i] = deq_elem(type, w, e0 + i);
    }
};

// Q8_0 (Dequantizer.cs:203-231): (sbyte)q * d, one 34-byte block per group
template <> struct PfW<PF_ROWS + FLLM_TYPE_Q8_0> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const uint8_t* p = w + (((int64_t)r * K + k0) >> 5) * 34;
        const float d = half_exact(deq_ld_u16(p));
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = (float)(int8_t)p[2 + i] * d;
    }
};

// Q4_0 (Dequantizer.cs:155-185): (nibble - 8) * d, low nibbles are elements 0..15
template <> struct PfW<PF_ROWS + FLLM_TYPE_Q4_0> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const uint8_t* p = w + (((int64_t)r * K + k0) >> 5) * 18;
        const float d = half_exact(deq_ld_u16(p));
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
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const int64_t e0 = (int64_t)r * K + k0;
        const uint8_t* p = w + (e0 >> 8) * 144;
        const int g = (int)((e0 & 255) >> 5);
        const float d = half_exact(deq_ld_u16(p)), dmin = half_exact(deq_ld_u16(p + 2));
        int sc, mn;
        kscale_min(p + 4, g, sc, mn);
        const float dg = d * (float)sc;
        const float mg = dmin * (float)mn;
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
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const int64_t e0 = (int64_t)r * K + k0;
        const uint8_t* p = w + (e0 >> 8) * 176;
        const int t0 = (int)(e0 & 255), g = t0 >> 5;
        const float d = half_exact(deq_ld_u16(p)), dmin = half_exact(deq_ld_u16(p + 2));
        int sc, mn;
        kscale_min(p + 4, g, sc, mn);
        const float dg = d * (float)sc;
        const float mg = dmin * (float)mn;
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
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const int64_t e0 = (int64_t)r * K + k0;
        const uint8_t* p = w + (e0 >> 8) * 210;
        const int i0 = (int)(e0 & 255);
        const float d = half_exact(deq_ld_u16(p + 208));
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
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const uint8_t* p = w + ((int64_t)r * K + k0) * 4;
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = bits_f32(deq_ld_u32(p + 4 * i));
    }
};
template <> struct PfW<PF_ROWS + FLLM_TYPE_F16> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const uint8_t* p = w + ((int64_t)r * K + k0) * 2;
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = half_exact(deq_ld_u16(p + 2 * i));
    }
};
template <> struct PfW<PF_ROWS + FLLM_TYPE_BF16> {
    struct Raw {};
    __device__ static void load(Raw&, const uint8_t*, int, int, int) {}
    __device__ static void deq(const Raw&, const uint8_t* __restrict__ w, int, int K, int r, int k0, float* v) {
        const uint8_t* p = w + ((int64_t)r * K + k0) * 2;
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = bf16_exact(deq_ld_u16(p + 2 * i));
    }
};

// ---- GEMM ---------------------------------------------------------------------------------------
// Workgroup tile: BM tokens (128 or 64) x 128 weight rows, 4 waves in a 2 x 2 arrangement, each
// (BM / 2) x 64 (BM / 32 x 4 MFMA tiles of 16 x 16). Per K step of 64 the workgroup stages X
// (copied) and W (dequantized, one 32-weight group per thread) into LDS as f32 rows. The K step is
// 4 blocks of 16; within a block, MFMA slice s (K = 4) takes from lane l the k index 4 (l >> 4) + s,
// so a lane reads its 4 slices' values as one 16-byte LDS load (the same permutation of k for A and
// B leaves the sum unchanged). MFMA 16x16x4 f32: lane l holds A row (l & 15) and B column (l & 15);
// D lane l holds rows 4 (l >> 4) .. + 3 of column l & 15.
constexpr int PF_BN = 128, PF_BK = 64;
constexpr int PF_LDF = PF_BK + 4;  // LDS row stride in floats (16 bytes of padding per row)

template <int BM>
static constexpr size_t pf_gemm_lds() {
    return sizeof(float) * (size_t)(BM + PF_BN) * PF_LDF;
}

// one 128-row column tile (rows n0.., tokens t0..) of segment sg
template <int WT, int BM>
__device__ __forceinline__ void pf_gemm_tile(const PfGemm& a, const PfSeg& sg, int n0, int t0, float* sx, float* sw) {
    constexpr int WM = BM / 2;   // tokens per wave
    constexpr int TI = WM / 16;  // MFMA tiles along the tokens
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    pf_f32x4 acc[TI][4];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = pf_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // this thread's share of a K step: X pieces c = tid + 256 i, and W group (row tid % 128, group
    // tid / 128): neighbouring lanes store neighbouring rows (68-float stride, 4 banks apart), so
    // the W tile goes into LDS without bank conflicts
    constexpr int XP = BM * 16 / 256;
    const int wrow = tid & (PF_BN - 1), wgrp = tid / PF_BN, wr = n0 + wrow;
    const bool wlive = wr < sg.N;
    using Raw = typename PfW<WT>::Raw;
    float4 xr[XP];
    Raw wraw;
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XP; i++) {
            const int c = tid + 256 * i, row = c >> 4, col = (c & 15) * 4, t = t0 + row, k = k0 + col;
            xr[i] = (t < a.T && k < a.K) ? *(const float4*)(a.x + (size_t)t * a.ldx + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if (wlive && k0 + 32 * wgrp < a.K) PfW<WT>::load(wraw, sg.w, a.K, wr, k0 + 32 * wgrp);
    };
    // this workgroup's part of K (the whole row unless the launch splits K)
    const int kb = (int)blockIdx.z * a.kpart, ke = kb + a.kpart < a.K ? kb + a.kpart : a.K;
    fetch(kb);
    for (int k0 = kb; k0 < ke; k0 += PF_BK) {
        __syncthreads();  // the previous step's operands have been read
#pragma unroll
        for (int i = 0; i < XP; i++) {
            const int c = tid + 256 * i;
            *(float4*)(sx + (c >> 4) * PF_LDF + (c & 15) * 4) = xr[i];
        }
        {
            float v[32];
            const int k = k0 + 32 * wgrp;
            if (wlive && k < a.K) {
                PfW<WT>::deq(wraw, sg.w, sg.type, a.K, wr, k, v);
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) v[i] = 0.0f;
            }
            float4* dst = (float4*)(sw + wrow * PF_LDF + 32 * wgrp);
#pragma unroll
            for (int i = 0; i < 8; i++) dst[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
        }
        // the next step's global loads fly while this step multiplies
        if (k0 + PF_BK < ke) fetch(k0 + PF_BK);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < PF_BK; kk += 16) {
            const int ko = kk + 4 * (lane >> 4);
            float4 av[TI], bv[4];
#pragma unroll
            for (int i = 0; i < TI; i++) av[i] = *(const float4*)(sx + (WM * wm + 16 * i + (lane & 15)) * PF_LDF + ko);
#pragma unroll
            for (int j = 0; j < 4; j++) bv[j] = *(const float4*)(sw + (64 * wn + 16 * j + (lane & 15)) * PF_LDF + ko);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < TI; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float as = s == 0 ? av[i].x : s == 1 ? av[i].y : s == 2 ? av[i].z : av[i].w;
                        const float bs = s == 0 ? bv[j].x : s == 1 ? bv[j].y : s == 2 ? bv[j].z : bv[j].w;
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(as, bs, acc[i][j], 0, 0, 0);
                    }
        }
    }
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = t0 + WM * wm + 16 * i + 4 * (lane >> 4) + e;
                const int n = n0 + 64 * wn + 16 * j + (lane & 15);
                if (t < a.T && n < sg.N) {
                    if (blockIdx.z == 0) {
                        float* p = sg.y + (size_t)t * sg.ldy + n;
                        *p = a.add ? *p + acc[i][j][e] : acc[i][j][e];
                    } else {
                        // K part z > 0: its slice of the scratch, at y's place in the shared rows
                        const size_t col = (size_t)(sg.y - a.seg[0].y);
                        a.part[(size_t)(blockIdx.z - 1) * a.T * sg.ldy + (size_t)t * sg.ldy + col + n] = acc[i][j][e];
                    }
                }
            }
}

typedef void (*PfGemmKernel)(const PfGemm);

// y[i] += part[0][i] + part[1][i] + ... (in that order) over n = T * ldy values
__global__ __launch_bounds__(256) void k_pf_split_add(float* __restrict__ y, const float* __restrict__ part, int nsp,
                                                      int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = y[i];
        for (int z = 0; z < nsp; z++) v += part[(int64_t)z * n + i];
        y[i] = v;
    }
}

// workgroup (x, y): column tile x of the launch's segments, token tile y
__device__ __forceinline__ int pf_seg_of(const PfGemm& a, int& bx) {
    int si = 0;
    while (si + 1 < a.nseg && bx >= a.seg[si].tiles) {
        bx -= a.seg[si].tiles;
        si++;
    }
    return si;
}

// tile-interleaved Q4_K / Q6_K segments
template <int BM>
__global__ __launch_bounds__(256) void k_pf_gemm_tiles(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) float pf_lds[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    const PfSeg& sg = a.seg[si];
    if (sg.type == FLLM_TYPE_Q6_K)
        pf_gemm_tile<FLLM_TYPE_Q6_K, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_lds, pf_lds + BM * PF_LDF);
    else if (sg.type == FLLM_TYPE_Q8_0)
        pf_gemm_tile<FLLM_TYPE_Q8_0, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_lds, pf_lds + BM * PF_LDF);
    else if (sg.type == FLLM_TYPE_Q5_K)
        pf_gemm_tile<FLLM_TYPE_Q5_K, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_lds, pf_lds + BM * PF_LDF);
    else
        pf_gemm_tile<FLLM_TYPE_Q4_K, BM>(a, sg, bx * PF_BN, blockIdx.y * BM, pf_lds, pf_lds + BM * PF_LDF);
}

// GGUF-row segments, all of type RT - PF_ROWS (RT = -1: any type, element-wise)
template <int BM, int RT>
__global__ __launch_bounds__(256) void k_pf_gemm_rows(const PfGemm a) {
    extern __shared__ __attribute__((aligned(16))) float pf_lds[];
    int bx = blockIdx.x;
    const int si = pf_seg_of(a, bx);
    pf_gemm_tile<RT, BM>(a, a.seg[si], bx * PF_BN, blockIdx.y * BM, pf_lds, pf_lds + BM * PF_LDF);
}

template <int BM>
static PfGemmKernel pf_rows_kernel(int type) {
    switch (type) {
        case FLLM_TYPE_Q8_0: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_Q8_0>;
        case FLLM_TYPE_Q4_0: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_Q4_0>;
        case FLLM_TYPE_Q4_K: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_Q4_K>;
        case FLLM_TYPE_Q5_K: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_Q5_K>;
        case FLLM_TYPE_Q6_K: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_Q6_K>;
        case FLLM_TYPE_F32: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_F32>;
        case FLLM_TYPE_F16: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_F16>;
        case FLLM_TYPE_BF16: return k_pf_gemm_rows<BM, PF_ROWS + FLLM_TYPE_BF16>;
        default: return k_pf_gemm_rows<BM, -1>;
    }
}

static hipError_t pf_lds_attr(const void* k, size_t bytes) {
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

hipError_t launch_pf_gemm(PfGemm a, int n_cu, hipStream_t st) {
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
    // 128-token tiles only for grids of at least four of them per CU: the 64-token tiles fit three
    // workgroups per CU (128-token ones two), and their finer grain wins below that (gate/up at
    // 511 tokens: 896 tiles of 128 tokens ran 3% slower than 1792 of 64)
    const bool tall = col_tiles * ((a.T + 127) / 128) >= 4 * (int64_t)(n_cu > 0 ? n_cu : 256);
    PfGemmKernel k;
    if (tiles) k = tall ? k_pf_gemm_tiles<128> : k_pf_gemm_tiles<64>;
    else k = tall ? pf_rows_kernel<128>(a.seg[0].type) : pf_rows_kernel<64>(a.seg[0].type);
    const size_t lds = tall ? pf_gemm_lds<128>() : pf_gemm_lds<64>();
    hipError_t e = pf_lds_attr((const void*)k, lds);
    if (e != hipSuccess) return e;
    const int bm = tall ? 128 : 64;
    // a short grid splits K (parts of whole 512-element multiples) when the segments fill the rows
    // of one buffer side by side and the scratch holds the extra parts
    int nsplit = 1;
    if (!tall && a.part != nullptr) {
        const int64_t base = col_tiles * ((a.T + bm - 1) / bm), want = 2 * (int64_t)(n_cu > 0 ? n_cu : 256);
        bool side_by_side = true;
        int64_t off = 0;
        for (int i = 0; i < a.nseg; i++) {
            const PfSeg& g = a.seg[i];
            side_by_side = side_by_side && g.ldy == a.seg[0].ldy && g.y - a.seg[0].y == off;
            off += g.N;
        }
        side_by_side = side_by_side && off == a.seg[0].ldy;
        while (side_by_side && nsplit < 4 && base * nsplit < want && a.K % (512 * nsplit) == 0 &&
               (size_t)(2 * nsplit - 1) * (size_t)a.T * (size_t)a.seg[0].ldy <= a.part_cap)
            nsplit *= 2;
    }
    a.nsplit = nsplit;
    a.kpart = a.K / nsplit;
    dim3 grid((unsigned)col_tiles, (unsigned)((a.T + bm - 1) / bm), (unsigned)nsplit);
    k<<<grid, 256, lds, st>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess || nsplit == 1) return e;
    const int64_t n = (int64_t)a.T * a.seg[0].ldy;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 2048) blocks = 2048;
    k_pf_split_add<<<blocks, 256, 0, st>>>(a.seg[0].y, a.part, nsplit - 1, n);
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
__global__ __launch_bounds__(256) void k_pf_qkv_post(float* __restrict__ qkv, int ldq, int pos0,
                                                     const float* __restrict__ bq, const float* __restrict__ bk,
                                                     const float* __restrict__ bv, const float2* __restrict__ rope,
                                                     int nh, int nkv, int hd, float* __restrict__ kc,
                                                     float* __restrict__ vc) {
    const int t = blockIdx.x, pos = pos0 + t, half = hd >> 1, qdim = nh * hd, kvdim = nkv * hd;
    float* row = qkv + (size_t)t * ldq;
    const float2* rp = rope + (size_t)pos * half;
    const int npairs = (nh + nkv) * half;
    for (int idx = threadIdx.x; idx < npairs; idx += 256) {
        const bool isq = idx < nh * half;
        const int li = isq ? idx : idx - nh * half;
        const int head = li / half, i = li % half, o = head * hd + 2 * i;
        const float* src = row + (isq ? 0 : qdim);
        float x0 = src[o], x1 = src[o + 1];
        const float* b = isq ? bq : bk;
        if (b) { x0 = x0 + b[o]; x1 = x1 + b[o + 1]; }
        const float2 cs = rp[i];
        const float y0 = x0 * cs.x - x1 * cs.y;
        const float y1 = x0 * cs.y + x1 * cs.x;
        if (isq) {
            row[o] = y0;
            row[o + 1] = y1;
        } else {
            kc[(size_t)pos * kvdim + o] = y0;
            kc[(size_t)pos * kvdim + o + 1] = y1;
        }
    }
    for (int i = threadIdx.x; i < kvdim; i += 256) {
        float v = row[qdim + kvdim + i];
        if (bv) v = v + bv[i];
        vc[(size_t)pos * kvdim + i] = v;
    }
}

hipError_t launch_pf_qkv_post(float* qkv, int ldq, int T, int pos0, const float* bq, const float* bk, const float* bv,
                              const float2* rope, int nh, int nkv, int hd, float* kc, float* vc, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    k_pf_qkv_post<<<T, 256, 0, st>>>(qkv, ldq, pos0, bq, bk, bv, rope, nh, nkv, hd, kc, vc);
    return hipGetLastError();
}

// Gemma2 post-norm: x += GemmaRmsNorm(tmp, w), eps 1e-6 (Gemma2ForwardPass.cs:90-96)
__global__ __launch_bounds__(256) void k_pf_postnorm_add(const float* __restrict__ tmp, int n, const float* __restrict__ w,
                                                         float* __restrict__ x) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    const float* tr = tmp + (size_t)t * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(tr[i], tr[i], ss);
    const float tot = pf_block_sum(ss, red);
    const float rms = 1.0f / sqrtf(tot / (float)n + 1e-6f);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float o = (tr[i] * rms) * (w[i] + 1.0f);
        x[(size_t)t * n + i] = x[(size_t)t * n + i] + o;
    }
}

hipError_t launch_pf_postnorm_add(const float* tmp, int T, int n, const float* w, float* x, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    k_pf_postnorm_add<<<T, 256, 0, st>>>(tmp, n, w, x);
    return hipGetLastError();
}

// ---- causal attention over the cache (ComputeAttention, LlamaForwardPass.cs:158-211 and the
// Mistral / Qwen2 / Gemma2 variants) ----------------------------------------------------------------
// Workgroup = (query head, block of 8 consecutive queries), one wave per query. Keys go in blocks
// of 64 rows of the head's kv head, staged in LDS (K rows padded to HD + 1 floats so that lane j
// reading row j is conflict-free). Per block a wave scores its 64 keys (lane = key), updates the
// running max / sum (online softmax) and adds p_j v_j to its output slice (lane = dims d, d + 64, ..).
constexpr int PF_AQ = 8, PF_AK = 64;

template <int HD>
static constexpr size_t pf_attn_lds() {
    return sizeof(float) * ((size_t)PF_AK * (HD + 1) + (size_t)PF_AK * HD + PF_AQ * PF_AK + PF_AQ * HD);
}

template <int HD>
__global__ __launch_bounds__(512) void k_pf_attn(const PfAttn a) {
    constexpr int DPL = HD / 64;  // output dims per lane
    extern __shared__ float pa_lds[];
    float* sk = pa_lds;                  // [PF_AK][HD + 1]
    float* sv = sk + PF_AK * (HD + 1);   // [PF_AK][HD]
    float* sp = sv + PF_AK * HD;         // [PF_AQ][PF_AK]
    float* sq = sp + PF_AQ * PF_AK;      // [PF_AQ][HD]
    const int h = blockIdx.x, qb = blockIdx.y * PF_AQ;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kvh = h / (a.nh / a.nkv);
    const int t = qb + wave;
    const bool live = t < a.T;
    const int pos = a.pos0 + (live ? t : a.T - 1);
    const int ws = pos + 1 - a.window > 0 ? pos + 1 - a.window : 0;
    for (int d = lane; d < HD; d += 64) sq[wave * HD + d] = live ? a.q[(size_t)t * a.ldq + h * HD + d] : 0.0f;
    // keys of the workgroup: from the first query's window start to the last live query
    const int tl = (qb + PF_AQ < a.T ? qb + PF_AQ : a.T) - 1;
    const int kend = a.pos0 + tl;
    const int kstart = a.pos0 + qb + 1 - a.window > 0 ? a.pos0 + qb + 1 - a.window : 0;
    const float inv_cap = a.softcap > 0.0f ? 1.0f / a.softcap : 0.0f;
    float m = -INFINITY, l = 0.0f;
    float acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) acc[e] = 0.0f;
    for (int kb = kstart; kb <= kend; kb += PF_AK) {
        __syncthreads();  // the previous block's rows have been read (and sq is written)
        for (int c = threadIdx.x; c < PF_AK * (HD / 4); c += 512) {
            const int j = c / (HD / 4), d4 = (c % (HD / 4)) * 4;
            const int key = kb + j < kend ? kb + j : kend;
            const size_t off = (size_t)key * a.kvdim + (size_t)kvh * HD + d4;
            const float4 kv = *(const float4*)(a.kc + off);
            float* kr = sk + j * (HD + 1) + d4;
            kr[0] = kv.x; kr[1] = kv.y; kr[2] = kv.z; kr[3] = kv.w;
            *(float4*)(sv + j * HD + d4) = *(const float4*)(a.vc + off);
        }
        __syncthreads();
        if (live && kb <= pos && kb + PF_AK - 1 >= ws) {  // the block meets [ws, pos]
            const int key = kb + lane;
            const bool valid = key >= ws && key <= pos;
            float s = -INFINITY;
            if (valid) {
                float dot = 0.0f;
                const float* qr = sq + wave * HD;
                const float* kr = sk + lane * (HD + 1);
#pragma unroll 8
                for (int d = 0; d < HD; d++) dot = fmaf(qr[d], kr[d], dot);
                s = dot * a.scale;
                if (a.softcap > 0.0f) s = tanhf(s * inv_cap) * a.softcap;
            }
            const float m_new = fmaxf(m, pf_wave_max(s));
            const float corr = expf(m - m_new);
            const float p = valid ? expf(s - m_new) : 0.0f;
            l = l * corr + pf_wave_sum(p);
            sp[wave * PF_AK + lane] = p;
            pf_wave_sync();
#pragma unroll
            for (int e = 0; e < DPL; e++) acc[e] *= corr;
            for (int j = 0; j < PF_AK; j++) {
                const float pj = sp[wave * PF_AK + j];
#pragma unroll
                for (int e = 0; e < DPL; e++) acc[e] = fmaf(pj, sv[j * HD + lane + 64 * e], acc[e]);
            }
            pf_wave_sync();  // sp is rewritten for the next block
            m = m_new;
        }
    }
    if (live) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int e = 0; e < DPL; e++) a.out[(size_t)t * a.nh * HD + h * HD + lane + 64 * e] = acc[e] * inv;
    }
}

hipError_t launch_pf_attn(const PfAttn& a, hipStream_t st) {
    if (a.T <= 0) return hipSuccess;
    if (a.nkv <= 0 || a.nh % a.nkv != 0 || a.kvdim != a.nkv * a.hd) return hipErrorInvalidValue;
    dim3 grid((unsigned)a.nh, (unsigned)((a.T + PF_AQ - 1) / PF_AQ));
    hipError_t e;
    switch (a.hd) {
        case 64:
            if ((e = pf_lds_attr((const void*)k_pf_attn<64>, pf_attn_lds<64>())) != hipSuccess) return e;
            k_pf_attn<64><<<grid, 512, pf_attn_lds<64>(), st>>>(a);
            break;
        case 128:
            if ((e = pf_lds_attr((const void*)k_pf_attn<128>, pf_attn_lds<128>())) != hipSuccess) return e;
            k_pf_attn<128><<<grid, 512, pf_attn_lds<128>(), st>>>(a);
            break;
        case 256:
            if ((e = pf_lds_attr((const void*)k_pf_attn<256>, pf_attn_lds<256>())) != hipSuccess) return e;
            k_pf_attn<256><<<grid, 512, pf_attn_lds<256>(), st>>>(a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fllm
