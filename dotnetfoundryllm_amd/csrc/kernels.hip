// kernels.hip — gfx950 kernels of the decode path.
//
// Compiled with -ffp-contract=off: every a*b+c written below stays two roundings unless an
// explicit fmaf() asks for one, so the dequantized values and the RoPE rotation follow the
// reference's operation order (the .NET JIT does not contract either).
#include "kernels.hpp"

#include <math.h>

namespace fllm {

// =====================================================================================
// Byte access helpers
// =====================================================================================
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
__device__ __forceinline__ uint32_t ld_u32b(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
// Hardware binary16 -> binary32 conversion (exact for every finite input).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, bytes);
}
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// =====================================================================================
// Exact element dequantization (Dequantizer.cs:68-456), one element at a time.
// Used by fllm_dequantize, the embedding lookup, norm/bias uploads and the generic GEMV.
// =====================================================================================
__device__ float deq_elem(int type, const uint8_t* w, int64_t e) {
    switch (type) {
        case FLLM_TYPE_F32: return bits_f32(ld_u32b(w + e * 4));
        case FLLM_TYPE_F16: return half_exact(ld_u16(w + e * 2));
        case FLLM_TYPE_BF16: return bf16_exact(ld_u16(w + e * 2));
        case FLLM_TYPE_Q4_0: {  // Dequantizer.cs:172-184
            const uint8_t* p = w + (e >> 5) * 18;
            int j = (int)(e & 31);
            float d = half_exact(ld_u16(p));
            uint32_t qs = p[2 + (j & 15)];
            int q = j < 16 ? (int)(qs & 0x0F) : (int)(qs >> 4);
            return (float)(q - 8) * d;
        }
        case FLLM_TYPE_Q8_0: {  // Dequantizer.cs:220-229
            const uint8_t* p = w + (e >> 5) * 34;
            float d = half_exact(ld_u16(p));
            return (float)(int8_t)p[2 + (e & 31)] * d;
        }
        case FLLM_TYPE_Q4_K: {  // Dequantizer.cs:268-292
            const uint8_t* p = w + (e >> 8) * 144;
            int i = (int)(e & 255), g = i >> 5, ii = i & 31;
            float d = half_exact(ld_u16(p)), dmin = half_exact(ld_u16(p + 2));
            int sc, mn;
            kscale_min(p + 4, g, sc, mn);
            float dg = d * (float)sc;
            float mg = dmin * (float)mn;
            uint32_t packed = p[16 + g * 16 + (ii >> 1)];
            int q = (ii & 1) == 0 ? (int)(packed & 0x0F) : (int)(packed >> 4);
            return dg * (float)q - mg;
        }
        case FLLM_TYPE_Q5_K: {  // Dequantizer.cs:333-366
            const uint8_t* p = w + (e >> 8) * 176;
            int t = (int)(e & 255), g = t >> 5;
            float d = half_exact(ld_u16(p)), dmin = half_exact(ld_u16(p + 2));
            int sc, mn;
            kscale_min(p + 4, g, sc, mn);
            float dg = d * (float)sc;
            float mg = dmin * (float)mn;
            uint32_t pl = p[48 + (t >> 1)];
            int lo = (t & 1) == 0 ? (int)(pl & 0x0F) : (int)(pl >> 4);
            int hi = (p[16 + (t >> 3)] >> (t & 7)) & 1;
            int q = (hi << 4) | lo;
            return dg * (float)q - mg;
        }
        case FLLM_TYPE_Q6_K: {  // Dequantizer.cs:395-416
            const uint8_t* p = w + (e >> 8) * 210;
            int i = (int)(e & 255);
            uint32_t qlb = p[i >> 1];
            int low = (i & 1) == 0 ? (int)(qlb & 0x0F) : (int)(qlb >> 4);
            int high = (p[128 + (i >> 2)] >> ((i & 3) * 2)) & 3;
            int q = ((high << 4) | low) - 32;
            int scale = (int8_t)p[192 + (i >> 4)];
            float d = half_exact(ld_u16(p + 208));
            return d * (float)scale * (float)q;
        }
        case FLLM_TYPE_Q8_K: {  // Dequantizer.cs:444-455
            const uint8_t* p = w + (e >> 8) * 292;
            float d = bits_f32(ld_u32b(p));
            return (float)(int8_t)p[4 + (e & 255)] * d;
        }
        default: return 0.0f;
    }
}

__global__ void k_dequant(int type, const uint8_t* __restrict__ src, int64_t n, float* __restrict__ dst) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride) dst[e] = deq_elem(type, src, e);
}

hipError_t launch_dequant(int type, const uint8_t* src, int64_t nelem, float* dst, hipStream_t st) {
    if (nelem <= 0) return hipSuccess;
    int64_t blocks = (nelem + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    k_dequant<<<(unsigned)blocks, 256, 0, st>>>(type, src, nelem, dst);
    return hipGetLastError();
}

// =====================================================================================
// Activation quantization for the int8 dot-product GEMV.
// A group of 32 floats v is written as s = amax/127 and integers X_i = rint(v_i*127/amax*2^16)
// split into three signed base-256 digits (X = b2*65536 + b1*256 + b0), so that
// sum_i q_i v_i = s * (D2 + D1/256 + D0/65536) with D_k = sum_i q_i b_k,i computed exactly by
// v_dot4_i32_i8. The representation error is at most s*2^-17 per element (about 2^-24 of the
// group's largest magnitude), i.e. float32 resolution. Digits are stored in the element order of
// the 4-bit formats: dword k (k<4) holds elements 8k+0,2,4,6 and dword 4+k holds 8k+1,3,5,7.
// =====================================================================================
__device__ void quantize_group(const float* v, uint4* parts, float4* stats) {
    float amax = 0.0f, s16a = 0.0f, s16b = 0.0f;
    for (int i = 0; i < 16; i++) { s16a += v[i]; amax = fmaxf(amax, fabsf(v[i])); }
    for (int i = 16; i < 32; i++) { s16b += v[i]; amax = fmaxf(amax, fabsf(v[i])); }
    float s = 0.0f, inv = 0.0f;
    if (amax > 0.0f) { s = amax / 127.0f; inv = 127.0f / amax; }
    uint32_t P[24];
    for (int i = 0; i < 24; i++) P[i] = 0;
    for (int i = 0; i < 32; i++) {
        int X = (int)rintf(v[i] * inv * 65536.0f);
        int b0 = (int)(int8_t)(X & 0xFF);
        int X1 = (X - b0) >> 8;
        int b1 = (int)(int8_t)(X1 & 0xFF);
        int b2 = (X1 - b1) >> 8;
        int k = i >> 3, j = i & 7;
        int dw = ((j & 1) ? 4 : 0) + k;
        int sh = (j >> 1) * 8;
        P[dw] |= (uint32_t)(b2 & 0xFF) << sh;
        P[8 + dw] |= (uint32_t)(b1 & 0xFF) << sh;
        P[16 + dw] |= (uint32_t)(b0 & 0xFF) << sh;
    }
    for (int i = 0; i < 6; i++) parts[i] = make_uint4(P[4 * i], P[4 * i + 1], P[4 * i + 2], P[4 * i + 3]);
    *stats = make_float4(s, s16a + s16b, s16a, s16b);
}

__global__ void k_quantize(const float* __restrict__ x, int64_t groups, uint4* parts, float4* stats) {
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    float v[32];
    for (int i = 0; i < 32; i++) v[i] = x[g * 32 + i];
    quantize_group(v, parts + g * 6, stats + g);
}

hipError_t launch_quantize(const float* x, int64_t n, XQ xq, hipStream_t st) {
    int64_t groups = n / 32;
    if (groups <= 0) return hipSuccess;
    k_quantize<<<(unsigned)((groups + 127) / 128), 128, 0, st>>>(x, groups, xq.parts, xq.stats);
    return hipGetLastError();
}

// =====================================================================================
// Fused dequant-GEMV, int8 dot-product path.
// One lane owns one 32-element group column j of the row (its activation digits stay in
// 24 VGPRs for the whole kernel); a wave covers a K-slice of S <= 64 group columns; a
// workgroup has one wave per K-slice and walks rows_per_wg rows in steps of 8, so each
// lane has 8 independent block loads in flight. Row sums are reduced across lanes with a
// transposing butterfly (8 rows per 34 lane operations) and across K-slices through LDS in a
// fixed order, so results are deterministic.
// =====================================================================================

// Q4_K group: Dequantizer.cs:268-292 as dg * sum(q x) - mg * sum(x).
__device__ __forceinline__ float gdot_q4k(const uint8_t* __restrict__ W, int64_t gi, const uint32_t* xp, float4 xs) {
    const uint8_t* blk = W + (gi >> 3) * 144;
    int g = (int)(gi & 7);
    uint4 hdr = *(const uint4*)blk;
    uint4 qs = *(const uint4*)(blk + 16 + g * 16);
    float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
    int sh = (g & 3) * 8;
    uint32_t a = (hdr.y >> sh) & 0xFF, b = (hdr.z >> sh) & 0xFF, c = (hdr.w >> sh) & 0xFF;
    int sc, mn;
    if (g < 4) { sc = (int)(a & 63); mn = (int)(b & 63); }
    else { sc = (int)((c & 15) | ((a >> 6) << 4)); mn = (int)((c >> 4) | ((b >> 6) << 4)); }
    float dg = d * (float)sc, mg = dmin * (float)mn;
    uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
    int D2 = 0, D1 = 0, D0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
        D2 = sdot4(lo, xp[k], D2); D2 = sdot4(hi, xp[4 + k], D2);
        D1 = sdot4(lo, xp[8 + k], D1); D1 = sdot4(hi, xp[12 + k], D1);
        D0 = sdot4(lo, xp[16 + k], D0); D0 = sdot4(hi, xp[20 + k], D0);
    }
    float t = (float)D2 + (float)D1 * 0.00390625f + (float)D0 * 1.52587890625e-05f;
    return dg * (xs.x * t) - mg * xs.y;
}

// Q5_K group: Dequantizer.cs:333-366; high bit of element t is bit t of qh dword g.
__device__ __forceinline__ float gdot_q5k(const uint8_t* __restrict__ W, int64_t gi, const uint32_t* xp, float4 xs) {
    const uint8_t* blk = W + (gi >> 3) * 176;
    int g = (int)(gi & 7);
    uint4 hdr = *(const uint4*)blk;
    uint32_t qh = *(const uint32_t*)(blk + 16 + g * 4);
    uint4 qs = *(const uint4*)(blk + 48 + g * 16);
    float d = h2f(hdr.x & 0xFFFFu), dmin = h2f(hdr.x >> 16);
    int sh = (g & 3) * 8;
    uint32_t a = (hdr.y >> sh) & 0xFF, b = (hdr.z >> sh) & 0xFF, c = (hdr.w >> sh) & 0xFF;
    int sc, mn;
    if (g < 4) { sc = (int)(a & 63); mn = (int)(b & 63); }
    else { sc = (int)((c & 15) | ((a >> 6) << 4)); mn = (int)((c >> 4) | ((b >> 6) << 4)); }
    float dg = d * (float)sc, mg = dmin * (float)mn;
    uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
    int D2 = 0, D1 = 0, D0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t bk = (qh >> (8 * k)) & 0xFFu;
        uint32_t lo = (q[k] & 0x0F0F0F0Fu) | (((bk & 0x55u) * 0x410410u) & 0x10101010u);
        uint32_t hi = ((q[k] >> 4) & 0x0F0F0F0Fu) | ((((bk >> 1) & 0x55u) * 0x410410u) & 0x10101010u);
        D2 = sdot4(lo, xp[k], D2); D2 = sdot4(hi, xp[4 + k], D2);
        D1 = sdot4(lo, xp[8 + k], D1); D1 = sdot4(hi, xp[12 + k], D1);
        D0 = sdot4(lo, xp[16 + k], D0); D0 = sdot4(hi, xp[20 + k], D0);
    }
    float t = (float)D2 + (float)D1 * 0.00390625f + (float)D0 * 1.52587890625e-05f;
    return dg * (xs.x * t) - mg * xs.y;
}

// Spread the 2-bit fields held in nibbles 0..3 of e into bytes 0..3.
__device__ __forceinline__ uint32_t spread4(uint32_t e) {
    e = (e | (e << 8)) & 0x00FF00FFu;
    return (e | (e << 4)) & 0x0F0F0F0Fu;
}

// Q6_K 32-element chunk c of a block: Dequantizer.cs:395-416 as
// (d*sc)*(sum(q6 x) - 32 sum(x)) per 16-element scale group. Blocks are 210 bytes, so the
// block start is only 2-byte aligned: dwords are loaded from the 4-byte-aligned address
// below it and re-aligned with v_alignbyte.
__device__ __forceinline__ float gdot_q6k(const uint8_t* __restrict__ W, int64_t gi, const uint32_t* xp, float4 xs) {
    const uint8_t* blk = W + (gi >> 3) * 210;
    int c = (int)(gi & 7);
    uint32_t mis = (uint32_t)((uintptr_t)blk & 3u);
    const uint32_t* b4 = (const uint32_t*)(blk - mis);
    uint32_t l0 = b4[4 * c], l1 = b4[4 * c + 1], l2 = b4[4 * c + 2], l3 = b4[4 * c + 3], l4 = b4[4 * c + 4];
    uint32_t L[4] = {alignb(l1, l0, mis), alignb(l2, l1, mis), alignb(l3, l2, mis), alignb(l4, l3, mis)};
    uint32_t h0 = b4[32 + 2 * c], h1 = b4[33 + 2 * c], h2 = b4[34 + 2 * c];
    uint32_t H[2] = {alignb(h1, h0, mis), alignb(h2, h1, mis)};
    uint32_t so = 192u + 2u * (uint32_t)c + mis;
    uint32_t sdw = b4[so >> 2];
    uint32_t ssh = (so & 3u) * 8u;
    int sca = (int)(int8_t)((sdw >> ssh) & 0xFFu);
    int scb = (int)(int8_t)((sdw >> (ssh + 8u)) & 0xFFu);
    float d = h2f((b4[52] >> (8u * mis)) & 0xFFFFu);
    int A2 = 0, A1 = 0, A0 = 0, B2 = 0, B1 = 0, B0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t hk = (H[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
        uint32_t lo = (L[k] & 0x0F0F0F0Fu) | (spread4(hk & 0x3333u) << 4);
        uint32_t hi = ((L[k] >> 4) & 0x0F0F0F0Fu) | (spread4((hk >> 2) & 0x3333u) << 4);
        if (k < 2) {
            A2 = sdot4(lo, xp[k], A2); A2 = sdot4(hi, xp[4 + k], A2);
            A1 = sdot4(lo, xp[8 + k], A1); A1 = sdot4(hi, xp[12 + k], A1);
            A0 = sdot4(lo, xp[16 + k], A0); A0 = sdot4(hi, xp[20 + k], A0);
        } else {
            B2 = sdot4(lo, xp[k], B2); B2 = sdot4(hi, xp[4 + k], B2);
            B1 = sdot4(lo, xp[8 + k], B1); B1 = sdot4(hi, xp[12 + k], B1);
            B0 = sdot4(lo, xp[16 + k], B0); B0 = sdot4(hi, xp[20 + k], B0);
        }
    }
    float ta = (float)A2 + (float)A1 * 0.00390625f + (float)A0 * 1.52587890625e-05f;
    float tb = (float)B2 + (float)B1 * 0.00390625f + (float)B0 * 1.52587890625e-05f;
    float ra = xs.x * ta - 32.0f * xs.z;
    float rb = xs.x * tb - 32.0f * xs.w;
    return (d * (float)sca) * ra + (d * (float)scb) * rb;
}

// Q8_0 block (34 bytes, 2-byte aligned): Dequantizer.cs:220-229 as d * sum(q x).
__device__ __forceinline__ float gdot_q8_0(const uint8_t* __restrict__ W, int64_t gi, const uint32_t* xp, float4 xs) {
    const uint8_t* blk = W + gi * 34;
    uint32_t mis = (uint32_t)((uintptr_t)blk & 3u);
    const uint32_t* b4 = (const uint32_t*)(blk - mis);
    uint32_t dw[10];
#pragma unroll
    for (int i = 0; i < 10; i++) dw[i] = b4[i];
    float d = h2f((dw[0] >> (8u * mis)) & 0xFFFFu);
    bool shifted = mis != 0;  // qs start: byte mis+2 -> dword (mis+2)>>2, shift (mis+2)&3
    uint32_t qv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) qv[i] = shifted ? dw[i + 1] : alignb(dw[i + 1], dw[i], 2);
    int D2 = 0, D1 = 0, D0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t ev = __builtin_amdgcn_perm(qv[2 * k + 1], qv[2 * k], 0x06040200u);
        uint32_t od = __builtin_amdgcn_perm(qv[2 * k + 1], qv[2 * k], 0x07050301u);
        D2 = sdot4(ev, xp[k], D2); D2 = sdot4(od, xp[4 + k], D2);
        D1 = sdot4(ev, xp[8 + k], D1); D1 = sdot4(od, xp[12 + k], D1);
        D0 = sdot4(ev, xp[16 + k], D0); D0 = sdot4(od, xp[20 + k], D0);
    }
    float t = (float)D2 + (float)D1 * 0.00390625f + (float)D0 * 1.52587890625e-05f;
    return d * (xs.x * t);
}

// Q4_0 block (18 bytes): Dequantizer.cs:172-184 as d * (sum(q x) - 8 sum(x)); low nibble of
// byte j is element j, high nibble element j+16.
__device__ __forceinline__ float gdot_q4_0(const uint8_t* __restrict__ W, int64_t gi, const uint32_t* xp, float4 xs) {
    const uint8_t* blk = W + gi * 18;
    uint32_t mis = (uint32_t)((uintptr_t)blk & 3u);
    const uint32_t* b4 = (const uint32_t*)(blk - mis);
    uint32_t dw[5];
#pragma unroll
    for (int i = 0; i < 5; i++) dw[i] = b4[i];
    float d = h2f((dw[0] >> (8u * mis)) & 0xFFFFu);
    bool shifted = mis != 0;
    uint32_t qv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) qv[i] = shifted ? dw[i + 1] : alignb(dw[i + 1], dw[i], 2);
    uint32_t nib[8];
#pragma unroll
    for (int i = 0; i < 4; i++) { nib[i] = qv[i] & 0x0F0F0F0Fu; nib[4 + i] = (qv[i] >> 4) & 0x0F0F0F0Fu; }
    int D2 = 0, D1 = 0, D0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t ev = __builtin_amdgcn_perm(nib[2 * k + 1], nib[2 * k], 0x06040200u);
        uint32_t od = __builtin_amdgcn_perm(nib[2 * k + 1], nib[2 * k], 0x07050301u);
        D2 = sdot4(ev, xp[k], D2); D2 = sdot4(od, xp[4 + k], D2);
        D1 = sdot4(ev, xp[8 + k], D1); D1 = sdot4(od, xp[12 + k], D1);
        D0 = sdot4(ev, xp[16 + k], D0); D0 = sdot4(od, xp[20 + k], D0);
    }
    float t = (float)D2 + (float)D1 * 0.00390625f + (float)D0 * 1.52587890625e-05f;
    return d * (xs.x * t - 8.0f * xs.y);
}

template <int T>
__device__ __forceinline__ float gdot(const uint8_t* __restrict__ W, int64_t gi, const uint32_t* xp, float4 xs) {
    if constexpr (T == FLLM_TYPE_Q4_K) return gdot_q4k(W, gi, xp, xs);
    else if constexpr (T == FLLM_TYPE_Q5_K) return gdot_q5k(W, gi, xp, xs);
    else if constexpr (T == FLLM_TYPE_Q6_K) return gdot_q6k(W, gi, xp, xs);
    else if constexpr (T == FLLM_TYPE_Q8_0) return gdot_q8_0(W, gi, xp, xs);
    else return gdot_q4_0(W, gi, xp, xs);
}

// Sum 8 per-lane values over the 64 lanes of a wave; lane l ends with the total of
// row ((l>>5)&1)*4 + ((l>>4)&1)*2 + ((l>>3)&1).
__device__ __forceinline__ float transpose_reduce8(const float* acc, int lane) {
    float v[4], w[2];
    bool b = (lane & 32) != 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float keep = b ? acc[i + 4] : acc[i];
        float send = b ? acc[i] : acc[i + 4];
        v[i] = keep + __shfl_xor(send, 32);
    }
    b = (lane & 16) != 0;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        float keep = b ? v[i + 2] : v[i];
        float send = b ? v[i] : v[i + 2];
        w[i] = keep + __shfl_xor(send, 16);
    }
    b = (lane & 8) != 0;
    float keep = b ? w[1] : w[0];
    float send = b ? w[0] : w[1];
    float u = keep + __shfl_xor(send, 8);
    u += __shfl_xor(u, 4);
    u += __shfl_xor(u, 2);
    u += __shfl_xor(u, 1);
    return u;
}

template <int T>
__global__ __launch_bounds__(1024) void k_gemv_q(const uint8_t* __restrict__ W, int rows, int G, int S,
                                                  int rows_per_wg, const uint4* __restrict__ xq,
                                                  const float4* __restrict__ xs, float* y,
                                                  const float* residual) {
    extern __shared__ float part[];  // [nslice][rows_per_wg]
    int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int nslice = blockDim.x >> 6;
    int j = wave * S + lane;
    bool active = lane < S && j < G;
    uint32_t xp[24];
    float4 st = make_float4(0.f, 0.f, 0.f, 0.f);
    if (active) {
#pragma unroll
        for (int i = 0; i < 6; i++) {
            uint4 u = xq[(int64_t)j * 6 + i];
            xp[4 * i] = u.x; xp[4 * i + 1] = u.y; xp[4 * i + 2] = u.z; xp[4 * i + 3] = u.w;
        }
        st = xs[j];
    } else {
#pragma unroll
        for (int i = 0; i < 24; i++) xp[i] = 0;
    }
    int r0 = blockIdx.x * rows_per_wg;
    for (int rb = 0; rb < rows_per_wg; rb += 8) {
        float acc[8];
#pragma unroll
        for (int rr = 0; rr < 8; rr++) {
            int r = r0 + rb + rr;
            acc[rr] = (active && r < rows) ? gdot<T>(W, (int64_t)r * G + j, xp, st) : 0.0f;
        }
        float tot = transpose_reduce8(acc, lane);
        if ((lane & 7) == 0) {
            int rr = ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
            part[wave * rows_per_wg + rb + rr] = tot;
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < rows_per_wg; t += blockDim.x) {
        int r = r0 + t;
        if (r < rows) {
            float s = 0.0f;
            for (int sl = 0; sl < nslice; sl++) s += part[sl * rows_per_wg + t];
            y[r] = residual ? residual[r] + s : s;
        }
    }
}

// =====================================================================================
// Float GEMV for F32 / F16 / BF16 weights (128-bit row loads; x from L2).
// =====================================================================================
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <int T>
__global__ __launch_bounds__(256) void k_gemv_f(const uint8_t* __restrict__ W, int64_t rows, int64_t cols,
                                                 const float* __restrict__ x, float* y, const float* residual) {
    int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= rows) return;
    constexpr int esz = (T == FLLM_TYPE_F32) ? 4 : 2;
    constexpr int per = 16 / esz;
    const uint4* rp = (const uint4*)(W + row * cols * esz);
    int64_t nvec = cols / per;
    const float4* x4 = (const float4*)x;
    float acc = 0.0f;
    for (int64_t v = lane; v < nvec; v += 64) {
        uint4 u = rp[v];
        if constexpr (T == FLLM_TYPE_F32) {
            float4 xv = x4[v];
            acc = fmaf(__uint_as_float(u.x), xv.x, acc);
            acc = fmaf(__uint_as_float(u.y), xv.y, acc);
            acc = fmaf(__uint_as_float(u.z), xv.z, acc);
            acc = fmaf(__uint_as_float(u.w), xv.w, acc);
        } else {
            float4 xa = x4[2 * v], xb = x4[2 * v + 1];
            uint32_t wd[4] = {u.x, u.y, u.z, u.w};
            float xs8[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float w0, w1;
                if constexpr (T == FLLM_TYPE_BF16) {
                    w0 = __uint_as_float(wd[i] << 16);
                    w1 = __uint_as_float(wd[i] & 0xFFFF0000u);
                } else {
                    w0 = h2f(wd[i] & 0xFFFFu);
                    w1 = h2f(wd[i] >> 16);
                }
                acc = fmaf(w0, xs8[2 * i], acc);
                acc = fmaf(w1, xs8[2 * i + 1], acc);
            }
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = residual ? residual[row] + acc : acc;
}

// Any type, any shape: element-wise exact dequant (slow path for Q8_K and odd shapes).
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t* __restrict__ W, int type, int64_t rows,
                                                       int64_t cols, const float* __restrict__ x, float* y,
                                                       const float* residual) {
    int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= rows) return;
    float acc = 0.0f;
    for (int64_t c = lane; c < cols; c += 64) acc = fmaf(deq_elem(type, W, row * cols + c), x[c], acc);
    acc = wave_sum(acc);
    if (lane == 0) y[row] = residual ? residual[row] + acc : acc;
}

hipError_t launch_gemv(const WMat& m, const float* xf, const XQ& xq, float* y, const float* residual,
                       hipStream_t st) {
    int t = m.type;
    // the int8 path holds one 32-element group column per lane and at most 16 waves per
    // workgroup, so it covers rows of up to 1024 groups (32768 elements)
    bool qpath = (t == FLLM_TYPE_Q4_K || t == FLLM_TYPE_Q5_K || t == FLLM_TYPE_Q6_K || t == FLLM_TYPE_Q8_0 ||
                  t == FLLM_TYPE_Q4_0) &&
                 (m.cols % 32 == 0) && m.cols <= 32768 && xq.parts != nullptr;
    if (qpath) {
        int G = (int)(m.cols / 32);
        int nslice = (G + 63) / 64;
        int S = (G + nslice - 1) / nslice;
        int rows_per_wg = m.rows >= 4096 ? 16 : 8;
        int grid = (int)((m.rows + rows_per_wg - 1) / rows_per_wg);
        size_t lds = sizeof(float) * (size_t)nslice * rows_per_wg;
        dim3 blk(64 * nslice);
        switch (t) {
            case FLLM_TYPE_Q4_K:
                k_gemv_q<FLLM_TYPE_Q4_K><<<grid, blk, lds, st>>>(m.w, (int)m.rows, G, S, rows_per_wg, xq.parts, xq.stats, y, residual);
                break;
            case FLLM_TYPE_Q5_K:
                k_gemv_q<FLLM_TYPE_Q5_K><<<grid, blk, lds, st>>>(m.w, (int)m.rows, G, S, rows_per_wg, xq.parts, xq.stats, y, residual);
                break;
            case FLLM_TYPE_Q6_K:
                k_gemv_q<FLLM_TYPE_Q6_K><<<grid, blk, lds, st>>>(m.w, (int)m.rows, G, S, rows_per_wg, xq.parts, xq.stats, y, residual);
                break;
            case FLLM_TYPE_Q8_0:
                k_gemv_q<FLLM_TYPE_Q8_0><<<grid, blk, lds, st>>>(m.w, (int)m.rows, G, S, rows_per_wg, xq.parts, xq.stats, y, residual);
                break;
            default:
                k_gemv_q<FLLM_TYPE_Q4_0><<<grid, blk, lds, st>>>(m.w, (int)m.rows, G, S, rows_per_wg, xq.parts, xq.stats, y, residual);
                break;
        }
        return hipGetLastError();
    }
    unsigned grid = (unsigned)((m.rows + 3) / 4);
    if (t == FLLM_TYPE_F32 && m.cols % 4 == 0)
        k_gemv_f<FLLM_TYPE_F32><<<grid, 256, 0, st>>>(m.w, m.rows, m.cols, xf, y, residual);
    else if (t == FLLM_TYPE_F16 && m.cols % 8 == 0)
        k_gemv_f<FLLM_TYPE_F16><<<grid, 256, 0, st>>>(m.w, m.rows, m.cols, xf, y, residual);
    else if (t == FLLM_TYPE_BF16 && m.cols % 8 == 0)
        k_gemv_f<FLLM_TYPE_BF16><<<grid, 256, 0, st>>>(m.w, m.rows, m.cols, xf, y, residual);
    else
        k_gemv_generic<<<grid, 256, 0, st>>>(m.w, t, m.rows, m.cols, xf, y, residual);
    return hipGetLastError();
}

// =====================================================================================
// Step parameters, embedding, norms
// =====================================================================================
__global__ void k_set_params(StepParams* p, int token, int pos, int cur_len) {
    p->token = token;
    p->pos = pos;
    p->cur_len = cur_len;
    p->argmax = -1;
}

hipError_t launch_set_params(StepParams* p, int token, int pos, int cur_len, hipStream_t st) {
    k_set_params<<<1, 1, 0, st>>>(p, token, pos, cur_len);
    return hipGetLastError();
}

// x = E[token] (LlamaForwardPass.cs:96); the row is dequantized exactly.
__global__ void k_embed(const uint8_t* __restrict__ emb, int type, int hidden, const StepParams* p, float* x) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    x[i] = deq_elem(type, emb, (int64_t)p->token * hidden + i);
}

hipError_t launch_embed(const uint8_t* emb, int type, int hidden, const StepParams* p, float* x, hipStream_t st) {
    k_embed<<<(hidden + 255) / 256, 256, 0, st>>>(emb, type, hidden, p, x);
    return hipGetLastError();
}

__device__ float block_sum(float v, float* red) {
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// RmsNorm (TensorOperations.cs:42-54) or GemmaRmsNorm (TensorOperations.cs:90-107), then the
// quantized copy of the normed vector for the next GEMV.
__global__ __launch_bounds__(1024) void k_rmsnorm_q(const float* __restrict__ x, const float* __restrict__ w, int n,
                                                     float eps, int kind, float* xn, uint4* parts, float4* stats) {
    extern __shared__ float sh[];  // n + 16
    float* red = sh + n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = x[i];
        sh[i] = v;
        ss = fmaf(v, v, ss);
    }
    float tot = block_sum(ss, red);
    float rms = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float t = sh[i] * rms;
        float o = kind ? t * (w[i] + 1.0f) : t * w[i];
        xn[i] = o;
        sh[i] = o;
    }
    __syncthreads();
    if (parts)
        for (int g = threadIdx.x; g < n / 32; g += blockDim.x) quantize_group(sh + g * 32, parts + g * 6, stats + g);
}

hipError_t launch_rmsnorm_q(const float* x, const float* w, int n, float eps, int norm_kind, float* xn, XQ xq,
                            hipStream_t st) {
    size_t lds = sizeof(float) * ((size_t)n + 16);
    k_rmsnorm_q<<<1, 1024, lds, st>>>(x, w, n, eps, norm_kind, xn, (n % 32 == 0) ? xq.parts : nullptr, xq.stats);
    return hipGetLastError();
}

// q/k/v bias (Qwen2ForwardPass.cs:83-85), RoPE with a host-built cos/sin table
// (TensorOperations.cs:250-260, interleaved pairs), then KvCache.Append (KvCache.cs:86-89).
__global__ void k_qkv_post(float* q, float* k, float* v, const float* bq, const float* bk, const float* bv,
                           const float2* __restrict__ rope, int nh, int nkv, int hd, float* kc, float* vc,
                           const StepParams* p) {
    int half = hd / 2;
    int kvdim = nkv * hd;
    int pos = p->pos, slot = p->cur_len;
    const float2* rp = rope + (int64_t)pos * half;
    int npairs = (nh + nkv) * half;
    int tid = blockIdx.x * blockDim.x + threadIdx.x;
    int nthr = gridDim.x * blockDim.x;
    for (int idx = tid; idx < npairs; idx += nthr) {
        bool isq = idx < nh * half;
        int li = isq ? idx : idx - nh * half;
        int head = li / half, i = li % half;
        float* vec = isq ? q : k;
        const float* bias = isq ? bq : bk;
        int o = head * hd + 2 * i;
        float x0 = vec[o], x1 = vec[o + 1];
        if (bias) { x0 = x0 + bias[o]; x1 = x1 + bias[o + 1]; }
        float2 cs = rp[i];
        float y0 = x0 * cs.x - x1 * cs.y;
        float y1 = x0 * cs.y + x1 * cs.x;
        vec[o] = y0;
        vec[o + 1] = y1;
        if (!isq) {
            kc[(int64_t)slot * kvdim + o] = y0;
            kc[(int64_t)slot * kvdim + o + 1] = y1;
        }
    }
    for (int idx = tid; idx < kvdim; idx += nthr) {
        float vv = v[idx];
        if (bv) vv = vv + bv[idx];
        v[idx] = vv;
        vc[(int64_t)slot * kvdim + idx] = vv;
    }
}

hipError_t launch_qkv_post(float* q, float* k, float* v, const float* bq, const float* bk, const float* bv,
                           const float2* rope, int n_heads, int n_kv, int head_dim, float* kcache, float* vcache,
                           const StepParams* p, hipStream_t st) {
    int work = (n_heads + n_kv) * head_dim / 2;
    int blocks = (work + 255) / 256;
    k_qkv_post<<<blocks, 256, 0, st>>>(q, k, v, bq, bk, bv, rope, n_heads, n_kv, head_dim, kcache, vcache, p);
    return hipGetLastError();
}

// =====================================================================================
// Attention: ComputeAttention (LlamaForwardPass.cs:158-211; Mistral window
// MistralForwardPass.cs:131; Gemma2 scale/softcap/window Gemma2ForwardPass.cs:126-185)
// as split-K decoding: workgroup (kv head, split) scores a contiguous slice of the attended
// range for the whole query group of that kv head (K/V rows read once per group).
// =====================================================================================
__global__ __launch_bounds__(256) void k_attn_partial(const float* __restrict__ q, const float* __restrict__ kc,
                                                       const float* __restrict__ vc, int nh, int nkv, int hd,
                                                       int window, float scale, float softcap, int nsplit,
                                                       int chunk_cap, float* part_o, float* part_ml,
                                                       const StepParams* p) {
    extern __shared__ float sh[];
    int kvh = blockIdx.x, split = blockIdx.y;
    int group = nh / nkv, kvdim = nkv * hd;
    int seq = p->pos + 1;
    int ws = seq - window;
    if (ws < 0) ws = 0;
    int alen = seq - ws;
    int chunk = (alen + nsplit - 1) / nsplit;
    int t0 = ws + split * chunk;
    int t1 = min(t0 + chunk, seq);
    int len = t1 - t0;
    int h0 = kvh * group;
    if (len <= 0) {
        for (int h = threadIdx.x; h < group; h += blockDim.x) {
            part_ml[((int64_t)(h0 + h) * nsplit + split) * 2] = -INFINITY;
            part_ml[((int64_t)(h0 + h) * nsplit + split) * 2 + 1] = 0.0f;
        }
        return;
    }
    float* qs = sh;                    // group * hd
    float* sc = sh + group * hd;       // group * chunk_cap
    for (int i = threadIdx.x; i < group * hd; i += blockDim.x) qs[i] = q[(int64_t)h0 * hd + i];
    __syncthreads();
    float inv_cap = softcap > 0.0f ? 1.0f / softcap : 0.0f;
    for (int idx = threadIdx.x; idx < group * len; idx += blockDim.x) {
        int h = idx / len, t = idx % len;
        const float4* kr = (const float4*)(kc + (int64_t)(t0 + t) * kvdim + (int64_t)kvh * hd);
        const float4* qq = (const float4*)(qs + h * hd);
        float s = 0.0f;
        for (int d4 = 0; d4 < hd / 4; d4++) {
            float4 kv = kr[d4], qv = qq[d4];
            s = fmaf(qv.x, kv.x, s);
            s = fmaf(qv.y, kv.y, s);
            s = fmaf(qv.z, kv.z, s);
            s = fmaf(qv.w, kv.w, s);
        }
        s = s * scale;
        if (softcap > 0.0f) s = tanhf(s * inv_cap) * softcap;
        sc[h * chunk_cap + t] = s;
    }
    __syncthreads();
    int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int h = wave; h < group; h += nw) {
        float m = -INFINITY;
        for (int t = lane; t < len; t += 64) m = fmaxf(m, sc[h * chunk_cap + t]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        float l = 0.0f;
        for (int t = lane; t < len; t += 64) {
            float e = expf(sc[h * chunk_cap + t] - m);
            sc[h * chunk_cap + t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            part_ml[((int64_t)(h0 + h) * nsplit + split) * 2] = m;
            part_ml[((int64_t)(h0 + h) * nsplit + split) * 2 + 1] = l;
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < group * hd; idx += blockDim.x) {
        int h = idx / hd, dd = idx % hd;
        const float* vp = vc + (int64_t)t0 * kvdim + (int64_t)kvh * hd + dd;
        float o = 0.0f;
        for (int t = 0; t < len; t++) o = fmaf(sc[h * chunk_cap + t], vp[(int64_t)t * kvdim], o);
        part_o[((int64_t)(h0 + h) * nsplit + split) * hd + dd] = o;
    }
}

__global__ __launch_bounds__(256) void k_attn_combine(const float* __restrict__ part_o,
                                                       const float* __restrict__ part_ml, int nsplit, int hd,
                                                       float* out, uint4* parts, float4* stats) {
    __shared__ float sh[256];
    int h = blockIdx.x, d = threadIdx.x;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) {
        float l = part_ml[((int64_t)h * nsplit + s) * 2 + 1];
        if (l > 0.0f) M = fmaxf(M, part_ml[((int64_t)h * nsplit + s) * 2]);
    }
    float L = 0.0f, o = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        float l = part_ml[((int64_t)h * nsplit + s) * 2 + 1];
        if (l > 0.0f) {
            float wgt = expf(part_ml[((int64_t)h * nsplit + s) * 2] - M);
            L += l * wgt;
            if (d < hd) o = fmaf(part_o[((int64_t)h * nsplit + s) * hd + d], wgt, o);
        }
    }
    float r = o / L;
    if (d < hd) {
        out[(int64_t)h * hd + d] = r;
        sh[d] = r;
    }
    __syncthreads();
    int ng = hd / 32;
    if (parts && d < ng) quantize_group(sh + d * 32, parts + ((int64_t)h * ng + d) * 6, stats + (int64_t)h * ng + d);
}

hipError_t launch_attention(const float* q, const float* kcache, const float* vcache, int n_heads, int n_kv,
                            int head_dim, int window, float scale, float softcap, int nsplit, float* part_o,
                            float* part_ml, float* out, XQ out_q, const StepParams* p, hipStream_t st) {
    int group = n_heads / n_kv;
    int chunk_cap = 256;
    size_t lds = sizeof(float) * ((size_t)group * head_dim + (size_t)group * chunk_cap);
    dim3 grid(n_kv, nsplit);
    k_attn_partial<<<grid, 256, lds, st>>>(q, kcache, vcache, n_heads, n_kv, head_dim, window, scale, softcap,
                                            nsplit, chunk_cap, part_o, part_ml, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    int bs = head_dim < 64 ? 64 : head_dim;
    k_attn_combine<<<n_heads, bs, 0, st>>>(part_o, part_ml, nsplit, head_dim, out,
                                           (head_dim % 32 == 0) ? out_q.parts : nullptr, out_q.stats);
    return hipGetLastError();
}

// =====================================================================================
// FFN gating: ComputeSiluFfn (LlamaForwardPass.cs:217-232), ComputeGeluFfn
// (Gemma2ForwardPass.cs:187-199); Silu/Gelu from TensorOperations.cs:57-117.
// =====================================================================================
__global__ __launch_bounds__(256) void k_act(const float* __restrict__ g, const float* __restrict__ u, int n,
                                              int act, float* h, uint4* parts, float4* stats) {
    __shared__ float sh[256];
    int i = blockIdx.x * 256 + threadIdx.x;
    float hv = 0.0f;
    if (i < n) {
        float gv = g[i];
        float a;
        if (act == 0) {
            float sig = 1.0f / (1.0f + expf(-gv));
            a = gv * sig;
        } else {
            float inner = 0.7978845608f * (gv + 0.044715f * gv * gv * gv);
            a = 0.5f * gv * (1.0f + tanhf(inner));
        }
        hv = a * u[i];
        h[i] = hv;
    }
    sh[threadIdx.x] = hv;
    __syncthreads();
    int gidx = blockIdx.x * 8 + threadIdx.x;
    if (parts && threadIdx.x < 8 && (gidx + 1) * 32 <= n)
        quantize_group(sh + threadIdx.x * 32, parts + (int64_t)gidx * 6, stats + gidx);
}

hipError_t launch_act(const float* g, const float* u, int n, int act, float* h, XQ hq, hipStream_t st) {
    k_act<<<(n + 255) / 256, 256, 0, st>>>(g, u, n, act, h, (n % 32 == 0) ? hq.parts : nullptr, hq.stats);
    return hipGetLastError();
}

// Gemma2 post-norms: x += GemmaRmsNorm(t, w) (Gemma2ForwardPass.cs:90-91, 95-96).
__global__ __launch_bounds__(1024) void k_postnorm_add(const float* __restrict__ t, const float* __restrict__ w,
                                                        int n, float* x) {
    __shared__ float red[16];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(t[i], t[i], ss);
    float tot = block_sum(ss, red);
    float rms = 1.0f / sqrtf(tot / (float)n + 1e-6f);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float o = (t[i] * rms) * (w[i] + 1.0f);
        x[i] = x[i] + o;
    }
}

hipError_t launch_postnorm_add(const float* t, const float* w, int n, float* x, hipStream_t st) {
    k_postnorm_add<<<1, 1024, 0, st>>>(t, w, n, x);
    return hipGetLastError();
}

// SoftCap (TensorOperations.cs:120-126).
__global__ void k_softcap(float* x, int64_t n, float cap) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float inv = 1.0f / cap;
    x[i] = tanhf(x[i] * inv) * cap;
}

hipError_t launch_softcap(float* x, int64_t n, float cap, hipStream_t st) {
    k_softcap<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(x, n, cap);
    return hipGetLastError();
}

// =====================================================================================
// Sampling: ArgMax (TensorOperations.cs:187-195 -> IndexOfMax) and top-k selection
// (TopKSampler.ApplyTopK, TopKSampler.cs:42-71).
// =====================================================================================
// Order-preserving key: NaN above everything, +0 above -0.
__device__ __forceinline__ uint32_t okey(float v) {
    uint32_t b = __float_as_uint(v);
    if (v != v) return 0xFFFFFFFFu;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int64_t n, StepParams* p) {
    __shared__ uint32_t sk[16];
    __shared__ int64_t si[16];
    uint32_t bk = 0;
    int64_t bi = -1;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        uint32_t k = okey(x[i]);
        if (bi < 0 || k > bk) { bk = k; bi = i; }
    }
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t ok = __shfl_xor(bk, o);
        int64_t oi = __shfl_xor(bi, o);
        bool take = oi >= 0 && (bi < 0 || ok > bk || (ok == bk && oi < bi));
        if (take) { bk = ok; bi = oi; }
    }
    if (lane == 0) { sk[wave] = bk; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t k = sk[0];
        int64_t idx = si[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) {
            if (si[w] >= 0 && (idx < 0 || sk[w] > k || (sk[w] == k && si[w] < idx))) { k = sk[w]; idx = si[w]; }
        }
        p->argmax = (int)idx;
    }
}

hipError_t launch_argmax(const float* x, int64_t n, StepParams* p, hipStream_t st) {
    k_argmax<<<1, 1024, 0, st>>>(x, n, p);
    return hipGetLastError();
}

// Scale by inv_temp in place (SamplerPipeline.cs:67-70), find the k-th largest value by a
// 4-pass radix select on order-preserving keys, and emit every index whose value is not
// below it (ties kept), in ascending index order.
__global__ __launch_bounds__(1024) void k_topk(float* x, int64_t n, float inv_temp, int k, int cap, int* ids,
                                                float* vals, int* count) {
    __shared__ int hist[256];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remain;
    __shared__ int scan[1024];
    int tid = threadIdx.x, nt = blockDim.x;
    if (inv_temp != 1.0f) {
        for (int64_t i = tid; i < n; i += nt) x[i] = x[i] * inv_temp;
        __threadfence_block();
    }
    if (tid == 0) { s_prefix = 0; s_mask = 0; s_remain = k; }
    __syncthreads();
    uint32_t thr = 0;
    if (k < n) {
        for (int pass = 0; pass < 4; pass++) {
            int shift = 24 - 8 * pass;
            for (int b = tid; b < 256; b += nt) hist[b] = 0;
            __syncthreads();
            uint32_t prefix = s_prefix, mask = s_mask;
            for (int64_t i = tid; i < n; i += nt) {
                uint32_t key = okey(x[i]);
                if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, rem = s_remain;
                for (int b = 255; b >= 0; b--) {
                    if (cum + hist[b] >= rem) {
                        s_prefix = prefix | ((uint32_t)b << shift);
                        s_mask = mask | (255u << shift);
                        s_remain = rem - cum;
                        break;
                    }
                    cum += hist[b];
                }
            }
            __syncthreads();
        }
        thr = s_prefix;
    }
    // stable compaction: thread t owns indices [t*per, (t+1)*per)
    int64_t per = (n + nt - 1) / nt;
    int64_t beg = (int64_t)tid * per, end = min(beg + per, n);
    int c = 0;
    for (int64_t i = beg; i < end; i++) c += okey(x[i]) >= thr ? 1 : 0;
    scan[tid] = c;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int t = 0; t < nt; t++) { int v = scan[t]; scan[t] = run; run += v; }
        *count = run;
    }
    __syncthreads();
    int off = scan[tid];
    for (int64_t i = beg; i < end; i++) {
        float v = x[i];
        if (okey(v) >= thr) {
            if (off < cap) { ids[off] = (int)i; vals[off] = v; }
            off++;
        }
    }
}

hipError_t launch_topk(float* x, int64_t n, float inv_temp, int k, int cap, int* ids, float* vals, int* count,
                       hipStream_t st) {
    k_topk<<<1, 1024, 0, st>>>(x, n, inv_temp, k, cap, ids, vals, count);
    return hipGetLastError();
}

__global__ void k_copy(const float* __restrict__ x, int n, float* dst) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = x[i];
}

hipError_t launch_copy_hidden(const float* x, int n, float* dst, hipStream_t st) {
    k_copy<<<(n + 255) / 256, 256, 0, st>>>(x, n, dst);
    return hipGetLastError();
}

}  // namespace fllm
