// gemv.hip — fused dequant-GEMV for the decode step (gfx950).
//
// LinearProjection (LlamaForwardPass.cs:237-260: y[i] = Dot(x, W[i])) over weights kept in their
// GGUF block layout, with the producer and consumer ops of each projection fused in:
//   prologue  x source: an F32 vector, RmsNorm / GemmaRmsNorm of the residual stream
//             (TensorOperations.cs:42-54, 90-107), or the embedding row of the step's token
//             (LlamaForwardPass.cs:96) followed by the norm;
//   epilogue  plain store (+ Qwen2 bias, Qwen2ForwardPass.cs:83-85), residual add
//             (LlamaForwardPass.cs:119,124), RoPE of q / k (TensorOperations.cs:250-260) with the
//             K/V cache store (KvCache.cs:86-89), SiLU/GELU gating of gate and up
//             (LlamaForwardPass.cs:217-232, Gemma2ForwardPass.cs:187-199), or LM-head logits with
//             the final softcap (Gemma2ForwardPass.cs:101-104) and each workgroup's share of
//             the greedy argmax (TensorOperations.cs:187-195).
//
// Work split. A row is G = cols/32 groups of 32 elements. A workgroup has nslice waves; lane
// `lane` of wave `w` owns group column j = w*S + lane for every row it visits, so the
// activation digits of that column stay in VGPRs for the whole kernel. The workgroup walks its
// row slots in batches of 8 rows: first the raw block words of all 8 rows are loaded (8
// independent loads per lane in flight), then they are dequantized and dotted in registers.
// Row sums are reduced across lanes by a transposing butterfly and across waves through LDS in
// a fixed order, so every result is deterministic.
//
// Activation representation. Each 32-element group v of the (normed) input is held as a scale
// s = amax/127 and integers X_i = rint(v_i * 2^16 / s) split into three signed base-256 digits,
// so sum_i q_i v_i = s * (D2 + D1/256 + D0/65536) with each D_k an exact v_dot4_i32_i8 sum over
// the integer weights q. The representation error is at most 2^-17 * s per element (about 2^-24
// of the group's largest magnitude), float32 resolution.
#include "gemv.hpp"

#include <math.h>

namespace fllm {

// ---- small helpers ----------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t alignb(uint32_t hi, uint32_t lo, uint32_t bytes) {
    return __builtin_amdgcn_alignbyte(hi, lo, bytes);
}
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
__device__ __forceinline__ float wsum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
// Order-preserving key of a float: NaN above everything, +0 above -0.
__device__ __forceinline__ uint32_t fkey(float v) {
    uint32_t b = __float_as_uint(v);
    if (v != v) return 0xFFFFFFFFu;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// 32 consecutive elements [e0, e0+32) of an F32 / F16 / BF16 row, exactly widened
// (Dequantizer.cs:68-137), with 16-byte loads (e0 is a multiple of 32). Quantized embedding
// rows are produced by a separate lookup kernel before the first projection.
__device__ __forceinline__ void deq32(int type, const uint8_t* __restrict__ w, int64_t e0, float* v) {
    if (type == FLLM_TYPE_F32) {
        const float4* p = (const float4*)(w + e0 * 4);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 t = p[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
    } else {
        const bool bf = type == FLLM_TYPE_BF16;
        const uint4* p = (const uint4*)(w + e0 * 2);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint4 t = p[i];
            uint32_t d[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                v[8 * i + 2 * k] = bf ? bf16_exact(d[k] & 0xFFFFu) : half_exact(d[k] & 0xFFFFu);
                v[8 * i + 2 * k + 1] = bf ? bf16_exact(d[k] >> 16) : half_exact(d[k] >> 16);
            }
        }
    }
}

// ---- activation digits ---------------------------------------------------------------------
// Digits are stored in the element order of the 4-bit formats: dword k (k<4) holds elements
// 8k+0,2,4,6 and dword 4+k holds 8k+1,3,5,7; xp[0..7] high digit, [8..15] middle, [16..23] low.
// st = {s, sum of the 32 values, sum of elements 0..15, sum of elements 16..31}.
__device__ __forceinline__ void quantize32(const float* v, uint32_t* xp, float4& st) {
    float amax = 0.0f, s16a = 0.0f, s16b = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) { s16a += v[i]; amax = fmaxf(amax, fabsf(v[i])); }
#pragma unroll
    for (int i = 16; i < 32; i++) { s16b += v[i]; amax = fmaxf(amax, fabsf(v[i])); }
    float s = 0.0f, inv = 0.0f;
    if (amax > 0.0f) { s = amax / 127.0f; inv = 127.0f / amax; }
#pragma unroll
    for (int i = 0; i < 24; i++) xp[i] = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        int X = (int)rintf(v[i] * inv * 65536.0f);
        int b0 = (int)(int8_t)(X & 0xFF);
        int X1 = (X - b0) >> 8;
        int b1 = (int)(int8_t)(X1 & 0xFF);
        int b2 = (X1 - b1) >> 8;
        int k = i >> 3, jj = i & 7;
        int dw = ((jj & 1) ? 4 : 0) + k;
        int sh = (jj >> 1) * 8;
        xp[dw] |= (uint32_t)(b2 & 0xFF) << sh;
        xp[8 + dw] |= (uint32_t)(b1 & 0xFF) << sh;
        xp[16 + dw] |= (uint32_t)(b0 & 0xFF) << sh;
    }
    st = make_float4(s, s16a + s16b, s16a, s16b);
}

__device__ __forceinline__ float digits_total(int D2, int D1, int D0) {
    return (float)D2 + (float)D1 * 0.00390625f + (float)D0 * 1.52587890625e-05f;
}

// ---- per-type block geometry, raw reads and group dots ------------------------------------
// The raw words of one 32-element group are read from the LDS copy of its block by ld() into a
// Raw<T>, then dotted by dot(). LDS pointers carry address space 3 so the reads are ds_read.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const uint8_t lds_u8;
typedef __attribute__((address_space(3))) const uint32_t lds_u32;
typedef __attribute__((address_space(3))) const u32x4 lds_v4;
typedef __attribute__((address_space(3))) u32x4 lds_v4w;
__device__ __forceinline__ uint4 lds_ld16(lds_u8* p) {
    u32x4 t = *(lds_v4*)p;
    return make_uint4(t.x, t.y, t.z, t.w);
}

// BB block bytes, GPB 32-element groups per block, N16 16-byte chunks that cover the blocks of a
// wave's slice of one row (at most 64 groups, plus 15 bytes of alignment), CPL chunks per lane.
template <int T> struct Geo;
template <> struct Geo<FLLM_TYPE_Q4_K> { static constexpr int BB = 144, GPB = 8; };
template <> struct Geo<FLLM_TYPE_Q5_K> { static constexpr int BB = 176, GPB = 8; };
template <> struct Geo<FLLM_TYPE_Q6_K> { static constexpr int BB = 210, GPB = 8; };
template <> struct Geo<FLLM_TYPE_Q8_0> { static constexpr int BB = 34, GPB = 1; };
template <> struct Geo<FLLM_TYPE_Q4_0> { static constexpr int BB = 18, GPB = 1; };
template <int T> struct Stage {
    static constexpr int BB = Geo<T>::BB, GPB = Geo<T>::GPB;
    static constexpr int MAXB = GPB == 8 ? 9 : 64;               // blocks touched by 64 groups
    static constexpr int N16 = (MAXB * BB + 15 + 15) / 16;       // chunks per row slice
    static constexpr int CPL = (N16 + 63) / 64;                  // chunks per lane per row
    static constexpr int RSB = N16 * 16 + 16;                    // LDS bytes per row slice (+ over-read slack)
};

template <int T> struct Raw;

// Q4_K (Dequantizer.cs:251-294): 144-byte blocks; group g = 32 elements with byte qs[g*16+i/2],
// low nibble for even i; dg = d*sc, mg = dmin*m; y = dg*q - mg.
template <> struct Raw<FLLM_TYPE_Q4_K> { uint4 hdr, qs; int g; };
__device__ __forceinline__ void ld(Raw<FLLM_TYPE_Q4_K>& r, lds_u8* blk, int g) {
    r.g = g;
    r.hdr = lds_ld16(blk);
    r.qs = lds_ld16(blk + 16 + g * 16);
}
__device__ __forceinline__ void kscale_regs(const uint4& hdr, int g, int& sc, int& mn) {
    int sh = (g & 3) * 8;
    uint32_t a = (hdr.y >> sh) & 0xFF, b = (hdr.z >> sh) & 0xFF, c = (hdr.w >> sh) & 0xFF;
    if (g < 4) { sc = (int)(a & 63); mn = (int)(b & 63); }
    else { sc = (int)((c & 15) | ((a >> 6) << 4)); mn = (int)((c >> 4) | ((b >> 6) << 4)); }
}
__device__ __forceinline__ float dot(const Raw<FLLM_TYPE_Q4_K>& r, const uint32_t* xp, float4 xs) {
    float d = h2f(r.hdr.x & 0xFFFFu), dmin = h2f(r.hdr.x >> 16);
    int sc, mn;
    kscale_regs(r.hdr, r.g, sc, mn);
    float dg = d * (float)sc, mg = dmin * (float)mn;
    uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
    int D2 = 0, D1 = 0, D0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
        D2 = sdot4(lo, xp[k], D2); D2 = sdot4(hi, xp[4 + k], D2);
        D1 = sdot4(lo, xp[8 + k], D1); D1 = sdot4(hi, xp[12 + k], D1);
        D0 = sdot4(lo, xp[16 + k], D0); D0 = sdot4(hi, xp[20 + k], D0);
    }
    return dg * (xs.x * digits_total(D2, D1, D0)) - mg * xs.y;
}

// Q5_K (Dequantizer.cs:316-368): 176-byte blocks; high bit of element t is bit t&7 of
// qh[t>>3], i.e. bit t of the group's qh dword; low nibble from qs[t>>1].
template <> struct Raw<FLLM_TYPE_Q5_K> { uint4 hdr, qs; uint32_t qh; int g; };
__device__ __forceinline__ void ld(Raw<FLLM_TYPE_Q5_K>& r, lds_u8* blk, int g) {
    r.g = g;
    r.hdr = lds_ld16(blk);
    r.qh = *(lds_u32*)(blk + 16 + g * 4);
    r.qs = lds_ld16(blk + 48 + g * 16);
}
__device__ __forceinline__ float dot(const Raw<FLLM_TYPE_Q5_K>& r, const uint32_t* xp, float4 xs) {
    float d = h2f(r.hdr.x & 0xFFFFu), dmin = h2f(r.hdr.x >> 16);
    int sc, mn;
    kscale_regs(r.hdr, r.g, sc, mn);
    float dg = d * (float)sc, mg = dmin * (float)mn;
    uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
    int D2 = 0, D1 = 0, D0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t bk = (r.qh >> (8 * k)) & 0xFFu;
        uint32_t lo = (q[k] & 0x0F0F0F0Fu) | (((bk & 0x55u) * 0x410410u) & 0x10101010u);
        uint32_t hi = ((q[k] >> 4) & 0x0F0F0F0Fu) | ((((bk >> 1) & 0x55u) * 0x410410u) & 0x10101010u);
        D2 = sdot4(lo, xp[k], D2); D2 = sdot4(hi, xp[4 + k], D2);
        D1 = sdot4(lo, xp[8 + k], D1); D1 = sdot4(hi, xp[12 + k], D1);
        D0 = sdot4(lo, xp[16 + k], D0); D0 = sdot4(hi, xp[20 + k], D0);
    }
    return dg * (xs.x * digits_total(D2, D1, D0)) - mg * xs.y;
}

// Q6_K (Dequantizer.cs:378-417): 210-byte blocks, linear layout: low nibble of element i in
// ql[i>>1], 2 high bits in qh[i>>2] at bit 2*(i&3), int8 scale sc[i>>4], d at bytes 208..209;
// y = (d*sc)*(q-32). Blocks are only 2-byte aligned: dwords are read from the 4-byte-aligned
// address below the block and re-aligned with v_alignbyte.
template <> struct Raw<FLLM_TYPE_Q6_K> { uint32_t l[5], h[3], s, d; uint32_t mis; int c; };
__device__ __forceinline__ void ld(Raw<FLLM_TYPE_Q6_K>& r, lds_u8* blk, int c) {
    r.c = c;
    r.mis = (uint32_t)(uintptr_t)blk & 3u;
    lds_u32* b4 = (lds_u32*)(blk - r.mis);
#pragma unroll
    for (int i = 0; i < 5; i++) r.l[i] = b4[4 * c + i];
#pragma unroll
    for (int i = 0; i < 3; i++) r.h[i] = b4[32 + 2 * c + i];
    r.s = b4[(192u + 2u * (uint32_t)c + r.mis) >> 2];
    r.d = b4[52];
}
__device__ __forceinline__ uint32_t spread4(uint32_t e) {
    e = (e | (e << 8)) & 0x00FF00FFu;
    return (e | (e << 4)) & 0x0F0F0F0Fu;
}
__device__ __forceinline__ float dot(const Raw<FLLM_TYPE_Q6_K>& r, const uint32_t* xp, float4 xs) {
    uint32_t mis = r.mis;
    uint32_t L[4] = {alignb(r.l[1], r.l[0], mis), alignb(r.l[2], r.l[1], mis), alignb(r.l[3], r.l[2], mis),
                     alignb(r.l[4], r.l[3], mis)};
    uint32_t H[2] = {alignb(r.h[1], r.h[0], mis), alignb(r.h[2], r.h[1], mis)};
    uint32_t ssh = ((192u + 2u * (uint32_t)r.c + mis) & 3u) * 8u;
    int sca = (int)(int8_t)((r.s >> ssh) & 0xFFu);
    int scb = (int)(int8_t)((r.s >> (ssh + 8u)) & 0xFFu);
    float d = h2f((r.d >> (8u * mis)) & 0xFFFFu);
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
    float ra = xs.x * digits_total(A2, A1, A0) - 32.0f * xs.z;
    float rb = xs.x * digits_total(B2, B1, B0) - 32.0f * xs.w;
    return (d * (float)sca) * ra + (d * (float)scb) * rb;
}

// Q8_0 (Dequantizer.cs:203-231): 34-byte blocks (2-byte aligned), y = (sbyte)q * d.
template <> struct Raw<FLLM_TYPE_Q8_0> { uint32_t dw[10]; uint32_t mis; };
__device__ __forceinline__ void ld(Raw<FLLM_TYPE_Q8_0>& r, lds_u8* blk, int) {
    r.mis = (uint32_t)(uintptr_t)blk & 3u;
    lds_u32* b4 = (lds_u32*)(blk - r.mis);
#pragma unroll
    for (int i = 0; i < 10; i++) r.dw[i] = b4[i];
}
__device__ __forceinline__ float dot(const Raw<FLLM_TYPE_Q8_0>& r, const uint32_t* xp, float4 xs) {
    float d = h2f((r.dw[0] >> (8u * r.mis)) & 0xFFFFu);
    bool shifted = r.mis != 0;  // quants start at byte mis+2: dword-aligned when mis == 2
    uint32_t qv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) qv[i] = shifted ? r.dw[i + 1] : alignb(r.dw[i + 1], r.dw[i], 2);
    int D2 = 0, D1 = 0, D0 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t ev = __builtin_amdgcn_perm(qv[2 * k + 1], qv[2 * k], 0x06040200u);
        uint32_t od = __builtin_amdgcn_perm(qv[2 * k + 1], qv[2 * k], 0x07050301u);
        D2 = sdot4(ev, xp[k], D2); D2 = sdot4(od, xp[4 + k], D2);
        D1 = sdot4(ev, xp[8 + k], D1); D1 = sdot4(od, xp[12 + k], D1);
        D0 = sdot4(ev, xp[16 + k], D0); D0 = sdot4(od, xp[20 + k], D0);
    }
    return d * (xs.x * digits_total(D2, D1, D0));
}

// Q4_0 (Dequantizer.cs:155-185): 18-byte blocks, y = (nib-8)*d; low nibble of byte j is
// element j, high nibble element j+16.
template <> struct Raw<FLLM_TYPE_Q4_0> { uint32_t dw[5]; uint32_t mis; };
__device__ __forceinline__ void ld(Raw<FLLM_TYPE_Q4_0>& r, lds_u8* blk, int) {
    r.mis = (uint32_t)(uintptr_t)blk & 3u;
    lds_u32* b4 = (lds_u32*)(blk - r.mis);
#pragma unroll
    for (int i = 0; i < 5; i++) r.dw[i] = b4[i];
}
__device__ __forceinline__ float dot(const Raw<FLLM_TYPE_Q4_0>& r, const uint32_t* xp, float4 xs) {
    float d = h2f((r.dw[0] >> (8u * r.mis)) & 0xFFFFu);
    bool shifted = r.mis != 0;
    uint32_t qv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) qv[i] = shifted ? r.dw[i + 1] : alignb(r.dw[i + 1], r.dw[i], 2);
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
    return d * (xs.x * digits_total(D2, D1, D0) - 8.0f * xs.y);
}

// Sum NR per-lane values over the 64 lanes of a wave with a transposing butterfly
// (NR*2 - 2 + log2(64/NR) lane exchanges); lane l ends with the total of row
// (l >> (6 - log2 NR)) & (NR-1), and lanes with l % (64/NR) == 0 hold distinct rows.
template <int NR>
__device__ __forceinline__ float transpose_reduce(const float* acc, int lane) {
    float v[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) v[i] = acc[i];
    int bit = 32;
#pragma unroll
    for (int n = NR; n > 1; n >>= 1) {
        const int half = n >> 1;
        const bool b = (lane & bit) != 0;
#pragma unroll
        for (int i = 0; i < half; i++) {
            float keep = b ? v[i + half] : v[i];
            float send = b ? v[i] : v[i + half];
            v[i] = keep + __shfl_xor(send, bit);
        }
        bit >>= 1;
    }
    float u = v[0];
#pragma unroll
    for (int o = 64 / NR / 2; o > 0; o >>= 1) u += __shfl_xor(u, o);
    return u;
}

template <int NR> struct Log2;
template <> struct Log2<4> { static constexpr int v = 2; };
template <> struct Log2<8> { static constexpr int v = 3; };

// ---- row batches staged through LDS -----------------------------------------------------------
// A wave's slice of a row (its S group columns) is a contiguous byte range of the block stream.
// The wave copies the 16-byte-aligned chunks covering it into its own LDS area with fully
// coalesced 16-byte loads (64 lanes x 16 B per instruction), then every lane reads its group's
// block fields from LDS. The loads of the next batch are issued before the current batch is
// dotted, so HBM latency overlaps the dequant arithmetic.
struct SliceGeom {
    int G, S, Sw;   // groups per row, groups per wave slice, groups in this wave's slice
    int wave;
};

template <int T, int NR>
struct Batch {
    uint4 c[NR][Stage<T>::CPL];
    uint32_t a0[NR];  // aligned start byte of each row slice (relative to the matrix)
    int n16[NR];      // chunks covering each row slice (0 = row outside the matrix)
};

template <int T, int NR>
__device__ __forceinline__ void issue_batch(Batch<T, NR>& bt, const uint8_t* __restrict__ W, int rows, int row0,
                                            const SliceGeom& sg, int lane) {
    using St = Stage<T>;
#pragma unroll
    for (int rr = 0; rr < NR; rr++) {
        int row = row0 + rr;
        bt.n16[rr] = 0;
        bt.a0[rr] = 0;
        if (row < rows && sg.Sw > 0) {
            int64_t g0 = (int64_t)row * sg.G + (int64_t)sg.wave * sg.S;
            int64_t b0 = g0 / St::GPB, b1 = (g0 + sg.Sw - 1) / St::GPB;
            int64_t by0 = b0 * St::BB, by1 = (b1 + 1) * St::BB;
            int64_t a0 = by0 & ~(int64_t)15;
            bt.a0[rr] = (uint32_t)(a0 & 0xFFFFFFFF);
            bt.n16[rr] = (int)((by1 - a0 + 15) >> 4);
            const uint4* src = (const uint4*)(W + a0);
#pragma unroll
            for (int k = 0; k < St::CPL; k++) {
                int ch = lane + 64 * k;
                if (ch < bt.n16[rr]) bt.c[rr][k] = src[ch];
            }
        }
    }
}

template <int T, int NR>
__device__ __forceinline__ void stage_batch(const Batch<T, NR>& bt, __attribute__((address_space(3))) uint8_t* wlds, int lane) {
    using St = Stage<T>;
#pragma unroll
    for (int rr = 0; rr < NR; rr++) {
#pragma unroll
        for (int k = 0; k < St::CPL; k++) {
            int ch = lane + 64 * k;
            if (ch < bt.n16[rr]) {
                const uint4 c = bt.c[rr][k];
                u32x4 t = {c.x, c.y, c.z, c.w};
                *(lds_v4w*)(wlds + rr * St::RSB + ch * 16) = t;
            }
        }
    }
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Dot the NR staged rows with this lane's group column; the wave's row sums go to part[0..NR).
template <int T, int NR>
__device__ __forceinline__ void dot_batch(const Batch<T, NR>& bt, lds_u8* wlds, int row0, const SliceGeom& sg,
                                          int j, bool active, const uint32_t* xp, float4 xs, int lane, float* part) {
    using St = Stage<T>;
    float acc[NR];
#pragma unroll
    for (int rr = 0; rr < NR; rr++) {
        acc[rr] = 0.0f;
        if (active && bt.n16[rr] > 0) {
            int64_t gi = (int64_t)(row0 + rr) * sg.G + j;
            int64_t blk = gi / St::GPB;
            uint32_t off = (uint32_t)((blk * St::BB) & 0xFFFFFFFF) - bt.a0[rr];
            Raw<T> r;
            ld(r, (lds_u8*)(wlds + rr * St::RSB + off), (int)(gi % St::GPB));
            acc[rr] = dot(r, xp, xs);
        }
    }
    float tot = transpose_reduce<NR>(acc, lane);
    if ((lane & (64 / NR - 1)) == 0) part[(lane >> (6 - Log2<NR>::v)) & (NR - 1)] = tot;
}

__device__ __forceinline__ float act_fn(float g, int act) {
    if (act == 0) {  // SiLU = x * Sigmoid(x) (TensorOperations.cs:57-87)
        float sig = 1.0f / (1.0f + expf(-g));
        return g * sig;
    }
    // GELU, tanh form (TensorOperations.cs:110-117)
    return 0.5f * g * (1.0f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g)));
}

// =====================================================================================
// The fused kernel.
// LDS: part[nslice][T] row partials (T = row slots of the workgroup), red[16], 16 u64 keys for the
// logits epilogue, then each wave's staging area (GEMV_NR row slices).
// =====================================================================================
constexpr int GEMV_NR = 4;  // rows per batch

__device__ __forceinline__ void epilogue(const GemvArgs& a, const GemvSeg& sg, const float* part, float* red, int nslice,
                                         int R, int T, int row_base, int wave, int lane) {
    if (a.glu) {
        // h = act(W_gate x) * (W_up x)
        for (int t = threadIdx.x; t < R; t += blockDim.x) {
            int r = row_base + t;
            if (r >= sg.rows) continue;
            float g = 0.0f, u = 0.0f;
            for (int sl = 0; sl < nslice; sl++) { g += part[sl * T + t]; u += part[sl * T + R + t]; }
            sg.out[r] = act_fn(g, a.act) * u;
        }
        return;
    }
    const int epi = sg.epi;
    if (epi == EPI_Q || epi == EPI_K) {
        // bias, then RoPE on interleaved pairs (2i, 2i+1) of each head
        const int half = a.hd >> 1;
        const float2* rp = a.rope + (int64_t)a.params->pos * half;
        const int slot = a.params->cur_len;
        for (int p = threadIdx.x; p < (R >> 1); p += blockDim.x) {
            int r = row_base + 2 * p;
            if (r >= sg.rows) continue;
            float x0 = 0.0f, x1 = 0.0f;
            for (int sl = 0; sl < nslice; sl++) { x0 += part[sl * T + 2 * p]; x1 += part[sl * T + 2 * p + 1]; }
            if (sg.bias) { x0 = x0 + sg.bias[r]; x1 = x1 + sg.bias[r + 1]; }
            float2 cs = rp[(r % a.hd) >> 1];
            float y0 = x0 * cs.x - x1 * cs.y;
            float y1 = x0 * cs.y + x1 * cs.x;
            if (epi == EPI_Q) {
                sg.out[r] = y0;
                sg.out[r + 1] = y1;
            } else {
                float* kc = a.kc + (int64_t)slot * a.kvdim;
                kc[r] = y0;
                kc[r + 1] = y1;
            }
        }
        return;
    }
    if (epi == EPI_LOGITS) {
        unsigned long long best = 0ull;
        for (int t = threadIdx.x; t < R; t += blockDim.x) {
            int r = row_base + t;
            if (r >= sg.rows) continue;
            float y = 0.0f;
            for (int sl = 0; sl < nslice; sl++) y += part[sl * T + t];
            if (a.softcap > 0.0f) y = tanhf(y * (1.0f / a.softcap)) * a.softcap;  // SoftCap
            sg.out[r] = y;
            // larger value wins; on equal values the lower index (IndexOfMax: first maximum)
            unsigned long long key = ((unsigned long long)fkey(y) << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)r);
            best = key > best ? key : best;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            unsigned long long ot = __shfl_xor(best, o);
            best = ot > best ? ot : best;
        }
        unsigned long long* keys = (unsigned long long*)(red + 16);
        if (lane == 0) keys[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < nslice; w++) best = keys[w] > best ? keys[w] : best;
            a.wg_keys[blockIdx.x] = best;  // reduced by the argmax kernel that follows
        }
        return;
    }
    for (int t = threadIdx.x; t < R; t += blockDim.x) {
        int r = row_base + t;
        if (r >= sg.rows) continue;
        float y = 0.0f;
        for (int sl = 0; sl < nslice; sl++) y += part[sl * T + t];
        if (epi == EPI_RESID) {
            sg.out[r] = sg.resid[r] + y;
        } else if (epi == EPI_V) {
            if (sg.bias) y = y + sg.bias[r];
            a.vc[(int64_t)a.params->cur_len * a.kvdim + r] = y;
        } else {
            if (sg.bias) y = y + sg.bias[r];
            sg.out[r] = y;
        }
    }
}

// PREFETCH: the next batch's loads are issued before the current batch is dotted (two batches of
// staging registers); without it the kernel fits the 128 VGPRs of 16-wave workgroups.
template <int T, bool PREFETCH>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, const GemvSeg& sg, int wg_in_seg) {
    constexpr int NR = GEMV_NR;
    extern __shared__ float lds[];
    const int nslice = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j = wave * a.S + lane;
    const bool active = lane < a.S && j < a.G;
    const int R = a.rpw;                 // rows per workgroup (multiple of 8)
    const int row_base = wg_in_seg * R;  // first row of this workgroup in its matrix (GLU: in gate and up)
    const int T_slots = a.glu ? 2 * R : R;
    float* part = lds;                   // [nslice][T_slots]
    float* red = lds + nslice * T_slots; // [16] floats, then 16 u64
    __attribute__((address_space(3))) uint8_t* wlds =
        (__attribute__((address_space(3))) uint8_t*)(red + 16 + 32) + wave * NR * Stage<T>::RSB;

    SliceGeom geo;
    geo.G = a.G;
    geo.S = a.S;
    geo.wave = wave;
    geo.Sw = min(a.S, a.G - wave * a.S);
    if (geo.Sw < 0) geo.Sw = 0;

    // first batch's weight loads go out before the activation prologue
    const GemvSeg& s1 = a.glu ? a.seg[1] : sg;
    Batch<T, NR> cur, nxt;
    issue_batch<T, NR>(cur, sg.w, sg.rows, row_base, geo, lane);

    // ---- prologue: this lane's 32 input values -----------------------------------------
    float v[32];
    if (a.xin == XIN_EMBED_NORM) {
        const int64_t tok = a.params->token;
        if (active) {
            deq32(a.emb_type, a.emb, tok * (int64_t)a.G * 32 + j * 32, v);
            if (blockIdx.x == 0) {
                float4* xo = (float4*)(a.x_out + j * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) xo[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
            }
        }
    } else if (active) {
        const float4* xi = (const float4*)(a.x + j * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 t = xi[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
    }
    if (!active) {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = 0.0f;
    }
    if (a.xin != XIN_F32) {
        // RmsNorm: rms = 1/sqrt(Dot(x,x)/n + eps); dst = (x*rms)*w  (Gemma: *(1+w), eps 1e-6)
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) ss = fmaf(v[i], v[i], ss);
        ss = wsum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int i = 0; i < nslice; i++) tot += red[i];
        float rms = 1.0f / sqrtf(tot / (float)(a.G * 32) + a.eps);
        if (active) {
            const float4* wv = (const float4*)(a.norm_w + j * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float4 w4 = wv[i];
                float ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float t = v[4 * i + e] * rms;
                    v[4 * i + e] = a.norm_kind ? t * (ww[e] + 1.0f) : t * ww[e];
                }
            }
        }
    }
    uint32_t xp[24];
    float4 xs;
    quantize32(v, xp, xs);

    // ---- row batches --------------------------------------------------------------------------
    for (int b = 0; b < T_slots; b += NR) {
        stage_batch<T, NR>(cur, wlds, lane);
        const int bn = b + NR;
        const bool more = bn < T_slots;
        const bool up = a.glu && bn >= R;
        const GemvSeg& m = up ? s1 : sg;
        if (PREFETCH && more) issue_batch<T, NR>(nxt, m.w, m.rows, row_base + (up ? bn - R : bn), geo, lane);
        wave_lds_sync();
        dot_batch<T, NR>(cur, wlds, row_base + ((a.glu && b >= R) ? b - R : b), geo, j, active, xp, xs, lane,
                         part + wave * T_slots + b);
        wave_lds_sync();
        if (PREFETCH) cur = nxt;
        else if (more) issue_batch<T, NR>(cur, m.w, m.rows, row_base + (up ? bn - R : bn), geo, lane);
    }
    __syncthreads();
    epilogue(a, sg, part, red, nslice, R, T_slots, row_base, wave, lane);
}

// WIDE: rows of more than 512 groups (up to 16 waves per workgroup), no prefetch.
template <bool WIDE>
__global__ __launch_bounds__(WIDE ? 1024 : 512) __attribute__((amdgpu_waves_per_eu(4))) void k_gemv_fused(const GemvArgs a) {
    int si = 0;
    while (si + 1 < a.nseg && (int)blockIdx.x >= a.seg[si + 1].wg_begin) si++;
    const GemvSeg& sg = a.seg[si];
    const int wg_in_seg = (int)blockIdx.x - sg.wg_begin;
    switch (sg.type) {
        case FLLM_TYPE_Q4_K: gemv_body<FLLM_TYPE_Q4_K, !WIDE>(a, sg, wg_in_seg); break;
        case FLLM_TYPE_Q5_K: gemv_body<FLLM_TYPE_Q5_K, !WIDE>(a, sg, wg_in_seg); break;
        case FLLM_TYPE_Q6_K: gemv_body<FLLM_TYPE_Q6_K, !WIDE>(a, sg, wg_in_seg); break;
        case FLLM_TYPE_Q8_0: gemv_body<FLLM_TYPE_Q8_0, !WIDE>(a, sg, wg_in_seg); break;
        default: gemv_body<FLLM_TYPE_Q4_0, !WIDE>(a, sg, wg_in_seg); break;
    }
}

// ---- host side ------------------------------------------------------------------------
bool gemv_fusable_type(int t) {
    return t == FLLM_TYPE_Q4_K || t == FLLM_TYPE_Q5_K || t == FLLM_TYPE_Q6_K || t == FLLM_TYPE_Q8_0 ||
           t == FLLM_TYPE_Q4_0;
}

static int stage_rsb(int t) {
    switch (t) {
        case FLLM_TYPE_Q4_K: return Stage<FLLM_TYPE_Q4_K>::RSB;
        case FLLM_TYPE_Q5_K: return Stage<FLLM_TYPE_Q5_K>::RSB;
        case FLLM_TYPE_Q6_K: return Stage<FLLM_TYPE_Q6_K>::RSB;
        case FLLM_TYPE_Q8_0: return Stage<FLLM_TYPE_Q8_0>::RSB;
        default: return Stage<FLLM_TYPE_Q4_0>::RSB;
    }
}

bool gemv_fusable_cols(int64_t cols) { return cols % 32 == 0 && cols >= 32 && cols <= 32768; }

// Fill G, S, rpw and the segments' workgroup ranges; rows_per_wg 0 = choose.
int gemv_plan(GemvArgs& a, int64_t cols, int n_cu, int rows_per_wg, int* block_threads, size_t* lds_bytes) {
    a.G = (int)(cols / 32);
    int nslice = (a.G + 63) / 64;
    a.S = (a.G + nslice - 1) / nslice;
    int64_t total_rows = 0;
    for (int i = 0; i < a.nseg; i++) total_rows += a.glu ? (i == 0 ? a.seg[i].rows : 0) : a.seg[i].rows;
    int rpw = rows_per_wg;
    if (rpw <= 0) {
        // aim for about 16 waves per CU over the launch, whole batches of 8 rows per workgroup
        int64_t target_wgs = (int64_t)n_cu * 16 / nslice;
        if (target_wgs < 1) target_wgs = 1;
        int64_t slots = a.glu ? 2 * total_rows : total_rows;
        int64_t per = (slots + target_wgs - 1) / target_wgs;
        if (a.glu) per = (per + 1) / 2;
        rpw = (int)((per + 7) / 8 * 8);
        if (rpw < 8) rpw = 8;
        if (rpw > 256) rpw = 256;
    }
    a.rpw = rpw;
    int wg = 0;
    for (int i = 0; i < a.nseg; i++) {
        a.seg[i].wg_begin = wg;
        if (a.glu && i > 0) { a.seg[i].wg_begin = 1 << 30; continue; }
        wg += (int)((a.seg[i].rows + rpw - 1) / rpw);
    }
    int T = a.glu ? 2 * rpw : rpw;
    int rsb = 0;
    for (int i = 0; i < a.nseg; i++) rsb = stage_rsb(a.seg[i].type) > rsb ? stage_rsb(a.seg[i].type) : rsb;
    *block_threads = 64 * nslice;
    // row partials, 16 reduction floats, 16 u64 keys, then every wave's staging area
    *lds_bytes = sizeof(float) * ((size_t)nslice * T + 48) + (size_t)nslice * GEMV_NR * rsb;
    return wg;
}

hipError_t launch_gemv_fused(const GemvArgs& a, int grid, int block_threads, size_t lds, hipStream_t st) {
    if (grid <= 0) return hipSuccess;
    if (block_threads <= 512)
        k_gemv_fused<false><<<grid, block_threads, lds, st>>>(a);
    else
        k_gemv_fused<true><<<grid, block_threads, lds, st>>>(a);
    return hipGetLastError();
}

}  // namespace fllm
