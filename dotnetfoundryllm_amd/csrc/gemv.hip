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
#include "actab.hpp"

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

// Weight loads with the non-temporal hint: every weight byte is read once per step, so the weight
// stream need not displace the activation tables, the epilogue operands and the kernels' code from
// the caches. nt16a / nt8a: 4-byte aligned (raw GGUF rows).
typedef uint32_t nt_u2 __attribute__((ext_vector_type(2)));
typedef uint32_t nt_u4a __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t nt_u2a __attribute__((ext_vector_type(2), aligned(4)));
__device__ __forceinline__ uint4 nt16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 nt16a(const uint8_t* p) {
    const nt_u4a v = __builtin_nontemporal_load((const nt_u4a*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 nt8(const uint8_t* p) {
    const nt_u2 v = __builtin_nontemporal_load((const nt_u2*)p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint2 nt8a(const uint8_t* p) {
    const nt_u2a v = __builtin_nontemporal_load((const nt_u2a*)p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t nt4(const uint8_t* p) { return __builtin_nontemporal_load((const uint32_t*)p); }
__device__ __forceinline__ uint16_t nt2(const uint8_t* p) { return __builtin_nontemporal_load((const uint16_t*)p); }

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
                if (ch < bt.n16[rr]) bt.c[rr][k] = nt16((const uint8_t*)(src + ch));
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

// =====================================================================================
// The fused kernel.
// LDS: part[nslice][T] row partials (T = row slots of the workgroup), red[16], 16 u64 keys for the
// logits epilogue, then each wave's staging area (GEMV_NR row slices).
// =====================================================================================
constexpr int GEMV_NR = 4;  // rows per batch

// Rows [row_base, row_base + R) of segment sg from the waves' partial sums part[nslice][T]. For the
// LM head, thread 0 folds this range's largest logit key into wg_best.
// The segment's fields come by value (a by-reference aggregate selected at run time would be
// copied to scratch memory).
__device__ __forceinline__ void tab_emit(const GemvArgs& a, float v, float sq, int row_base, int rows, int lane);

struct EpiSeg {
    int rows, epi;
    float* out;
    const float* bias;
    const float* resid;
    // pre: this thread's residual (pr) and consumer norm weight (pw) of a residual add were
    // loaded ahead (the matrix-core kernels load them for a workgroup's first tile with its table)
    int pre;
    float pr, pw;
};

__device__ __forceinline__ void epilogue(const GemvArgs& a, const EpiSeg sg, const float* part, float* red, int nslice,
                                         int R, int T, int row_base, int wave, int lane, unsigned long long& wg_best) {
    // value and squared raw output of this thread's row, for the activation table of the consumer
    float tv = 0.0f, tq = 0.0f;
    if (a.glu) {
        // h = act(W_gate x) * (W_up x)
        for (int t = threadIdx.x; t < R; t += nslice * 64) {
            int r = row_base + t;
            if (r >= sg.rows) continue;
            float g = 0.0f, u = 0.0f;
            for (int sl = 0; sl < nslice; sl++) { g += part[sl * T + t]; u += part[sl * T + R + t]; }
            tv = act_fn(g, a.act) * u;
            sg.out[r] = tv;
        }
        if (a.tab_out && wave == 0) tab_emit(a, tv, 0.0f, row_base, sg.rows, lane);
        return;
    }
    const int epi = sg.epi;
    if (epi == EPI_Q || epi == EPI_K) {
        // bias, then RoPE on interleaved pairs (2i, 2i+1) of each head
        const int half = a.hd >> 1;
        const float2* rp = a.rope + (int64_t)a.params->pos * half;
        const int slot = a.params->cur_len;
        for (int p = threadIdx.x; p < (R >> 1); p += nslice * 64) {
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
        for (int t = threadIdx.x; t < R; t += nslice * 64) {
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
            wg_best = best > wg_best ? best : wg_best;
        }
        return;
    }
    for (int t = threadIdx.x; t < R; t += nslice * 64) {
        int r = row_base + t;
        if (r >= sg.rows) continue;
        float y = 0.0f;
        for (int sl = 0; sl < nslice; sl++) y += part[sl * T + t];
        if (epi == EPI_RESID) {
            const float xr = (sg.pre ? sg.pr : sg.resid[r]) + y;
            sg.out[r] = xr;
            tq = xr * xr;
            if (a.tab_w) {
                const float w = sg.pre ? sg.pw : a.tab_w[r];
                tv = xr * (a.tab_kind ? 1.0f + w : w);
            } else {
                tv = xr;
            }
        } else if (epi == EPI_V) {
            if (sg.bias) y = y + sg.bias[r];
            a.vc[(int64_t)a.params->cur_len * a.kvdim + r] = y;
        } else {
            if (sg.bias) y = y + sg.bias[r];
            sg.out[r] = y;
        }
    }
    if (a.tab_out && epi == EPI_RESID && wave == 0) tab_emit(a, tv, tq, row_base, sg.rows, lane);
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
    unsigned long long best = 0ull;
    epilogue(a, EpiSeg{sg.rows, sg.epi, sg.out, sg.bias, sg.resid}, part, red, nslice, R, T_slots, row_base, wave, lane, best);
    if (sg.epi == EPI_LOGITS && threadIdx.x == 0) a.wg_keys[blockIdx.x] = best;  // reduced by the argmax kernel
}

// =====================================================================================
// Matrix-core (MFMA) variant for rows that are whole 256-element chunks.
//
// v_mfma_i32_16x16x64_i8 computes D[16x16] += A[16x64] B[64x16] in int32. Lane l supplies A row
// l%16 and B column l%16, both for the 16 k values of quarter l/16, and receives D column l%16,
// rows 4*(l/16) .. +3. Here B column n is weight row n of a 16-row tile, quarter Q of a chunk is
// the lane's own share of the chunk's bytes, and A row m = 4Q' + d holds activation digit d of the
// elements of quarter Q' (zero elsewhere). So lane (n, Q) loads the weights it multiplies and
// receives the three digit sums of (row n, quarter Q) in its own D registers: digit combination
// and the per-group block scales are applied lane-locally.
//
// In 4 MFMA steps a lane covers groups Q and Q+4 of the chunk (32 elements each): step s is half
// s&1 (elements 16(s&1) .. +15) of group Q + 4*(s>>1). Inside a step's 16-byte fragment, byte `by`
// of dword j holds element 4*by + j of that half, for the weights (built from the GGUF bytes in
// registers) and for the activation digits alike.
//
// Activation table (LDS, and in global memory when a producer epilogue writes it): per chunk 48
// uint4 digit entries [step][quarter][digit], then per chunk 8 float4 group stats. Each 16-element
// half is quantized on its own: X = rint(v * 65536 * 127 / amax), split into signed base-256 digits
// X = 65536 b2 + 256 b1 + b0 (digit 0 = b2). Stats of group g: {scale of half 0, scale of half 1,
// sum of half 0, sum of half 1}, scale = amax / 127, sums over the unquantized values.
// =====================================================================================
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x4 lds_f4;
typedef __attribute__((address_space(3))) u32x4 lds_tab;
// 16 and 8 bytes at 4-byte-aligned global addresses (Q6_K blocks are 210 bytes)
typedef u32x4 u32x4a __attribute__((aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef u32x2 u32x2a __attribute__((aligned(4)));

constexpr int MF_TILE = 16;        // weight rows per MFMA tile
// zeroed uint4 entries in LDS read as the A operand by lanes that carry no table row: as many as
// the table entries one wave's KC chunks span
#define MF_ZERO_ENTRIES(kc) ((kc) * 48)

// bytes of 256 elements (one chunk) for the MFMA-capable types
__host__ __device__ constexpr int mf_chunk_bytes(int t) {
    return t == FLLM_TYPE_Q4_K ? 144 : t == FLLM_TYPE_Q6_K ? 210 : t == FLLM_TYPE_Q8_0 ? 272 : t == FLLM_TYPE_Q5_K ? 176 : 0;
}


// One thread: the digit entries of group g (0..7) of chunk b from its 32 values; returns the
// group stats.
__device__ __forceinline__ void atab_write(lds_tab* atab, int b, int g, const float* v, float4* st) {
    float sc[2], sm[2];
    int X[32];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float amax = 0.0f, sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) { sum += v[16 * h + i]; amax = fmaxf(amax, fabsf(v[16 * h + i])); }
        float inv;
        half_scale(amax, sc[h], inv);
        sm[h] = sum;
#pragma unroll
        for (int i = 0; i < 16; i++) X[16 * h + i] = quant_x(v[16 * h + i], inv);
    }
    const int q = g & 3, s0 = 2 * (g >> 2);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        uint32_t w[3][4];
        // dword j of each digit entry: bytes from elements j, 4 + j, 8 + j, 12 + j
#pragma unroll
        for (int j = 0; j < 4; j++)
            digits3_pack4(X[16 * h + j], X[16 * h + 4 + j], X[16 * h + 8 + j], X[16 * h + 12 + j], w[0][j], w[1][j],
                          w[2][j]);
#pragma unroll
        for (int d = 0; d < 3; d++) {
            u32x4 e4 = {w[d][0], w[d][1], w[d][2], w[d][3]};
            atab[atab_index(b, s0 + h, q, d)] = e4;
        }
    }
    *st = make_float4(sc[0], sc[1], sm[0], sm[1]);
}

// One thread: the digit entries of half h of group g (0..7) of chunk b from its 16 values (the
// arithmetic of atab_write for one half); returns the half's scale and sum.
__device__ __forceinline__ void atab_write_half(lds_tab* atab, int b, int g, int h, const float* v, float& sc,
                                                float& sm) {
    float amax = 0.0f, sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) { sum += v[i]; amax = fmaxf(amax, fabsf(v[i])); }
    float inv;
    half_scale(amax, sc, inv);
    sm = sum;
    int X[16];
#pragma unroll
    for (int e = 0; e < 16; e++) X[e] = quant_x(v[e], inv);
    uint32_t w[3][4];
#pragma unroll
    for (int j = 0; j < 4; j++) digits3_pack4(X[j], X[4 + j], X[8 + j], X[12 + j], w[0][j], w[1][j], w[2][j]);
#pragma unroll
    for (int d = 0; d < 3; d++) {
        u32x4 e4 = {w[d][0], w[d][1], w[d][2], w[d][3]};
        atab[atab_index(b, 2 * (g >> 2) + h, g & 3, d)] = e4;
    }
}

// Producer side of the table, for a consumer whose columns are this launch's rows: lanes 0..15 of
// the calling wave hold v for rows row_base .. row_base + 15 (one half of a group; other lanes hold
// 0) and sq, the square of the raw output for the consumer's RMSNorm. Writes the half's three
// digit entries, its scale and sum, and its sum of squares.
__device__ __forceinline__ void tab_emit(const GemvArgs& a, float v, float sq, int row_base, int rows, int lane) {
    float amax = fabsf(v), sum = v, ssq = sq;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, o));
        sum += __shfl_xor(sum, o);
        ssq += __shfl_xor(ssq, o);
    }
    float sc, inv;
    half_scale(amax, sc, inv);
    const int X = quant_x(v, inv);
    const int h16 = row_base >> 4, g32 = h16 >> 1, half = h16 & 1, b = g32 >> 3, gg = g32 & 7;
    const int s = 2 * (gg >> 2) + half, q = gg & 3, j = lane & 3;
    // dword j of each digit entry: bytes from elements j, 4 + j, 8 + j, 12 + j
    uint32_t w2, w1, w0;
    digits3_pack4(__shfl(X, j), __shfl(X, j + 4), __shfl(X, j + 8), __shfl(X, j + 12), w2, w1, w0);
    uint32_t* tab = (uint32_t*)a.tab_out;
    if (lane < 4) {
        tab[4 * atab_index(b, s, q, 0) + j] = w2;
        tab[4 * atab_index(b, s, q, 1) + j] = w1;
        tab[4 * atab_index(b, s, q, 2) + j] = w0;
    }
    if (lane == 0) {
        float* st = (float*)(tab + 4 * (size_t)(rows / 256) * 48) + 4 * (8 * b + gg);
        st[half] = sc;
        st[2 + half] = sum;
        if (a.ssq_out) a.ssq_out[h16] = ssq;
    }
}

// D2 + D1 / 256 + D0 / 65536 of a lane's three digit sums (D.x = D2 .. D.z = D0, each at most
// 64 * 128 * 128 in magnitude, so 256 D1 + D0 fits an int32): two conversions and one fma
__device__ __forceinline__ float mf_total(const v4i& D) {
    return fmaf((float)(D.y * 256 + D.z), 1.52587890625e-05f, (float)D.x);
}

// ---- Q4_K (Dequantizer.cs:251-294): 16-byte-aligned 144-byte blocks ---------------------------
// Group g's 32 elements are bytes 16g .. 16g+15 of qs, element i in the low (even i) or high nibble
// of byte i/2.
struct MfQ4K { uint4 hdr, qa, qb; };
__device__ __forceinline__ void mf_issue(MfQ4K& r, const uint8_t* __restrict__ W, uint32_t off, int c, int, int q) {
    const uint8_t* p = W + off + (uint32_t)(c * 144);
    r.hdr = nt16(p);
    r.qa = nt16(p + 16 + 16 * q);   // group q
    r.qb = nt16(p + 80 + 16 * q);   // group q + 4
}
// the same fields from a LAYOUT_TILES region (lane = 16 q + n)
__device__ __forceinline__ void mf_issue_tiles(MfQ4K& r, const uint8_t* __restrict__ reg, int lane, int n) {
    r.hdr = nt16(reg + 2048 + 16 * n);
    r.qa = nt16(reg + 16 * lane);
    r.qb = nt16(reg + 1024 + 16 * lane);
}

// fragment of one half-group from its 8 qs bytes: dword j = elements j, 4+j, 8+j, 12+j
__device__ __forceinline__ v4i q4_frag(uint32_t w0, uint32_t w1) {
    const uint32_t E = __builtin_amdgcn_perm(w1, w0, 0x06040200u);  // bytes 0, 2, 4, 6: elements 4by, 4by+1
    const uint32_t O = __builtin_amdgcn_perm(w1, w0, 0x07050301u);  // bytes 1, 3, 5, 7: elements 4by+2, 4by+3
    v4i r = {(int)(E & 0x0F0F0F0Fu), (int)((E >> 4) & 0x0F0F0F0Fu), (int)(O & 0x0F0F0F0Fu),
             (int)((O >> 4) & 0x0F0F0F0Fu)};
    return r;
}

// The tile layout (k_pack_tiles) stores each 8-byte half of a group's qs as bytes 0, 2, 4, 6, 1, 3,
// 5, 7, so its two dwords are q4_frag's E and O already: the fragment is four masks.
struct MfQ4KT : MfQ4K {};
__device__ __forceinline__ v4i q4_frag_t(uint32_t E, uint32_t O) {
    v4i r = {(int)(E & 0x0F0F0F0Fu), (int)((E >> 4) & 0x0F0F0F0Fu), (int)(O & 0x0F0F0F0Fu),
             (int)((O >> 4) & 0x0F0F0F0Fu)};
    return r;
}

// 4 MFMAs over groups q and q+4 and their block scales; this lane's part of row n.
template <bool TILES>
__device__ __forceinline__ float mf_compute_q4k(const MfQ4K& r, const v4i* A, const f32x4& sA, const f32x4& sB, int q) {
    const v4i z = {0, 0, 0, 0};
    auto frag = [](uint32_t w0, uint32_t w1) { return TILES ? q4_frag_t(w0, w1) : q4_frag(w0, w1); };
    const v4i D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], frag(r.qa.x, r.qa.y), z, 0, 0, 0);
    const v4i D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], frag(r.qa.z, r.qa.w), z, 0, 0, 0);
    const v4i D2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], frag(r.qb.x, r.qb.y), z, 0, 0, 0);
    const v4i D3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], frag(r.qb.z, r.qb.w), z, 0, 0, 0);
    // DecodeKScaleMin (Dequantizer.cs:506-521) for groups q (< 4) and q + 4
    const int sh = 8 * q;
    const uint32_t a = (r.hdr.y >> sh) & 0xFF, b = (r.hdr.z >> sh) & 0xFF, c = (r.hdr.w >> sh) & 0xFF;
    const int scA = (int)(a & 63), mnA = (int)(b & 63);
    const int scB = (int)((c & 15) | ((a >> 6) << 4)), mnB = (int)((c >> 4) | ((b >> 6) << 4));
    const float d = h2f(r.hdr.x & 0xFFFFu), dmin = h2f(r.hdr.x >> 16);
    const float dgA = d * (float)scA, mgA = dmin * (float)mnA;
    const float dgB = d * (float)scB, mgB = dmin * (float)mnB;
    const float tA = fmaf(sA.x, mf_total(D0), sA.y * mf_total(D1));
    const float tB = fmaf(sB.x, mf_total(D2), sB.y * mf_total(D3));
    const float y = fmaf(dgA, tA, -mgA * (sA.z + sA.w));
    return y + fmaf(dgB, tB, -mgB * (sB.z + sB.w));
}

__device__ __forceinline__ float mf_compute(const MfQ4K& r, const v4i* A, const f32x4& sA, const f32x4& sB, int q,
                                            int) {
    return mf_compute_q4k<false>(r, A, sA, sB, q);
}
__device__ __forceinline__ float mf_compute(const MfQ4KT& r, const v4i* A, const f32x4& sA, const f32x4& sB, int q,
                                            int) {
    return mf_compute_q4k<true>(r, A, sA, sB, q);
}

// ---- Q6_K (Dequantizer.cs:378-417): 210-byte blocks -------------------------------------------
// A block starts 0 or 2 bytes past a 4-byte boundary (mis); each lane loads the dword-aligned
// windows of its fields and realigns them in registers. ql of group g: bytes 16g .. +15, qh of
// group g: bytes 128 + 8g .. +7, int8 scales at 192 (one per 16 elements), f16 d at 208.
struct MfQ6K { uint32_t la[5], lb[5], ha[3], hb[3], sa, sb, d; };
__device__ __forceinline__ void mf_issue(MfQ6K& r, const uint8_t* __restrict__ W, uint32_t off, int c, int mis,
                                         int q) {
    const uint8_t* blk = W + off + (uint32_t)(c * 210);
    const uint8_t* p = blk - mis;
    uint4 t = nt16a(p + 16 * q);
    r.la[0] = t.x; r.la[1] = t.y; r.la[2] = t.z; r.la[3] = t.w;
    r.la[4] = nt4(p + 16 + 16 * q);
    t = nt16a(p + 64 + 16 * q);
    r.lb[0] = t.x; r.lb[1] = t.y; r.lb[2] = t.z; r.lb[3] = t.w;
    r.lb[4] = nt4(p + 80 + 16 * q);
    uint2 h = nt8a(p + 128 + 8 * q);
    r.ha[0] = h.x; r.ha[1] = h.y;
    r.ha[2] = nt4(p + 136 + 8 * q);
    h = nt8a(p + 160 + 8 * q);
    r.hb[0] = h.x; r.hb[1] = h.y;
    r.hb[2] = nt4(p + 168 + 8 * q);
    r.sa = nt2(blk + 192 + 2 * q);  // scales 2q, 2q + 1
    r.sb = nt2(blk + 200 + 2 * q);  // scales 2q + 8, 2q + 9
    r.d = nt2(blk + 208);
}

// fragment of one half-group: 8 ql bytes (2 dwords) and the 4 qh bytes of those 16 elements;
// byte `by` of dword j = element 4by + j: low nibble of ql byte 2by + (j>>1), 2 high bits =
// field j of qh byte by
__device__ __forceinline__ v4i q6_frag(uint32_t l0, uint32_t l1, uint32_t hq) {
    uint32_t E = __builtin_amdgcn_perm(l1, l0, 0x06040200u);  // ql bytes 0,2,4,6
    uint32_t O = __builtin_amdgcn_perm(l1, l0, 0x07050301u);  // ql bytes 1,3,5,7
    uint32_t f0 = (E & 0x0F0F0F0Fu) | ((hq & 0x03030303u) << 4);
    uint32_t f1 = ((E >> 4) & 0x0F0F0F0Fu) | (((hq >> 2) & 0x03030303u) << 4);
    uint32_t f2 = (O & 0x0F0F0F0Fu) | (((hq >> 4) & 0x03030303u) << 4);
    uint32_t f3 = ((O >> 4) & 0x0F0F0F0Fu) | (((hq >> 6) & 0x03030303u) << 4);
    v4i r = {(int)f0, (int)f1, (int)f2, (int)f3};
    return r;
}

__device__ __forceinline__ float mf_compute(const MfQ6K& r, const v4i* A, const f32x4& sA, const f32x4& sB, int,
                                            int mis) {
    uint32_t la[4], lb[4], ha[2], hb[2];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        la[i] = __builtin_amdgcn_alignbyte(r.la[i + 1], r.la[i], mis);
        lb[i] = __builtin_amdgcn_alignbyte(r.lb[i + 1], r.lb[i], mis);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        ha[i] = __builtin_amdgcn_alignbyte(r.ha[i + 1], r.ha[i], mis);
        hb[i] = __builtin_amdgcn_alignbyte(r.hb[i + 1], r.hb[i], mis);
    }
    const v4i z = {0, 0, 0, 0};
    const v4i D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], q6_frag(la[0], la[1], ha[0]), z, 0, 0, 0);
    const v4i D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], q6_frag(la[2], la[3], ha[1]), z, 0, 0, 0);
    const v4i D2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], q6_frag(lb[0], lb[1], hb[0]), z, 0, 0, 0);
    const v4i D3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], q6_frag(lb[2], lb[3], hb[1]), z, 0, 0, 0);
    // y = (d * sc) * (q - 32) per element: (d * sc) * (s_x T - 32 * sum of the 16 activations)
    const float d = h2f(r.d);
    float y = (float)(int8_t)(r.sa & 0xFF) * fmaf(sA.x, mf_total(D0), -32.0f * sA.z);
    y = fmaf((float)(int8_t)(r.sa >> 8), fmaf(sA.y, mf_total(D1), -32.0f * sA.w), y);
    y = fmaf((float)(int8_t)(r.sb & 0xFF), fmaf(sB.x, mf_total(D2), -32.0f * sB.z), y);
    y = fmaf((float)(int8_t)(r.sb >> 8), fmaf(sB.y, mf_total(D3), -32.0f * sB.w), y);
    return d * y;
}

// Q6_K from a LAYOUT_TILES region: the lane's ql, qh and scale bytes are 4-byte aligned there
struct MfQ6KT { uint4 la, lb, h; uint32_t s, d; };
__device__ __forceinline__ void mf_issue_tiles(MfQ6KT& r, const uint8_t* __restrict__ reg, int lane, int n) {
    r.la = nt16(reg + 16 * lane);         // ql 16q .. 16q + 15
    r.lb = nt16(reg + 1024 + 16 * lane);  // ql 64 + 16q ..
    r.h = nt16(reg + 2048 + 16 * lane);   // qh 8q .. 8q + 7, qh 32 + 8q .. 32 + 8q + 7
    r.s = nt4(reg + 3072 + 4 * lane);     // scales 2q, 2q + 1, 8 + 2q, 9 + 2q
    r.d = nt2(reg + 3328 + 2 * n);
}

__device__ __forceinline__ float mf_compute(const MfQ6KT& r, const v4i* A, const f32x4& sA, const f32x4& sB, int,
                                            int) {
    const v4i z = {0, 0, 0, 0};
    const v4i D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], q6_frag(r.la.x, r.la.y, r.h.x), z, 0, 0, 0);
    const v4i D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], q6_frag(r.la.z, r.la.w, r.h.y), z, 0, 0, 0);
    const v4i D2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], q6_frag(r.lb.x, r.lb.y, r.h.z), z, 0, 0, 0);
    const v4i D3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], q6_frag(r.lb.z, r.lb.w, r.h.w), z, 0, 0, 0);
    const float d = h2f(r.d);
    float y = (float)(int8_t)(r.s & 0xFF) * fmaf(sA.x, mf_total(D0), -32.0f * sA.z);
    y = fmaf((float)(int8_t)((r.s >> 8) & 0xFF), fmaf(sA.y, mf_total(D1), -32.0f * sA.w), y);
    y = fmaf((float)(int8_t)((r.s >> 16) & 0xFF), fmaf(sB.x, mf_total(D2), -32.0f * sB.z), y);
    y = fmaf((float)(int8_t)(r.s >> 24), fmaf(sB.y, mf_total(D3), -32.0f * sB.w), y);
    return d * y;
}

// register image of one chunk of one lane, per weight type and layout
template <int T, bool IL> struct MfPick;
template <> struct MfPick<FLLM_TYPE_Q4_K, false> { using Raw = MfQ4K; };
template <> struct MfPick<FLLM_TYPE_Q4_K, true> { using Raw = MfQ4KT; };
template <> struct MfPick<FLLM_TYPE_Q6_K, false> { using Raw = MfQ6K; };
template <> struct MfPick<FLLM_TYPE_Q6_K, true> { using Raw = MfQ6KT; };

// ---- Q8_0 (Dequantizer.cs:203-231), tile-interleaved only: 8 blocks of 34 bytes per chunk ------
// In LAYOUT_TILES each 16-element half of a group is stored in the activation table's element
// order (byte 4 j + by = element 4 by + j), so the loaded dwords are the MFMA operand as they are;
// the lane's two block scales (groups q and q + 4) share one dword.
struct MfQ8T { uint4 a0, a1, b0, b1; uint32_t d; };
__device__ __forceinline__ void mf_issue_tiles(MfQ8T& r, const uint8_t* __restrict__ reg, int lane, int n) {
    r.a0 = nt16(reg + 16 * lane);         // group q, elements 0 .. 15
    r.a1 = nt16(reg + 1024 + 16 * lane);  // group q, elements 16 .. 31
    r.b0 = nt16(reg + 2048 + 16 * lane);  // group q + 4
    r.b1 = nt16(reg + 3072 + 16 * lane);
    r.d = nt4(reg + 4096 + 16 * n + 4 * (lane >> 4));
}
__device__ __forceinline__ v4i mf_v4i(const uint4& u) {
    v4i r = {(int)u.x, (int)u.y, (int)u.z, (int)u.w};
    return r;
}
// y = d_q * sum over group q of q_i x_i + d_{q+4} * (group q + 4): (sbyte)q * d per element
__device__ __forceinline__ float mf_compute(const MfQ8T& r, const v4i* A, const f32x4& sA, const f32x4& sB, int,
                                            int) {
    const v4i z = {0, 0, 0, 0};
    const v4i D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], mf_v4i(r.a0), z, 0, 0, 0);
    const v4i D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], mf_v4i(r.a1), z, 0, 0, 0);
    const v4i D2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], mf_v4i(r.b0), z, 0, 0, 0);
    const v4i D3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], mf_v4i(r.b1), z, 0, 0, 0);
    const float dq = h2f(r.d & 0xFFFFu), dq4 = h2f(r.d >> 16);
    return fmaf(dq, fmaf(sA.x, mf_total(D0), sA.y * mf_total(D1)), dq4 * fmaf(sB.x, mf_total(D2), sB.y * mf_total(D3)));
}
template <> struct MfPick<FLLM_TYPE_Q8_0, true> { using Raw = MfQ8T; };

// ---- Q5_K (Dequantizer.cs:316-368), tile-interleaved only ---------------------------------------
// Low nibbles as Q4_K (group g = qs bytes 16 g .. 16 g + 15); the 32 high bits of a group are
// regrouped at pack time so that bit 8 by + 4 h + j is the bit of element 16 h + 4 by + j: the high
// bits of fragment dword j of half h are then (H >> (4 h + j)) & 0x01010101, shifted to bit 4.
struct MfQ5KT { uint4 hdr, qa, qb; uint2 h; };
__device__ __forceinline__ void mf_issue_tiles(MfQ5KT& r, const uint8_t* __restrict__ reg, int lane, int n) {
    r.qa = nt16(reg + 16 * lane);         // qs of group q
    r.qb = nt16(reg + 1024 + 16 * lane);  // qs of group q + 4
    r.h = nt8(reg + 2048 + 8 * lane);     // high bits of groups q and q + 4
    r.hdr = nt16(reg + 2560 + 16 * n);    // d, dmin, scales
}
// q4_frag with bit 4 of each byte from the regrouped high bits of half h
__device__ __forceinline__ v4i q5_frag(uint32_t w0, uint32_t w1, uint32_t H, int h) {
    v4i f = q4_frag(w0, w1);
    f.x |= (int)(((H >> (4 * h + 0)) & 0x01010101u) << 4);
    f.y |= (int)(((H >> (4 * h + 1)) & 0x01010101u) << 4);
    f.z |= (int)(((H >> (4 * h + 2)) & 0x01010101u) << 4);
    f.w |= (int)(((H >> (4 * h + 3)) & 0x01010101u) << 4);
    return f;
}
__device__ __forceinline__ float mf_compute(const MfQ5KT& r, const v4i* A, const f32x4& sA, const f32x4& sB, int q,
                                            int) {
    const v4i z = {0, 0, 0, 0};
    const v4i D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], q5_frag(r.qa.x, r.qa.y, r.h.x, 0), z, 0, 0, 0);
    const v4i D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], q5_frag(r.qa.z, r.qa.w, r.h.x, 1), z, 0, 0, 0);
    const v4i D2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], q5_frag(r.qb.x, r.qb.y, r.h.y, 0), z, 0, 0, 0);
    const v4i D3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], q5_frag(r.qb.z, r.qb.w, r.h.y, 1), z, 0, 0, 0);
    // DecodeKScaleMin (Dequantizer.cs:506-521) for groups q (< 4) and q + 4, as Q4_K
    const int sh = 8 * q;
    const uint32_t a = (r.hdr.y >> sh) & 0xFF, b = (r.hdr.z >> sh) & 0xFF, c = (r.hdr.w >> sh) & 0xFF;
    const int scA = (int)(a & 63), mnA = (int)(b & 63);
    const int scB = (int)((c & 15) | ((a >> 6) << 4)), mnB = (int)((c >> 4) | ((b >> 6) << 4));
    const float d = h2f(r.hdr.x & 0xFFFFu), dmin = h2f(r.hdr.x >> 16);
    const float dgA = d * (float)scA, mgA = dmin * (float)mnA;
    const float dgB = d * (float)scB, mgB = dmin * (float)mnB;
    const float tA = fmaf(sA.x, mf_total(D0), sA.y * mf_total(D1));
    const float tB = fmaf(sB.x, mf_total(D2), sB.y * mf_total(D3));
    const float y = fmaf(dgA, tA, -mgA * (sA.z + sA.w));
    return y + fmaf(dgB, tB, -mgB * (sB.z + sB.w));
}
template <> struct MfPick<FLLM_TYPE_Q5_K, true> { using Raw = MfQ5KT; };

// Persistent workgroup body of the MFMA variant for weight type T. The launch's rows form units:
// one 16-row tile, or for GLU the gate and up tiles of the same 16 rows. Workgroup w takes units
// w, w + grid, w + 2 grid, ...; each of its nw waves covers KC consecutive chunks of every row
// (NB = nw KC chunks, or fewer for a ragged row), so all waves walk the same (tile, chunk) item
// sequence: item i is chunk i % KC of the workgroup's tile i / KC. Items stream through a ring of
// chunk loads in flight (MfRing) that runs across tile and unit boundaries; the first loads go out
// before the activation prologue. A lane's load addresses are its tile row's offset (computed once
// per tile) plus constants; with
// LAYOUT_TILES (IL) the tile offset is the same for all lanes of a wave and each load instruction
// of a wave reads one contiguous piece.
constexpr int MF_RING = 4;
// ring depth of a kernel (measured: deeper rings do not pay, a Q6_K ring of 8 is slower)
template <int T, int KC> struct MfRing { static constexpr int v = MF_RING; };

// unit u -> matrix of tile ts (0: gate / the segment's own, 1: up), its rows, first row, segment
__device__ __forceinline__ void mf_tile_of(const GemvArgs& a, int u, int ts, const uint8_t*& W, int& rows, int& row0,
                                           int& si) {
    const int ub1 = a.seg[1].wg_begin, ub2 = a.seg[2].wg_begin;
    si = (a.nseg > 2 && u >= ub2) ? 2 : (a.nseg > 1 && u >= ub1) ? 1 : 0;
    const int tile = u - (si == 2 ? ub2 : si == 1 ? ub1 : 0);
    const int mi = si + ts;
    W = mi == 0 ? a.seg[0].w : (mi == 1 ? a.seg[1].w : a.seg[2].w);
    rows = mi == 0 ? a.seg[0].rows : (mi == 1 ? a.seg[1].rows : a.seg[2].rows);
    row0 = tile * MF_TILE;
}

// workgroup tile t (its units are ufirst, ufirst + ustride, ...): its matrix and the byte offset of
// chunk kb0 of row n of the tile (IL: of the tile's region of chunk kb0; rb is the bytes of a row,
// so row0 * rb is where the tile's regions start)
template <bool IL>
__device__ __forceinline__ uint32_t mf_tile_base(const GemvArgs& a, int ufirst, int ustride, int t, int ltpu,
                                                 uint32_t rb, uint32_t kboff, int n, const uint8_t*& W) {
    const int u = ufirst + (t >> ltpu) * ustride;
    int rows, row0, si;
    mf_tile_of(a, u, t & ((1 << ltpu) - 1), W, rows, row0, si);
    const int row = IL ? row0 : min(row0 + n, rows - 1);
    return (uint32_t)row * rb + kboff;
}

// read instead of the activation table when there is none (keeps the prologue's loads unconditional)
__device__ u32x4 mf_tab_dummy[1];

// Per-workgroup state of the MFMA body that the item step reads.
struct MfCtx {
    lds_tab* at;        // this lane's A fragments of chunk kb0 (or the zero block)
    lds_f4* stats;
    float* part;
    float* red;
    uint32_t rb, kboff;
    float xs;
    int kb0, q, m, lane, wave, nw, ltpu, T_slots, ufirst, ustride, items;
    int cmax;  // ragged rows: chunks kb0 + c with c > cmax lie past the row (padding of the last wave)
    // residual and norm weight of row 16 * tile + (thread & 15) of the first tile (pre_on: it is a
    // residual add), loaded with the table
    int pre_on;
    float pre_r, pre_w;
};

// issue the loads of chunk kb0 + c of the tile at offset off of W into r
template <int T, bool IL, bool RAGGED = false>
__device__ __forceinline__ void mf_load(typename MfPick<T, IL>::Raw& r, const uint8_t* W, uint32_t off, int c,
                                        const MfCtx& x) {
    // ragged rows: a padding chunk re-reads the row's last one (its activations are zero)
    if constexpr (RAGGED) c = c < x.cmax ? c : x.cmax;
    if constexpr (IL) mf_issue_tiles(r, W + off + (uint32_t)(c * MF_TILE * mf_chunk_bytes(T)), x.lane, x.m);
    else mf_issue(r, W, off, c, ((x.kb0 + c) & 1) * 2, x.q);
}

// One item: chunk c = r % KC of workgroup tile i / KC, from ring slot r % RING. With refill the
// slot is reloaded with item i + RING. Every item but the last RING of the workgroup refills,
// and the choice is a compile-time constant of the unrolled item position, so the number of loads
// in flight at every wait is known at compile time.
template <int T, int KC, bool IL, bool REFILL, bool RAGGED = false>
__device__ __forceinline__ void mf_item(const GemvArgs& a, const MfCtx& x, typename MfPick<T, IL>::Raw* ring, int i, int r,
                                        float& y, uint32_t& offr, const uint8_t*& Wr, unsigned long long& best) {
    constexpr int LKC = KC == 1 ? 0 : KC == 2 ? 1 : KC == 4 ? 2 : 3;
    constexpr int RING = MfRing<T, KC>::v;
    const int c = r & (KC - 1), slot = r & (RING - 1), b = x.kb0 + c;
    v4i A[4];
#pragma unroll
    for (int s = 0; s < 4; s++) A[s] = *(__attribute__((address_space(3))) const v4i*)&x.at[(4 * c + s) * 12];
    const f32x4 sa = x.stats[b * 8 + x.q], sb = x.stats[b * 8 + x.q + 4];
    y += mf_compute(ring[slot], A, sa, sb, x.q, (b & 1) * 2);
    // finish this item's arithmetic here (sinking it to the tile's end keeps every item's MFMA
    // results live)
    __asm__ volatile("" : "+v"(y));
    if (REFILL) {
        const int cn = (r + RING) & (KC - 1);
        if (cn == 0) offr = mf_tile_base<IL>(a, x.ufirst, x.ustride, (i + RING) >> LKC, x.ltpu, x.rb, x.kboff, x.m, Wr);
        mf_load<T, IL, RAGGED>(ring[slot], Wr, offr, cn, x);
    }
    // keep each item's fragment reads next to its MFMAs
    __builtin_amdgcn_sched_barrier(0);
    if (c == KC - 1) {
        // last chunk of the tile: the four quarters of row n, then this wave's partial
        const int ti = i >> LKC, tt = ti & ((1 << x.ltpu) - 1);
        float yt = y + __shfl_xor(y, 16);
        yt += __shfl_xor(yt, 32);
        if (x.lane < 16) x.part[x.wave * x.T_slots + tt * MF_TILE + x.lane] = yt * x.xs;
        y = 0.0f;
        if (tt == (1 << x.ltpu) - 1) {
            // last tile of the unit (same item in every wave): combine the waves, epilogue
            const uint8_t* Wu;
            int rows, row0, si;
            mf_tile_of(a, x.ufirst + (ti >> x.ltpu) * x.ustride, 0, Wu, rows, row0, si);
            __syncthreads();
            const EpiSeg es{si == 0 ? a.seg[0].rows : si == 1 ? a.seg[1].rows : a.seg[2].rows,
                            si == 0 ? a.seg[0].epi : si == 1 ? a.seg[1].epi : a.seg[2].epi,
                            si == 0 ? a.seg[0].out : si == 1 ? a.seg[1].out : a.seg[2].out,
                            si == 0 ? a.seg[0].bias : si == 1 ? a.seg[1].bias : a.seg[2].bias,
                            si == 0 ? a.seg[0].resid : si == 1 ? a.seg[1].resid : a.seg[2].resid,
                            x.pre_on && (ti >> x.ltpu) == 0, x.pre_r, x.pre_w};
            epilogue(a, es, x.part, x.red, x.nw, MF_TILE, x.T_slots, row0, x.wave, x.lane, best);
            __syncthreads();
        }
    }
}

// The last N items of a workgroup (N < 2 RING, first item at a multiple of RING) as straight-line
// code: the first N - RING refill, the rest do not. One instantiation per remainder keeps the
// per-item refill choice a compile-time constant, as in the main loop (a runtime choice per item
// keeps both variants' registers live).
template <int T, int KC, bool IL, bool RAGGED, int N>
__device__ __forceinline__ void mf_tail(const GemvArgs& a, const MfCtx& x, typename MfPick<T, IL>::Raw* ring, int i0,
                                        float& y, uint32_t& offr, const uint8_t*& Wr, unsigned long long& best) {
    constexpr int RING = MfRing<T, KC>::v;
#pragma unroll
    for (int r = 0; r < N; r++) {
        if (r + RING < N) mf_item<T, KC, IL, true, RAGGED>(a, x, ring, i0 + r, r, y, offr, Wr, best);
        else mf_item<T, KC, IL, false, RAGGED>(a, x, ring, i0 + r, r, y, offr, Wr, best);
    }
}

// The Gemma-2 post-norm prologue with two threads per 32-element group (Gemma2ForwardPass.cs:90-96),
// thread half hh of group g (live: g < G) holding its 16 values of x2, x, post_w and the norm weight:
// the new residual is x + (x2 * rms(x2)) * (post_w + 1), the operation order of the separate
// post-norm kernel, stored by workgroup 0, then normalized as XIN_NORM into the table.
__device__ __forceinline__ void post_prologue_half(const GemvArgs& a, MfCtx& x, lds_tab* atab, int g, int hh,
                                                   bool live, const float* t2, float* xv, const float* pw,
                                                   const float* wv) {
    float ss = 0.0f;
    if (live) {
#pragma unroll
        for (int i = 0; i < 16; i++) ss = fmaf(t2[i], t2[i], ss);
    }
    ss = wsum(ss);
    if (x.lane == 0) x.red[x.wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < x.nw; i++) tot += x.red[i];
    const float prms = 1.0f / sqrtf(tot / (float)(a.G * 32) + 1e-6f);
    __syncthreads();  // x.red is reused below
    float ssq = 0.0f;
    if (live) {
#pragma unroll
        for (int i = 0; i < 16; i++) xv[i] = xv[i] + (t2[i] * prms) * (pw[i] + 1.0f);
#pragma unroll
        for (int i = 0; i < 16; i++) ssq = fmaf(xv[i], xv[i], ssq);
    }
    ssq = wsum(ssq);
    if (x.lane == 0) x.red[x.wave] = ssq;
    __syncthreads();
    tot = 0.0f;
    for (int i = 0; i < x.nw; i++) tot += x.red[i];
    const float scale = 1.0f / sqrtf(tot / (float)(a.G * 32) + a.eps);  // rms
    float hsc = 0.0f, hsm = 0.0f;
    if (live) {
        const int e0 = g * 32 + 16 * hh;
        if (blockIdx.x == 0) {
            float4* xo = (float4*)(a.x_out + e0);
#pragma unroll
            for (int i = 0; i < 4; i++) xo[i] = make_float4(xv[4 * i], xv[4 * i + 1], xv[4 * i + 2], xv[4 * i + 3]);
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float t = xv[i] * scale;
            xv[i] = a.norm_kind ? t * (wv[i] + 1.0f) : t * wv[i];
        }
        atab_write_half(atab, g >> 3, g & 7, hh, xv, hsc, hsm);
    }
    // the group's stats {scale of half 0, of half 1, sum of half 0, of half 1} from the pair
    const float osc = __shfl_xor(hsc, 1), osm = __shfl_xor(hsm, 1);
    if (live && hh == 0) {
        const f32x4 stv = {hsc, osc, hsm, osm};
        x.stats[(g >> 3) * 8 + (g & 7)] = stv;
    }
}

// the 16 values of half hh of group g of the post-norm's four vectors
__device__ __forceinline__ void post_load_half(const GemvArgs& a, int g, int hh, float* t2, float* xv, float* pw,
                                               float* wv) {
    const int e0 = g * 32 + 16 * hh;
    const float4* ti = (const float4*)(a.x2 + e0);
    const float4* xi = (const float4*)(a.x + e0);
    const float4* pi = (const float4*)(a.post_w + e0);
    const float4* wi = (const float4*)(a.norm_w + e0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 t = ti[i], u = xi[i], p4 = pi[i], w4 = wi[i];
        t2[4 * i] = t.x; t2[4 * i + 1] = t.y; t2[4 * i + 2] = t.z; t2[4 * i + 3] = t.w;
        xv[4 * i] = u.x; xv[4 * i + 1] = u.y; xv[4 * i + 2] = u.z; xv[4 * i + 3] = u.w;
        pw[4 * i] = p4.x; pw[4 * i + 1] = p4.y; pw[4 * i + 2] = p4.z; pw[4 * i + 3] = p4.w;
        wv[4 * i] = w4.x; wv[4 * i + 1] = w4.y; wv[4 * i + 2] = w4.z; wv[4 * i + 3] = w4.w;
    }
}

// Input kinds of the matrix-core body's instantiations. XK_TAB: an activation table (XIN_TAB).
// XK_ANY: a vector quantized here, its kind chosen at run time (XIN_F32 / XIN_NORM /
// XIN_EMBED_NORM / XIN_POST). XK_F32: a plain f32 vector (XIN_F32), each thread's 32-element group
// loaded before the weight ring, so the table is ready when those loads return instead of behind
// the ring's (a wave's loads return in order), and without the other kinds' registers.
// XK_POST: a Gemma-2 post-norm folded in (XIN_POST) with two threads per 32-element group, its four
// vectors loaded before the weight ring.
enum { XK_TAB = 0, XK_ANY = 1, XK_F32 = 2, XK_POST = 3 };

// XK: the input kind (above). The workgroup is number wg of ng that share units [u0, u0 + nu) of
// the launch.
// RAGGED: the row's NB chunks do not split evenly: the nw waves of KC chunks cover nw * KC >= NB,
// and the last wave's chunks past the row have zero activations (their weight loads re-read the
// row's last chunk), so they add nothing.
template <int T, int KC, int XK, bool IL, bool RAGGED = false>
__device__ __forceinline__ void mfma_body(const GemvArgs& a, int u0, int nu, int wg, int ng) {
    constexpr bool TABIN = XK == XK_TAB;
    using Raw = typename MfPick<T, IL>::Raw;
    constexpr int CB = mf_chunk_bytes(T);
    constexpr int LKC = KC == 1 ? 0 : KC == 2 ? 1 : KC == 4 ? 2 : 3;
    constexpr int RING = MfRing<T, KC>::v;
    constexpr int U = KC > RING ? KC : RING;  // items per unrolled iteration
    extern __shared__ float lds[];
    MfCtx x;
    x.nw = a.nw;  // blockDim.x / 64 (the kernel argument avoids reading the dispatch packet)
    x.wave = threadIdx.x >> 6;
    x.lane = threadIdx.x & 63;
    x.q = x.lane >> 4;
    x.m = x.lane & 15;
    const bool a_live = (x.m >> 2) == x.q && (x.m & 3) < 3;  // A row m = 4Q' + d lives in quarter Q'
    const int NB = a.G / 8;            // chunks per row (NB == nw * KC unless RAGGED)
    const int NBP = RAGGED ? x.nw * KC : NB;  // chunk slots of the table in LDS
    x.kb0 = x.wave * KC;
    x.cmax = NB - 1 - x.kb0;
    x.ltpu = a.glu ? 1 : 0;            // log2 of tiles per unit
    x.T_slots = MF_TILE << x.ltpu;
    x.part = lds;                              // [nw][T_slots]
    x.red = lds + x.nw * x.T_slots;            // [16] + 16 u64
    lds_tab* zeros = (lds_tab*)(x.red + 48);   // A operand of lanes without a table row
    lds_tab* atab = zeros + MF_ZERO_ENTRIES(KC);
    x.stats = (lds_f4*)(atab + NBP * 48);
    // fragment (chunk kb0 + c, step s) of this lane: x.at[(4c + s) * 12]
    lds_tab* const abase = a_live ? atab + atab_index(x.kb0, 0, x.m >> 2, x.m & 3) : zeros;
    x.rb = (uint32_t)NB * CB;
    x.kboff = (uint32_t)x.kb0 * (IL ? MF_TILE * CB : CB);
    x.ufirst = u0 + wg;
    x.ustride = ng;
    const int my_units = (nu - wg + ng - 1) / ng;
    x.items = (my_units << x.ltpu) * KC;

    // ---- a table input: each wave copies the part its own chunks use (digit entries of chunks
    // kb0 .. kb0 + KC - 1, their stats) and sums its share of the squares. These loads go out before
    // the weight ring, so waiting for them is not waiting for weights; fixed counts with clamped
    // indices keep the wait counts exact.
    constexpr int TDL = (KC * 48 + 63) / 64, TSL = (KC * 16 + 63) / 64;
    // (without a table the loads all read one dummy entry and go unused)
    u32x4 tdig[TDL];
    float tsq[TSL];
    constexpr bool tab_in = TABIN;
    const int tm = tab_in ? 1 : 0;
    const u32x4* tsrc = tab_in ? (const u32x4*)a.xtab : mf_tab_dummy;
    // (ragged rows: entries of chunks past the row read entry 0 and are replaced by zeros)
#pragma unroll
    for (int k = 0; k < TDL; k++) {
        const int e = min(x.lane + 64 * k, KC * 48 - 1);
        const bool live = !RAGGED || x.kb0 + e / 48 < NB;
        tdig[k] = tsrc[tm * (live ? x.kb0 * 48 + e : 0)];
    }
    const int es = min(x.lane, KC * 8 - 1);
    const bool st_live = !RAGGED || x.kb0 + es / 8 < NB;
    u32x4 tst = tsrc[tm * (st_live ? NB * 48 + x.kb0 * 8 + es : 0)];
    const int sm = (tab_in && a.xssq) ? 1 : 0;
    const float* sp = sm ? a.xssq : (const float*)mf_tab_dummy;
#pragma unroll
    for (int k = 0; k < TSL; k++) {
        const int e = min(x.lane + 64 * k, KC * 16 - 1);
        const bool live = !RAGGED || x.kb0 + e / 16 < NB;
        tsq[k] = sp[sm * (live ? x.kb0 * 16 + e : 0)];
    }
    if constexpr (RAGGED) {
        const u32x4 z4 = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < TDL; k++)
            if (x.kb0 + min(x.lane + 64 * k, KC * 48 - 1) / 48 >= NB) tdig[k] = z4;
        if (!st_live) tst = z4;
#pragma unroll
        for (int k = 0; k < TSL; k++)
            if (x.kb0 + min(x.lane + 64 * k, KC * 16 - 1) / 16 >= NB) tsq[k] = 0.0f;
    }
    // XK_F32: with 8 or 4 chunks per wave a wave quantizes its own chunks' groups (one per lane, or
    // a 16-element half per lane), so it needs no other wave's entries (XL: lanes per group); with
    // fewer, thread t takes group t of the row (XL = 0). Threads past the groups read the row's last
    // group and write nothing.
    constexpr int XL = XK != XK_F32 ? 0 : KC == 8 ? 1 : KC == 4 ? 2 : 0;
    constexpr int XN = XK != XK_F32 ? 1 : XL == 2 ? 16 : 32;
    const int xgrp = XL == 1 ? x.kb0 * 8 + x.lane : XL == 2 ? x.kb0 * 8 + (x.lane >> 1) : (int)threadIdx.x;
    float xg[XN];
    if constexpr (XK == XK_F32) {
        const float4* xi = (const float4*)(a.x + min(xgrp, a.G - 1) * 32 + (XL == 2 ? 16 * (x.lane & 1) : 0));
#pragma unroll
        for (int i = 0; i < XN / 4; i++) {
            const float4 t = xi[i];
            xg[4 * i] = t.x; xg[4 * i + 1] = t.y; xg[4 * i + 2] = t.z; xg[4 * i + 3] = t.w;
        }
    }
    // XK_POST: this thread's half group of the post-norm's vectors (threads past the row's groups
    // read its last group and write nothing)
    constexpr int PN = XK == XK_POST ? 16 : 1;
    float p_t2[PN], p_xv[PN], p_pw[PN], p_wv[PN];
    if constexpr (XK == XK_POST)
        post_load_half(a, min((int)threadIdx.x >> 1, a.G - 1), (int)threadIdx.x & 1, p_t2, p_xv, p_pw, p_wv);
    // the residual and the consumer's norm weight of the first tile's rows, when it is a residual
    // add: written by earlier launches, so they go out with the table rather than after the last
    // weights (where they would add a round trip to the epilogue)
    {
        const uint8_t* Wu;
        int rows_u, row0_u, si_u;
        mf_tile_of(a, x.ufirst, 0, Wu, rows_u, row0_u, si_u);
        const float* rs = si_u == 0 ? a.seg[0].resid : si_u == 1 ? a.seg[1].resid : a.seg[2].resid;
        const int epi_u = si_u == 0 ? a.seg[0].epi : si_u == 1 ? a.seg[1].epi : a.seg[2].epi;
        x.pre_on = (!a.glu && epi_u == EPI_RESID && rs != nullptr && x.items > 0) ? 1 : 0;
        const int rr = min(row0_u + (int)(threadIdx.x & 15), rows_u - 1);
        const float* rp = x.pre_on ? rs + rr : (const float*)mf_tab_dummy;
        const float* wp = (x.pre_on && a.tab_w) ? a.tab_w + rr : (const float*)mf_tab_dummy;
        x.pre_r = *rp;
        x.pre_w = *wp;
    }
    __builtin_amdgcn_sched_barrier(0);
    // every wave's input loads are issued before any wave's weight ring: a CU serves a wave's
    // loads in the order the waves issued them, so the table would otherwise wait behind the other
    // waves' rings (a barrier without a memory fence: nothing waits for the loads here)
    if constexpr (XK != XK_ANY) __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    Raw ring[RING];
    const uint8_t* Wr = a.seg[0].w;  // matrix and lane offset of the tile of the latest load
    uint32_t offr = 0;
#pragma unroll
    for (int r = 0; r < RING; r++) {
        const int c = r & (KC - 1);
        // fewer items than ring slots (a single tile of KC < RING chunks): reload its last chunk
        if (c == 0 && r < x.items) offr = mf_tile_base<IL>(a, x.ufirst, x.ustride, r >> LKC, x.ltpu, x.rb, x.kboff, x.m, Wr);
        mf_load<T, IL, RAGGED>(ring[r], Wr, offr, c, x);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- prologue: the activation table -------------------------------------------------------
    // (a wave-local table: every wave writes the zero block itself, so no wave waits for another)
    constexpr bool WAVE_LOCAL = XL != 0 || TABIN;
    for (int e = WAVE_LOCAL ? x.lane : (int)threadIdx.x; e < MF_ZERO_ENTRIES(KC); e += WAVE_LOCAL ? 64 : x.nw * 64) {
        const u32x4 z4 = {0u, 0u, 0u, 0u};
        zeros[e] = z4;
    }
    if constexpr (RAGGED && !TABIN) {
        // the vector prologue below fills the row's chunks; the padding chunks' digits and stats
        // are zero
        const u32x4 z4 = {0u, 0u, 0u, 0u};
        for (int e = NB * 48 + threadIdx.x; e < NBP * 48; e += x.nw * 64) atab[e] = z4;
        const f32x4 zf = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int e = NB * 8 + threadIdx.x; e < NBP * 8; e += x.nw * 64) x.stats[e] = zf;
    }
    x.xs = 1.0f;  // RMSNorm factor of a table of raw (weighted) values
    if constexpr (tab_in) {
#pragma unroll
        for (int k = 0; k < TDL; k++) atab[x.kb0 * 48 + min(x.lane + 64 * k, KC * 48 - 1)] = tdig[k];
        x.stats[x.kb0 * 8 + min(x.lane, KC * 8 - 1)] = *(const f32x4*)&tst;
        if (a.xssq) {
            // the RMSNorm factor needs every wave's share of the sum of squares
            float s2 = 0.0f;
#pragma unroll
            for (int k = 0; k < TSL; k++) s2 += x.lane + 64 * k < KC * 16 ? tsq[k] : 0.0f;
            s2 = wsum(s2);
            if (x.lane == 0) x.red[x.wave] = s2;
            __syncthreads();
            float tot = 0.0f;
            for (int i = 0; i < x.nw; i++) tot += x.red[i];
            x.xs = 1.0f / sqrtf(tot / (float)(a.G * 32) + a.eps);
        }
    } else if constexpr (XK == XK_F32) {
        // (a wave's items read only its own chunks' entries)
        const int g = xgrp;
        if constexpr (XL == 2) {
            float hsc = 0.0f, hsm = 0.0f;
            atab_write_half(atab, g >> 3, g & 7, x.lane & 1, xg, hsc, hsm);
            // the group's stats {scale of half 0, of half 1, sum of half 0, of half 1} from the pair
            const float osc = __shfl_xor(hsc, 1), osm = __shfl_xor(hsm, 1);
            if ((x.lane & 1) == 0) {
                const f32x4 stv = {hsc, osc, hsm, osm};
                x.stats[(g >> 3) * 8 + (g & 7)] = stv;
            }
        } else if (XL == 1 ? x.lane < 8 * KC : g < a.G) {
            float4 st;
            atab_write(atab, g >> 3, g & 7, xg, &st);
            f32x4 stv = {st.x, st.y, st.z, st.w};
            x.stats[(g >> 3) * 8 + (g & 7)] = stv;
        }
    } else if constexpr (XK == XK_POST) {
        const int g = (int)threadIdx.x >> 1;
        post_prologue_half(a, x, atab, g, (int)threadIdx.x & 1, g < a.G, p_t2, p_xv, p_pw, p_wv);
    } else if (a.xin == XIN_POST && 2 * a.G <= x.nw * 64) {
        // two threads per 32-element group (one per 16-element half, the table's quantization
        // unit): x2, x, post_w and the norm weight all load at once and stay in registers across
        // the two reductions
        const int g = (int)threadIdx.x >> 1, hh = (int)threadIdx.x & 1;
        const bool live = g < a.G;
        float t2[16], xv[16], pw[16], wv[16];
        if (live) post_load_half(a, g, hh, t2, xv, pw, wv);
        post_prologue_half(a, x, atab, g, hh, live, t2, xv, pw, wv);
    } else if (a.xin == XIN_POST && a.G <= x.nw * 64) {
        // Gemma-2 post-norm folded in (Gemma2ForwardPass.cs:90-96), one 32-element group per
        // thread: x2 and x stay in registers across the two reductions, so every vector is read
        // once. The new residual is x + (x2 * rms(x2)) * (post_w + 1), the operation order of the
        // separate post-norm kernel, then normalized as XIN_NORM.
        const int g = (int)threadIdx.x;
        const bool live = g < a.G;
        float t2[32], xv[32];
        float ss = 0.0f;
        if (live) {
            const float4* ti = (const float4*)(a.x2 + g * 32);
            const float4* xi = (const float4*)(a.x + g * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 t = ti[i], u = xi[i];
                t2[4 * i] = t.x; t2[4 * i + 1] = t.y; t2[4 * i + 2] = t.z; t2[4 * i + 3] = t.w;
                xv[4 * i] = u.x; xv[4 * i + 1] = u.y; xv[4 * i + 2] = u.z; xv[4 * i + 3] = u.w;
            }
#pragma unroll
            for (int i = 0; i < 32; i++) ss = fmaf(t2[i], t2[i], ss);
        }
        ss = wsum(ss);
        if (x.lane == 0) x.red[x.wave] = ss;
        __syncthreads();
        float tot = 0.0f;
        for (int i = 0; i < x.nw; i++) tot += x.red[i];
        const float prms = 1.0f / sqrtf(tot / (float)(a.G * 32) + 1e-6f);
        __syncthreads();  // x.red is reused below
        float ssq = 0.0f;
        if (live) {
            const float4* pw = (const float4*)(a.post_w + g * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 w4 = pw[i];
                const float ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) xv[4 * i + e] = xv[4 * i + e] + (t2[4 * i + e] * prms) * (ww[e] + 1.0f);
            }
#pragma unroll
            for (int i = 0; i < 32; i++) ssq = fmaf(xv[i], xv[i], ssq);
        }
        ssq = wsum(ssq);
        if (x.lane == 0) x.red[x.wave] = ssq;
        __syncthreads();
        tot = 0.0f;
        for (int i = 0; i < x.nw; i++) tot += x.red[i];
        const float scale = 1.0f / sqrtf(tot / (float)(a.G * 32) + a.eps);  // rms
        if (live) {
            if (blockIdx.x == 0) {
                float4* xo = (float4*)(a.x_out + g * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) xo[i] = make_float4(xv[4 * i], xv[4 * i + 1], xv[4 * i + 2], xv[4 * i + 3]);
            }
            const float4* wv = (const float4*)(a.norm_w + g * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 w4 = wv[i];
                const float ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float t = xv[4 * i + e] * scale;
                    xv[4 * i + e] = a.norm_kind ? t * (ww[e] + 1.0f) : t * ww[e];
                }
            }
            float4 st;
            atab_write(atab, g >> 3, g & 7, xv, &st);
            f32x4 stv = {st.x, st.y, st.z, st.w};
            x.stats[(g >> 3) * 8 + (g & 7)] = stv;
        }
    } else {
        // XIN_POST over more groups than threads: the scale of the post-norm over x2 first, then
        // the rows below recompute the new residual
        float prms = 1.0f;
        if (a.xin == XIN_POST) {
            float ss = 0.0f;
            for (int g = threadIdx.x; g < a.G; g += x.nw * 64) {
                const float4* ti = (const float4*)(a.x2 + g * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float4 t = ti[i];
                    ss = fmaf(t.x, t.x, ss);
                    ss = fmaf(t.y, t.y, ss);
                    ss = fmaf(t.z, t.z, ss);
                    ss = fmaf(t.w, t.w, ss);
                }
            }
            ss = wsum(ss);
            if (x.lane == 0) x.red[x.wave] = ss;
            __syncthreads();
            float tot = 0.0f;
            for (int i = 0; i < x.nw; i++) tot += x.red[i];
            prms = 1.0f / sqrtf(tot / (float)(a.G * 32) + 1e-6f);
            __syncthreads();  // x.red is reused below
        }
        // this group's input row: the embedding row, x, or (XIN_POST) the new residual
        auto row = [&](int g, float* v) {
            if (a.xin == XIN_EMBED_NORM) {
                deq32(a.emb_type, a.emb, (int64_t)a.params->token * a.G * 32 + g * 32, v);
                return;
            }
            const float4* xi = (const float4*)(a.x + g * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) { float4 t = xi[i]; v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w; }
            if (a.xin == XIN_POST) {
                const float4* ti = (const float4*)(a.x2 + g * 32);
                const float4* pw = (const float4*)(a.post_w + g * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float4 t = ti[i], w4 = pw[i];
                    v[4 * i] = v[4 * i] + (t.x * prms) * (w4.x + 1.0f);
                    v[4 * i + 1] = v[4 * i + 1] + (t.y * prms) * (w4.y + 1.0f);
                    v[4 * i + 2] = v[4 * i + 2] + (t.z * prms) * (w4.z + 1.0f);
                    v[4 * i + 3] = v[4 * i + 3] + (t.w * prms) * (w4.w + 1.0f);
                }
            }
        };
        float scale = 1.0f;
        if (a.xin != XIN_F32) {
            float ssq = 0.0f;
            for (int g = threadIdx.x; g < a.G; g += x.nw * 64) {
                float v[32];
                row(g, v);
#pragma unroll
                for (int i = 0; i < 32; i++) ssq = fmaf(v[i], v[i], ssq);
            }
            ssq = wsum(ssq);
            if (x.lane == 0) x.red[x.wave] = ssq;
            __syncthreads();
            float tot = 0.0f;
            for (int i = 0; i < x.nw; i++) tot += x.red[i];
            scale = 1.0f / sqrtf(tot / (float)(a.G * 32) + a.eps);  // rms
        }
        for (int g = threadIdx.x; g < a.G; g += x.nw * 64) {
            float v[32];
            row(g, v);
            if ((a.xin == XIN_EMBED_NORM || a.xin == XIN_POST) && blockIdx.x == 0) {
                float4* xo = (float4*)(a.x_out + g * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) xo[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
            }
            if (a.xin != XIN_F32) {
                const float4* wv = (const float4*)(a.norm_w + g * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float4 w4 = wv[i];
                    float ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        float t = v[4 * i + e] * scale;
                        v[4 * i + e] = a.norm_kind ? t * (ww[e] + 1.0f) : t * ww[e];
                    }
                }
            }
            float4 st;
            atab_write(atab, g >> 3, g & 7, v, &st);
            f32x4 stv = {st.x, st.y, st.z, st.w};
            x.stats[(g >> 3) * 8 + (g & 7)] = stv;
        }
    }
    if constexpr (WAVE_LOCAL) {
        // a wave's items read only its own chunks' entries, written by its own lanes (the table
        // input's copy or the f32 input's quantization)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
        __syncthreads();
    }

    // ---- items ----------------------------------------------------------------------------------
    unsigned long long best = 0ull;
    float y = 0.0f;
    if constexpr (KC >= RING) {
        // whole iterations of one tile; the last one refills only its own items RING ahead
        const int n_it = x.items / U;
        for (int it = 0; it + 1 < n_it; it++) {
            x.at = abase;
            __asm__ volatile("" : "+v"(x.at));  // re-read the fragments from LDS each iteration
#pragma unroll
            for (int r = 0; r < U; r++) mf_item<T, KC, IL, true, RAGGED>(a, x, ring, it * U + r, r, y, offr, Wr, best);
        }
        x.at = abase;
        __asm__ volatile("" : "+v"(x.at));
        const int i0 = (n_it - 1) * U;
#pragma unroll
        for (int r = 0; r < U - RING; r++) mf_item<T, KC, IL, true, RAGGED>(a, x, ring, i0 + r, r, y, offr, Wr, best);
#pragma unroll
        for (int r = U - RING; r < U; r++) mf_item<T, KC, IL, false, RAGGED>(a, x, ring, i0 + r, r, y, offr, Wr, best);
    } else if constexpr (KC == RING / 2) {
        // U == RING items per iteration while the item RING ahead of each exists, then the last
        // 0 .. U + RING - 1 items (a multiple of KC) as one straight-line tail
        int i0 = 0;
        for (; i0 + U + RING <= x.items; i0 += U) {
            x.at = abase;
            __asm__ volatile("" : "+v"(x.at));
#pragma unroll
            for (int r = 0; r < U; r++) mf_item<T, KC, IL, true, RAGGED>(a, x, ring, i0 + r, r, y, offr, Wr, best);
        }
        x.at = abase;
        __asm__ volatile("" : "+v"(x.at));
        switch (x.items - i0) {
            case 2: mf_tail<T, KC, IL, RAGGED, 2>(a, x, ring, i0, y, offr, Wr, best); break;
            case 4: mf_tail<T, KC, IL, RAGGED, 4>(a, x, ring, i0, y, offr, Wr, best); break;
            case 6: mf_tail<T, KC, IL, RAGGED, 6>(a, x, ring, i0, y, offr, Wr, best); break;
            default: break;
        }
    } else {
        for (int i0 = 0; i0 < x.items; i0 += U) {
            x.at = abase;
            __asm__ volatile("" : "+v"(x.at));
#pragma unroll
            for (int r = 0; r < U; r++) {
                const int i = i0 + r;
                if (i >= x.items) break;
                if (i + RING < x.items) mf_item<T, KC, IL, true, RAGGED>(a, x, ring, i, r, y, offr, Wr, best);
                else mf_item<T, KC, IL, false, RAGGED>(a, x, ring, i, r, y, offr, Wr, best);
            }
        }
    }
    if (a.seg[0].epi == EPI_LOGITS && threadIdx.x == 0) a.wg_keys[blockIdx.x] = best;  // reduced by the argmax kernel
}

// one kernel per (weight type, chunks per wave, input kind, weight layout), each with its own
// register allocation; every segment of such a launch has the same weight type and layout
template <int T, int KC, int XK, bool IL>
__global__ __launch_bounds__(512) void k_gemv_mfma(const GemvArgs a) {
    mfma_body<T, KC, XK, IL>(a, 0, a.nunits, (int)blockIdx.x, (int)gridDim.x);
}

// Two weight types in one launch (q and k in Q4_K, v in Q6_K): the first mix_wg workgroups take the
// Q4_K units [0, mix_unit), the others the Q6_K units after them.
template <int KC, int XK, bool IL>
__global__ __launch_bounds__(512) void k_gemv_mfma_mix(const GemvArgs a) {
    if ((int)blockIdx.x < a.mix_wg)
        mfma_body<FLLM_TYPE_Q4_K, KC, XK, IL>(a, 0, a.mix_unit, (int)blockIdx.x, a.mix_wg);
    else
        mfma_body<FLLM_TYPE_Q6_K, KC, XK, IL>(a, a.mix_unit, a.nunits - a.mix_unit, (int)blockIdx.x - a.mix_wg,
                                             (int)gridDim.x - a.mix_wg);
}

// waves per workgroup and chunks per wave (*kc) for rows of NB chunks: 10 or 14 chunks as 4 per
// wave with the last wave partly past the row (a ragged row: 2 chunks per wave would leave one
// workgroup of 5 or 7 waves per CU at its register count); else an even split over at most 8 waves
// of 1, 2, 4 or 8 chunks (4 preferred), else 8 chunks per wave over up to 10 waves with the last one
// partly past the row (e.g. 74 chunks); 0: no split
static int mf_split(int NB, int* kc) {
    if (NB == 10 || NB == 14) {
        *kc = 4;
        return (NB + 3) / 4;
    }
    const int order[4] = {4, 8, 2, 1};
    for (int c : order)
        if (NB % c == 0 && NB / c <= 8) {
            *kc = c;
            return NB / c;
        }
    if (NB > 64 && NB <= 80) {
        *kc = 8;
        return (NB + 7) / 8;
    }
    *kc = 0;
    return 0;
}
static int mf_waves(int NB) {
    int kc;
    return mf_split(NB, &kc);
}
static int mf_kc(int NB) {
    int kc;
    mf_split(NB, &kc);
    return kc;
}
static bool mf_ragged(int NB) {
    int kc;
    const int nw = mf_split(NB, &kc);
    return nw > 0 && nw * kc != NB;
}

// ragged rows (chunks that do not split evenly): KC chunks per wave, the last wave partly past the row
template <int T, int KC, int XK>
__global__ __launch_bounds__(KC == 8 ? 640 : 512) void k_gemv_mfma_r(const GemvArgs a) {
    mfma_body<T, KC, XK, true, true>(a, 0, a.nunits, (int)blockIdx.x, (int)gridDim.x);
}

typedef void (*MfKernel)(const GemvArgs);
template <int T, int XK, bool IL>
static MfKernel mf_kernel_kc(int kc) {
    switch (kc) {
        case 1: return k_gemv_mfma<T, 1, XK, IL>;
        case 2: return k_gemv_mfma<T, 2, XK, IL>;
        case 4: return k_gemv_mfma<T, 4, XK, IL>;
        default: return k_gemv_mfma<T, 8, XK, IL>;
    }
}
// XK_F32 for a plain vector input (one weight type, rows that split evenly), else XK_TAB / XK_ANY
template <int T, bool IL>
static MfKernel mf_kernel_in(int xk, int kc) {
    return xk == XK_TAB ? mf_kernel_kc<T, XK_TAB, IL>(kc) : xk == XK_F32 ? mf_kernel_kc<T, XK_F32, IL>(kc)
                                                                         : mf_kernel_kc<T, XK_ANY, IL>(kc);
}
template <bool TABIN, bool IL>
static MfKernel mf_kernel_mix(int kc) {
    constexpr int XK = TABIN ? XK_TAB : XK_ANY;
    switch (kc) {
        case 1: return k_gemv_mfma_mix<1, XK, IL>;
        case 2: return k_gemv_mfma_mix<2, XK, IL>;
        case 4: return k_gemv_mfma_mix<4, XK, IL>;
        default: return k_gemv_mfma_mix<8, XK, IL>;
    }
}
template <int T>
static MfKernel mf_kernel_ragged(int xk, int kc) {
    if (kc == 4)
        return xk == XK_TAB ? k_gemv_mfma_r<T, 4, XK_TAB> : xk == XK_POST ? k_gemv_mfma_r<T, 4, XK_POST> : k_gemv_mfma_r<T, 4, XK_ANY>;
    if (kc == 8)
        return xk == XK_TAB ? k_gemv_mfma_r<T, 8, XK_TAB> : xk == XK_POST ? k_gemv_mfma_r<T, 8, XK_POST> : k_gemv_mfma_r<T, 8, XK_ANY>;
    return nullptr;
}
template <bool IL>
static MfKernel mf_kernel_layout(const GemvArgs& a, int kc) {
    const bool tab = a.xin == XIN_TAB;
    if constexpr (IL) {
        if (mf_ragged(a.G / 8)) {
            // the post-norm's two threads per group: 2 G <= the workgroup's threads
            const int xk = tab ? XK_TAB : (a.xin == XIN_POST && 2 * a.G <= 64 * a.nw) ? XK_POST : XK_ANY;
            switch (a.seg[0].type) {
                case FLLM_TYPE_Q4_K: return mf_kernel_ragged<FLLM_TYPE_Q4_K>(xk, kc);
                case FLLM_TYPE_Q6_K: return mf_kernel_ragged<FLLM_TYPE_Q6_K>(xk, kc);
                case FLLM_TYPE_Q8_0: return mf_kernel_ragged<FLLM_TYPE_Q8_0>(xk, kc);
                default: return mf_kernel_ragged<FLLM_TYPE_Q5_K>(xk, kc);
            }
        }
    }
    if (a.mix_wg > 0) return tab ? mf_kernel_mix<true, IL>(kc) : mf_kernel_mix<false, IL>(kc);
    const int xk = tab ? XK_TAB : a.xin == XIN_F32 ? XK_F32 : XK_ANY;
    if constexpr (IL) {
        if (a.seg[0].type == FLLM_TYPE_Q8_0) return mf_kernel_in<FLLM_TYPE_Q8_0, true>(xk, kc);
        if (a.seg[0].type == FLLM_TYPE_Q5_K) return mf_kernel_in<FLLM_TYPE_Q5_K, true>(xk, kc);
    }
    if (a.seg[0].type == FLLM_TYPE_Q6_K) return mf_kernel_in<FLLM_TYPE_Q6_K, IL>(xk, kc);
    return mf_kernel_in<FLLM_TYPE_Q4_K, IL>(xk, kc);
}
// the kernel of a planned launch (a.mix_wg > 0: two weight types)
static MfKernel mf_kernel(const GemvArgs& a, int kc) {
    return a.seg[0].layout == LAYOUT_TILES ? mf_kernel_layout<true>(a, kc) : mf_kernel_layout<false>(a, kc);
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

// The matrix-core variant takes launches whose rows are whole 256-element chunks, with one
// MFMA-capable weight type for all segments, and a wave count that divides the chunks per row.

static bool mfma_ok(const GemvArgs& a, int64_t cols) {
    const int NB = (int)(cols / 256);
    if (cols % 256 != 0 || mf_waves(NB) == 0) return false;
    // ragged rows: tile-interleaved matrices of one type
    for (int i = 0; i < a.nseg; i++) {
        if (mf_ragged(NB) && (a.seg[i].layout != LAYOUT_TILES || a.seg[i].type != a.seg[0].type)) return false;
        const int t = a.seg[i].type;
        if (mf_chunk_bytes(t) == 0) return false;
        // byte offsets within a matrix are 32-bit
        if ((uint64_t)a.seg[i].rows * (uint64_t)NB * (uint64_t)mf_chunk_bytes(t) >= (1ull << 32)) return false;
        // one layout per launch; tiles hold whole 16-row tiles
        if (a.seg[i].layout != a.seg[0].layout) return false;
        if (a.seg[i].layout == LAYOUT_TILES) {
            if (a.seg[i].rows % MF_TILE != 0 || ((uintptr_t)a.seg[i].w & 15) != 0) return false;
            if (t != a.seg[0].type && (a.glu || t != FLLM_TYPE_Q6_K || a.seg[0].type != FLLM_TYPE_Q4_K)) return false;
            if (i > 0 && t == FLLM_TYPE_Q4_K && a.seg[i - 1].type != FLLM_TYPE_Q4_K) return false;
            continue;
        }
        if (t == FLLM_TYPE_Q8_0 || t == FLLM_TYPE_Q5_K) return false;  // read tile-interleaved only
        // one type, or Q4_K segments followed by Q6_K ones (the two-type kernel; not for GLU)
        if (t != a.seg[0].type && (a.glu || t != FLLM_TYPE_Q6_K || a.seg[0].type != FLLM_TYPE_Q4_K)) return false;
        if (i > 0 && t == FLLM_TYPE_Q4_K && a.seg[i - 1].type != FLLM_TYPE_Q4_K) return false;
        // Q4_K rows are read as aligned 16-byte pieces; Q6_K as dword-aligned windows whose 0-or-2
        // byte phase follows the chunk index (an even number of chunks per row)
        const uintptr_t w = (uintptr_t)a.seg[i].w;
        if (t == FLLM_TYPE_Q4_K && (w & 15) != 0) return false;
        if (t == FLLM_TYPE_Q6_K && ((w & 3) != 0 || NB % 2 != 0)) return false;
    }
    return true;
}

static size_t mf_lds_split(int nw, int kc, bool glu) {
    const int T = (glu ? 2 : 1) * MF_TILE;
    // row partials, 48 floats, zero block, table (nw * kc chunk slots), and one wave's worth of
    // padding after the table
    return sizeof(float) * ((size_t)nw * T + 48) + (size_t)(MF_ZERO_ENTRIES(kc) + (size_t)nw * kc * MF_TAB_ENTRIES + 64) * 16;
}
static size_t mf_lds(int NB, bool glu) {
    int kc;
    const int nw = mf_split(NB, &kc);
    return mf_lds_split(nw, kc, glu);
}

bool gemv_uses_mfma(const GemvArgs& a, int64_t cols) {
    return mfma_ok(a, cols) && mf_lds((int)(cols / 256), a.glu != 0) <= 160 * 1024;
}

size_t gemv_tab_bytes(int64_t cols) { return (size_t)(cols / 256) * MF_TAB_ENTRIES * 16; }

static int plan_mfma(GemvArgs& a, int64_t cols, int n_cu, int* block_threads, size_t* lds_bytes) {
    a.mfma = 1;
    a.G = (int)(cols / 32);
    a.S = 0;
    a.rpw = MF_TILE;
    const int NB = (int)(cols / 256);
    int kc;
    const int nw = mf_split(NB, &kc);
    int units = 0;
    for (int i = 0; i < a.nseg; i++) {
        a.seg[i].wg_begin = units;  // first unit of the segment
        if (a.glu && i > 0) { a.seg[i].wg_begin = 1 << 30; continue; }
        units += (a.seg[i].rows + MF_TILE - 1) / MF_TILE;
    }
    a.nunits = units;
    a.chunks_per_wave = kc;
    // two weight types: units of the Q6_K segments come after the Q4_K ones
    a.mix_wg = 0;
    a.mix_unit = units;
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].type != a.seg[0].type) { a.mix_unit = a.seg[i].wg_begin; a.mix_wg = 1; break; }
    *block_threads = 64 * nw;
    a.nw = nw;
    *lds_bytes = mf_lds_split(nw, kc, a.glu != 0);
    // persistent grid: as many workgroups as fit on the device at once
    MfKernel k = mf_kernel(a, kc);
    (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k, *block_threads, *lds_bytes) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    int grid = n_cu * per_cu;
    if (grid > units) grid = units;
    if (a.mix_wg > 0) {
        // workgroups for each type in proportion to its units, at least one each
        if (grid < 2) grid = 2;
        int ga = (int)(((int64_t)grid * a.mix_unit + units / 2) / units);
        if (ga < 1) ga = 1;
        if (ga > grid - 1) ga = grid - 1;
        if (ga > a.mix_unit) ga = a.mix_unit;
        if (grid - ga > units - a.mix_unit) grid = ga + (units - a.mix_unit);
        a.mix_wg = ga;
    }
    return grid;
}

// Fill G, S, rpw and the segments' workgroup ranges; rows_per_wg 0 = choose.
int gemv_plan(GemvArgs& a, int64_t cols, int n_cu, int rows_per_wg, int* block_threads, size_t* lds_bytes) {
    a.mfma = 0;
    if (rows_per_wg <= 0 && gemv_uses_mfma(a, cols)) return plan_mfma(a, cols, n_cu, block_threads, lds_bytes);
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

bool gemv_tiles_shape_ok(int type, int64_t rows, int64_t cols) {
    if (mf_chunk_bytes(type) == 0 || rows <= 0 || rows % MF_TILE != 0 || rows > (1 << 30) || cols % 256 != 0) return false;
    const int NB = (int)(cols / 256);
    if (mf_waves(NB) == 0 || mf_lds(NB, true) > 160 * 1024) return false;
    return (uint64_t)rows * (uint64_t)NB * (uint64_t)mf_chunk_bytes(type) < (1ull << 32);
}

// LAYOUT_TILES of a Q4_K, Q6_K or Q8_0 matrix (rows a multiple of 16, NB chunks of 256 elements per
// row): the blocks of tile t (rows 16t .. 16t + 15) in chunk column kb fill region t * NB + kb of 16
// chunk sizes, laid out so that matrix-core lane L = 16 q + n (tile row n, quarter q) finds its part
// of row n as 16-byte pieces at 16 L of 1 KiB slices, and the fields a row's four lanes share at n:
//   Q4_K, 2304 B: [0, 1024) qs bytes 16q .. 16q + 15; [1024, 2048) qs bytes 64 + 16q .. ;
//                 [2048, 2304) block bytes 0 .. 15 (d, dmin, scales) at 16 n
//   Q6_K, 3360 B: [0, 1024) ql 16q .. ; [1024, 2048) ql 64 + 16q .. ; [2048, 3072) qh 8q .. 8q + 7
//                 then qh 32 + 8q .. ; [3072, 3328) scales 2q, 2q + 1, 8 + 2q, 9 + 2q at 4 L;
//                 [3328, 3360) d at 2 n
//   Q8_0, 4352 B: [0, 1024) int8 0 .. 15 of block q; [1024, 2048) its 16 .. 31; [2048, 4096) the same
//                 for block q + 4; each 16-byte piece in element order 4 by + j at byte 4 j + by (the
//                 activation table's); [4096, 4352) d of blocks q and q + 4 as one dword at 16 n + 4 q
//   Q5_K, 2816 B: [0, 1024) qs bytes 16q .. ; [1024, 2048) qs bytes 64 + 16q .. ; [2048, 2560) the high
//                 bits of groups q and q + 4 (qh bits 32 g .. 32 g + 31) as two dwords at 8 L, each with
//                 the bit of element 16 h + 4 by + j at bit 8 by + 4 h + j; [2560, 2816) block bytes
//                 0 .. 15 at 16 n
// Every block byte (for Q5_K's high bits: every bit) has exactly one place, so the regrouped matrix
// dequantizes to the same values.
// One thread per (row, chunk).
__global__ void k_pack_tiles(int type, const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int rows, int NB) {
    const int64_t nchunk = (int64_t)rows * NB;
    const int cb = mf_chunk_bytes(type);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nchunk; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / NB;
        const int kb = (int)(i % NB), n = (int)(r & 15);
        const uint8_t* b = src + i * cb;  // the row's chunk kb: one K-quant block, or 8 Q8_0 blocks
        uint8_t* reg = dst + ((r >> 4) * NB + kb) * 16 * cb;
        if (type == FLLM_TYPE_Q5_K) {
            for (int g = 0; g < 8; g++) {
                const int q = g & 3, L = 16 * q + n;
                for (int j = 0; j < 16; j++) reg[(g < 4 ? 0 : 1024) + 16 * L + j] = b[48 + 16 * g + j];
                const uint32_t hs = (uint32_t)b[16 + 4 * g] | ((uint32_t)b[17 + 4 * g] << 8) |
                                    ((uint32_t)b[18 + 4 * g] << 16) | ((uint32_t)b[19 + 4 * g] << 24);
                uint32_t hr = 0u;
                for (int e = 0; e < 32; e++) {
                    const int h = e >> 4, by = (e >> 2) & 3, j = e & 3;
                    hr |= ((hs >> e) & 1u) << (8 * by + 4 * h + j);
                }
                uint8_t* hp = reg + 2048 + 8 * L + (g < 4 ? 0 : 4);
                hp[0] = (uint8_t)hr; hp[1] = (uint8_t)(hr >> 8); hp[2] = (uint8_t)(hr >> 16); hp[3] = (uint8_t)(hr >> 24);
            }
            for (int j = 0; j < 16; j++) reg[2560 + 16 * n + j] = b[j];
            continue;
        }
        if (type == FLLM_TYPE_Q8_0) {
            for (int g = 0; g < 8; g++) {
                const uint8_t* blk = b + 34 * g;
                const int q = g & 3, L = 16 * q + n, base = (g < 4 ? 0 : 2048) + 16 * L;
                for (int e = 0; e < 32; e++) {
                    const int h = e >> 4, ee = e & 15;
                    reg[base + 1024 * h + 4 * (ee & 3) + (ee >> 2)] = blk[2 + e];
                }
                reg[4096 + 16 * n + 4 * q + (g < 4 ? 0 : 2)] = blk[0];
                reg[4096 + 16 * n + 4 * q + (g < 4 ? 0 : 2) + 1] = blk[1];
            }
            continue;
        }
        for (int q = 0; q < 4; q++) {
            const int L = 16 * q + n;
            if (type == FLLM_TYPE_Q6_K) {
                for (int j = 0; j < 16; j++) reg[16 * L + j] = b[16 * q + j];
                for (int j = 0; j < 16; j++) reg[1024 + 16 * L + j] = b[64 + 16 * q + j];
                for (int j = 0; j < 8; j++) reg[2048 + 16 * L + j] = b[128 + 8 * q + j];
                for (int j = 0; j < 8; j++) reg[2048 + 16 * L + 8 + j] = b[160 + 8 * q + j];
                reg[3072 + 4 * L] = b[192 + 2 * q];
                reg[3072 + 4 * L + 1] = b[193 + 2 * q];
                reg[3072 + 4 * L + 2] = b[200 + 2 * q];
                reg[3072 + 4 * L + 3] = b[201 + 2 * q];
            } else {
                // Q4_K: each 8-byte half of a group's qs stored as its bytes 0, 2, 4, 6, 1, 3, 5, 7
                for (int j = 0; j < 16; j++) reg[16 * L + j] = b[16 + 16 * q + q4t_src_byte(j)];
                for (int j = 0; j < 16; j++) reg[1024 + 16 * L + j] = b[80 + 16 * q + q4t_src_byte(j)];
            }
        }
        if (type == FLLM_TYPE_Q6_K) {
            reg[3328 + 2 * n] = b[208];
            reg[3328 + 2 * n + 1] = b[209];
        } else {
            for (int j = 0; j < 16; j++) reg[2048 + 16 * n + j] = b[j];
        }
    }
}

hipError_t launch_pack_tiles(int type, const uint8_t* src, uint8_t* dst, int64_t rows, int64_t cols, hipStream_t st) {
    if (!gemv_tiles_shape_ok(type, rows, cols)) return hipErrorInvalidValue;
    const int64_t nblk = rows * (cols / 256);
    const int64_t grid = (nblk + 255) / 256 < 65536 ? (nblk + 255) / 256 : 65536;
    k_pack_tiles<<<(int)grid, 256, 0, st>>>(type, src, dst, (int)rows, (int)(cols / 256));
    return hipGetLastError();
}

hipError_t launch_gemv_fused(const GemvArgs& a, int grid, int block_threads, size_t lds, hipStream_t st) {
    if (grid <= 0) return hipSuccess;
    // the matrix-core prologue always reads its input: the table, or the vector (cols floats)
    if (a.mfma && (a.xin == XIN_TAB ? a.xtab == nullptr : a.x == nullptr)) return hipErrorInvalidValue;
    // LAYOUT_TILES matrices are read only by the matrix-core variant
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].layout == LAYOUT_TILES && !a.mfma) return hipErrorInvalidValue;
    if (a.xin == XIN_POST && (!a.mfma || a.x2 == nullptr || a.post_w == nullptr || a.x_out == nullptr || a.x_out == a.x))
        return hipErrorInvalidValue;
    if (a.mfma) {
        // the kernel's chunks per wave and wave count must be the plan's: a ragged row only as its
        // split, an even one covered exactly by at most 8 waves
        const int NB = a.G / 8, kc = a.chunks_per_wave;
        int kc_split;
        const int nw_split = mf_split(NB, &kc_split);
        const bool ragged = mf_ragged(NB);
        if (block_threads != 64 * a.nw || (kc != 1 && kc != 2 && kc != 4 && kc != 8) ||
            (ragged ? (kc != kc_split || a.nw != nw_split) : (a.nw < 1 || a.nw > 8 || a.nw * kc != NB)))
            return hipErrorInvalidValue;
        const MfKernel k = mf_kernel(a, kc);
        if (k == nullptr) return hipErrorInvalidValue;
        k<<<grid, block_threads, lds, st>>>(a);
    } else if (block_threads <= 512)
        k_gemv_fused<false><<<grid, block_threads, lds, st>>>(a);
    else
        k_gemv_fused<true><<<grid, block_threads, lds, st>>>(a);
    return hipGetLastError();
}

}  // namespace fllm
