/*
 * oracle.c — CPU restatement of DotNetFoundryLLM's decode path (test infrastructure only).
 *
 * Only tests/, the smoke check and bench.py's cpu_baseline leg use this file, as the
 * checker. It follows the reference's C# line by line; citations are relative to the
 * reference repository root. It is compiled with -ffp-contract=off so that a*b-c stays two
 * roundings, as the .NET JIT emits it (no FMA contraction).
 *
 * Parity status of each part (what pins it):
 *  - orc_half_to_float / orc_bf16_to_float / orc_dequantize: pinned by the reference's
 *    known-answer tests (DequantizerTests.cs), exhaustive 16-bit tables against numpy's
 *    IEEE conversions, and brute-force checks of the K-quant scale unpacking.
 *  - orc_dot / orc_linear: pinned against float64 brute force within float32 rounding
 *    bounds; the exact summation order of System.Numerics.Tensors 10.0.7's Dot is not
 *    vendored and stays unpinned at the bit level (tolerance-pinned only).
 *  - norms, activations, softcap, softmax, RoPE: closed forms checked in tests; bit-level
 *    parity with TensorPrimitives' vectorised Exp/Tanh/Sigmoid is unpinned.
 *  - argmax / top-k: integer-exact; pinned by the reference's sampler tests.
 *  - xoshiro256** (orc_xoshiro_*): integer-exact; pinned by published known answers that no
 *    code here computes: SplitMix64 from seeds 1234567 (Rosetta Code) and 0 (Vigna's
 *    splitmix64.c outputs) as the seeded state, and the xoshiro256** vector from the state
 *    {1, 2, 3, 4} (rand_xoshiro's reference test; its first three values follow by hand);
 *    NextFloat by its closed form on those outputs (tests/test_oracle_ops.py).
 *  - top-p (orc_apply_top_p): pinned by TopPSamplerTests.cs's cases and by the nucleus
 *    invariants (kept mass reaches p, dropping the smallest kept entry falls below it, every
 *    kept probability is at least every dropped one); the order among equal probabilities at
 *    the edge follows a stable sort, where the reference's Array.Sort is unstable (unpinned).
 *  - repetition penalty (orc_repetition_penalty): IEEE division / multiplication per listed
 *    id, pinned by RepetitionPenaltySamplerTests.cs's cases and closed forms (k repeats of a
 *    positive logit divide it k times).
 *  - forward pass: invariants (context of one => attention returns v0, GQA mapping,
 *    window start) and the reference's deterministic 2-layer fixtures.
 *  - row-parallel mode (orc_set_threads): pinned by bit-equality with one thread on every
 *    function it splits (tests/test_oracle_forward.py).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_E_RANGE (-1)
#define ORC_E_ARG (-2)
#define ORC_E_INVALID (-3)
#define ORC_E_NOTSUP (-4)

/* ---------------------------------------------------------------------------------
 * Row-parallel mode (orc_set_threads). The reference is single-threaded; splitting the rows
 * of a projection, the heads of an attention or the blocks of a dequantization over threads
 * leaves every output element computed by the same function on the same operands in the same
 * order, so results are bit-identical to one thread. It only makes the full-size models
 * tractable as a checker.
 * ------------------------------------------------------------------------------- */
#define ORC_MAX_THREADS 64
typedef void (*orc_task)(void* arg, int64_t begin, int64_t end);

static struct {
    int n;                         /* threads including the caller */
    pthread_t th[ORC_MAX_THREADS];
    pthread_mutex_t mu;
    pthread_cond_t go, done;
    unsigned long gen;
    int pending, quit;
    orc_task fn;
    void* arg;
    int64_t total;
} pool = {1, {0}, PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER, PTHREAD_COND_INITIALIZER, 0, 0, 0, 0, 0, 0};

static void pool_slice(int i, int n, int64_t total, int64_t* b, int64_t* e) {
    *b = total * i / n;
    *e = total * (i + 1) / n;
}

static void* pool_worker(void* p) {
    int id = (int)(intptr_t)p;
    unsigned long seen = 0;
    for (;;) {
        pthread_mutex_lock(&pool.mu);
        while (pool.gen == seen && !pool.quit) pthread_cond_wait(&pool.go, &pool.mu);
        if (pool.quit) { pthread_mutex_unlock(&pool.mu); return NULL; }
        seen = pool.gen;
        orc_task fn = pool.fn;
        void* arg = pool.arg;
        int64_t total = pool.total, b, e;
        int n = pool.n;
        pthread_mutex_unlock(&pool.mu);
        pool_slice(id, n, total, &b, &e);
        if (b < e) fn(arg, b, e);
        pthread_mutex_lock(&pool.mu);
        if (--pool.pending == 0) pthread_cond_signal(&pool.done);
        pthread_mutex_unlock(&pool.mu);
    }
}

/* Runs fn over [0, total) split into pool.n contiguous ranges, the caller taking the first. */
static void pool_run(orc_task fn, void* arg, int64_t total) {
    int n = pool.n;
    if (n <= 1 || total < 2) { if (total > 0) fn(arg, 0, total); return; }
    pthread_mutex_lock(&pool.mu);
    pool.fn = fn;
    pool.arg = arg;
    pool.total = total;
    pool.pending = n - 1;
    pool.gen++;
    pthread_cond_broadcast(&pool.go);
    pthread_mutex_unlock(&pool.mu);
    int64_t b, e;
    pool_slice(0, n, total, &b, &e);
    if (b < e) fn(arg, b, e);
    pthread_mutex_lock(&pool.mu);
    while (pool.pending > 0) pthread_cond_wait(&pool.done, &pool.mu);
    pthread_mutex_unlock(&pool.mu);
}

int orc_set_threads(int n) {
    if (n < 1) n = 1;
    if (n > ORC_MAX_THREADS) n = ORC_MAX_THREADS;
    if (n == pool.n) return n;
    if (pool.n > 1) {
        pthread_mutex_lock(&pool.mu);
        pool.quit = 1;
        pthread_cond_broadcast(&pool.go);
        pthread_mutex_unlock(&pool.mu);
        for (int i = 1; i < pool.n; i++) pthread_join(pool.th[i], NULL);
    }
    pool.quit = 0;
    pool.gen = 0;
    pool.n = 1;
    for (int i = 1; i < n; i++) {
        if (pthread_create(&pool.th[i], NULL, pool_worker, (void*)(intptr_t)i) != 0) break;
        pool.n = i + 1;
    }
    return pool.n;
}

int orc_get_threads(void) { return pool.n; }

/* ---------------------------------------------------------------------------------
 * Scalar conversions. Dequantizer.HalfToFloat (Dequantizer.cs:49-51) is the exact
 * IEEE binary16 -> binary32 widening; BFloat16ToFloat (Dequantizer.cs:57-59) is bits<<16.
 * ------------------------------------------------------------------------------- */
static float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    if (exp == 0) {
        if (man == 0) return bits_to_float(sign);
        /* subnormal: value = man * 2^-24, exactly representable in binary32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return bits_to_float(sign | 0x7F800000u | (man << 13));
    return bits_to_float(sign | ((exp + 112) << 23) | (man << 13));
}

float orc_bf16_to_float(uint16_t b) { return bits_to_float((uint32_t)b << 16); }

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Dequantizer.DecodeKScaleMin (Dequantizer.cs:506-521). */
void orc_decode_kscale_min(const uint8_t* packed, int g, int* scale, int* min) {
    if (g < 4) {
        *scale = packed[g] & 0x3F;
        *min = packed[g + 4] & 0x3F;
        return;
    }
    int i = g - 4;
    *scale = (packed[g + 4] & 0x0F) | ((packed[i] >> 6) << 4);
    *min = (packed[g + 4] >> 4) | ((packed[i + 4] >> 6) << 4);
}

/* Dequantizer.ElementCount (Dequantizer.cs:466-479). */
int orc_element_count(int type, int64_t nbytes, int64_t* out) {
    switch (type) {
        case 0: *out = nbytes / 4; return ORC_OK;
        case 1: *out = nbytes / 2; return ORC_OK;
        case 2: *out = nbytes / 18 * 32; return ORC_OK;
        case 8: *out = nbytes / 34 * 32; return ORC_OK;
        case 12: *out = nbytes / 144 * 256; return ORC_OK;
        case 13: *out = nbytes / 176 * 256; return ORC_OK;
        case 14: *out = nbytes / 210 * 256; return ORC_OK;
        case 15: *out = nbytes / 292 * 256; return ORC_OK;
        case 30: *out = nbytes / 2; return ORC_OK;
        default: return ORC_E_NOTSUP;
    }
}

static int block_geometry(int type, int64_t* bb, int64_t* be) {
    switch (type) {
        case 0: *bb = 4; *be = 1; return ORC_OK;
        case 1: case 30: *bb = 2; *be = 1; return ORC_OK;
        case 2: *bb = 18; *be = 32; return ORC_OK;
        case 8: *bb = 34; *be = 32; return ORC_OK;
        case 12: *bb = 144; *be = 256; return ORC_OK;
        case 13: *bb = 176; *be = 256; return ORC_OK;
        case 14: *bb = 210; *be = 256; return ORC_OK;
        case 15: *bb = 292; *be = 256; return ORC_OK;
        default: return ORC_E_NOTSUP;
    }
}

/* The per-type routines of Dequantizer.cs over blocks [b0, b1). */
static void dequant_blocks(int type, const uint8_t* src, float* dst, int64_t b0, int64_t b1) {
    int64_t bb = 1, be = 1;
    block_geometry(type, &bb, &be);
    for (int64_t b = b0; b < b1; b++) {
        const uint8_t* blk = src + b * bb;
        float* o = dst + b * be;
        switch (type) {
            case 0: /* DequantizeF32 (Dequantizer.cs:68-85) */
                o[0] = bits_to_float(rd32(blk));
                break;
            case 1: /* DequantizeF16 (Dequantizer.cs:94-111) */
                o[0] = orc_half_to_float(rd16(blk));
                break;
            case 30: /* DequantizeBF16 (Dequantizer.cs:120-137) */
                o[0] = orc_bf16_to_float(rd16(blk));
                break;
            case 2: { /* DequantizeQ4_0 (Dequantizer.cs:155-185) */
                float d = orc_half_to_float(rd16(blk));
                for (int j = 0; j < 16; j++) {
                    uint8_t qs = blk[2 + j];
                    o[j] = (float)((qs & 0x0F) - 8) * d;
                    o[j + 16] = (float)((qs >> 4) - 8) * d;
                }
                break;
            }
            case 8: { /* DequantizeQ8_0 (Dequantizer.cs:203-231) */
                float d = orc_half_to_float(rd16(blk));
                for (int j = 0; j < 32; j++) o[j] = (float)(int8_t)blk[2 + j] * d;
                break;
            }
            case 12: { /* DequantizeQ4_K (Dequantizer.cs:251-294) */
                float d = orc_half_to_float(rd16(blk));
                float dmin = orc_half_to_float(rd16(blk + 2));
                const uint8_t* scales = blk + 4;
                const uint8_t* qs = blk + 16;
                for (int g = 0; g < 8; g++) {
                    int sc, mn;
                    orc_decode_kscale_min(scales, g, &sc, &mn);
                    float dg = d * (float)sc;
                    float mg = dmin * (float)mn;
                    for (int i = 0; i < 32; i++) {
                        uint8_t packed = qs[g * 16 + (i >> 1)];
                        int q = (i & 1) == 0 ? (packed & 0x0F) : (packed >> 4);
                        o[g * 32 + i] = dg * (float)q - mg;
                    }
                }
                break;
            }
            case 13: { /* DequantizeQ5_K (Dequantizer.cs:316-368) */
                float d = orc_half_to_float(rd16(blk));
                float dmin = orc_half_to_float(rd16(blk + 2));
                const uint8_t* scales = blk + 4;
                const uint8_t* qh = blk + 16;
                const uint8_t* qs = blk + 48;
                for (int g = 0; g < 8; g++) {
                    int sc, mn;
                    orc_decode_kscale_min(scales, g, &sc, &mn);
                    float dg = d * (float)sc;
                    float mg = dmin * (float)mn;
                    for (int i = 0; i < 32; i++) {
                        int t = g * 32 + i;
                        uint8_t pl = qs[t >> 1];
                        int lo = (t & 1) == 0 ? (pl & 0x0F) : (pl >> 4);
                        int hi = (qh[t >> 3] >> (t & 7)) & 1;
                        int q = (hi << 4) | lo;
                        o[g * 32 + i] = dg * (float)q - mg;
                    }
                }
                break;
            }
            case 14: { /* DequantizeQ6_K (Dequantizer.cs:378-417) */
                const uint8_t* ql = blk;
                const uint8_t* qh = blk + 128;
                const uint8_t* scales = blk + 192;
                float d = orc_half_to_float(rd16(blk + 208));
                for (int i = 0; i < 256; i++) {
                    uint8_t qlb = ql[i >> 1];
                    int low = (i & 1) == 0 ? (qlb & 0x0F) : (qlb >> 4);
                    int high = (qh[i >> 2] >> ((i & 3) * 2)) & 3;
                    int q = ((high << 4) | low) - 32;
                    int scale = (int8_t)scales[i >> 4];
                    o[i] = d * (float)scale * (float)q;
                }
                break;
            }
            case 15: { /* DequantizeQ8_K (Dequantizer.cs:427-456) */
                float d = bits_to_float(rd32(blk));
                for (int i = 0; i < 256; i++) o[i] = (float)(int8_t)blk[4 + i] * d;
                break;
            }
        }
    }
}

typedef struct { int type; const uint8_t* src; float* dst; } dequant_job;
static void dequant_task(void* a, int64_t b0, int64_t b1) {
    dequant_job* j = (dequant_job*)a;
    dequant_blocks(j->type, j->src, j->dst, b0, b1);
}

/* Dequantizer.Dequantize dispatch (Dequantizer.cs:488-504) and the per-type routines. */
int orc_dequantize(int type, const uint8_t* src, int64_t nbytes, float* dst, int64_t n) {
    int64_t bb, be;
    if (block_geometry(type, &bb, &be) != ORC_OK) return ORC_E_NOTSUP;
    if (nbytes % bb != 0) return ORC_E_ARG;           /* "Source length must be a multiple" */
    int64_t nblk = nbytes / bb;
    if (n < nblk * be) return ORC_E_ARG;              /* "Destination must hold at least" */
    dequant_job j = {type, src, dst};
    if (nblk >= 4096) pool_run(dequant_task, &j, nblk);
    else dequant_blocks(type, src, dst, 0, nblk);
    return ORC_OK;
}

/* ---------------------------------------------------------------------------------
 * TensorOperations (src/DotNetFoundryLLM.Tensors/TensorOperations.cs).
 * ------------------------------------------------------------------------------- */

/* TensorOperations.Dot -> TensorPrimitives.Dot (TensorOperations.cs:170-171): a float32
 * dot product. Eight partial sums stand in for the library's SIMD lanes. */
float orc_dot(const float* a, const float* b, int64_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) acc[j] += a[i + j] * b[i + j];
    float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    for (; i < n; i++) s += a[i] * b[i];
    return s;
}

typedef struct { const float* x; const float* W; float* y; int64_t cols; } linear_job;
static void linear_task(void* a, int64_t r0, int64_t r1) {
    linear_job* j = (linear_job*)a;
    for (int64_t i = r0; i < r1; i++) j->y[i] = orc_dot(j->x, j->W + (size_t)i * (size_t)j->cols, j->cols);
}

/* LinearProjection (LlamaForwardPass.cs:237-260): y[i] = Dot(x, W[i*cols .. +cols]).
 * Rows are split over the row-parallel threads; each row is the same orc_dot call. */
void orc_linear(const float* x, const float* W, float* y, int64_t rows, int64_t cols) {
    linear_job j = {x, W, y, cols};
    if (rows * cols >= (1 << 16)) pool_run(linear_task, &j, rows);
    else linear_task(&j, 0, rows);
}

/* RmsNorm (TensorOperations.cs:42-54). */
int orc_rmsnorm(const float* x, const float* w, float* dst, int64_t n, float eps) {
    float sumsq = orc_dot(x, x, n);
    float rms = 1.0f / sqrtf(sumsq / (float)n + eps);
    for (int64_t i = 0; i < n; i++) dst[i] = x[i] * rms;
    for (int64_t i = 0; i < n; i++) dst[i] = dst[i] * w[i];
    return ORC_OK;
}

/* GemmaRmsNorm (TensorOperations.cs:90-107): eps fixed at 1e-6, scale (1 + w).
 * x and dst may alias (Gemma2ForwardPass.cs:90,95 pass the same span). */
void orc_gemma_rmsnorm(const float* x, const float* w, float* dst, int64_t n) {
    float sumsq = orc_dot(x, x, n);
    float rms = 1.0f / sqrtf(sumsq / (float)n + 1e-6f);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t i = 0; i < n; i++) tmp[i] = x[i] * rms;
    for (int64_t i = 0; i < n; i++) dst[i] = w[i] + 1.0f;
    for (int64_t i = 0; i < n; i++) dst[i] = tmp[i] * dst[i];
    free(tmp);
}

/* Silu (TensorOperations.cs:57-87): x * Sigmoid(x), Sigmoid = 1/(1+e^-x). */
void orc_silu(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float sig = 1.0f / (1.0f + expf(-x[i]));
        x[i] = x[i] * sig;
    }
}

/* Gelu, tanh form (TensorOperations.cs:110-117), same operation order. */
void orc_gelu(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
        x[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* SoftCap (TensorOperations.cs:120-126): cap * tanh(x * (1/cap)). */
void orc_softcap(float* x, int64_t n, float cap) {
    float inv = 1.0f / cap;
    for (int64_t i = 0; i < n; i++) x[i] = x[i] * inv;
    for (int64_t i = 0; i < n; i++) x[i] = tanhf(x[i]);
    for (int64_t i = 0; i < n; i++) x[i] = x[i] * cap;
}

/* Softmax (TensorOperations.cs:23-39): max, subtract, exp, sum, divide if sum != 0. */
void orc_softmax(float* x, int64_t n) {
    if (n <= 0) return;
    float mx = x[0];
    for (int64_t i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    for (int64_t i = 0; i < n; i++) x[i] = x[i] + (-mx);
    for (int64_t i = 0; i < n; i++) x[i] = expf(x[i]);
    float fs = 0.0f; /* summation order of TensorPrimitives.Sum is unpinned */
    for (int64_t i = 0; i < n; i++) fs += x[i];
    if (fs != 0.0f)
        for (int64_t i = 0; i < n; i++) x[i] = x[i] / fs;
}

/* RoPE inverse frequencies (LlamaForwardPass.cs:64-70): 1f / Pow(base, 2f*i/headDim). */
void orc_rope_inv_freqs(float base, int head_dim, float* inv) {
    for (int i = 0; i < head_dim / 2; i++) {
        float e = (2.0f * (float)i) / (float)head_dim;
        inv[i] = 1.0f / powf(base, e);
    }
}

/* ApplyRope(Span, float position, freqs) (TensorOperations.cs:250-260): interleaved pairs. */
void orc_apply_rope(float* x, float pos, const float* inv, int half) {
    for (int i = 0; i < half; i++) {
        float theta = pos * inv[i];
        float c = cosf(theta), s = sinf(theta);
        float x0 = x[2 * i], x1 = x[2 * i + 1];
        x[2 * i] = x0 * c - x1 * s;
        x[2 * i + 1] = x0 * s + x1 * c;
    }
}

/* ArgMax -> TensorPrimitives.IndexOfMax (TensorOperations.cs:187-195): index of the first
 * maximum; a NaN wins at its first occurrence; +0 is greater than -0. */
int64_t orc_argmax(const float* x, int64_t n) {
    if (n <= 0) return -1;
    int64_t best = 0;
    if (isnan(x[0])) return 0;
    for (int64_t i = 1; i < n; i++) {
        float v = x[i], b = x[best];
        if (isnan(v)) return i;
        if (v > b || (v == b && v == 0.0f && !signbit(v) && signbit(b))) best = i;
    }
    return best;
}

/* ---------------------------------------------------------------------------------
 * XoshiroRandom (src/DotNetFoundryLLM.Core/XoshiroRandom.cs:4-49): SplitMix64 seeding,
 * xoshiro256** step, NextFloat = (float)((x >> 11) * 2^-53).
 * ------------------------------------------------------------------------------- */
static uint64_t splitmix64(uint64_t* x) {
    *x += 0x9e3779b97f4a7c15ULL;
    uint64_t z = *x;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void orc_xoshiro_init(orc_xoshiro* r, uint64_t seed) {
    r->s0 = splitmix64(&seed);
    r->s1 = splitmix64(&seed);
    r->s2 = splitmix64(&seed);
    r->s3 = splitmix64(&seed);
}
uint64_t orc_xoshiro_next(orc_xoshiro* r) {
    uint64_t result = rotl64(r->s1 * 5, 7) * 9;
    uint64_t t = r->s1 << 17;
    r->s2 ^= r->s0;
    r->s3 ^= r->s1;
    r->s1 ^= r->s2;
    r->s0 ^= r->s3;
    r->s2 ^= t;
    r->s3 = rotl64(r->s3, 45);
    return result;
}
float orc_xoshiro_next_float(orc_xoshiro* r) {
    return (float)((double)(orc_xoshiro_next(r) >> 11) * (1.0 / 9007199254740992.0));
}

/* TopKSampler.PartialSortDescending / Partition (TopKSampler.cs:78-115), mirrored so the
 * threshold is the same element the reference picks. */
static int64_t topk_partition(float* s, int64_t left, int64_t right) {
    int64_t mid = left + (right - left) / 2;
    float t;
    if (s[left] < s[mid]) { t = s[left]; s[left] = s[mid]; s[mid] = t; }
    if (s[left] < s[right]) { t = s[left]; s[left] = s[right]; s[right] = t; }
    if (s[mid] < s[right]) { t = s[mid]; s[mid] = s[right]; s[right] = t; }
    float pivot = s[left];
    int64_t i = left + 1;
    for (int64_t j = left + 1; j <= right; j++) {
        if (s[j] > pivot) { t = s[i]; s[i] = s[j]; s[j] = t; i++; }
    }
    t = s[left]; s[left] = s[i - 1]; s[i - 1] = t;
    return i - 1;
}

float orc_topk_threshold(const float* logits, int64_t n, int k) {
    float* s = (float*)malloc(sizeof(float) * (size_t)n);
    memcpy(s, logits, sizeof(float) * (size_t)n);
    int64_t left = 0, right = n - 1, target = k - 1;
    while (left < right) {
        int64_t p = topk_partition(s, left, right);
        if (p == target) break;
        if (p < target) left = p + 1; else right = p - 1;
    }
    float th = s[k - 1];
    free(s);
    return th;
}

/* TopKSampler.ApplyTopK (TopKSampler.cs:42-71): values below the k-th largest -> -inf. */
void orc_apply_topk(float* logits, int64_t n, int k) {
    if (k >= n) return;
    float th = orc_topk_threshold(logits, n, k);
    for (int64_t i = 0; i < n; i++)
        if (logits[i] < th) logits[i] = -INFINITY;
}

/* TemperatureSampler.SampleFromProbabilities (TemperatureSampler.cs:53-70). */
int64_t orc_sample_from_probs(const float* probs, int64_t n, orc_xoshiro* r) {
    float u = orc_xoshiro_next_float(r);
    float cum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        cum += probs[i];
        if (u < cum) return i;
    }
    for (int64_t i = n - 1; i >= 0; i--)
        if (probs[i] > 0.0f) return i;
    return n - 1;
}

/* SamplerPipeline.Sample (SamplerPipeline.cs:58-89) with topP == 1. */
int64_t orc_sampler_pipeline(float* logits, int64_t n, float temperature, int top_k, orc_xoshiro* r) {
    return orc_sampler_pipeline_p(logits, n, temperature, top_k, 1.0f, r);
}

/* Descending probability, ties by ascending index: the order a stable sort gives. The reference
 * sorts with Array.Sort (introsort, unstable), so which of several equal probabilities at the
 * nucleus edge come first is not pinned; distinct values order the same either way. */
static const float* g_topp_probs;
static int cmp_desc_prob(const void* a, const void* b) {
    int64_t ia = *(const int64_t*)a, ib = *(const int64_t*)b;
    float pa = g_topp_probs[ia], pb = g_topp_probs[ib];
    if (pa > pb) return -1;
    if (pa < pb) return 1;
    return ia < ib ? -1 : (ia > ib ? 1 : 0);
}

/* TopPSampler.ApplyTopP (TopPSampler.cs:60-110): keep the smallest prefix of the descending order
 * whose running f32 sum reaches p, zero the rest, divide by the f32 sum of what is left. */
void orc_apply_top_p(float* probs, int64_t n, float p) {
    if (p >= 1.0f || n <= 0) return;
    int64_t* idx = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
    float* copy = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t i = 0; i < n; i++) { idx[i] = i; copy[i] = probs[i]; }
    g_topp_probs = copy;
    qsort(idx, (size_t)n, sizeof(int64_t), cmp_desc_prob);
    float cum = 0.0f;
    int reached = 0;
    for (int64_t r = 0; r < n; r++) {
        if (reached) probs[idx[r]] = 0.0f;
        else {
            cum += probs[idx[r]];
            if (cum >= p) reached = 1;
        }
    }
    float sum = 0.0f; /* TensorPrimitives.Sum order unpinned */
    for (int64_t i = 0; i < n; i++) sum += probs[i];
    if (sum > 0.0f)
        for (int64_t i = 0; i < n; i++) probs[i] = probs[i] / sum;
    free(idx);
    free(copy);
}

/* SamplerPipeline.Sample (SamplerPipeline.cs:58-89): temperature, top-k, softmax, top-p, draw. */
int64_t orc_sampler_pipeline_p(float* logits, int64_t n, float temperature, int top_k, float top_p, orc_xoshiro* r) {
    if (temperature == 0.0f) return orc_argmax(logits, n);
    if (temperature != 1.0f) {
        float inv = 1.0f / temperature;
        for (int64_t i = 0; i < n; i++) logits[i] = logits[i] * inv;
    }
    if (top_k > 0) orc_apply_topk(logits, n, top_k);
    orc_softmax(logits, n);
    if (top_p < 1.0f) orc_apply_top_p(logits, n, top_p);
    return orc_sample_from_probs(logits, n, r);
}

/* LlamaLanguageModel.ApplyRepetitionPenalty (LlamaLanguageModel.cs:357-373): for every id of the
 * generated list in order (repeats apply again), l > 0 ? l / penalty : l * penalty; ids outside
 * [0, n) are skipped. */
void orc_repetition_penalty(float* logits, int64_t n, const int32_t* ids, int64_t n_ids, float penalty) {
    for (int64_t j = 0; j < n_ids; j++) {
        int32_t id = ids[j];
        if ((uint32_t)id < (uint64_t)n) {
            if (logits[id] > 0.0f) logits[id] = logits[id] / penalty;
            else logits[id] = logits[id] * penalty;
        }
    }
}

/* ---------------------------------------------------------------------------------
 * Model weights (LlamaWeights / Qwen2Weights / Gemma2Weights) and the forward passes.
 * ------------------------------------------------------------------------------- */
enum { A_LLAMA = 0, A_MISTRAL = 1, A_QWEN2 = 2, A_GEMMA2 = 3 };
enum {
    S_TOKEN_EMBD = 0, S_OUTPUT_NORM = 1, S_OUTPUT = 2,
    S_ATTN_NORM = 10, S_Q = 11, S_K = 12, S_V = 13, S_O = 14, S_BQ = 15, S_BK = 16, S_BV = 17,
    S_POST_ATTN = 18, S_FFN_NORM = 19, S_GATE = 20, S_UP = 21, S_DOWN = 22, S_POST_FFN = 23
};
#define NSLOT_L 14

struct orc_model {
    orc_desc d;
    int qdim, kvdim;
    float* tok_embd;
    float* out_norm;
    float* output;
    int output_tied;
    float** layer[NSLOT_L]; /* indexed by slot - 10 */
    float* inv_freq;
};

struct orc_fwd {
    orc_model* m;
    int32_t max_seq, cur_len, next_layer;
    float **keys, **vals;
    float *x, *xn, *q, *k, *v, *att, *ffa, *ffb, *logits, *scores;
    float* hidden; /* (n_layers+1) * hidden */
    int lim_layers, lim_head;
};

static int64_t slot_elems(const orc_model* m, int slot) {
    const orc_desc* d = &m->d;
    int64_t h = d->hidden;
    switch (slot) {
        case S_TOKEN_EMBD: case S_OUTPUT: return (int64_t)d->vocab * h;
        case S_OUTPUT_NORM: case S_ATTN_NORM: case S_POST_ATTN: case S_FFN_NORM: case S_POST_FFN: return h;
        case S_Q: return (int64_t)m->qdim * h;
        case S_K: case S_V: return (int64_t)m->kvdim * h;
        case S_O: return h * m->qdim;
        case S_BQ: return m->qdim;
        case S_BK: case S_BV: return m->kvdim;
        case S_GATE: case S_UP: return (int64_t)d->ffn * h;
        case S_DOWN: return h * d->ffn;
        default: return -1;
    }
}

orc_model* orc_model_create(const orc_desc* d) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->d = *d;
    m->qdim = d->n_heads * d->head_dim;
    m->kvdim = d->n_kv_heads * d->head_dim;
    for (int s = 0; s < NSLOT_L; s++) m->layer[s] = (float**)calloc((size_t)d->n_layers, sizeof(float*));
    m->inv_freq = (float*)calloc((size_t)(d->head_dim / 2 + 1), sizeof(float));
    return m;
}

void orc_model_destroy(orc_model* m) {
    if (!m) return;
    free(m->tok_embd);
    free(m->out_norm);
    if (!m->output_tied) free(m->output);
    for (int s = 0; s < NSLOT_L; s++) {
        for (int l = 0; l < m->d.n_layers; l++) free(m->layer[s][l]);
        free(m->layer[s]);
    }
    free(m->inv_freq);
    free(m);
}

/* LoadTensor (GgufModelLoader.cs:409-418): new float[expected]; Dequantize(type, raw, dst). */
int orc_model_set(orc_model* m, int slot, int layer, int type, const uint8_t* bytes, int64_t nbytes) {
    int64_t n = slot_elems(m, slot);
    if (n < 0) return ORC_E_RANGE;
    float* dst = (float*)calloc((size_t)n, sizeof(float));
    if (!dst) return ORC_E_ARG;
    int rc = orc_dequantize(type, bytes, nbytes, dst, n);
    if (rc != ORC_OK) { free(dst); return rc; }
    float** where;
    if (slot == S_TOKEN_EMBD) where = &m->tok_embd;
    else if (slot == S_OUTPUT_NORM) where = &m->out_norm;
    else if (slot == S_OUTPUT) where = &m->output;
    else {
        if (layer < 0 || layer >= m->d.n_layers) { free(dst); return ORC_E_RANGE; }
        where = &m->layer[slot - 10][layer];
    }
    free(*where);
    *where = dst;
    return ORC_OK;
}

int orc_model_finalize(orc_model* m) {
    if (!m->tok_embd || !m->out_norm) return ORC_E_INVALID;
    if (!m->output) { m->output = m->tok_embd; m->output_tied = 1; } /* GgufModelLoader.cs:365-366 */
    int need[] = {S_ATTN_NORM, S_Q, S_K, S_V, S_O, S_FFN_NORM, S_GATE, S_UP, S_DOWN};
    for (int l = 0; l < m->d.n_layers; l++) {
        for (unsigned i = 0; i < sizeof(need) / sizeof(need[0]); i++)
            if (!m->layer[need[i] - 10][l]) return ORC_E_INVALID;
        if (m->d.arch == A_QWEN2 && (!m->layer[S_BQ - 10][l] || !m->layer[S_BK - 10][l] || !m->layer[S_BV - 10][l]))
            return ORC_E_INVALID;
        if (m->d.arch == A_GEMMA2 && (!m->layer[S_POST_ATTN - 10][l] || !m->layer[S_POST_FFN - 10][l]))
            return ORC_E_INVALID;
    }
    orc_rope_inv_freqs(m->d.rope_base, m->d.head_dim, m->inv_freq);
    return ORC_OK;
}

orc_fwd* orc_fwd_create(orc_model* m, int32_t max_seq) {
    orc_fwd* f = (orc_fwd*)calloc(1, sizeof(orc_fwd));
    const orc_desc* d = &m->d;
    f->m = m;
    f->max_seq = max_seq > 0 ? max_seq : d->max_ctx;
    f->keys = (float**)calloc((size_t)d->n_layers, sizeof(float*));
    f->vals = (float**)calloc((size_t)d->n_layers, sizeof(float*));
    for (int l = 0; l < d->n_layers; l++) {
        f->keys[l] = (float*)calloc((size_t)f->max_seq * (size_t)m->kvdim, sizeof(float));
        f->vals[l] = (float*)calloc((size_t)f->max_seq * (size_t)m->kvdim, sizeof(float));
    }
    f->x = (float*)calloc((size_t)d->hidden, sizeof(float));
    f->xn = (float*)calloc((size_t)d->hidden, sizeof(float));
    f->q = (float*)calloc((size_t)m->qdim, sizeof(float));
    f->k = (float*)calloc((size_t)m->kvdim, sizeof(float));
    f->v = (float*)calloc((size_t)m->kvdim, sizeof(float));
    f->att = (float*)calloc((size_t)m->qdim, sizeof(float));
    f->ffa = (float*)calloc((size_t)d->ffn, sizeof(float));
    f->ffb = (float*)calloc((size_t)d->ffn, sizeof(float));
    f->logits = (float*)calloc((size_t)d->vocab, sizeof(float));
    /* one score row per query head, so heads can run on separate threads */
    f->scores = (float*)calloc(((size_t)f->max_seq + 1) * (size_t)d->n_heads, sizeof(float));
    f->hidden = (float*)calloc((size_t)(d->n_layers + 1) * (size_t)d->hidden, sizeof(float));
    f->lim_layers = d->n_layers;
    f->lim_head = d->vocab;
    return f;
}

void orc_fwd_destroy(orc_fwd* f) {
    if (!f) return;
    for (int l = 0; l < f->m->d.n_layers; l++) { free(f->keys[l]); free(f->vals[l]); }
    free(f->keys); free(f->vals);
    free(f->x); free(f->xn); free(f->q); free(f->k); free(f->v); free(f->att);
    free(f->ffa); free(f->ffb); free(f->logits); free(f->scores); free(f->hidden);
    free(f);
}

/* KvCache.Clear (KvCache.cs:138-144). */
void orc_fwd_reset(orc_fwd* f) { f->cur_len = 0; f->next_layer = 0; }
void orc_fwd_limit(orc_fwd* f, int n_layers, int head_rows) { f->lim_layers = n_layers; f->lim_head = head_rows; }
int32_t orc_fwd_length(orc_fwd* f) { return f->cur_len; }

/* KvCache.Append (KvCache.cs:59-97), including evict-oldest-half (KvCache.cs:152-173). */
static int kv_append(orc_fwd* f, int layer) {
    int kvdim = f->m->kvdim;
    if (layer != f->next_layer) return ORC_E_INVALID;
    if (f->cur_len >= f->max_seq) {
        int keep = f->max_seq / 2;
        size_t src = (size_t)keep * kvdim, len = (size_t)(f->max_seq - keep) * kvdim;
        for (int l = 0; l < f->m->d.n_layers; l++) {
            memmove(f->keys[l], f->keys[l] + src, len * sizeof(float));
            memset(f->keys[l] + len, 0, src * sizeof(float));
            memmove(f->vals[l], f->vals[l] + src, len * sizeof(float));
            memset(f->vals[l] + len, 0, src * sizeof(float));
        }
        f->cur_len = keep;
    }
    size_t off = (size_t)f->cur_len * kvdim;
    memcpy(f->keys[layer] + off, f->k, sizeof(float) * (size_t)kvdim);
    memcpy(f->vals[layer] + off, f->v, sizeof(float) * (size_t)kvdim);
    f->next_layer++;
    if (f->next_layer == f->m->d.n_layers) { f->next_layer = 0; f->cur_len++; }
    return ORC_OK;
}

/* KvCache.GetKeys effective length (KvCache.cs:100-116). */
static int kv_effective(const orc_fwd* f, int layer) {
    int e = f->cur_len;
    if (f->next_layer > 0 && layer < f->next_layer) e++;
    return e;
}

typedef struct { orc_fwd* f; int layer, ws, seq_len; float scale; } attn_job;

/* One query head of ComputeAttention: scores over [ws, seq_len), optional Gemma softcap,
 * softmax, weighted sum of values. */
static void attn_heads(void* a, int64_t h0, int64_t h1) {
    attn_job* j = (attn_job*)a;
    orc_fwd* f = j->f;
    orc_model* m = f->m;
    const orc_desc* d = &m->d;
    int hd = d->head_dim, kvdim = m->kvdim, group = d->n_heads / d->n_kv_heads;
    int ws = j->ws, seq_len = j->seq_len, alen = seq_len - ws;
    const float* K = f->keys[j->layer];
    const float* V = f->vals[j->layer];
    for (int64_t h = h0; h < h1; h++) {
        int kh = (int)h / group;
        float* scores = f->scores + (size_t)h * ((size_t)f->max_seq + 1);
        const float* qh = f->q + (size_t)h * hd;
        for (int t = ws; t < seq_len; t++)
            scores[t - ws] = orc_dot(qh, K + (size_t)t * kvdim + (size_t)kh * hd, hd) * j->scale;
        if (d->arch == A_GEMMA2 && d->attn_softcap > 0.0f) orc_softcap(scores, alen, d->attn_softcap);
        orc_softmax(scores, alen);
        float* out = f->att + (size_t)h * hd;
        for (int t = ws; t < seq_len; t++) {
            const float* vv = V + (size_t)t * kvdim + (size_t)kh * hd;
            float w = scores[t - ws];
            for (int e = 0; e < hd; e++) out[e] += w * vv[e];
        }
    }
}

/* ComputeAttention (LlamaForwardPass.cs:158-211; MistralForwardPass.cs:121-175 window;
 * Gemma2ForwardPass.cs:126-185 scale, softcap, window). Heads are independent and may run on
 * the row-parallel threads. */
static int attention(orc_fwd* f, int layer, int seq_len, int window) {
    orc_model* m = f->m;
    const orc_desc* d = &m->d;
    int hd = d->head_dim;
    float scale = d->arch == A_GEMMA2 ? d->attn_scale : 1.0f / sqrtf((float)hd);
    if (seq_len > kv_effective(f, layer)) return ORC_E_RANGE; /* Span.Slice past the cache */
    int ws = seq_len - window;
    if (ws < 0) ws = 0;
    memset(f->att, 0, sizeof(float) * (size_t)m->qdim);
    attn_job j = {f, layer, ws, seq_len, scale};
    if ((int64_t)(seq_len - ws) * m->qdim >= 4096) pool_run(attn_heads, &j, d->n_heads);
    else attn_heads(&j, 0, d->n_heads);
    return ORC_OK;
}

static void rope_heads(orc_fwd* f, float* vec, int nheads, int position) {
    const orc_desc* d = &f->m->d;
    float pos = (d->rope_scaled && d->rope_scale > 0.0f) ? (float)position / d->rope_scale : (float)position;
    for (int h = 0; h < nheads; h++) orc_apply_rope(vec + (size_t)h * d->head_dim, pos, f->m->inv_freq, d->head_dim / 2);
}

static void norm(const orc_desc* d, const float* x, const float* w, float* dst) {
    if (d->arch == A_GEMMA2) orc_gemma_rmsnorm(x, w, dst, d->hidden);
    else orc_rmsnorm(x, w, dst, d->hidden, d->norm_eps);
}

/* IForwardPass.Forward for the four architectures (LlamaForwardPass.cs:82-130,
 * MistralForwardPass.cs:63-100, Qwen2ForwardPass.cs:62-103, Gemma2ForwardPass.cs:62-105). */
int orc_forward(orc_fwd* f, int32_t token, int32_t position) {
    orc_model* m = f->m;
    const orc_desc* d = &m->d;
    int h = d->hidden;
    if (token < 0 || token >= d->vocab) return ORC_E_RANGE;
    memcpy(f->x, m->tok_embd + (size_t)token * h, sizeof(float) * (size_t)h);
    for (int l = 0; l < f->lim_layers; l++) {
#define W(slot) (m->layer[(slot) - 10][l])
        norm(d, f->x, W(S_ATTN_NORM), f->xn);
        orc_linear(f->xn, W(S_Q), f->q, m->qdim, h);
        orc_linear(f->xn, W(S_K), f->k, m->kvdim, h);
        orc_linear(f->xn, W(S_V), f->v, m->kvdim, h);
        if (d->arch == A_QWEN2) {
            for (int i = 0; i < m->qdim; i++) f->q[i] = f->q[i] + W(S_BQ)[i];
            for (int i = 0; i < m->kvdim; i++) f->k[i] = f->k[i] + W(S_BK)[i];
            for (int i = 0; i < m->kvdim; i++) f->v[i] = f->v[i] + W(S_BV)[i];
        }
        rope_heads(f, f->q, d->n_heads, position);
        rope_heads(f, f->k, d->n_kv_heads, position);
        int rc = kv_append(f, l);
        if (rc != ORC_OK) return rc;
        int window = 0x7FFFFFFF;
        if (d->arch == A_MISTRAL) window = d->sliding_window;
        if (d->arch == A_GEMMA2 && (l % 2) == 0) window = d->sliding_window;
        rc = attention(f, l, position + 1, window);
        if (rc != ORC_OK) return rc;
        orc_linear(f->att, W(S_O), f->xn, h, m->qdim);
        if (d->arch == A_GEMMA2) orc_gemma_rmsnorm(f->xn, W(S_POST_ATTN), f->xn, h);
        for (int i = 0; i < h; i++) f->x[i] = f->x[i] + f->xn[i];
        norm(d, f->x, W(S_FFN_NORM), f->xn);
        orc_linear(f->xn, W(S_GATE), f->ffa, d->ffn, h);
        if (d->arch == A_GEMMA2) orc_gelu(f->ffa, d->ffn); else orc_silu(f->ffa, d->ffn);
        orc_linear(f->xn, W(S_UP), f->ffb, d->ffn, h);
        for (int i = 0; i < d->ffn; i++) f->ffa[i] *= f->ffb[i];
        orc_linear(f->ffa, W(S_DOWN), f->xn, h, d->ffn);
        if (d->arch == A_GEMMA2) orc_gemma_rmsnorm(f->xn, W(S_POST_FFN), f->xn, h);
        for (int i = 0; i < h; i++) f->x[i] = f->x[i] + f->xn[i];
        memcpy(f->hidden + (size_t)l * h, f->x, sizeof(float) * (size_t)h);
#undef W
    }
    norm(d, f->x, m->out_norm, f->xn);
    memcpy(f->hidden + (size_t)d->n_layers * h, f->xn, sizeof(float) * (size_t)h);
    orc_linear(f->xn, m->output, f->logits, f->lim_head, h);
    if (d->arch == A_GEMMA2 && d->final_softcap > 0.0f) orc_softcap(f->logits, f->lim_head, d->final_softcap);
    return ORC_OK;
}

const float* orc_logits(orc_fwd* f) { return f->logits; }

int orc_fwd_hidden(orc_fwd* f, int layer, float* dst, int64_t n) {
    int h = f->m->d.hidden;
    if (layer < 0 || layer > f->m->d.n_layers) return ORC_E_RANGE;
    if (n < h) return ORC_E_ARG;
    memcpy(dst, f->hidden + (size_t)layer * h, sizeof(float) * (size_t)h);
    return ORC_OK;
}

int orc_fwd_kv(orc_fwd* f, int layer, int kind, float* dst, int64_t n) {
    if (layer < 0 || layer >= f->m->d.n_layers) return ORC_E_RANGE;
    int64_t cnt = (int64_t)kv_effective(f, layer) * f->m->kvdim;
    if (n < cnt) return ORC_E_ARG;
    memcpy(dst, (kind == 0 ? f->keys : f->vals)[layer], sizeof(float) * (size_t)cnt);
    return ORC_OK;
}
