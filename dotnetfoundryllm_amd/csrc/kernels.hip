// kernels.hip — gfx950 kernels of the decode path.
//
// Compiled with -ffp-contract=off: every a*b+c written below stays two roundings unless an
// explicit fmaf() asks for one, so the dequantized values and the RoPE rotation follow the
// reference's operation order (the .NET JIT does not contract either).
#include "kernels.hpp"

#include "deq.hpp"
#include "gemv.hpp"

#include <math.h>

namespace fllm {

// Hardware binary16 -> binary32 conversion (exact for every finite input).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
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
// Float GEMV for F32 / F16 / BF16 weights (128-bit row loads; x from L2).
// =====================================================================================
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// weight rows are read once per step: non-temporal loads keep them from displacing what is reused
typedef uint32_t kf_u4 __attribute__((ext_vector_type(4)));

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
        const kf_u4 uv = __builtin_nontemporal_load((const kf_u4*)(rp + v));
        const uint4 u = make_uint4(uv.x, uv.y, uv.z, uv.w);
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

hipError_t launch_gemv_tiles(const WMat& m, const float* xf, float* y, int n_cu, hipStream_t st) {
    GemvArgs a{};
    a.nseg = 1;
    a.seg[0].w = m.w;
    a.seg[0].type = m.type;
    a.seg[0].layout = LAYOUT_TILES;
    a.seg[0].rows = (int)m.rows;
    a.seg[0].epi = EPI_STORE;
    a.seg[0].out = y;
    a.xin = XIN_F32;
    a.x = xf;
    if (!gemv_tiles_shape_ok(m.type, m.rows, m.cols) || !gemv_uses_mfma(a, m.cols)) return hipErrorInvalidValue;
    int threads;
    size_t lds;
    const int grid = gemv_plan(a, m.cols, n_cu, 0, &threads, &lds);
    return launch_gemv_fused(a, grid, threads, lds, st);
}

hipError_t launch_gemv(const WMat& m, const float* xf, float* y, const float* residual, int n_cu, hipStream_t st) {
    int t = m.type;
    if (gemv_fusable_type(t) && gemv_fusable_cols(m.cols)) {
        GemvArgs a{};
        a.nseg = 1;
        a.seg[0].w = m.w;
        a.seg[0].type = t;
        a.seg[0].rows = (int)m.rows;
        a.seg[0].epi = residual ? EPI_RESID : EPI_STORE;
        a.seg[0].out = y;
        a.seg[0].resid = residual;
        a.xin = XIN_F32;
        a.x = xf;
        int threads;
        size_t lds;
        int grid = gemv_plan(a, m.cols, n_cu, 0, &threads, &lds);
        return launch_gemv_fused(a, grid, threads, lds, st);
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
    p->nstep = 0;
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

// RmsNorm (TensorOperations.cs:42-54) or GemmaRmsNorm (TensorOperations.cs:90-107) into xn.
__global__ __launch_bounds__(1024) void k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w, int n,
                                                   float eps, int kind, float* xn) {
    __shared__ float red[16];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(x[i], x[i], ss);
    float tot = block_sum(ss, red);
    float rms = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float t = x[i] * rms;
        xn[i] = kind ? t * (w[i] + 1.0f) : t * w[i];
    }
}

hipError_t launch_rmsnorm(const float* x, const float* w, int n, float eps, int norm_kind, float* xn, hipStream_t st) {
    k_rmsnorm<<<1, 1024, 0, st>>>(x, w, n, eps, norm_kind, xn);
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
                                                       float* out) {
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
    if (d < hd) out[(int64_t)h * hd + d] = o / L;
}

hipError_t launch_attention(const float* q, const float* kcache, const float* vcache, int n_heads, int n_kv,
                            int head_dim, int window, float scale, float softcap, int nsplit, float* part_o,
                            float* part_ml, float* out, const StepParams* p, hipStream_t st) {
    int group = n_heads / n_kv;
    int chunk_cap = 256;
    size_t lds = sizeof(float) * ((size_t)group * head_dim + (size_t)group * chunk_cap);
    dim3 grid(n_kv, nsplit);
    k_attn_partial<<<grid, 256, lds, st>>>(q, kcache, vcache, n_heads, n_kv, head_dim, window, scale, softcap,
                                            nsplit, chunk_cap, part_o, part_ml, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    int bs = head_dim < 64 ? 64 : head_dim;
    k_attn_combine<<<n_heads, bs, 0, st>>>(part_o, part_ml, nsplit, head_dim, out);
    return hipGetLastError();
}

// =====================================================================================
// FFN gating: ComputeSiluFfn (LlamaForwardPass.cs:217-232), ComputeGeluFfn
// (Gemma2ForwardPass.cs:187-199); Silu/Gelu from TensorOperations.cs:57-117.
// =====================================================================================
__global__ __launch_bounds__(256) void k_act(const float* __restrict__ g, const float* __restrict__ u, int n,
                                              int act, float* h) {
    int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    h[i] = act_fn(g[i], act) * u[i];
}

hipError_t launch_act(const float* g, const float* u, int n, int act, float* h, hipStream_t st) {
    k_act<<<(n + 255) / 256, 256, 0, st>>>(g, u, n, act, h);
    return hipGetLastError();
}

// Gemma2 post-norms: x += GemmaRmsNorm(t, w) (Gemma2ForwardPass.cs:90-91, 95-96).
__global__ __launch_bounds__(1024) void k_postnorm_add(const float* __restrict__ t, const float* __restrict__ w,
                                                        int n, const float* xi, float* xo) {
    __shared__ float red[16];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss = fmaf(t[i], t[i], ss);
    float tot = block_sum(ss, red);
    float rms = 1.0f / sqrtf(tot / (float)n + 1e-6f);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float o = (t[i] * rms) * (w[i] + 1.0f);
        xo[i] = xi[i] + o;
    }
}

hipError_t launch_postnorm_add(const float* t, const float* w, int n, const float* x_in, float* x_out, hipStream_t st) {
    k_postnorm_add<<<1, 1024, 0, st>>>(t, w, n, x_in, x_out);
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

// Key of the top-k selection: TopKSampler compares floats with > and < (TopKSampler.cs:55-60,
// 93-105), under which -0 equals +0, so both zeros map to the key of +0.
__device__ __forceinline__ uint32_t tkey(float v) { return okey(v == 0.0f ? 0.0f : v); }

// First index of the maximum (IndexOfMax semantics). With tokens_out set, also publishes the
// token as the next step's input and advances the step parameters (device-side greedy loop).
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int64_t n, StepParams* p, int* tokens_out,
                                                 int tokens_cap) {
    __shared__ uint32_t sk[16];
    __shared__ int64_t si[16];
    uint32_t bk = 0;
    int64_t bi = -1;
    const int64_t nt = blockDim.x, step = nt * 8;
    for (int64_t base = threadIdx.x; base < n; base += step) {  // 8 loads in flight per thread
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = base + j * nt < n ? x[base + j * nt] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {  // ascending index within the thread: the first maximum stays
            int64_t i = base + j * nt;
            uint32_t k = okey(v[j]);
            if (i < n && (bi < 0 || k > bk)) { bk = k; bi = i; }
        }
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
        if (tokens_out) {
            if (p->nstep >= 0 && p->nstep < tokens_cap) tokens_out[p->nstep] = (int)idx;
            p->nstep = p->nstep + 1;
            p->token = (int)idx;
            p->pos = p->pos + 1;
            p->cur_len = p->cur_len + 1;
        }
    }
}

hipError_t launch_argmax(const float* x, int64_t n, StepParams* p, int* tokens_out, int tokens_cap, hipStream_t st) {
    k_argmax<<<1, 1024, 0, st>>>(x, n, p, tokens_out, tokens_cap);
    return hipGetLastError();
}

// Per 4096-entry segment of x: the key (order key << 32) | ~index of its first maximum (the LM head
// epilogue's key format, so k_argmax_keys reduces them); 16 loads per thread in flight.
__global__ __launch_bounds__(256) void k_argmax_seg(const float* __restrict__ x, int64_t n,
                                                    unsigned long long* __restrict__ keys) {
    const int64_t base = (int64_t)blockIdx.x * 4096;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int64_t i = base + threadIdx.x + 256 * j;
        v[j] = i < n ? x[i] : 0.0f;
    }
    unsigned long long best = 0ull;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int64_t i = base + threadIdx.x + 256 * j;
        const unsigned long long k = ((unsigned long long)okey(v[j]) << 32) | (0xFFFFFFFFu - (uint32_t)i);
        if (i < n && k > best) best = k;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long ot = __shfl_xor(best, o);
        best = ot > best ? ot : best;
    }
    __shared__ unsigned long long sk[4];
    if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) best = sk[w] > best ? sk[w] : best;
        keys[blockIdx.x] = best;
    }
}

// Reduce the LM head's per-workgroup keys ((order key << 32) | ~row) to the first index of the
// maximum, then advance the step like k_argmax with tokens_out.
__global__ __launch_bounds__(256) void k_argmax_keys(const unsigned long long* __restrict__ keys, int n, StepParams* p,
                                                     int* tokens_out, int tokens_cap) {
    __shared__ unsigned long long sk[4];
    unsigned long long best = 0ull;
    for (int i = threadIdx.x; i < n; i += blockDim.x) best = keys[i] > best ? keys[i] : best;
    for (int o = 32; o > 0; o >>= 1) {
        unsigned long long ot = __shfl_xor(best, o);
        best = ot > best ? ot : best;
    }
    if ((threadIdx.x & 63) == 0) sk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = sk[w] > best ? sk[w] : best;
        int idx = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
        p->argmax = idx;
        if (p->nstep >= 0 && p->nstep < tokens_cap) tokens_out[p->nstep] = idx;
        p->nstep = p->nstep + 1;
        p->token = idx;
        p->pos = p->pos + 1;
        p->cur_len = p->cur_len + 1;
    }
}

hipError_t launch_argmax_keys(const unsigned long long* keys, int n, StepParams* p, int* tokens_out, int tokens_cap,
                              hipStream_t st) {
    k_argmax_keys<<<1, 256, 0, st>>>(keys, n, p, tokens_out, tokens_cap);
    return hipGetLastError();
}

int argmax_segments(int64_t n) { return (int)((n + 4095) / 4096); }

hipError_t launch_argmax_seg(const float* x, int64_t n, unsigned long long* keys, hipStream_t st) {
    if (n <= 0 || n > 0xFFFFFFFFll) return hipErrorInvalidValue;
    k_argmax_seg<<<argmax_segments(n), 256, 0, st>>>(x, n, keys);
    return hipGetLastError();
}

// ---- helpers of the one-workgroup sampling kernels (1024 threads, 16 waves) ---------------
// The ordered passes (stable compaction, running sums) work on 64-element chunks: a wave takes
// chunks wave, wave + 16, ... with coalesced loads, a ballot gives the chunk's count and each
// lane's rank inside it, and a block scan over the per-chunk totals (in LDS) gives each chunk's
// offset. SAMPLE_MAX_CHUNKS bounds the vocabulary at 262144 entries.
constexpr int SAMPLE_MAX_CHUNKS = SAMPLE_MAX_VOCAB / 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ unsigned long long lanes_below() {
    int l = lane_id();
    return l ? (~0ull >> (64 - l)) : 0ull;
}

// Exclusive prefix over the block of one value per thread (Hillis-Steele in LDS); returns the
// thread's exclusive prefix and writes the block total.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T v, T* buf, T* total) {
    int t = threadIdx.x, nt = blockDim.x;
    buf[t] = v;
    __syncthreads();
    for (int o = 1; o < nt; o <<= 1) {
        T a = t >= o ? buf[t - o] : (T)0;
        __syncthreads();
        buf[t] += a;
        __syncthreads();
    }
    T incl = buf[t];
    *total = buf[nt - 1];
    __syncthreads();
    return incl - v;
}

// In place exclusive prefix over arr[0..nch) (nch <= 4 * blockDim.x); returns the total.
template <typename T>
__device__ __forceinline__ T chunks_excl_scan(T* arr, int nch, T* buf) {
    const int per = 4, b0 = threadIdx.x * per;
    T loc = 0;
    for (int c = b0; c < b0 + per && c < nch; c++) loc += arr[c];
    T total;
    T run = block_excl_scan(loc, buf, &total);
    for (int c = b0; c < b0 + per && c < nch; c++) {
        T v = arr[c];
        arr[c] = run;
        run += v;
    }
    __syncthreads();
    return total;
}

// hist[bin] += 1 for every lane with `take`, one LDS atomic per distinct bin of the wave (the bins
// of nearby logits coincide, and same-address atomics from many lanes serialise). Called with all
// 64 lanes of the wave active.
__device__ __forceinline__ void wave_hist_add(int* hist, bool take, uint32_t bin) {
    unsigned long long act = __ballot(take);
    while (act) {
        int leader = __ffsll((long long)act) - 1;
        uint32_t lb = __shfl(bin, leader);
        unsigned long long same = __ballot(take && bin == lb);
        if (lane_id() == leader) atomicAdd(&hist[lb], (int)__popcll(same));
        act &= ~same;
    }
}

// One pass of a one-workgroup kernel over src[0..n): f(i, v) for i = tid, tid + nt, ... with
// v = src[i] (0 past n, where f must check i < n itself). A thread's loads of a batch are issued
// together, so a pass costs one memory round trip per B elements of a thread rather than one per
// element. The trip count is uniform, so f may use wave-wide ballots and shuffles.
template <int B, typename F>
__device__ __forceinline__ void pass_strided(const float* __restrict__ src, int n, F f) {
    const int nt = blockDim.x, tid = threadIdx.x;
    for (int base = 0; base < n; base += nt * B) {
        float v[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            int i = base + j * nt + tid;
            v[j] = i < n ? src[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < B; j++) f(base + j * nt + tid, v[j]);
    }
}

// The same over 64-element chunks: wave w takes chunks w, w + 16, ..., lane l element 64c + l;
// f(c, i, v) runs for every chunk c < nch with the whole wave active.
template <int B, typename F>
__device__ __forceinline__ void pass_chunks(const float* __restrict__ src, int n, int nch, F f) {
    const int nw = blockDim.x >> 6, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int c0 = wave; c0 < nch; c0 += nw * B) {
        float v[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            int c = c0 + j * nw, i = (c << 6) + lane;
            v[j] = (c < nch && i < n) ? src[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < B; j++) {
            int c = c0 + j * nw;
            if (c < nch) f(c, (c << 6) + lane, v[j]);
        }
    }
}
constexpr int SAMPLE_BATCH = 16;

// ---- top-k (SamplerPipeline.cs:67-74, TopKSampler.ApplyTopK TopKSampler.cs:42-71) ------------
// Scale by inv_temp in place, then emit every index whose scaled value is at least the k-th
// largest (ties kept), in ascending index order, with its value. Two forms:
//  - sample select over a grid (k <= 256, n >= 4096): one workgroup takes a threshold t from an
//    evenly spaced sample of the scaled values, ranked so that a few hundred entries reach it;
//    segments of 4096 entries (one workgroup each) scale their entries and count those reaching
//    t, then gather them in index order into a candidate buffer; one workgroup finds the exact
//    k-th largest among the candidates and emits. When fewer than k or more than 4096 entries
//    reach t, that last workgroup runs the full select instead. A pass over the logits by one
//    workgroup is bound by one CU's outstanding misses (about 25 us for 150k entries), so the
//    full-width passes run on the grid;
//  - the full select in one workgroup: a 4-pass radix select on order-preserving keys and a
//    stable compaction.
constexpr int TOPK_NS = 2048, TOPK_SEG = 4096;

// The bucket of a descending radix-select step: with `above` already counted above this digit's
// buckets, the bucket b whose range holds the P-th unit from the top, i.e.
// above + sum(hist[b+1..255]) < P <= above + sum(hist[b..255]). Threads 0..255 each take one bin
// (wave prefix sums over bins 255, 254, ...; blockDim.x >= 256); all threads return b (or -1 when
// the total stays below P) and *before = above + sum(hist[b+1..255]). Two barriers, no serial scan.
template <typename T>
__device__ int find_bucket_desc(const T* hist, T above, T P, T* before_out, T* wtot, int* s_b) {
    const int t = threadIdx.x, lane = t & 63;
    T h = 0, incl = 0;
    if (t < 256) {
        h = hist[255 - t];
        incl = h;
        for (int o = 1; o < 64; o <<= 1) {
            T a = __shfl_up(incl, o);
            if (lane >= o) incl += a;
        }
        if (lane == 63) wtot[t >> 6] = incl;
    }
    if (t == 0) *s_b = -1;
    __syncthreads();
    if (t < 256) {
        T before = above;
        for (int w = 0; w < (t >> 6); w++) before += wtot[w];
        before += incl - h;
        if (before < P && P - before <= h) {  // exactly one bin: the running sum is monotone
            *s_b = 255 - t;
            *before_out = before;
        }
    }
    __syncthreads();
    return *s_b;
}

// Copies the first nseg entries of a per-segment array into LDS (nseg <= blockDim.x), one load per
// thread, so that one thread can then combine them in order without a chain of memory loads.
template <typename T>
__device__ __forceinline__ void load_segs(const T* __restrict__ src, int nseg, T* dst) {
    if ((int)threadIdx.x < nseg) dst[threadIdx.x] = src[threadIdx.x];
    __syncthreads();
}

// Full radix select + stable compaction over x[0..n) (already scaled); one workgroup of 1024.
__device__ void topk_radix_emit(const float* __restrict__ x, int n, int k, int cap, int* ids, float* vals,
                                int* count) {
    __shared__ int hist[256];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remain, s_before, s_wtot[4], s_b;
    __shared__ int chunk[SAMPLE_MAX_CHUNKS];
    __shared__ int scan[1024];
    const int tid = threadIdx.x, nt = blockDim.x, lane = lane_id();
    const int nch = (n + 63) >> 6;
    if (tid == 0) { s_prefix = 0; s_mask = 0; s_remain = k; }
    __syncthreads();
    uint32_t thr = 0;
    if (k < n) {
        for (int pass = 0; pass < 4; pass++) {
            const int shift = 24 - 8 * pass;
            for (int b = tid; b < 256; b += nt) hist[b] = 0;
            __syncthreads();
            const uint32_t prefix = s_prefix, mask = s_mask;
            pass_strided<SAMPLE_BATCH>(x, n, [&](int i, float v) {
                uint32_t key = tkey(v);
                wave_hist_add(hist, i < n && (key & mask) == prefix, (key >> shift) & 255u);
            });
            __syncthreads();
            const int rem = s_remain;
            const int b = find_bucket_desc(hist, 0, rem, &s_before, s_wtot, &s_b);
            if (tid == 0) {  // b >= 0: the counts above the prefix sum to at least rem
                s_prefix = prefix | ((uint32_t)b << shift);
                s_mask = mask | (255u << shift);
                s_remain = rem - s_before;
            }
            __syncthreads();
        }
        thr = s_prefix;
    }
    // stable compaction: survivors per 64-element chunk, chunk offsets, then ranks by ballot
    pass_chunks<SAMPLE_BATCH>(x, n, nch, [&](int c, int i, float v) {
        unsigned long long m = __ballot(i < n && tkey(v) >= thr);
        if (lane == 0) chunk[c] = (int)__popcll(m);
    });
    __syncthreads();
    int total = chunks_excl_scan(chunk, nch, scan);
    if (tid == 0) *count = total;
    pass_chunks<SAMPLE_BATCH>(x, n, nch, [&](int c, int i, float v) {
        bool keep = i < n && tkey(v) >= thr;
        unsigned long long m = __ballot(keep);
        if (keep) {
            int off = chunk[c] + (int)__popcll(m & lanes_below());
            if (off < cap) { ids[off] = i; vals[off] = v; }
        }
    });
}

// Exact k-th largest among the nc candidates (values cv, indices ci, in ascending index order)
// and the survivors emitted in that order; one workgroup of 1024, nc <= TOPK_CMAX.
__device__ void topk_select_candidates(const float* __restrict__ cv, const int* __restrict__ ci, int nc, int k,
                                       int cap, int* ids, float* vals, int* count) {
    __shared__ float lv[TOPK_CMAX];
    __shared__ int hist[256];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remain, s_before, s_wtot[4], s_b;
    __shared__ int scan[1024];
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int j = tid; j < nc; j += nt) lv[j] = cv[j];
    if (tid == 0) { s_prefix = 0; s_mask = 0; s_remain = k; }
    __syncthreads();
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        for (int b = tid; b < 256; b += nt) hist[b] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask;
        for (int j = tid; j < nc; j += nt) {
            uint32_t key = tkey(lv[j]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
        }
        __syncthreads();
        const int rem = s_remain;
        const int b = find_bucket_desc(hist, 0, rem, &s_before, s_wtot, &s_b);
        if (tid == 0) {
            s_prefix = prefix | ((uint32_t)b << shift);
            s_mask = mask | (255u << shift);
            s_remain = rem - s_before;
        }
        __syncthreads();
    }
    const uint32_t thr = s_prefix;
    const int per = (TOPK_CMAX + nt - 1) / nt, b0 = tid * per;
    int cnt = 0;
    for (int j = b0; j < b0 + per && j < nc; j++) cnt += tkey(lv[j]) >= thr ? 1 : 0;
    int total;
    int off = block_excl_scan(cnt, scan, &total);
    for (int j = b0; j < b0 + per && j < nc; j++) {
        float v = lv[j];
        if (tkey(v) >= thr) {
            if (off < cap) { ids[off] = ci[j]; vals[off] = v; }
            off++;
        }
    }
    if (tid == 0) *count = total;
}

__global__ __launch_bounds__(1024) void k_topk(float* x, int64_t n64, float inv_temp, int k, int cap, int* ids,
                                                float* vals, int* count) {
    const int n = (int)n64;
    if (inv_temp != 1.0f)
        pass_strided<SAMPLE_BATCH>(x, n, [&](int i, float v) { if (i < n) x[i] = v * inv_temp; });
    __syncthreads();
    topk_radix_emit(x, n, k, cap, ids, vals, count);
}

// The sample's threshold: among the keys of the scaled values at j * n / NS, the r-th largest
// (radix select) with r = 4 k NS / n + 8 (about 4 k + 8 n / NS entries of the whole reach it).
__global__ __launch_bounds__(1024) void k_topk_sample(const float* __restrict__ x, int n, float inv_temp, int k,
                                                      TopkScratch* sc) {
    __shared__ uint32_t samp[TOPK_NS];
    __shared__ int hist[256];
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_remain, s_before, s_wtot[4], s_b;
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int j = tid; j < TOPK_NS; j += nt) {
        float v = x[(int)(((int64_t)j * n) / TOPK_NS)];
        samp[j] = tkey(inv_temp != 1.0f ? v * inv_temp : v);
    }
    if (tid == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_remain = (int)min((int64_t)TOPK_NS, (int64_t)4 * k * TOPK_NS / n + 8);  // rank r in the sample
    }
    for (int pass = 0; pass < 4; pass++) {  // radix select of the sample's r-th largest key
        const int shift = 24 - 8 * pass;
        for (int b = tid; b < 256; b += nt) hist[b] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix, mask = s_mask;
        for (int j = tid; j < TOPK_NS; j += nt) {
            uint32_t key = samp[j];
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
        }
        __syncthreads();
        const int rem = s_remain;
        const int b = find_bucket_desc(hist, 0, rem, &s_before, s_wtot, &s_b);
        if (tid == 0) {
            s_prefix = prefix | ((uint32_t)b << shift);
            s_mask = mask | (255u << shift);
            s_remain = rem - s_before;
        }
        __syncthreads();
    }
    if (tid == 0) sc->t = s_prefix;
}

// Segment blockIdx.x (TOPK_SEG entries, 16 per thread): scale in place, count keys >= t.
__global__ __launch_bounds__(256) void k_topk_count(float* x, int n, float inv_temp, TopkScratch* sc) {
    __shared__ int red[4];
    const uint32_t t = sc->t;
    const int beg = blockIdx.x * TOPK_SEG, tid = threadIdx.x;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + j * 256 + tid;
        v[j] = i < n ? x[i] : 0.0f;
    }
    int c = 0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + j * 256 + tid;
        if (i < n) {
            float w = v[j];
            if (inv_temp != 1.0f) {
                w = w * inv_temp;
                x[i] = w;
            }
            c += tkey(w) >= t ? 1 : 0;
        }
    }
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
    if (lane_id() == 0) red[tid >> 6] = c;
    __syncthreads();
    if (tid == 0) sc->wg_cnt[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// Segment blockIdx.x: its offset among the candidates (counts of the segments before it), then
// its entries with keys >= t written there in index order (64-entry chunks ranked by ballot).
__global__ __launch_bounds__(256) void k_topk_gather(const float* __restrict__ x, int n, int k, int nseg,
                                                     TopkScratch* sc) {
    __shared__ int cc[TOPK_SEG / 64];
    __shared__ int segc[TOPK_MAX_SEG];
    __shared__ int s_off, s_total;
    const uint32_t t = sc->t;
    load_segs(sc->wg_cnt, nseg, segc);
    if (threadIdx.x == 0) {
        int o = 0, tot = 0;
        for (int h = 0; h < nseg; h++) {
            o += h < (int)blockIdx.x ? segc[h] : 0;
            tot += segc[h];
        }
        s_off = o;
        s_total = tot;
    }
    __syncthreads();
    const int off = s_off, total = s_total;
    if (blockIdx.x == 0 && threadIdx.x == 0) sc->nc = total;
    if (total < k || total > TOPK_CMAX) return;  // uniform: the finishing kernel runs the full select
    const int wave = threadIdx.x >> 6, lane = lane_id(), beg = blockIdx.x * TOPK_SEG;
    float v[16];
    unsigned long long m[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + ((wave * 16 + j) << 6) + lane;
        v[j] = i < n ? x[i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + ((wave * 16 + j) << 6) + lane;
        m[j] = __ballot(i < n && tkey(v[j]) >= t);
        if (lane == 0) cc[wave * 16 + j] = (int)__popcll(m[j]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int q = 0; q < TOPK_SEG / 64; q++) { int c = cc[q]; cc[q] = run; run += c; }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; j++) {
        if ((m[j] >> lane) & 1ull) {
            int i = beg + ((wave * 16 + j) << 6) + lane;
            int o = off + cc[wave * 16 + j] + (int)__popcll(m[j] & lanes_below());
            sc->cand_v[o] = v[j];
            sc->cand_i[o] = i;
        }
    }
}

__global__ __launch_bounds__(1024) void k_topk_finish(const float* __restrict__ x, int n, int k, int cap, int* ids,
                                                       float* vals, int* count, const TopkScratch* sc) {
    const int nc = sc->nc;
    if (nc >= k && nc <= TOPK_CMAX) topk_select_candidates(sc->cand_v, sc->cand_i, nc, k, cap, ids, vals, count);
    else topk_radix_emit(x, n, k, cap, ids, vals, count);  // x was scaled by k_topk_count
}

hipError_t launch_topk(float* x, int64_t n, float inv_temp, int k, int cap, int* ids, float* vals, int* count,
                       TopkScratch* sc, hipStream_t st) {
    const int nseg = (int)((n + TOPK_SEG - 1) / TOPK_SEG);
    if (sc && k <= 256 && k < n && n >= 2 * TOPK_NS && nseg <= TOPK_MAX_SEG) {
        k_topk_sample<<<1, 1024, 0, st>>>(x, (int)n, inv_temp, k, sc);
        k_topk_count<<<nseg, 256, 0, st>>>(x, (int)n, inv_temp, sc);
        k_topk_gather<<<nseg, 256, 0, st>>>(x, (int)n, k, nseg, sc);
        k_topk_finish<<<1, 1024, 0, st>>>(x, (int)n, k, cap, ids, vals, count, sc);
    } else {
        k_topk<<<1, 1024, 0, st>>>(x, n, inv_temp, k, cap, ids, vals, count);
    }
    return hipGetLastError();
}

// LlamaLanguageModel.ApplyRepetitionPenalty (LlamaLanguageModel.cs:357-373): for each listed id
// in [0, n), in list order, l > 0 ? l / penalty : l * penalty, repeats applying again. Distinct ids
// are independent, so the repeats of one id are counted first and then applied in sequence by a
// single thread, which gives the list-order result bit for bit. counts holds n zeros on entry and
// is left zeroed: exactly one exchange per id returns its count, every other returns 0.
__global__ __launch_bounds__(1024) void k_rep_penalty(float* x, int n, const int* __restrict__ ids, int n_ids,
                                                      float penalty, int* counts) {
    for (int j = threadIdx.x; j < n_ids; j += blockDim.x) {
        int id = ids[j];
        if ((unsigned)id < (unsigned)n) atomicAdd(&counts[id], 1);
    }
    __threadfence();  // every add has completed before any thread exchanges a counter
    __syncthreads();
    for (int j = threadIdx.x; j < n_ids; j += blockDim.x) {
        int id = ids[j];
        if ((unsigned)id >= (unsigned)n) continue;
        int c = atomicExch(&counts[id], 0);
        if (c == 0) continue;
        float v = x[id];
        for (int r = 0; r < c; r++) v = v > 0.0f ? v / penalty : v * penalty;
        x[id] = v;
    }
}

hipError_t launch_rep_penalty(float* x, int n, const int* ids, int n_ids, float penalty, int* counts,
                              hipStream_t st) {
    k_rep_penalty<<<1, 1024, 0, st>>>(x, n, ids, n_ids, penalty, counts);
    return hipGetLastError();
}

// ---- nucleus sampler ------------------------------------------------------------------
// Probability masses as unsigned 64-bit fixed point with 2^63 = 1: integer sums are exact and
// independent of the order they are formed in.
__device__ __forceinline__ unsigned long long fix63(float p) {
    return (unsigned long long)((double)p * 9223372036854775808.0);
}

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, T* red, Op op) {
    for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o));
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (int)(blockDim.x >> 6);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    T r = red[0];
    for (int w = 1; w < nw; w++) r = op(r, red[w]);  // same order in every thread
    return r;
}

// SamplerPipeline.Sample (SamplerPipeline.cs:58-89) with topK disabled, on the device logits:
// scale by inv_temp in place (stage 1), softmax (stage 3, TensorOperations.cs:23-39: max,
// exp(x - max), divide by the sum) into pr, nucleus of top_p (stage 4, TopPSampler.ApplyTopP
// TopPSampler.cs:60-110: the shortest prefix of the descending order whose mass reaches top_p,
// equal probabilities by ascending index, then divided by the kept sum), and the draw (stage 5,
// TemperatureSampler.SampleFromProbabilities TemperatureSampler.cs:53-70: the first index whose
// running sum exceeds u, else the last nonzero index). Masses and running sums are exact
// fixed-point integers where the reference accumulates in f32 order, so the chosen token can
// differ only where u or top_p lies within f32 rounding of a boundary.
// Every full-width pass runs over segments of NUC_SEG entries, one workgroup of 256 each (16
// entries per thread); per-segment results (max, sums, tie counts, masses) go through the
// scratch, whose f32 sums are taken in segment order, so results are deterministic. The nucleus
// edge tau comes from a 4-level radix select over the probabilities' bit patterns weighted by
// mass: each level's segments add their workgroup histogram into the scratch, and every
// workgroup of the next level re-derives the selection from the levels before it.
constexpr int NUC_SEG = 4096;

template <typename T>
__device__ __forceinline__ T wg256_sum(T v, T* red) {  // ordered: lanes by xor tree, then waves 0..3
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// Loads the first `levels` mass histograms and derives the selection: tau's bits so far (prefix
// under mask), the mass strictly above them (above), or `all` when the whole mass stays below P.
struct NucSel {
    uint32_t prefix, mask;
    unsigned long long above;
    int all;
};
__device__ NucSel nuc_select(const NucleusScratch* sc, int levels, unsigned long long P, unsigned long long* lh,
                             NucSel* out) {
    __shared__ unsigned long long s_before, s_wtot[4];
    __shared__ int s_b;
    for (int j = threadIdx.x; j < levels * 256; j += blockDim.x) lh[j] = sc->hist[j >> 8][j & 255];
    __syncthreads();
    NucSel r{0u, 0u, 0ull, 0};
    for (int L = 0; L < levels; L++) {  // every thread follows the same selections
        const int b = find_bucket_desc(lh + L * 256, r.above, P, &s_before, s_wtot, &s_b);
        if (b < 0) {
            r.all = 1;
            break;
        }
        const int shift = 24 - 8 * L;
        r.prefix |= (uint32_t)b << shift;
        r.mask |= 255u << shift;
        r.above = s_before;
        __syncthreads();  // s_before is rewritten by the next level
    }
    if (threadIdx.x == 0) *out = r;
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(256) void k_nuc_max(float* x, int n, float inv_temp, NucleusScratch* sc) {
    __shared__ float red[4];
    const int beg = blockIdx.x * NUC_SEG, tid = threadIdx.x;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) { int i = beg + j * 256 + tid; v[j] = i < n ? x[i] : -INFINITY; }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + j * 256 + tid;
        if (i < n) {
            if (inv_temp != 1.0f) { v[j] = v[j] * inv_temp; x[i] = v[j]; }
            m = fmaxf(m, v[j]);
        }
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) sc->seg_max[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ __launch_bounds__(256) void k_nuc_exp(const float* __restrict__ x, int n, float* pr, int nseg,
                                                 NucleusScratch* sc) {
    __shared__ float red[4];
    __shared__ float segv[NUC_MAX_SEG];
    __shared__ float s_m;
    const int beg = blockIdx.x * NUC_SEG, tid = threadIdx.x;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) { int i = beg + j * 256 + tid; v[j] = i < n ? x[i] : 0.0f; }
    load_segs(sc->seg_max, nseg, segv);
    if (tid == 0) {
        float m = -INFINITY;
        for (int h = 0; h < nseg; h++) m = fmaxf(m, segv[h]);
        s_m = m;
    }
    __syncthreads();
    const float mx = s_m;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + j * 256 + tid;
        if (i < n) {
            float e = expf(v[j] + (-mx));
            pr[i] = e;
            sum += e;
        }
    }
    sum = wg256_sum(sum, red);
    if (tid == 0) sc->seg_sum[blockIdx.x] = sum;
}

// p = e / sum; with top_p < 1 the level-0 mass histogram, else the draw's segment masses.
__global__ __launch_bounds__(256) void k_nuc_norm(float* pr, int n, float top_p, int nseg, NucleusScratch* sc) {
    __shared__ unsigned long long hist[256];
    __shared__ unsigned long long redu[4];
    __shared__ int redi[4];
    __shared__ float s_sum;
    __shared__ float segv[NUC_MAX_SEG];
    const int beg = blockIdx.x * NUC_SEG, tid = threadIdx.x;
    hist[tid] = 0ull;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) { int i = beg + j * 256 + tid; v[j] = i < n ? pr[i] : 0.0f; }
    load_segs(sc->seg_sum, nseg, segv);
    if (tid == 0) {
        float t = 0.0f;
        for (int h = 0; h < nseg; h++) t += segv[h];
        s_sum = t;
    }
    __syncthreads();
    const float sum = s_sum;
    unsigned long long mass = 0;
    int last = -1;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + j * 256 + tid;
        if (i < n) {
            float p = v[j] / sum;
            pr[i] = p;
            if (top_p < 1.0f) atomicAdd(&hist[__float_as_uint(p) >> 24], fix63(p));
            else {
                mass += fix63(p);
                if (p > 0.0f) last = i;
            }
        }
    }
    if (top_p < 1.0f) {
        __syncthreads();
        if (hist[tid]) atomicAdd(&sc->hist[0][tid], hist[tid]);
    } else {
        mass = wg256_sum(mass, redu);
        for (int o = 32; o > 0; o >>= 1) last = max(last, __shfl_xor(last, o));
        if ((tid & 63) == 0) redi[tid >> 6] = last;
        __syncthreads();
        if (tid == 0) {
            sc->seg_mass[blockIdx.x] = mass;
            sc->seg_last[blockIdx.x] = max(max(redi[0], redi[1]), max(redi[2], redi[3]));
        }
    }
}

// Radix level `level` (1..3) of the nucleus edge over the entries that match the levels before.
__global__ __launch_bounds__(256) void k_nuc_hist(const float* __restrict__ pr, int n, float top_p, int level,
                                                  NucleusScratch* sc) {
    __shared__ unsigned long long lh[3 * 256];
    __shared__ unsigned long long hist[256];
    __shared__ NucSel s_sel;
    const int beg = blockIdx.x * NUC_SEG, tid = threadIdx.x;
    hist[tid] = 0ull;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) { int i = beg + j * 256 + tid; v[j] = i < n ? pr[i] : 0.0f; }
    const NucSel sel = nuc_select(sc, level, fix63(top_p), lh, &s_sel);
    if (sel.all) return;  // uniform
    const int shift = 24 - 8 * level;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + j * 256 + tid;
        uint32_t key = __float_as_uint(v[j]);
        if (i < n && (key & sel.mask) == sel.prefix) atomicAdd(&hist[(key >> shift) & 255u], fix63(v[j]));
    }
    __syncthreads();
    if (hist[tid]) atomicAdd(&sc->hist[level][tid], hist[tid]);
}

// Entries equal to the edge tau in each segment.
__global__ __launch_bounds__(256) void k_nuc_ties(const float* __restrict__ pr, int n, float top_p,
                                                  NucleusScratch* sc) {
    __shared__ unsigned long long lh[4 * 256];
    __shared__ int red[4];
    __shared__ NucSel s_sel;
    const int beg = blockIdx.x * NUC_SEG, tid = threadIdx.x;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) { int i = beg + j * 256 + tid; v[j] = i < n ? pr[i] : 0.0f; }
    const NucSel sel = nuc_select(sc, 4, fix63(top_p), lh, &s_sel);
    int c = 0;
    if (!sel.all) {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            int i = beg + j * 256 + tid;
            c += (i < n && __float_as_uint(v[j]) == sel.prefix) ? 1 : 0;
        }
    }
    c = wg256_sum(c, red);
    if (tid == 0) sc->seg_tie[blockIdx.x] = c;
}

// Keep the nucleus (entries above tau, and the first m entries equal to it in index order),
// zero the rest, and the kept f32 sum per segment.
__global__ __launch_bounds__(256) void k_nuc_keep(float* pr, int n, float top_p, int nseg, NucleusScratch* sc) {
    __shared__ unsigned long long lh[4 * 256];
    __shared__ int cc[NUC_SEG / 64];
    __shared__ float red[4];
    __shared__ NucSel s_sel;
    __shared__ unsigned long long s_tie0, s_ntie;
    __shared__ int segt[NUC_MAX_SEG];
    const int beg = blockIdx.x * NUC_SEG, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // 64-entry chunks: wave w takes chunks 16w .. 16w+15 of the segment, lane l entry l of each
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + ((wave * 16 + j) << 6) + lane;
        v[j] = i < n ? pr[i] : 0.0f;
    }
    load_segs(sc->seg_tie, nseg, segt);
    if (tid == 0) {
        unsigned long long t0 = 0, nt = 0;
        for (int h = 0; h < nseg; h++) {
            unsigned long long c = (unsigned long long)segt[h];
            t0 += h < (int)blockIdx.x ? c : 0ull;
            nt += c;
        }
        s_tie0 = t0;
        s_ntie = nt;
    }
    const NucSel sel = nuc_select(sc, 4, fix63(top_p), lh, &s_sel);
    const uint32_t tau = sel.prefix;
    const bool all = sel.all != 0;
    unsigned long long tm[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + ((wave * 16 + j) << 6) + lane;
        tm[j] = __ballot(!all && i < n && __float_as_uint(v[j]) == tau);
        if (lane == 0) cc[wave * 16 + j] = (int)__popcll(tm[j]);
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int q = 0; q < NUC_SEG / 64; q++) { int c = cc[q]; cc[q] = run; run += c; }
    }
    __syncthreads();
    const unsigned long long ntie = s_ntie, tie0 = s_tie0;
    unsigned long long m = ntie;
    if (!all) {
        unsigned long long ft = fix63(__uint_as_float(tau)), need = fix63(top_p) - sel.above;
        if (ft > 0) {
            unsigned long long q = (need + ft - 1) / ft;
            m = q < ntie ? q : ntie;
        }
    }
    float kept = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + ((wave * 16 + j) << 6) + lane;
        if (i < n) {
            uint32_t key = __float_as_uint(v[j]);
            bool tie = (tm[j] >> lane) & 1ull;
            bool keep = all || key > tau ||
                        (tie && tie0 + (unsigned long long)cc[wave * 16 + j] + __popcll(tm[j] & lanes_below()) < m);
            if (!keep) pr[i] = 0.0f;
            else kept += v[j];
        }
    }
    kept = wg256_sum(kept, red);
    if (tid == 0) sc->seg_kept[blockIdx.x] = kept;
}

// Divide by the kept sum; the draw's segment masses and last nonzero entries.
__global__ __launch_bounds__(256) void k_nuc_renorm(float* pr, int n, int nseg, NucleusScratch* sc) {
    __shared__ unsigned long long redu[4];
    __shared__ int redi[4];
    __shared__ float s_kept;
    __shared__ float segv[NUC_MAX_SEG];
    const int beg = blockIdx.x * NUC_SEG, tid = threadIdx.x;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) { int i = beg + j * 256 + tid; v[j] = i < n ? pr[i] : 0.0f; }
    load_segs(sc->seg_kept, nseg, segv);
    if (tid == 0) {
        float t = 0.0f;
        for (int h = 0; h < nseg; h++) t += segv[h];
        s_kept = t;
    }
    __syncthreads();
    const float kept = s_kept;
    unsigned long long mass = 0;
    int last = -1;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int i = beg + j * 256 + tid;
        if (i < n) {
            float p = v[j];
            if (kept > 0.0f) {
                p = p / kept;
                pr[i] = p;
            }
            mass += fix63(p);
            if (p > 0.0f) last = i;
        }
    }
    mass = wg256_sum(mass, redu);
    for (int o = 32; o > 0; o >>= 1) last = max(last, __shfl_xor(last, o));
    if ((tid & 63) == 0) redi[tid >> 6] = last;
    __syncthreads();
    if (tid == 0) {
        sc->seg_mass[blockIdx.x] = mass;
        sc->seg_last[blockIdx.x] = max(max(redi[0], redi[1]), max(redi[2], redi[3]));
    }
}

// The draw: the segment whose running mass passes U, then the entry inside it (thread t walks
// entries 16t .. 16t+15 of the segment after an exclusive scan of the threads' masses); the last
// nonzero entry when rounding leaves the total below U. Leaves the mass histograms zeroed.
__global__ __launch_bounds__(256) void k_nuc_draw(const float* __restrict__ pr, int n, float u, int nseg,
                                                  NucleusScratch* sc, int* out_token) {
    __shared__ unsigned long long buf[256];
    __shared__ int s_seg, s_last, s_found;
    __shared__ unsigned long long s_base;
    __shared__ unsigned long long segm[NUC_MAX_SEG];
    __shared__ int segl[NUC_MAX_SEG];
    const int tid = threadIdx.x;
    const unsigned long long U = fix63(u);
    load_segs(sc->seg_mass, nseg, segm);
    load_segs(sc->seg_last, nseg, segl);
    if (tid == 0) {
        unsigned long long run = 0;
        int seg = -1, last = -1;
        for (int h = 0; h < nseg; h++) {
            unsigned long long mh = segm[h];
            if (seg < 0 && U < run + mh) { seg = h; s_base = run; }
            run += mh;
            last = max(last, segl[h]);
        }
        s_seg = seg;
        s_last = last;
        s_found = 0x7fffffff;
    }
    __syncthreads();
    const int seg = s_seg;
    if (seg >= 0) {
        const int b0 = seg * NUC_SEG + tid * 16;
        float v[16];
        unsigned long long part = 0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            v[j] = b0 + j < n ? pr[b0 + j] : 0.0f;
            part += fix63(v[j]);
        }
        unsigned long long total;
        unsigned long long run = s_base + block_excl_scan(part, buf, &total);
        if (U >= run && U < run + part) {
            for (int j = 0; j < 16; j++) {
                run += fix63(v[j]);
                if (U < run) { s_found = b0 + j; break; }
            }
        }
    }
    for (int j = tid; j < 4 * 256; j += blockDim.x) sc->hist[j >> 8][j & 255] = 0ull;
    __syncthreads();
    if (tid == 0) {
        int f = s_found;
        *out_token = f != 0x7fffffff ? f : (s_last >= 0 ? s_last : n - 1);
    }
}

hipError_t launch_sample_nucleus(float* x, int n, float inv_temp, float top_p, float u, float* pr, int* out_token,
                                 NucleusScratch* sc, hipStream_t st) {
    const int nseg = (n + NUC_SEG - 1) / NUC_SEG;
    if (nseg > NUC_MAX_SEG) return hipErrorInvalidValue;
    k_nuc_max<<<nseg, 256, 0, st>>>(x, n, inv_temp, sc);
    k_nuc_exp<<<nseg, 256, 0, st>>>(x, n, pr, nseg, sc);
    k_nuc_norm<<<nseg, 256, 0, st>>>(pr, n, top_p, nseg, sc);
    if (top_p < 1.0f) {
        for (int level = 1; level < 4; level++) k_nuc_hist<<<nseg, 256, 0, st>>>(pr, n, top_p, level, sc);
        k_nuc_ties<<<nseg, 256, 0, st>>>(pr, n, top_p, sc);
        k_nuc_keep<<<nseg, 256, 0, st>>>(pr, n, top_p, nseg, sc);
        k_nuc_renorm<<<nseg, 256, 0, st>>>(pr, n, nseg, sc);
    }
    k_nuc_draw<<<1, 256, 0, st>>>(pr, n, u, nseg, sc, out_token);
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
