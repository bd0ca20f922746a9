// api.hip — the C ABI of libfllm_hip.so (include/fllm.h): device context, model weights in
// GGUF block layout, per-request sequences (device KV cache + scratch + stream), the decode
// step (eager or replayed from a captured HIP graph) and the verification/microbenchmark
// entry points. No C++ exception crosses the ABI.
#include <math.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "attention.hpp"
#include "gemv.hpp"
#include "kernels.hpp"
#include "prefill.hpp"
#include "staging.hpp"

using namespace fllm;

// =====================================================================================
// errors
// =====================================================================================
static thread_local std::string g_err;

static int32_t fail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t _e = (expr);                                                                \
        if (_e != hipSuccess) return fail(FLLM_E_DEVICE, "%s: %s", #expr, hipGetErrorString(_e)); \
    } while (0)

#define NOT_NULL(p)                                                  \
    do {                                                             \
        if (!(p)) return fail(FLLM_E_NULL, "%s must not be null", #p); \
    } while (0)

extern "C" const char* fllm_last_error(void) { return g_err.c_str(); }
extern "C" int32_t fllm_version(void) { return 100; }

// =====================================================================================
// objects
// =====================================================================================
struct fllm_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int n_cu = 0;
    int64_t hbm = 0;
    Staging stage;
    uint8_t* scratch = nullptr;  // this device's address of the no-allocation scratch array
    hipError_t scratch_err = hipSuccess;  // why it could not be resolved, if so
};

// Scratch of fllm_dequantize_noalloc: the staged source blocks (kNoallocSrcBytes plus the slack the
// dequant kernel may read past them) and the dequantized floats (kNoallocElems). Each device holds
// its own copy for the life of the process. On the host the array's name is no device address: its
// per-device address comes from hipGetSymbolAddress at context creation (g_scratch_dev).
static const size_t kNoallocSrcBytes = FLLM_NOALLOC_MAX_BYTES;
static const size_t kNoallocElems = FLLM_NOALLOC_MAX_ELEMS;
static const size_t kNoallocSrcRegion = kNoallocSrcBytes + 256;
static __device__ __align__(256) uint8_t scratch[kNoallocSrcRegion + kNoallocElems * sizeof(float)];

static const int kMaxDevices = 64;
static uint8_t* g_scratch_dev[kMaxDevices];  // per device, set once with that device current
static std::mutex g_scratch_mu;
// held by fllm_dequantize_noalloc from its first copy to its stream sync, so calls from other
// threads or contexts on the same device take the array one after the other
static std::mutex g_scratch_use[kMaxDevices];

// Resolves this device's scratch address once (the device is current).
static hipError_t scratch_init(int device, uint8_t** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[device]) {
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_dev[device] = (uint8_t*)ptr;
    }
    *out = g_scratch_dev[device];
    return hipSuccess;
}

struct fllm_buf {
    fllm_ctx* ctx = nullptr;
    uint8_t* ptr = nullptr;
    uint64_t n = 0;
};

static const uint64_t kPad = 256;  // slack after every weight allocation for aligned over-reads

struct Tensor {
    uint8_t* ptr = nullptr;
    int layout = LAYOUT_ROWS;  // LAYOUT_TILES once finalize regroups it for the matrix-core GEMV
    int type = -1;
    int64_t rows = 0, cols = 0;
    uint64_t bytes = 0;
    int wexp = 0;  // batched prefill: 2^-wexp brings the largest |w| into [2^14, 2^15) (pf_wexp)
    bool present() const { return ptr != nullptr; }
    WMat mat() const { return WMat{ptr, type, rows, cols}; }
};

struct Layer {
    Tensor q, k, v, o, gate, up, down;
    float *attn_norm = nullptr, *ffn_norm = nullptr, *post_attn = nullptr, *post_ffn = nullptr;
    float *bq = nullptr, *bk = nullptr, *bv = nullptr;
};

struct fllm_model {
    fllm_ctx* ctx = nullptr;
    fllm_model_desc d{};
    int qdim = 0, kvdim = 0;
    Tensor tok_embd, output;
    bool output_tied = false;
    float* out_norm = nullptr;
    std::vector<Layer> layers;
    std::vector<float> inv_freq;
    bool finalized = false;
    uint64_t layer_bytes = 0, head_bytes = 0;
    // LlamaWeights.Dispose (LlamaWeights.cs:93-107): fllm_model_destroy marks the model disposed;
    // its device memory is released when the last sequence created from it is destroyed
    int n_seqs = 0;
    bool disposed = false;
};

struct ProfAgg {
    int64_t launches = 0;
    double ms = 0, bytes = 0;
};

struct fllm_seq {
    fllm_model* m = nullptr;
    hipStream_t st = nullptr;
    int max_seq = 0;
    int cur_len = 0;
    int next_layer = 0;           // KvCache._nextLayerToAppend (KvCache.cs:69-96)
    bool was_evicted = false;     // KvCache.WasEvicted (KvCache.cs:56)
    int nsplit = 1;               // chunks of the generic attention kernel
    int attn_nc = 1;              // chunks per kv head of the fast attention kernel
    size_t attn_lds = 0;
    bool attn_fast = false;
    // the fast attention merges its chunks inside its own launch (fllm_seq_set_attention_merge;
    // by default when one wave per query head of a group and one load pass per head suffice, i.e.
    // at most 4 query heads per kv head and 32 chunks); attn_cnt: its per-kv-head counters (zero
    // between launches)
    bool attn_merge_in = false;
    unsigned* attn_cnt = nullptr;
    bool fused = false;           // layers run as fused GEMV launches
    bool head_fused = false;
    bool argmax_valid = false;    // params->argmax holds the argmax of the current logits
    float *kc = nullptr, *vc = nullptr;
    float2* rope = nullptr;
    StepParams* params = nullptr;
    float *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr;
    float* x2 = nullptr;  // second residual buffer of the fused Gemma-2 post-norms
    float *g = nullptr, *u = nullptr, *h = nullptr, *tmp = nullptr, *logits = nullptr;
    float *part_o = nullptr, *part_ml = nullptr;
    unsigned long long* head_keys = nullptr;  // per-workgroup argmax keys of the fused LM head
    // activation tables written by matrix-core epilogues for the next matrix-core launch: of the
    // residual stream times the next RMSNorm weight (with per-16-row sums of squares), and of the
    // FFN activation
    float *tab_x = nullptr, *ssq_x = nullptr, *tab_h = nullptr;
    float* tab_att = nullptr;  // table of the attention output, written by the attention merge
    int* tokens_out = nullptr;
    int *topk_ids = nullptr, *topk_count = nullptr;
    float* topk_vals = nullptr;
    int topk_cap = 0;
    float* probs = nullptr;       // distribution left by the nucleus sampler (vocab floats)
    int* samp_token = nullptr;    // its drawn token
    // pinned host block the samplers' results come back through (the count, the first kPinCand
    // candidate ids and values; a drawn token), so each call is one DMA round trip
    int32_t* pin = nullptr;
    int* pen_counts = nullptr;    // repetition-penalty counters (vocab ints, zero between calls)
    int* pen_ids = nullptr;       // the penalised ids of the last call (device copy)
    TopkScratch* topk_sc = nullptr;  // grid top-k: threshold, segment counts, candidates
    NucleusScratch* nuc_sc = nullptr;  // grid nucleus sampler: edge histograms, segment results
    int pen_cap = 0;
    float* hidden_dbg = nullptr;
    bool debug = false;
    bool use_graph = true;
    bool graph_valid = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    // profiling
    bool profile = false;
    std::vector<hipEvent_t> ev;
    std::vector<std::pair<std::string, double>> pending;  // name, bytes per pending launch
    std::map<std::string, ProfAgg> agg;
    std::vector<std::string> agg_order;
    std::vector<std::string> launch_names;  // every profiled launch in order (bounded)
    std::vector<void*> allocs;
    // batched prefill: passes of up to pf_chunk tokens; scratch for pf_cap rows, sized by the
    // prompts seen (a multiple of 256 up to min(max_seq, pf_chunk)) and grown when a longer one comes
    int pf_chunk = 4096, pf_cap = 0, pf_ldx = 0;
    std::vector<void*> pf_allocs;
    float *pf_x = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_att = nullptr, *pf_gu = nullptr, *pf_tmp = nullptr;
    float* pf_part = nullptr;  // K-split partial products of the short GEMM launches
    size_t pf_part_cap = 0;
    _Float16* pf_xh = nullptr;  // fp16 hi / lo planes of the current GEMM input
    float* pf_xs = nullptr;     // their per-row scales
    _Float16* pf_kvh = nullptr;  // head_dim 256: fp16 planes of a layer's cached K / V (every position)
    int* pf_kvs = nullptr;
    int pf_kvblk = 0;
    int* pf_tok = nullptr;
};

// =====================================================================================
// context
// =====================================================================================
extern "C" int32_t fllm_ctx_create(int32_t device, fllm_ctx** out) {
    NOT_NULL(out);
    *out = nullptr;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(FLLM_E_ARG_RANGE, "device %d outside [0,%d)", device, n);
    if (device >= kMaxDevices) return fail(FLLM_E_NOT_SUPPORTED, "device %d: at most %d devices", device, kMaxDevices);
    HIP_TRY(hipSetDevice(device));
    fllm_ctx* c = new fllm_ctx();
    c->device = device;
    // only fllm_dequantize_noalloc needs the scratch address: a failure is kept for it to report
    c->scratch_err = scratch_init(device, &c->scratch);
    if (c->scratch_err != hipSuccess) (void)hipGetLastError();
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) { delete c; return fail(FLLM_E_DEVICE, "hipStreamCreate: %s", hipGetErrorString(e)); }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
        c->n_cu = prop.multiProcessorCount;
        c->hbm = (int64_t)prop.totalGlobalMem;
    }
    *out = c;
    return FLLM_OK;
}

extern "C" int32_t fllm_ctx_destroy(fllm_ctx* ctx) {
    if (!ctx) return FLLM_OK;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    staging_free(ctx->stage);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return FLLM_OK;
}

extern "C" int32_t fllm_ctx_sync(fllm_ctx* ctx) {
    NOT_NULL(ctx);
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return FLLM_OK;
}

extern "C" int32_t fllm_ctx_device_info(fllm_ctx* ctx, int32_t* n_cu, int64_t* hbm_bytes) {
    NOT_NULL(ctx);
    if (n_cu) *n_cu = ctx->n_cu;
    if (hbm_bytes) *hbm_bytes = ctx->hbm;
    return FLLM_OK;
}

// =====================================================================================
// element counts and dequantization (Dequantizer.cs:466-504)
// =====================================================================================
extern "C" int32_t fllm_element_count(int32_t type, int64_t nbytes, int64_t* out) {
    NOT_NULL(out);
    if (!type_supported(type)) return fail(FLLM_E_NOT_SUPPORTED, "Tensor type %d is not supported for dequantization.", type);
    TypeInfo ti = type_info(type);
    *out = nbytes / ti.block_bytes * ti.block_elems;
    return FLLM_OK;
}

extern "C" int32_t fllm_dequantize(fllm_ctx* ctx, int32_t type, const void* src, uint64_t nbytes, float* dst, int64_t n) {
    NOT_NULL(ctx);
    if (!type_supported(type)) return fail(FLLM_E_NOT_SUPPORTED, "Tensor type %d is not supported for dequantization.", type);
    TypeInfo ti = type_info(type);
    if (nbytes % (uint64_t)ti.block_bytes != 0)
        return fail(FLLM_E_ARG, "Source length must be a multiple of %d for type %d.", ti.block_bytes, type);
    int64_t elems = (int64_t)(nbytes / ti.block_bytes) * ti.block_elems;
    if (n < elems) return fail(FLLM_E_ARG, "Destination must hold at least %lld floats.", (long long)elems);
    if (elems == 0) return FLLM_OK;
    NOT_NULL(src);
    NOT_NULL(dst);
    HIP_TRY(hipSetDevice(ctx->device));
    uint8_t* dsrc = nullptr;
    float* ddst = nullptr;
    HIP_TRY(hipMalloc(&dsrc, nbytes + kPad));
    hipError_t e = hipMalloc(&ddst, sizeof(float) * (size_t)elems);
    if (e != hipSuccess) { hipFree(dsrc); return fail(FLLM_E_OOM, "hipMalloc: %s", hipGetErrorString(e)); }
    e = hipMemcpyAsync(dsrc, src, nbytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = launch_dequant(type, dsrc, elems, ddst, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dst, ddst, sizeof(float) * (size_t)elems, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    hipFree(dsrc);
    hipFree(ddst);
    if (e != hipSuccess) return fail(FLLM_E_DEVICE, "dequantize: %s", hipGetErrorString(e));
    return FLLM_OK;
}

// fllm_dequantize without allocating: the source blocks and the floats go through this device's
// scratch array (its address resolved at context creation), so nothing is allocated or freed.
// The call is synchronous and holds the device's lock on the array for its whole use, so calls
// from several threads or contexts on one device are serialized rather than racing.
extern "C" int32_t fllm_dequantize_noalloc(fllm_ctx* ctx, int32_t type, const void* src, uint64_t nbytes, float* dst,
                                           int64_t n) {
    NOT_NULL(ctx);
    if (!type_supported(type)) return fail(FLLM_E_NOT_SUPPORTED, "Tensor type %d is not supported for dequantization.", type);
    TypeInfo ti = type_info(type);
    if (nbytes % (uint64_t)ti.block_bytes != 0)
        return fail(FLLM_E_ARG, "Source length must be a multiple of %d for type %d.", ti.block_bytes, type);
    int64_t elems = (int64_t)(nbytes / ti.block_bytes) * ti.block_elems;
    if (n < elems) return fail(FLLM_E_ARG, "Destination must hold at least %lld floats.", (long long)elems);
    if (nbytes > kNoallocSrcBytes || elems > (int64_t)kNoallocElems)
        return fail(FLLM_E_ARG,
                    "fllm_dequantize_noalloc takes at most %llu source bytes and %llu elements (got %llu bytes, %lld "
                    "elements); use fllm_dequantize",
                    (unsigned long long)kNoallocSrcBytes, (unsigned long long)kNoallocElems,
                    (unsigned long long)nbytes, (long long)elems);
    if (elems == 0) return FLLM_OK;
    NOT_NULL(src);
    NOT_NULL(dst);
    if (!ctx->scratch)
        return fail(FLLM_E_DEVICE, "hipGetSymbolAddress(scratch) failed at context creation: %s",
                    hipGetErrorString(ctx->scratch_err));
    HIP_TRY(hipSetDevice(ctx->device));
    std::lock_guard<std::mutex> use(g_scratch_use[ctx->device]);
    uint8_t* dsrc = ctx->scratch;
    float* ddst = (float*)(ctx->scratch + kNoallocSrcRegion);
    hipError_t e = hipMemcpyAsync(dsrc, src, nbytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = launch_dequant(type, dsrc, elems, ddst, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dst, ddst, sizeof(float) * (size_t)elems, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return fail(FLLM_E_DEVICE, "dequantize_noalloc: %s", hipGetErrorString(e));
    return FLLM_OK;
}

// =====================================================================================
// buffers and the standalone GEMV
// =====================================================================================
extern "C" int32_t fllm_buf_create(fllm_ctx* ctx, uint64_t nbytes, fllm_buf** out) {
    NOT_NULL(ctx);
    NOT_NULL(out);
    *out = nullptr;
    HIP_TRY(hipSetDevice(ctx->device));
    uint8_t* p = nullptr;
    hipError_t e = hipMalloc(&p, nbytes + kPad);
    if (e != hipSuccess) return fail(FLLM_E_OOM, "hipMalloc(%llu): %s", (unsigned long long)nbytes, hipGetErrorString(e));
    e = hipMemsetAsync(p + nbytes, 0, kPad, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { hipFree(p); return fail(FLLM_E_DEVICE, "hipMemset: %s", hipGetErrorString(e)); }
    fllm_buf* b = new fllm_buf();
    b->ctx = ctx;
    b->ptr = p;
    b->n = nbytes;
    *out = b;
    return FLLM_OK;
}

extern "C" int32_t fllm_buf_destroy(fllm_buf* b) {
    if (!b) return FLLM_OK;
    hipSetDevice(b->ctx->device);
    hipStreamSynchronize(b->ctx->stream);
    hipFree(b->ptr);
    delete b;
    return FLLM_OK;
}

extern "C" int32_t fllm_buf_write(fllm_buf* b, uint64_t offset, const void* src, uint64_t n) {
    NOT_NULL(b);
    if (offset > b->n || n > b->n - offset) return fail(FLLM_E_ARG, "write [%llu,+%llu) outside buffer of %llu bytes",
                                                        (unsigned long long)offset, (unsigned long long)n, (unsigned long long)b->n);
    if (n == 0) return FLLM_OK;
    NOT_NULL(src);
    HIP_TRY(hipSetDevice(b->ctx->device));
    HIP_TRY(hipMemcpyAsync(b->ptr + offset, src, n, hipMemcpyHostToDevice, b->ctx->stream));
    HIP_TRY(hipStreamSynchronize(b->ctx->stream));
    return FLLM_OK;
}

extern "C" int32_t fllm_buf_read(fllm_buf* b, uint64_t offset, void* dst, uint64_t n) {
    NOT_NULL(b);
    if (offset > b->n || n > b->n - offset) return fail(FLLM_E_ARG, "read [%llu,+%llu) outside buffer of %llu bytes",
                                                        (unsigned long long)offset, (unsigned long long)n, (unsigned long long)b->n);
    if (n == 0) return FLLM_OK;
    NOT_NULL(dst);
    HIP_TRY(hipSetDevice(b->ctx->device));
    HIP_TRY(hipMemcpyAsync(dst, b->ptr + offset, n, hipMemcpyDeviceToHost, b->ctx->stream));
    HIP_TRY(hipStreamSynchronize(b->ctx->stream));
    return FLLM_OK;
}

static int32_t check_gemv_args(int32_t type, fllm_buf* w, uint64_t w_offset, int64_t rows, int64_t cols, fllm_buf* x,
                               fllm_buf* y) {
    NOT_NULL(w);
    NOT_NULL(x);
    NOT_NULL(y);
    if (!type_supported(type)) return fail(FLLM_E_NOT_SUPPORTED, "Tensor type %d is not supported.", type);
    if (rows <= 0 || cols <= 0) return fail(FLLM_E_ARG, "rows and cols must be positive");
    TypeInfo ti = type_info(type);
    if ((rows * cols) % ti.block_elems != 0) return fail(FLLM_E_ARG, "rows*cols must be a whole number of blocks");
    if (w_offset % 16 != 0) return fail(FLLM_E_ARG, "weight offset must be 16-byte aligned");
    uint64_t wb = type_bytes(type, rows * cols);
    if (w_offset > w->n || wb > w->n - w_offset) return fail(FLLM_E_ARG, "weight buffer too small");
    if ((uint64_t)cols * 4 > x->n) return fail(FLLM_E_ARG, "x buffer too small");
    if ((uint64_t)rows * 4 > y->n) return fail(FLLM_E_ARG, "y buffer too small");
    return FLLM_OK;
}

extern "C" int32_t fllm_gemv(fllm_ctx* ctx, int32_t type, fllm_buf* w, uint64_t w_offset, int64_t rows, int64_t cols,
                             fllm_buf* x, fllm_buf* y) {
    NOT_NULL(ctx);
    int32_t rc = check_gemv_args(type, w, w_offset, rows, cols, x, y);
    if (rc) return rc;
    HIP_TRY(hipSetDevice(ctx->device));
    WMat m{w->ptr + w_offset, type, rows, cols};
    HIP_TRY(launch_gemv(m, (const float*)x->ptr, (float*)y->ptr, nullptr, ctx->n_cu, ctx->stream));
    return FLLM_OK;
}

extern "C" int32_t fllm_gemv_pack(fllm_ctx* ctx, int32_t type, fllm_buf* src, uint64_t src_offset, int64_t rows,
                                  int64_t cols, fllm_buf* dst) {
    NOT_NULL(ctx);
    NOT_NULL(src);
    NOT_NULL(dst);
    if (!type_supported(type)) return fail(FLLM_E_NOT_SUPPORTED, "Tensor type %d is not supported.", type);
    if (rows <= 0 || cols <= 0) return fail(FLLM_E_ARG, "rows and cols must be positive");
    if (!gemv_tiles_shape_ok(type, rows, cols))
        return fail(FLLM_E_NOT_SUPPORTED, "no tile layout for type %d, %lld x %lld", type, (long long)rows, (long long)cols);
    if (src_offset % 16 != 0) return fail(FLLM_E_ARG, "source offset must be 16-byte aligned");
    const uint64_t nb = type_bytes(type, rows * cols);
    if (src_offset > src->n || nb > src->n - src_offset) return fail(FLLM_E_ARG, "source buffer too small");
    if (nb > dst->n) return fail(FLLM_E_ARG, "destination buffer too small");
    if (dst == src) return fail(FLLM_E_ARG, "the regrouping is not in place");
    HIP_TRY(hipSetDevice(ctx->device));
    HIP_TRY(launch_pack_tiles(type, src->ptr + src_offset, dst->ptr, rows, cols, ctx->stream));
    return FLLM_OK;
}

static int32_t check_layout(int32_t type, int64_t rows, int64_t cols, uint64_t w_offset, int32_t layout) {
    if (layout == FLLM_LAYOUT_GGUF) return FLLM_OK;
    if (layout != FLLM_LAYOUT_TILES) return fail(FLLM_E_ARG_RANGE, "unknown layout %d", layout);
    if (w_offset != 0) return fail(FLLM_E_ARG, "a tile-interleaved matrix starts at offset 0");
    if (!gemv_tiles_shape_ok(type, rows, cols))
        return fail(FLLM_E_NOT_SUPPORTED, "no tile layout for type %d, %lld x %lld", type, (long long)rows, (long long)cols);
    return FLLM_OK;
}

extern "C" int32_t fllm_gemv_ex(fllm_ctx* ctx, int32_t type, fllm_buf* w, uint64_t w_offset, int64_t rows, int64_t cols,
                                fllm_buf* x, fllm_buf* y, int32_t layout) {
    NOT_NULL(ctx);
    int32_t rc = check_gemv_args(type, w, w_offset, rows, cols, x, y);
    if (rc == FLLM_OK) rc = check_layout(type, rows, cols, w_offset, layout);
    if (rc) return rc;
    HIP_TRY(hipSetDevice(ctx->device));
    WMat m{w->ptr + w_offset, type, rows, cols};
    if (layout == FLLM_LAYOUT_TILES) HIP_TRY(launch_gemv_tiles(m, (const float*)x->ptr, (float*)y->ptr, ctx->n_cu, ctx->stream));
    else HIP_TRY(launch_gemv(m, (const float*)x->ptr, (float*)y->ptr, nullptr, ctx->n_cu, ctx->stream));
    return FLLM_OK;
}

extern "C" int32_t fllm_gemv_time_ex(fllm_ctx* ctx, int32_t type, fllm_buf* const* w, int32_t n_w, int64_t rows,
                                     int64_t cols, fllm_buf* x, fllm_buf* y, int32_t iters, int32_t layout,
                                     double* avg_us) {
    NOT_NULL(ctx);
    NOT_NULL(w);
    NOT_NULL(avg_us);
    if (n_w <= 0 || iters <= 0) return fail(FLLM_E_ARG, "n_w and iters must be positive");
    for (int i = 0; i < n_w; i++) {
        int32_t rc = check_gemv_args(type, w[i], 0, rows, cols, x, y);
        if (rc == FLLM_OK) rc = check_layout(type, rows, cols, 0, layout);
        if (rc) return rc;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t err = hipEventCreate(&e0);
    if (err == hipSuccess) err = hipEventCreate(&e1);
    if (err == hipSuccess) err = hipEventRecord(e0, ctx->stream);
    for (int i = 0; i < iters && err == hipSuccess; i++) {
        WMat m{w[i % n_w]->ptr, type, rows, cols};
        err = layout == FLLM_LAYOUT_TILES ? launch_gemv_tiles(m, (const float*)x->ptr, (float*)y->ptr, ctx->n_cu, ctx->stream)
                                          : launch_gemv(m, (const float*)x->ptr, (float*)y->ptr, nullptr, ctx->n_cu, ctx->stream);
    }
    if (err == hipSuccess) err = hipEventRecord(e1, ctx->stream);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (err != hipSuccess) return fail(FLLM_E_DEVICE, "gemv_time: %s", hipGetErrorString(err));
    *avg_us = ms * 1000.0 / iters;
    return FLLM_OK;
}

extern "C" int32_t fllm_gemv_time(fllm_ctx* ctx, int32_t type, fllm_buf* const* w, int32_t n_w, int64_t rows,
                                  int64_t cols, fllm_buf* x, fllm_buf* y, int32_t iters, double* avg_us) {
    NOT_NULL(ctx);
    NOT_NULL(w);
    NOT_NULL(avg_us);
    if (n_w <= 0 || iters <= 0) return fail(FLLM_E_ARG, "n_w and iters must be positive");
    for (int i = 0; i < n_w; i++) {
        int32_t rc = check_gemv_args(type, w[i], 0, rows, cols, x, y);
        if (rc) return rc;
    }
    HIP_TRY(hipSetDevice(ctx->device));
    std::vector<hipEvent_t> ev(2 * (size_t)iters);
    for (auto& e : ev) HIP_TRY(hipEventCreate(&e));
    hipError_t err = hipSuccess;
    for (int i = 0; i < iters && err == hipSuccess; i++) {
        WMat m{w[i % n_w]->ptr, type, rows, cols};
        err = hipEventRecord(ev[2 * i], ctx->stream);
        if (err == hipSuccess) err = launch_gemv(m, (const float*)x->ptr, (float*)y->ptr, nullptr, ctx->n_cu, ctx->stream);
        if (err == hipSuccess) err = hipEventRecord(ev[2 * i + 1], ctx->stream);
    }
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    double tot = 0;
    for (int i = 0; i < iters && err == hipSuccess; i++) {
        float ms = 0;
        err = hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]);
        tot += ms;
    }
    for (auto& e : ev) hipEventDestroy(e);
    if (err != hipSuccess) return fail(FLLM_E_DEVICE, "gemv_time: %s", hipGetErrorString(err));
    *avg_us = tot * 1000.0 / iters;
    return FLLM_OK;
}

// =====================================================================================
// model
// =====================================================================================
extern "C" int32_t fllm_model_create(fllm_ctx* ctx, const fllm_model_desc* desc, fllm_model** out) {
    NOT_NULL(ctx);
    NOT_NULL(desc);
    NOT_NULL(out);
    *out = nullptr;
    const fllm_model_desc& d = *desc;
    if (d.arch < FLLM_ARCH_LLAMA || d.arch > FLLM_ARCH_GEMMA2)
        return fail(FLLM_E_NOT_SUPPORTED, "Architecture %d is not supported.", d.arch);
    // LlamaForwardPass.cs:48-52 head configuration check
    if (d.n_kv_heads <= 0 || d.n_heads <= 0 || d.n_kv_heads > d.n_heads || d.n_heads % d.n_kv_heads != 0)
        return fail(FLLM_E_ARG_RANGE, "Invalid attention head configuration: NumHeads=%d, NumKvHeads=%d.", d.n_heads, d.n_kv_heads);
    if (d.n_layers <= 0 || d.hidden <= 0 || d.ffn <= 0 || d.vocab <= 0 || d.head_dim <= 0 || d.max_ctx <= 0)
        return fail(FLLM_E_ARG, "model dimensions must be positive");
    if (d.head_dim % 2 != 0) return fail(FLLM_E_ARG, "headDim must be even.");
    if (d.head_dim % 4 != 0 || d.head_dim > 256) return fail(FLLM_E_NOT_SUPPORTED, "head_dim %d not supported (multiple of 4, <= 256)", d.head_dim);
    fllm_model* m = new fllm_model();
    m->ctx = ctx;
    m->d = d;
    m->qdim = d.n_heads * d.head_dim;
    m->kvdim = d.n_kv_heads * d.head_dim;
    m->layers.resize((size_t)d.n_layers);
    *out = m;
    return FLLM_OK;
}

static void free_tensor(Tensor& t) {
    if (t.ptr) hipFree(t.ptr);
    t = Tensor();
}

static void model_free(fllm_model* m) {
    hipSetDevice(m->ctx->device);
    hipDeviceSynchronize();
    free_tensor(m->tok_embd);
    if (!m->output_tied) free_tensor(m->output);
    if (m->out_norm) hipFree(m->out_norm);
    for (auto& L : m->layers) {
        free_tensor(L.q); free_tensor(L.k); free_tensor(L.v); free_tensor(L.o);
        free_tensor(L.gate); free_tensor(L.up); free_tensor(L.down);
        float* vecs[] = {L.attn_norm, L.ffn_norm, L.post_attn, L.post_ffn, L.bq, L.bk, L.bv};
        for (float* p : vecs)
            if (p) hipFree(p);
    }
    delete m;
}

// ObjectDisposedException.ThrowIf(_disposed, this) of LlamaWeights.ThrowIfDisposed
// (LlamaWeights.cs:138-139), checked by Forward before anything runs (LlamaForwardPass.cs:87).
#define NOT_DISPOSED(m)                                                                                \
    do {                                                                                               \
        if ((m)->disposed) return fail(FLLM_E_DISPOSED, "Cannot access a disposed object. Object name: 'LlamaWeights'."); \
    } while (0)

extern "C" int32_t fllm_model_destroy(fllm_model* m) {
    if (!m) return FLLM_OK;
    if (m->disposed) return FLLM_OK;  // Dispose is idempotent (LlamaWeights.cs:95-98)
    m->disposed = true;
    if (m->n_seqs == 0) model_free(m);
    return FLLM_OK;
}

// Expected (rows, cols) of a slot, as LoadTensor's expectedElements (GgufModelLoader.cs:338-366).
static bool slot_shape(const fllm_model* m, int slot, int64_t& rows, int64_t& cols, bool& vec) {
    const fllm_model_desc& d = m->d;
    vec = false;
    switch (slot) {
        case FLLM_SLOT_TOKEN_EMBD: case FLLM_SLOT_OUTPUT: rows = d.vocab; cols = d.hidden; return true;
        case FLLM_SLOT_ATTN_Q: rows = m->qdim; cols = d.hidden; return true;
        case FLLM_SLOT_ATTN_K: case FLLM_SLOT_ATTN_V: rows = m->kvdim; cols = d.hidden; return true;
        case FLLM_SLOT_ATTN_OUTPUT: rows = d.hidden; cols = m->qdim; return true;
        case FLLM_SLOT_FFN_GATE: case FLLM_SLOT_FFN_UP: rows = d.ffn; cols = d.hidden; return true;
        case FLLM_SLOT_FFN_DOWN: rows = d.hidden; cols = d.ffn; return true;
        case FLLM_SLOT_OUTPUT_NORM: case FLLM_SLOT_ATTN_NORM: case FLLM_SLOT_POST_ATTN_NORM:
        case FLLM_SLOT_FFN_NORM: case FLLM_SLOT_POST_FFN_NORM:
            rows = 1; cols = d.hidden; vec = true; return true;
        case FLLM_SLOT_ATTN_Q_BIAS: rows = 1; cols = m->qdim; vec = true; return true;
        case FLLM_SLOT_ATTN_K_BIAS: case FLLM_SLOT_ATTN_V_BIAS: rows = 1; cols = m->kvdim; vec = true; return true;
        default: return false;
    }
}

extern "C" int32_t fllm_model_upload(fllm_model* m, int32_t slot, int32_t layer, int32_t type, const void* bytes,
                                     uint64_t nbytes) {
    NOT_NULL(m);
    NOT_DISPOSED(m);
    if (m->finalized) return fail(FLLM_E_INVALID_OP, "model already finalized");
    int64_t rows, cols;
    bool vec;
    if (!slot_shape(m, slot, rows, cols, vec)) return fail(FLLM_E_ARG_RANGE, "unknown tensor slot %d", slot);
    bool per_layer = slot >= 10;
    if (per_layer && (layer < 0 || layer >= m->d.n_layers))
        return fail(FLLM_E_ARG_RANGE, "Layer index must be in [0, %d].", m->d.n_layers - 1);
    if (!type_supported(type)) return fail(FLLM_E_NOT_SUPPORTED, "Tensor type %d is not supported for dequantization.", type);
    TypeInfo ti = type_info(type);
    int64_t n = rows * cols;
    if (n % ti.block_elems != 0) return fail(FLLM_E_ARG, "tensor of %lld elements is not a whole number of type-%d blocks", (long long)n, type);
    uint64_t want = type_bytes(type, n);
    if (nbytes != want)
        return fail(FLLM_E_ARG, "tensor slot %d: %llu bytes given, %llu expected for %lld elements of type %d", slot,
                    (unsigned long long)nbytes, (unsigned long long)want, (long long)n, type);
    NOT_NULL(bytes);
    hipStream_t st = m->ctx->stream;
    HIP_TRY(hipSetDevice(m->ctx->device));
    uint8_t* dev = nullptr;
    hipError_t e = hipMalloc(&dev, nbytes + kPad);
    if (e != hipSuccess) return fail(FLLM_E_OOM, "hipMalloc(%llu): %s", (unsigned long long)nbytes, hipGetErrorString(e));
    // every tensor through the pinned staging pair: the host reads the caller's bytes (a mapped
    // file, say), no device copy does
    e = staged_upload(m->ctx->stage, st, dev, (const uint8_t*)bytes, nbytes);
    if (e == hipSuccess) e = hipMemsetAsync(dev + nbytes, 0, kPad, st);
    if (e != hipSuccess) {
        hipStreamSynchronize(st);  // copies already enqueued into dev
        hipFree(dev);
        return fail(FLLM_E_DEVICE, "upload: %s", hipGetErrorString(e));
    }
    if (vec) {
        // norms and biases: dequantize once to F32 on the device
        float* f = nullptr;
        e = hipMalloc(&f, sizeof(float) * (size_t)n);
        if (e == hipSuccess) e = launch_dequant(type, dev, n, f, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        hipFree(dev);
        if (e != hipSuccess) { if (f) hipFree(f); return fail(FLLM_E_DEVICE, "upload: %s", hipGetErrorString(e)); }
        float** where = nullptr;
        if (slot == FLLM_SLOT_OUTPUT_NORM) where = &m->out_norm;
        else {
            Layer& L = m->layers[(size_t)layer];
            switch (slot) {
                case FLLM_SLOT_ATTN_NORM: where = &L.attn_norm; break;
                case FLLM_SLOT_FFN_NORM: where = &L.ffn_norm; break;
                case FLLM_SLOT_POST_ATTN_NORM: where = &L.post_attn; break;
                case FLLM_SLOT_POST_FFN_NORM: where = &L.post_ffn; break;
                case FLLM_SLOT_ATTN_Q_BIAS: where = &L.bq; break;
                case FLLM_SLOT_ATTN_K_BIAS: where = &L.bk; break;
                default: where = &L.bv; break;
            }
        }
        if (*where) hipFree(*where);
        *where = f;
        return FLLM_OK;
    }
    e = hipStreamSynchronize(st);
    if (e != hipSuccess) { hipFree(dev); return fail(FLLM_E_DEVICE, "upload: %s", hipGetErrorString(e)); }
    Tensor t;
    t.ptr = dev; t.type = type; t.rows = rows; t.cols = cols; t.bytes = nbytes;
    Tensor* where = nullptr;
    if (slot == FLLM_SLOT_TOKEN_EMBD) where = &m->tok_embd;
    else if (slot == FLLM_SLOT_OUTPUT) where = &m->output;
    else {
        Layer& L = m->layers[(size_t)layer];
        switch (slot) {
            case FLLM_SLOT_ATTN_Q: where = &L.q; break;
            case FLLM_SLOT_ATTN_K: where = &L.k; break;
            case FLLM_SLOT_ATTN_V: where = &L.v; break;
            case FLLM_SLOT_ATTN_OUTPUT: where = &L.o; break;
            case FLLM_SLOT_FFN_GATE: where = &L.gate; break;
            case FLLM_SLOT_FFN_UP: where = &L.up; break;
            default: where = &L.down; break;
        }
    }
    free_tensor(*where);
    *where = t;
    return FLLM_OK;
}

// true when the decode launch over these matrices (GLU: gate, up) runs the matrix-core variant with
// them regrouped into LAYOUT_TILES
static bool tiles_launch_ok(const Tensor* const* t, int n, int glu) {
    GemvArgs a{};
    a.nseg = n;
    a.glu = glu;
    for (int i = 0; i < n; i++) {
        if (!gemv_tiles_shape_ok(t[i]->type, t[i]->rows, t[i]->cols) || t[i]->cols != t[0]->cols) return false;
        a.seg[i].w = t[i]->ptr; a.seg[i].layout = LAYOUT_TILES; a.seg[i].type = t[i]->type; a.seg[i].rows = (int)t[i]->rows;
    }
    return gemv_uses_mfma(a, t[0]->cols);
}

// regroup one matrix into LAYOUT_TILES on the device (same bytes, new allocation)
static hipError_t pack_tiles(fllm_model* m, Tensor& t) {
    if (t.layout == LAYOUT_TILES) return hipSuccess;
    uint8_t* dev = nullptr;
    hipError_t e = hipMalloc(&dev, t.bytes + kPad);
    if (e != hipSuccess) return e;
    hipStream_t st = m->ctx->stream;
    e = launch_pack_tiles(t.type, t.ptr, dev, t.rows, t.cols, st);
    if (e == hipSuccess) e = hipMemsetAsync(dev + t.bytes, 0, kPad, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) { hipFree(dev); return e; }
    hipFree(t.ptr);
    t.ptr = dev;
    t.layout = LAYOUT_TILES;
    return hipSuccess;
}

extern "C" int32_t fllm_model_finalize(fllm_model* m) {
    NOT_NULL(m);
    NOT_DISPOSED(m);
    if (m->finalized) return FLLM_OK;
    const fllm_model_desc& d = m->d;
    if (!m->tok_embd.present()) return fail(FLLM_E_INVALID_OP, "Required tensor 'token_embd.weight' not found in GGUF file.");
    if (!m->out_norm) return fail(FLLM_E_INVALID_OP, "Required tensor 'output_norm.weight' not found in GGUF file.");
    for (int l = 0; l < d.n_layers; l++) {
        Layer& L = m->layers[(size_t)l];
        struct { bool ok; const char* name; } req[] = {
            {L.attn_norm != nullptr, "attn_norm.weight"}, {L.q.present(), "attn_q.weight"},
            {L.k.present(), "attn_k.weight"}, {L.v.present(), "attn_v.weight"},
            {L.o.present(), "attn_output.weight"}, {L.ffn_norm != nullptr, "ffn_norm.weight"},
            {L.gate.present(), "ffn_gate.weight"}, {L.up.present(), "ffn_up.weight"},
            {L.down.present(), "ffn_down.weight"},
            {d.arch != FLLM_ARCH_QWEN2 || L.bq, "attn_q.bias"}, {d.arch != FLLM_ARCH_QWEN2 || L.bk, "attn_k.bias"},
            {d.arch != FLLM_ARCH_QWEN2 || L.bv, "attn_v.bias"},
            {d.arch != FLLM_ARCH_GEMMA2 || L.post_attn, "post_attn_norm.weight"},
            {d.arch != FLLM_ARCH_GEMMA2 || L.post_ffn, "post_ffn_norm.weight"},
        };
        for (auto& r : req)
            if (!r.ok) return fail(FLLM_E_INVALID_OP, "Required tensor 'blk.%d.%s' not found in GGUF file.", l, r.name);
    }
    if (!m->output.present()) {  // GgufModelLoader.cs:365-366: tied LM head
        m->output = m->tok_embd;
        m->output_tied = true;
    }
    // Matrices whose decode launches run on the matrix cores are regrouped by 16-row tile, so that
    // every load instruction of a wave reads contiguous memory; the token embedding (and a head
    // tied to it) keeps its rows for the lookup.
    std::vector<Tensor*> to_pack;
    for (Layer& L : m->layers) {
        const Tensor* qkv[3] = {&L.q, &L.k, &L.v};
        if (tiles_launch_ok(qkv, 3, 0)) { to_pack.push_back(&L.q); to_pack.push_back(&L.k); to_pack.push_back(&L.v); }
        const Tensor* gu[2] = {&L.gate, &L.up};
        if (tiles_launch_ok(gu, 2, 1)) { to_pack.push_back(&L.gate); to_pack.push_back(&L.up); }
        const Tensor* o[1] = {&L.o};
        if (tiles_launch_ok(o, 1, 0)) to_pack.push_back(&L.o);
        const Tensor* dn[1] = {&L.down};
        if (tiles_launch_ok(dn, 1, 0)) to_pack.push_back(&L.down);
    }
    const Tensor* head[1] = {&m->output};
    if (!m->output_tied && tiles_launch_ok(head, 1, 0)) to_pack.push_back(&m->output);
    HIP_TRY(hipSetDevice(m->ctx->device));
    {
        // the largest |w| of every projection matrix, for the batched prefill's fp16 split (read in
        // GGUF row layout, before the regrouping)
        std::vector<Tensor*> mats;
        for (Layer& L : m->layers) {
            Tensor* ts[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
            for (Tensor* t : ts) mats.push_back(t);
        }
        unsigned* dmax = nullptr;
        hipError_t e = hipMalloc(&dmax, sizeof(unsigned) * mats.size());
        if (e == hipSuccess) e = hipMemsetAsync(dmax, 0, sizeof(unsigned) * mats.size(), m->ctx->stream);
        for (size_t i = 0; i < mats.size() && e == hipSuccess; i++)
            e = launch_pf_wmax(mats[i]->type, mats[i]->ptr, mats[i]->rows * mats[i]->cols, dmax + i, m->ctx->stream);
        std::vector<unsigned> hmax(mats.size(), 0u);
        if (e == hipSuccess)
            e = hipMemcpyAsync(hmax.data(), dmax, sizeof(unsigned) * mats.size(), hipMemcpyDeviceToHost, m->ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->ctx->stream);
        if (dmax) hipFree(dmax);
        if (e != hipSuccess) return fail(FLLM_E_DEVICE, "weight range: %s", hipGetErrorString(e));
        for (size_t i = 0; i < mats.size(); i++) mats[i]->wexp = pf_wexp(hmax[i]);
    }
    for (Tensor* t : to_pack) {
        hipError_t e = pack_tiles(m, *t);
        if (e != hipSuccess) return fail(FLLM_E_DEVICE, "weight regrouping: %s", hipGetErrorString(e));
    }
    // RoPE inverse frequencies (LlamaForwardPass.cs:64-70), computed on the host with powf.
    int half = d.head_dim / 2;
    m->inv_freq.resize((size_t)half);
    for (int i = 0; i < half; i++) {
        float e = (2.0f * (float)i) / (float)d.head_dim;
        m->inv_freq[(size_t)i] = 1.0f / powf(d.rope_base, e);
    }
    uint64_t lb = 0;
    for (auto& L : m->layers) lb += L.q.bytes + L.k.bytes + L.v.bytes + L.o.bytes + L.gate.bytes + L.up.bytes + L.down.bytes;
    m->layer_bytes = lb;
    m->head_bytes = m->output.bytes;
    m->finalized = true;
    return FLLM_OK;
}

extern "C" int32_t fllm_model_get_desc(fllm_model* m, fllm_model_desc* out) {
    NOT_NULL(m);
    NOT_NULL(out);
    *out = m->d;
    return FLLM_OK;
}

extern "C" int32_t fllm_model_weight_bytes(fllm_model* m, uint64_t* layer_bytes, uint64_t* head_bytes) {
    NOT_NULL(m);
    if (!m->finalized) return fail(FLLM_E_INVALID_OP, "model not finalized");
    if (layer_bytes) *layer_bytes = m->layer_bytes;
    if (head_bytes) *head_bytes = m->head_bytes;
    return FLLM_OK;
}

// =====================================================================================
// sequence
// =====================================================================================
template <typename T>
static hipError_t seq_alloc(fllm_seq* s, T** p, size_t count) {
    void* v = nullptr;
    hipError_t e = hipMalloc(&v, sizeof(T) * (count ? count : 1));
    if (e == hipSuccess) {
        s->allocs.push_back(v);
        *p = (T*)v;
    }
    return e;
}

static void seq_free(fllm_seq* s) {
    if (s->pin) hipHostFree(s->pin);
    for (void* p : s->pf_allocs) hipFree(p);
    if (s->gexec) hipGraphExecDestroy(s->gexec);
    if (s->graph) hipGraphDestroy(s->graph);
    for (void* p : s->allocs) hipFree(p);
    for (auto e : s->ev) hipEventDestroy(e);
    if (s->st) hipStreamDestroy(s->st);
    delete s;
}

extern "C" int32_t fllm_seq_create(fllm_model* m, int32_t max_seq, fllm_seq** out) {
    NOT_NULL(m);
    NOT_NULL(out);
    *out = nullptr;
    NOT_DISPOSED(m);
    if (!m->finalized) return fail(FLLM_E_INVALID_OP, "model not finalized");
    if (max_seq < 0) return fail(FLLM_E_ARG_RANGE, "max_seq must be >= 0");
    const fllm_model_desc& d = m->d;
    HIP_TRY(hipSetDevice(m->ctx->device));
    fllm_seq* s = new fllm_seq();
    s->m = m;
    s->max_seq = max_seq > 0 ? max_seq : d.max_ctx;
    s->nsplit = (s->max_seq + 255) / 256;
    s->attn_fast = attn_fast_supported(d.head_dim, d.n_heads / d.n_kv_heads, s->max_seq);
    s->attn_nc = attn_chunks(d.n_kv_heads, s->max_seq, m->ctx->n_cu > 0 ? m->ctx->n_cu : 256);
    s->attn_lds = attn_lds_bytes(d.head_dim, d.n_heads / d.n_kv_heads, s->attn_nc, s->max_seq);
    // (Llama-3-8B at 4 heads / 32 chunks: 1.572 -> 1.566 ms per step, Gemma-2-9B at 2 / 32 and
    // 6144 positions 3.290 -> 3.257; Qwen2-7B at 7 / 64 and 2048 positions 1.719 -> 1.934: the
    // merging workgroup's two passes over 64 chunks for 7 heads cost more than a second launch)
    s->attn_merge_in = d.n_heads / d.n_kv_heads <= 4 && s->attn_nc <= 32;
    s->fused = s->attn_fast && gemv_fusable_cols(d.hidden) && gemv_fusable_cols(m->qdim) && gemv_fusable_cols(d.ffn);
    for (const Layer& Lr : m->layers) {
        const Tensor* ts[] = {&Lr.q, &Lr.k, &Lr.v, &Lr.o, &Lr.gate, &Lr.up, &Lr.down};
        for (const Tensor* t : ts) s->fused = s->fused && gemv_fusable_type(t->type);
        s->fused = s->fused && Lr.gate.type == Lr.up.type;  // gate and up share one fused launch
    }
    s->head_fused = s->fused && gemv_fusable_type(m->output.type);
    hipError_t e = hipStreamCreateWithFlags(&s->st, hipStreamNonBlocking);
    if (e != hipSuccess) { s->st = nullptr; seq_free(s); return fail(FLLM_E_DEVICE, "hipStreamCreate: %s", hipGetErrorString(e)); }
    size_t L = (size_t)d.n_layers, kv = (size_t)m->kvdim, H = (size_t)d.hidden, F = (size_t)d.ffn;
    size_t kvsz = L * (size_t)s->max_seq * kv;
    int half = d.head_dim / 2;
    s->topk_cap = d.vocab;
#define ALLOC(ptr, n) \
    if (e == hipSuccess) e = seq_alloc(s, &(ptr), (n))
    ALLOC(s->kc, kvsz);
    ALLOC(s->vc, kvsz);
    ALLOC(s->rope, (size_t)s->max_seq * half);
    ALLOC(s->params, 1);
    ALLOC(s->x, H);
    ALLOC(s->xn, H);
    ALLOC(s->q, (size_t)m->qdim);
    ALLOC(s->k, kv);
    ALLOC(s->v, kv);
    ALLOC(s->att, (size_t)m->qdim);
    ALLOC(s->g, F);
    ALLOC(s->u, F);
    ALLOC(s->h, F);
    ALLOC(s->tmp, H);
    ALLOC(s->logits, (size_t)d.vocab);
    size_t nparts = (size_t)(s->nsplit > s->attn_nc ? s->nsplit : s->attn_nc);
    ALLOC(s->part_o, (size_t)d.n_heads * nparts * d.head_dim);
    ALLOC(s->part_ml, (size_t)d.n_heads * nparts * 2);
    ALLOC(s->head_keys, (size_t)d.vocab / 8 + 1);
    ALLOC(s->tab_x, gemv_tab_bytes(d.hidden) / 4 + 4);
    ALLOC(s->ssq_x, H / 16 + 1);
    ALLOC(s->tab_h, gemv_tab_bytes(d.ffn) / 4 + 4);
    ALLOC(s->tab_att, gemv_tab_bytes(m->qdim) / 4 + 4);
    ALLOC(s->tokens_out, (size_t)s->max_seq);
    ALLOC(s->topk_ids, (size_t)d.vocab);
    ALLOC(s->topk_vals, (size_t)d.vocab);
    ALLOC(s->topk_count, 1);
    ALLOC(s->probs, (size_t)d.vocab);
    ALLOC(s->samp_token, 1);
    ALLOC(s->pen_counts, (size_t)d.vocab);
    ALLOC(s->topk_sc, 1);
    ALLOC(s->nuc_sc, 1);
    ALLOC(s->hidden_dbg, (L + 1) * H);
    ALLOC(s->x2, H);
    ALLOC(s->attn_cnt, (size_t)attn_cnt_words(d.n_kv_heads));
#undef ALLOC
    if (e != hipSuccess) { seq_free(s); return fail(FLLM_E_OOM, "sequence allocation: %s", hipGetErrorString(e)); }
    // RoPE table: theta = scaledPos * inv[i] (LlamaForwardPass.cs:137-147), cos/sin on the host.
    std::vector<float2> tab((size_t)s->max_seq * half);
    for (int p = 0; p < s->max_seq; p++) {
        float sp = (d.rope_scaled && d.rope_scale > 0.0f) ? (float)p / d.rope_scale : (float)p;
        for (int i = 0; i < half; i++) {
            float th = sp * m->inv_freq[(size_t)i];
            tab[(size_t)p * half + i] = make_float2(cosf(th), sinf(th));
        }
    }
    e = hipMemcpyAsync(s->rope, tab.data(), sizeof(float2) * tab.size(), hipMemcpyHostToDevice, s->st);
    if (e == hipSuccess) e = hipMemsetAsync(s->kc, 0, sizeof(float) * kvsz, s->st);
    if (e == hipSuccess) e = hipMemsetAsync(s->params, 0, sizeof(StepParams), s->st);
    if (e == hipSuccess) e = hipMemsetAsync(s->vc, 0, sizeof(float) * kvsz, s->st);
    if (e == hipSuccess) e = hipMemsetAsync(s->pen_counts, 0, sizeof(int) * (size_t)d.vocab, s->st);
    if (e == hipSuccess) e = hipMemsetAsync(s->nuc_sc, 0, sizeof(NucleusScratch), s->st);
    if (e == hipSuccess) e = hipMemsetAsync(s->attn_cnt, 0, sizeof(unsigned) * (size_t)attn_cnt_words(d.n_kv_heads), s->st);
    if (e == hipSuccess) e = hipStreamSynchronize(s->st);
    if (e != hipSuccess) { seq_free(s); return fail(FLLM_E_DEVICE, "sequence init: %s", hipGetErrorString(e)); }
    m->n_seqs++;
    *out = s;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_destroy(fllm_seq* s) {
    if (!s) return FLLM_OK;
    fllm_model* m = s->m;
    hipSetDevice(m->ctx->device);
    hipStreamSynchronize(s->st);
    seq_free(s);
    // the last sequence of a disposed model releases its weights
    if (--m->n_seqs == 0 && m->disposed) model_free(m);
    return FLLM_OK;
}

// KvCache.Clear (KvCache.cs:138-144)
extern "C" int32_t fllm_seq_reset(fllm_seq* s) {
    NOT_NULL(s);
    HIP_TRY(hipStreamSynchronize(s->st));
    s->cur_len = 0;
    s->next_layer = 0;
    s->was_evicted = false;
    return FLLM_OK;
}

extern "C" int32_t fllm_kv_was_evicted(fllm_seq* s, int32_t* out) {
    NOT_NULL(s);
    NOT_NULL(out);
    *out = s->was_evicted ? 1 : 0;
    return FLLM_OK;
}

// KvCache.EvictOldestHalf (KvCache.cs:152-173): in every layer, positions [keep, max) move down to
// [0, max - keep) and [max - keep, max) are cleared; the length becomes keep = max / 2. For an odd
// capacity the two ranges share one position, so the move is split in two copies that do not
// overlap (the first reads that position before the second overwrites it; both are stream-ordered).
static hipError_t kv_evict(fllm_seq* s) {
    const size_t kvb = sizeof(float) * (size_t)s->m->kvdim;
    const size_t pitch = kvb * (size_t)s->max_seq;
    const int max = s->max_seq, keep = max / 2, len = max - keep;
    const size_t L = (size_t)s->m->d.n_layers;
    hipError_t e = hipSuccess;
    for (float* c : {s->kc, s->vc}) {
        uint8_t* base = (uint8_t*)c;
        if (keep > 0 && e == hipSuccess)
            e = hipMemcpy2DAsync(base, pitch, base + keep * kvb, pitch, keep * kvb, L, hipMemcpyDeviceToDevice, s->st);
        if (len > keep && keep > 0 && e == hipSuccess)  // capacity 1 keeps nothing: the row stays
            e = hipMemcpy2DAsync(base + keep * kvb, pitch, base + (size_t)(2 * keep) * kvb, pitch,
                                 (size_t)(len - keep) * kvb, L, hipMemcpyDeviceToDevice, s->st);
        if (keep > 0 && e == hipSuccess)
            e = hipMemset2DAsync(base + (size_t)len * kvb, pitch, 0, (size_t)keep * kvb, L, s->st);
    }
    if (e != hipSuccess) return e;
    s->cur_len = keep;
    s->was_evicted = true;
    return hipSuccess;
}

// The length GetKeys / GetValues return for a layer (KvCache.cs:109-115): one more than the
// current length for the layers already appended at the position being filled.
static int kv_effective(const fllm_seq* s, int layer) {
    return s->cur_len + ((s->next_layer > 0 && layer < s->next_layer) ? 1 : 0);
}

extern "C" int32_t fllm_kv_length(fllm_seq* s, int32_t layer, int32_t* out) {
    NOT_NULL(s);
    NOT_NULL(out);
    if (layer < 0 || layer >= s->m->d.n_layers)
        return fail(FLLM_E_ARG_RANGE, "Layer index must be in [0, %d].", s->m->d.n_layers - 1);
    *out = kv_effective(s, layer);
    return FLLM_OK;
}

// KvCache.Append (KvCache.cs:59-97): host slices of kv_dim floats, layers in order, the oldest half
// evicted when the cache is full.
extern "C" int32_t fllm_kv_append(fllm_seq* s, int32_t layer, const float* keys, int64_t n_keys,
                                  const float* values, int64_t n_values) {
    NOT_NULL(s);
    const int L = s->m->d.n_layers, kvdim = s->m->kvdim;
    if (layer < 0 || layer >= L) return fail(FLLM_E_ARG_RANGE, "Layer index must be in [0, %d].", L - 1);
    if (layer != s->next_layer)
        return fail(FLLM_E_INVALID_OP,
                    "KV cache append order violation: expected layer %d but received layer %d. "
                    "Append layers sequentially for each token position.", s->next_layer, layer);
    if (n_keys != kvdim || n_values != kvdim)
        return fail(FLLM_E_ARG, "Key/value slice length must be %d but got key=%lld, value=%lld.", kvdim,
                    (long long)n_keys, (long long)n_values);
    NOT_NULL(keys);
    NOT_NULL(values);
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    if (s->cur_len >= s->max_seq) HIP_TRY(kv_evict(s));
    size_t off = ((size_t)layer * s->max_seq + (size_t)s->cur_len) * kvdim;
    HIP_TRY(hipMemcpyAsync(s->kc + off, keys, sizeof(float) * kvdim, hipMemcpyHostToDevice, s->st));
    HIP_TRY(hipMemcpyAsync(s->vc + off, values, sizeof(float) * kvdim, hipMemcpyHostToDevice, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    if (++s->next_layer == L) {
        s->next_layer = 0;
        s->cur_len++;
    }
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_length(fllm_seq* s, int32_t* len) {
    NOT_NULL(s);
    NOT_NULL(len);
    *len = s->cur_len;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_capacity(fllm_seq* s, int32_t* cap) {
    NOT_NULL(s);
    NOT_NULL(cap);
    *cap = s->max_seq;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_get_model(fllm_seq* s, fllm_model** out) {
    NOT_NULL(s);
    NOT_NULL(out);
    *out = s->m;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_set_graph(fllm_seq* s, int32_t enable) {
    NOT_NULL(s);
    s->use_graph = enable != 0;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_set_prefill_chunk(fllm_seq* s, int32_t tokens) {
    NOT_NULL(s);
    if (tokens < 1) return fail(FLLM_E_ARG_RANGE, "prefill chunk must be >= 1 token");
    s->pf_chunk = tokens;  // later prefills; the scratch grows at the next one if it needs to
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_set_debug(fllm_seq* s, int32_t enable) {
    NOT_NULL(s);
    if (s->debug != (enable != 0)) s->graph_valid = false;
    s->debug = enable != 0;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_set_attention_merge(fllm_seq* s, int32_t in_launch) {
    NOT_NULL(s);
    s->attn_merge_in = in_launch != 0;
    s->graph_valid = false;  // the next graph replay captures the launches again
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_sync(fllm_seq* s) {
    NOT_NULL(s);
    HIP_TRY(hipStreamSynchronize(s->st));
    return FLLM_OK;
}

// ---- profiling helpers ------------------------------------------------------------
static hipError_t prof_begin(fllm_seq* s, const char* name, double bytes) {
    if (!s->profile) return hipSuccess;
    size_t i = s->pending.size();
    while (s->ev.size() < 2 * (i + 1)) {
        hipEvent_t e;
        hipError_t r = hipEventCreate(&e);
        if (r != hipSuccess) return r;
        s->ev.push_back(e);
    }
    s->pending.emplace_back(name, bytes);
    if (s->launch_names.size() < (1u << 20)) s->launch_names.emplace_back(name);
    return hipEventRecord(s->ev[2 * i], s->st);
}

static hipError_t prof_end(fllm_seq* s) {
    if (!s->profile) return hipSuccess;
    size_t i = s->pending.size() - 1;
    return hipEventRecord(s->ev[2 * i + 1], s->st);
}

static hipError_t prof_collect(fllm_seq* s) {
    if (!s->profile || s->pending.empty()) return hipSuccess;
    hipError_t e = hipStreamSynchronize(s->st);
    if (e != hipSuccess) return e;
    for (size_t i = 0; i < s->pending.size(); i++) {
        float ms = 0;
        e = hipEventElapsedTime(&ms, s->ev[2 * i], s->ev[2 * i + 1]);
        if (e != hipSuccess) return e;
        auto it = s->agg.find(s->pending[i].first);
        if (it == s->agg.end()) {
            s->agg_order.push_back(s->pending[i].first);
            it = s->agg.emplace(s->pending[i].first, ProfAgg()).first;
        }
        it->second.launches++;
        it->second.ms += ms;
        it->second.bytes += s->pending[i].second;
    }
    s->pending.clear();
    return hipSuccess;
}

static const char* gemv_name(int type) {
    switch (type) {
        case FLLM_TYPE_Q4_K: return "gemv_q4_k";
        case FLLM_TYPE_Q5_K: return "gemv_q5_k";
        case FLLM_TYPE_Q6_K: return "gemv_q6_k";
        case FLLM_TYPE_Q8_0: return "gemv_q8_0";
        case FLLM_TYPE_Q4_0: return "gemv_q4_0";
        case FLLM_TYPE_F32: return "gemv_f32";
        case FLLM_TYPE_F16: return "gemv_f16";
        case FLLM_TYPE_BF16: return "gemv_bf16";
        default: return "gemv_generic";
    }
}

#define STEP(name, bytes, call)                          \
    do {                                                 \
        hipError_t _e = prof_begin(s, (name), (bytes));  \
        if (_e == hipSuccess) _e = (call);               \
        if (_e == hipSuccess) _e = prof_end(s);          \
        if (_e != hipSuccess) return _e;                 \
    } while (0)

static int layer_window(const fllm_model_desc& d, int l) {
    if (d.arch == FLLM_ARCH_MISTRAL) return d.sliding_window;             // MistralForwardPass.cs:131
    if (d.arch == FLLM_ARCH_GEMMA2 && (l % 2) == 0) return d.sliding_window;  // Gemma2ForwardPass.cs:87
    return 0x7FFFFFFF;
}

// arguments of the fast decode attention of layer l (tab: it also writes the output projection's table)
static AttnArgs attn_args(const fllm_seq* s, int l, const float* kc, const float* vc, bool tab) {
    const fllm_model_desc& d = s->m->d;
    const bool gemma = d.arch == FLLM_ARCH_GEMMA2;
    AttnArgs a{};
    a.q = s->q; a.kc = kc; a.vc = vc;
    a.nh = d.n_heads; a.nkv = d.n_kv_heads; a.hd = d.head_dim; a.kvdim = s->m->kvdim;
    a.window = layer_window(d, l); a.scale = d.attn_scale; a.softcap = gemma ? d.attn_softcap : 0.0f;
    a.nc = s->attn_nc; a.part_o = s->part_o; a.part_ml = s->part_ml;
    a.out = s->att; a.params = s->params;
    a.tab_out = tab ? s->tab_att : nullptr;
    return a;
}

// K and V rows attended (at most the whole cache) plus q and the output
static double attn_bytes(const fllm_seq* s) {
    return 8.0 * (double)s->m->kvdim * (double)s->max_seq + 8.0 * s->m->qdim;
}

static hipError_t attention_step(fllm_seq* s, int l, const float* kc, const float* vc, bool tab) {
    const fllm_model_desc& d = s->m->d;
    bool gemma = d.arch == FLLM_ARCH_GEMMA2;
    int window = layer_window(d, l);
    float softcap = gemma ? d.attn_softcap : 0.0f;
    const double bytes = attn_bytes(s);
    if (s->attn_fast) {
        const AttnArgs a = attn_args(s, l, kc, vc, tab);
        const double merge_bytes = 4.0 * (double)d.n_heads * s->attn_nc * (d.head_dim + 2) + 4.0 * s->m->qdim;
        if (s->attn_merge_in) {
            STEP("attention", bytes + merge_bytes, launch_attn_merged(a, s->attn_lds, s->attn_cnt, s->st));
        } else {
            STEP("attention", bytes, launch_attn_partial(a, s->attn_lds, s->st));
            STEP("attention_merge", merge_bytes, launch_attn_merge(a, s->st));
        }
    } else {
        STEP("attention", bytes,
             launch_attention(s->q, kc, vc, d.n_heads, d.n_kv_heads, d.head_dim, window, d.attn_scale, softcap,
                              s->nsplit, s->part_o, s->part_ml, s->att, s->params, s->st));
    }
    return hipSuccess;
}

static GemvSeg seg_of(const Tensor& t, int epi, float* out, const float* bias, const float* resid) {
    GemvSeg g{};
    g.w = t.ptr; g.layout = t.layout; g.type = t.type; g.rows = (int)t.rows;
    g.epi = epi; g.out = out; g.bias = bias; g.resid = resid;
    return g;
}

static hipError_t fused_step(fllm_seq* s, const char* name, GemvArgs& a, int64_t cols, double bytes) {
    int threads;
    size_t lds;
    int grid = gemv_plan(a, cols, s->m->ctx->n_cu > 0 ? s->m->ctx->n_cu : 256, 0, &threads, &lds);
    STEP(name, bytes, launch_gemv_fused(a, grid, threads, lds, s->st));
    return hipSuccess;
}

// y = W x (+ res), one launch per matrix
static hipError_t gemv_step(fllm_seq* s, const Tensor& t, const float* xf, float* y, const float* res) {
    double bytes = (double)t.bytes + 4.0 * (double)(t.cols + t.rows);
    if (t.layout == LAYOUT_TILES) {
        // a regrouped matrix is read by the matrix-core variant, as a one-segment launch
        GemvArgs a{};
        a.nseg = 1;
        a.seg[0] = seg_of(t, res ? EPI_RESID : EPI_STORE, y, nullptr, res);
        a.xin = XIN_F32;
        a.x = xf;
        return fused_step(s, gemv_name(t.type), a, t.cols, bytes);
    }
    STEP(gemv_name(t.type), bytes, launch_gemv(t.mat(), xf, y, res, s->m->ctx->n_cu, s->st));
    return hipSuccess;
}

// LM head, logits softcap, greedy argmax and the step advance (generic kernels).
static hipError_t head_generic(fllm_seq* s) {
    fllm_model* m = s->m;
    const fllm_model_desc& d = m->d;
    bool gemma = d.arch == FLLM_ARCH_GEMMA2;
    float eps = gemma ? 1e-6f : d.norm_eps;
    int H = d.hidden;
    STEP("rmsnorm", 12.0 * H, launch_rmsnorm(s->x, m->out_norm, H, eps, gemma ? 1 : 0, s->xn, s->st));
    if (s->debug) STEP("debug_copy", 8.0 * H, launch_copy_hidden(s->xn, H, s->hidden_dbg + (size_t)d.n_layers * H, s->st));
    hipError_t e = gemv_step(s, m->output, s->xn, s->logits, nullptr);
    if (e != hipSuccess) return e;
    if (gemma && d.final_softcap > 0.0f) STEP("softcap", 8.0 * d.vocab, launch_softcap(s->logits, d.vocab, d.final_softcap, s->st));
    // (one kernel per profiled step: the segment keys, then their reduction and the step advance)
    STEP("argmax_segments", 4.0 * d.vocab, launch_argmax_seg(s->logits, d.vocab, s->head_keys, s->st));
    STEP("argmax", 8.0 * argmax_segments(d.vocab),
         launch_argmax_keys(s->head_keys, argmax_segments(d.vocab), s->params, s->tokens_out, s->max_seq, s->st));
    return hipSuccess;
}

// true when a launch over these matrices (GLU: gate, up) runs the matrix-core variant
static bool mfma_launch(const Tensor* const* t, int n, int glu, int64_t cols) {
    GemvArgs a{};
    a.nseg = n;
    a.glu = glu;
    for (int i = 0; i < n; i++) {
        a.seg[i].w = t[i]->ptr; a.seg[i].layout = t[i]->layout; a.seg[i].type = t[i]->type; a.seg[i].rows = (int)t[i]->rows;
    }
    return gemv_uses_mfma(a, cols);
}

// Decode step as fused launches: per layer [norm + QKV + RoPE + KV store], attention,
// [Wo + residual], [norm + gate/up + activation], [down + residual]; then [norm + LM head +
// softcap + argmax + step advance]. Gemma2's post-norms are separate small kernels.
// Between matrix-core launches the activation vector travels as its quantized table: the
// residual epilogues (Wo, down) write the table of x times the next RMSNorm weight plus partial
// sums of squares, the gate/up epilogue the table of the FFN activation, and the next launch
// copies it instead of quantizing the vector in every workgroup.
static hipError_t enqueue_body_fused(fllm_seq* s) {
    fllm_model* m = s->m;
    const fllm_model_desc& d = m->d;
    bool gemma = d.arch == FLLM_ARCH_GEMMA2;
    int H = d.hidden, kvdim = m->kvdim;
    float eps = gemma ? 1e-6f : d.norm_eps;
    int nk = gemma ? 1 : 0;
    size_t layer_kv = (size_t)s->max_seq * kvdim;
    // F32 / F16 / BF16 embedding rows are read by the first projection's prologue; quantized
    // ones go through the element-wise lookup kernel first
    int et = m->tok_embd.type;
    bool emb_fused = et == FLLM_TYPE_F32 || et == FLLM_TYPE_F16 || et == FLLM_TYPE_BF16;
    if (!emb_fused) STEP("embed", 4.0 * H, launch_embed(m->tok_embd.ptr, et, H, s->params, s->x, s->st));
    const Tensor* head_t[1] = {&m->output};
    const bool head_mf = s->head_fused && !s->debug && mfma_launch(head_t, 1, 0, H);
    bool xtab = false;  // tab_x / ssq_x hold the table of the current x for the next launch's norm
    // Gemma-2 post-norms (x += GemmaRmsNorm(tmp, w) after o and after down): the pending one (its
    // weight pend) is folded into the prologue of the next launch that normalizes x on the matrix
    // cores (XIN_POST), which stores the new residual in the other of two buffers; cur is the
    // current residual buffer. The last one of the step goes into s->x, the head's input.
    const bool post_fuse = gemma && !s->debug;
    float* cur = s->x;
    float* alt = s->x2;
    const float* pend = nullptr;
    auto fold_post = [&](GemvArgs& a, int cols) -> hipError_t {
        if (pend == nullptr) return hipSuccess;
        if (a.xin == XIN_NORM && gemv_uses_mfma(a, cols)) {
            a.xin = XIN_POST;
            a.x = cur; a.x2 = s->tmp; a.post_w = pend; a.x_out = alt;
            std::swap(cur, alt);
        } else {
            STEP("postnorm_add", 12.0 * H, launch_postnorm_add(s->tmp, pend, H, cur, cur, s->st));
        }
        pend = nullptr;
        return hipSuccess;
    };
    for (int l = 0; l < d.n_layers; l++) {
        const Layer& L = m->layers[(size_t)l];
        float* kc = s->kc + (size_t)l * layer_kv;
        float* vc = s->vc + (size_t)l * layer_kv;
        const Tensor* gu_t[2] = {&L.gate, &L.up};
        const Tensor* o_t[1] = {&L.o};
        const Tensor* dn_t[1] = {&L.down};
        const bool o_mf = mfma_launch(o_t, 1, 0, m->qdim), gu_mf = mfma_launch(gu_t, 2, 1, H);
        const bool dn_mf = mfma_launch(dn_t, 1, 0, d.ffn);
        {
            // q, k and v in one launch (the matrix-core variant takes Q4_K q/k with a Q6_K v)
            GemvArgs a{};
            a.nseg = 3;
            a.seg[0] = seg_of(L.q, EPI_Q, s->q, L.bq, nullptr);
            a.seg[1] = seg_of(L.k, EPI_K, nullptr, L.bk, nullptr);
            a.seg[2] = seg_of(L.v, EPI_V, nullptr, L.bv, nullptr);
            const double bytes = (double)(L.q.bytes + L.k.bytes + L.v.bytes) + 4.0 * (L.q.rows + L.k.rows + L.v.rows);
            a.xin = (l == 0 && emb_fused) ? XIN_EMBED_NORM : XIN_NORM;
            a.x = cur; a.x_out = cur; a.norm_w = L.attn_norm; a.eps = eps; a.norm_kind = nk;
            if (xtab && gemv_uses_mfma(a, H)) { a.xin = XIN_TAB; a.xtab = s->tab_x; a.xssq = s->ssq_x; }
            a.emb = m->tok_embd.ptr; a.emb_type = m->tok_embd.type; a.params = s->params;
            a.rope = s->rope; a.hd = d.head_dim; a.kc = kc; a.vc = vc; a.kvdim = kvdim;
            hipError_t e = fold_post(a, H);
            if (e != hipSuccess) return e;
            e = fused_step(s, "qkv_rope_kv", a, H, bytes + 8.0 * H);
            if (e != hipSuccess) return e;
        }
        // the attention merge writes the output projection's activation table when that runs on
        // the matrix cores
        const bool atab = s->attn_fast && o_mf;
        hipError_t e = attention_step(s, l, kc, vc, atab);
        if (e != hipSuccess) return e;
        {
            GemvArgs a{};
            a.nseg = 1;
            a.seg[0] = gemma ? seg_of(L.o, EPI_STORE, s->tmp, nullptr, nullptr) : seg_of(L.o, EPI_RESID, cur, nullptr, cur);
            a.xin = XIN_F32;
            a.x = s->att;
            if (atab) { a.xin = XIN_TAB; a.xtab = s->tab_att; }
            xtab = !gemma && o_mf && gu_mf;
            if (xtab) { a.tab_out = s->tab_x; a.ssq_out = s->ssq_x; a.tab_w = L.ffn_norm; a.tab_kind = nk; }
            e = fused_step(s, "attn_output", a, m->qdim, (double)L.o.bytes + 4.0 * (m->qdim + 2.0 * H));
            if (e != hipSuccess) return e;
            if (gemma && post_fuse) pend = L.post_attn;
            else if (gemma) STEP("postnorm_add", 12.0 * H, launch_postnorm_add(s->tmp, L.post_attn, H, cur, cur, s->st));
        }
        const bool htab = gu_mf && dn_mf;
        {
            GemvArgs a{};
            a.nseg = 2;
            a.glu = 1;
            a.act = gemma ? 1 : 0;
            a.seg[0] = seg_of(L.gate, EPI_STORE, s->h, nullptr, nullptr);
            a.seg[1] = seg_of(L.up, EPI_STORE, nullptr, nullptr, nullptr);
            a.xin = XIN_NORM;
            a.x = cur; a.norm_w = L.ffn_norm; a.eps = eps; a.norm_kind = nk;
            if (xtab) { a.xin = XIN_TAB; a.xtab = s->tab_x; a.xssq = s->ssq_x; }
            if (htab) a.tab_out = s->tab_h;
            if ((e = fold_post(a, H)) != hipSuccess) return e;
            e = fused_step(s, "ffn_gate_up", a, H, (double)(L.gate.bytes + L.up.bytes) + 4.0 * (2.0 * H + d.ffn));
            if (e != hipSuccess) return e;
        }
        {
            GemvArgs a{};
            a.nseg = 1;
            a.seg[0] = gemma ? seg_of(L.down, EPI_STORE, s->tmp, nullptr, nullptr) : seg_of(L.down, EPI_RESID, cur, nullptr, cur);
            a.xin = XIN_F32;
            a.x = s->h;
            if (htab) { a.xin = XIN_TAB; a.xtab = s->tab_h; }
            // the next consumer of x: the next layer's q/k/v, or the LM head
            bool next_mf = head_mf;
            const float* next_w = m->out_norm;
            if (l + 1 < d.n_layers) {
                const Layer& N = m->layers[(size_t)l + 1];
                const Tensor* qkv_t[3] = {&N.q, &N.k, &N.v};
                next_mf = mfma_launch(qkv_t, 3, 0, H);
                next_w = N.attn_norm;
            }
            xtab = !gemma && dn_mf && next_mf;
            if (xtab) { a.tab_out = s->tab_x; a.ssq_out = s->ssq_x; a.tab_w = next_w; a.tab_kind = nk; }
            e = fused_step(s, "ffn_down", a, d.ffn, (double)L.down.bytes + 4.0 * (d.ffn + 2.0 * H));
            if (e != hipSuccess) return e;
            if (gemma && post_fuse) pend = L.post_ffn;
            else if (gemma) STEP("postnorm_add", 12.0 * H, launch_postnorm_add(s->tmp, L.post_ffn, H, cur, cur, s->st));
        }
        if (s->debug) STEP("debug_copy", 8.0 * H, launch_copy_hidden(cur, H, s->hidden_dbg + (size_t)l * H, s->st));
    }
    // the step's last post-norm, into s->x (where the head reads the residual)
    if (pend != nullptr) {
        STEP("postnorm_add", 12.0 * H, launch_postnorm_add(s->tmp, pend, H, cur, s->x, s->st));
        pend = nullptr;
        cur = s->x;
    }
    if (!s->head_fused || s->debug) return head_generic(s);
    GemvArgs a{};
    a.nseg = 1;
    a.seg[0] = seg_of(m->output, EPI_LOGITS, s->logits, nullptr, nullptr);
    a.xin = XIN_NORM;
    a.x = s->x; a.norm_w = m->out_norm; a.eps = eps; a.norm_kind = nk;
    if (xtab && head_mf) { a.xin = XIN_TAB; a.xtab = s->tab_x; a.xssq = s->ssq_x; }
    a.softcap = (gemma && d.final_softcap > 0.0f) ? d.final_softcap : 0.0f;
    a.wg_keys = s->head_keys; a.params = s->params;
    int threads;
    size_t lds;
    int grid = gemv_plan(a, H, m->ctx->n_cu > 0 ? m->ctx->n_cu : 256, 0, &threads, &lds);
    STEP("lm_head", (double)m->output.bytes + 4.0 * (2.0 * H + d.vocab), launch_gemv_fused(a, grid, threads, lds, s->st));
    STEP("argmax", 8.0 * grid, launch_argmax_keys(s->head_keys, grid, s->params, s->tokens_out, s->max_seq, s->st));
    return hipSuccess;
}

// The decode step as one kernel per reference op (any tensor type and shape).
static hipError_t enqueue_body_generic(fllm_seq* s) {
    fllm_model* m = s->m;
    const fllm_model_desc& d = m->d;
    bool gemma = d.arch == FLLM_ARCH_GEMMA2;
    int H = d.hidden, kvdim = m->kvdim;
    float eps = gemma ? 1e-6f : d.norm_eps;
    int nk = gemma ? 1 : 0;
    size_t layer_kv = (size_t)s->max_seq * kvdim;
    STEP("embed", 4.0 * H, launch_embed(m->tok_embd.ptr, m->tok_embd.type, H, s->params, s->x, s->st));
    for (int l = 0; l < d.n_layers; l++) {
        const Layer& L = m->layers[(size_t)l];
        STEP("rmsnorm", 12.0 * H, launch_rmsnorm(s->x, L.attn_norm, H, eps, nk, s->xn, s->st));
        hipError_t e;
        if ((e = gemv_step(s, L.q, s->xn, s->q, nullptr)) != hipSuccess) return e;
        if ((e = gemv_step(s, L.k, s->xn, s->k, nullptr)) != hipSuccess) return e;
        if ((e = gemv_step(s, L.v, s->xn, s->v, nullptr)) != hipSuccess) return e;
        float* kc = s->kc + (size_t)l * layer_kv;
        float* vc = s->vc + (size_t)l * layer_kv;
        STEP("qkv_rope_kvstore", 8.0 * (m->qdim + 2 * kvdim),
             launch_qkv_post(s->q, s->k, s->v, L.bq, L.bk, L.bv, s->rope, d.n_heads, d.n_kv_heads, d.head_dim, kc, vc,
                             s->params, s->st));
        if ((e = attention_step(s, l, kc, vc, false)) != hipSuccess) return e;
        if (gemma) {
            if ((e = gemv_step(s, L.o, s->att, s->tmp, nullptr)) != hipSuccess) return e;
            STEP("postnorm_add", 12.0 * H, launch_postnorm_add(s->tmp, L.post_attn, H, s->x, s->x, s->st));
        } else {
            if ((e = gemv_step(s, L.o, s->att, s->x, s->x)) != hipSuccess) return e;
        }
        STEP("rmsnorm", 12.0 * H, launch_rmsnorm(s->x, L.ffn_norm, H, eps, nk, s->xn, s->st));
        if ((e = gemv_step(s, L.gate, s->xn, s->g, nullptr)) != hipSuccess) return e;
        if ((e = gemv_step(s, L.up, s->xn, s->u, nullptr)) != hipSuccess) return e;
        STEP("ffn_act", 12.0 * d.ffn, launch_act(s->g, s->u, d.ffn, gemma ? 1 : 0, s->h, s->st));
        if (gemma) {
            if ((e = gemv_step(s, L.down, s->h, s->tmp, nullptr)) != hipSuccess) return e;
            STEP("postnorm_add", 12.0 * H, launch_postnorm_add(s->tmp, L.post_ffn, H, s->x, s->x, s->st));
        } else {
            if ((e = gemv_step(s, L.down, s->h, s->x, s->x)) != hipSuccess) return e;
        }
        if (s->debug) STEP("debug_copy", 8.0 * H, launch_copy_hidden(s->x, H, s->hidden_dbg + (size_t)l * H, s->st));
    }
    return head_generic(s);
}

static hipError_t enqueue_body(fllm_seq* s) { return s->fused ? enqueue_body_fused(s) : enqueue_body_generic(s); }

static int32_t enqueue_step(fllm_seq* s, int token, int pos) {
    if (token >= 0) HIP_TRY(launch_set_params(s->params, token, pos, s->cur_len, s->st));
    bool graph = s->use_graph && !s->profile;
    if (!graph) {
        hipError_t e = enqueue_body(s);
        if (e != hipSuccess) return fail(FLLM_E_DEVICE, "decode step: %s", hipGetErrorString(e));
        e = prof_collect(s);
        if (e != hipSuccess) return fail(FLLM_E_DEVICE, "profile: %s", hipGetErrorString(e));
        return FLLM_OK;
    }
    if (!s->graph_valid) {
        if (s->gexec) { hipGraphExecDestroy(s->gexec); s->gexec = nullptr; }
        if (s->graph) { hipGraphDestroy(s->graph); s->graph = nullptr; }
        HIP_TRY(hipStreamBeginCapture(s->st, hipStreamCaptureModeThreadLocal));
        hipError_t e = enqueue_body(s);
        hipGraph_t g = nullptr;
        hipError_t e2 = hipStreamEndCapture(s->st, &g);
        if (e != hipSuccess) { if (g) hipGraphDestroy(g); return fail(FLLM_E_DEVICE, "capture: %s", hipGetErrorString(e)); }
        if (e2 != hipSuccess) return fail(FLLM_E_DEVICE, "hipStreamEndCapture: %s", hipGetErrorString(e2));
        s->graph = g;
        HIP_TRY(hipGraphInstantiate(&s->gexec, s->graph, nullptr, nullptr, 0));
        s->graph_valid = true;
    }
    HIP_TRY(hipGraphLaunch(s->gexec, s->st));
    return FLLM_OK;
}

// KvCache.Append's order check for layer 0 (KvCache.cs:69-74), the first thing a Forward call
// does to the cache.
#define APPEND_ORDER_OK(s)                                                                               \
    do {                                                                                                 \
        if ((s)->next_layer != 0)                                                                        \
            return fail(FLLM_E_INVALID_OP,                                                               \
                        "KV cache append order violation: expected layer %d but received layer 0. "      \
                        "Append layers sequentially for each token position.", (s)->next_layer);        \
    } while (0)

extern "C" int32_t fllm_forward(fllm_seq* s, int32_t token, int32_t position) {
    NOT_NULL(s);
    NOT_DISPOSED(s->m);
    const fllm_model_desc& d = s->m->d;
    if (token < 0 || token >= d.vocab)
        return fail(FLLM_E_ARG_RANGE, "Token id %d is outside the valid vocabulary range [0, %d].", token, d.vocab - 1);
    if (position < 0) return fail(FLLM_E_ARG_RANGE, "position %d must be >= 0", position);
    APPEND_ORDER_OK(s);
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    // Layer 0's Append evicts the oldest half of a full cache (KvCache.cs:82-85).
    if (s->cur_len >= s->max_seq) HIP_TRY(kv_evict(s));
    if (position > s->cur_len) {
        // The reference appends layer 0 at the current length, then attention slices positions
        // [0, position] of a cache that holds cur_len + 1 and throws (LlamaForwardPass.cs:186-188):
        // the cache is left expecting layer 1. That state is kept here, with layer 0's row at the
        // slot cleared to zeros instead of the failed token's keys and values (the slot may hold a
        // row of an earlier use of the cache, before a reset or an eviction).
        const size_t row = (size_t)s->cur_len * s->m->kvdim;
        const size_t nb = sizeof(float) * (size_t)s->m->kvdim;
        HIP_TRY(hipMemsetAsync(s->kc + row, 0, nb, s->st));
        HIP_TRY(hipMemsetAsync(s->vc + row, 0, nb, s->st));
        if (++s->next_layer == d.n_layers) {
            s->next_layer = 0;
            s->cur_len++;
        }
        return fail(FLLM_E_ARG_RANGE, "position %d outside the cached range [0, %d]", position, kv_effective(s, 0) - 1);
    }
    int32_t rc = enqueue_step(s, token, position);
    if (rc) return rc;
    s->cur_len++;
    s->argmax_valid = true;
    return FLLM_OK;
}

extern "C" int32_t fllm_decode_greedy(fllm_seq* s, int32_t token, int32_t position, int32_t n_steps, int32_t* out_tokens) {
    NOT_NULL(s);
    const fllm_model_desc& d = s->m->d;
    if (n_steps < 0) return fail(FLLM_E_ARG_RANGE, "n_steps must be >= 0");
    NOT_DISPOSED(s->m);
    if (n_steps == 0) return FLLM_OK;
    NOT_NULL(out_tokens);
    APPEND_ORDER_OK(s);
    if (token < 0 || token >= d.vocab)
        return fail(FLLM_E_ARG_RANGE, "Token id %d is outside the valid vocabulary range [0, %d].", token, d.vocab - 1);
    if (position < 0 || position > s->cur_len)
        return fail(FLLM_E_ARG_RANGE, "position %d outside the cached range [0, %d]", position, s->cur_len);
    if ((int64_t)s->cur_len + n_steps > s->max_seq)
        return fail(FLLM_E_ARG_RANGE, "%d steps from length %d exceed the KV cache capacity (%d positions)", n_steps,
                    s->cur_len, s->max_seq);
    if (s->profile) return fail(FLLM_E_INVALID_OP, "the device-side decode loop does not run in profile mode");
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    // parameters once; every replayed step then feeds its greedy token to the next on the device
    HIP_TRY(launch_set_params(s->params, token, position, s->cur_len, s->st));
    for (int i = 0; i < n_steps; i++) {
        int32_t rc;
        if (s->use_graph) {
            rc = FLLM_OK;
            if (!s->graph_valid) {
                // capture without touching the parameters the first step already holds
                rc = enqueue_step(s, -1, -1);
            } else {
                hipError_t e = hipGraphLaunch(s->gexec, s->st);
                if (e != hipSuccess) rc = fail(FLLM_E_DEVICE, "hipGraphLaunch: %s", hipGetErrorString(e));
            }
        } else {
            hipError_t e = enqueue_body(s);
            rc = e == hipSuccess ? FLLM_OK : fail(FLLM_E_DEVICE, "decode step: %s", hipGetErrorString(e));
        }
        if (rc) return rc;
        s->cur_len++;
    }
    HIP_TRY(hipMemcpyAsync(out_tokens, s->tokens_out, sizeof(int32_t) * (size_t)n_steps, hipMemcpyDeviceToHost, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    s->argmax_valid = true;
    return FLLM_OK;
}

// ---- batched prefill ---------------------------------------------------------------------------

// the batched path covers the fast attention's head dims and 32-aligned projection widths
static bool prefill_batched_ok(const fllm_seq* s) {
    const fllm_model_desc& d = s->m->d;
    const int hd = d.head_dim;
    return (hd == 64 || hd == 128 || hd == 256) && d.n_kv_heads > 0 && d.n_heads % d.n_kv_heads == 0 &&
           d.hidden % 32 == 0 && s->m->qdim % 32 == 0 && d.ffn % 32 == 0;
}

// tokens per pass of a prefill of n tokens: at most pf_chunk and the capacity
static int prefill_pass(const fllm_seq* s) {
    return s->max_seq < s->pf_chunk ? s->max_seq : s->pf_chunk;
}

static void prefill_release(fllm_seq* s) {
    for (void* p : s->pf_allocs) hipFree(p);
    s->pf_allocs.clear();
    s->pf_x = s->pf_xn = s->pf_qkv = s->pf_att = s->pf_gu = s->pf_tmp = s->pf_part = nullptr;
    s->pf_xh = nullptr;
    s->pf_xs = nullptr;
    s->pf_kvh = nullptr;
    s->pf_kvs = nullptr;
    s->pf_kvblk = 0;
    s->pf_tok = nullptr;
    s->pf_cap = 0;
    s->pf_part_cap = 0;
}

// scratch for passes over n tokens: rows for min(pass, n rounded up to 256); kept and reused while
// it holds enough (about 0.4 MB per row at 8B-model widths), replaced by a larger one otherwise
static hipError_t prefill_alloc(fllm_seq* s, int n) {
    const int pass = prefill_pass(s);
    int want = (n + 255) / 256 * 256;
    want = want < pass ? want : pass;
    if (s->pf_cap >= want) return hipSuccess;
    if (s->pf_cap > 0) {
        hipError_t e = hipStreamSynchronize(s->st);  // nothing queued may still use the old rows
        if (e != hipSuccess) return e;
        prefill_release(s);
    }
    const fllm_model& m = *s->m;
    const int cap = want;
    size_t ldx = (size_t)std::max(m.d.hidden, m.d.ffn);
    ldx = (ldx + 3) / 4 * 4;
    const size_t H = (size_t)m.d.hidden, C = (size_t)cap;
    hipError_t e = hipSuccess;
    auto pf_alloc = [&](auto** ptr, size_t count) {
        if (e != hipSuccess) return;
        void* v = nullptr;
        e = hipMalloc(&v, sizeof(**ptr) * (count ? count : 1));
        if (e == hipSuccess) {
            s->pf_allocs.push_back(v);
            *ptr = (std::remove_reference_t<decltype(*ptr)>)v;
        }
    };
#define PF_ALLOC(ptr, count) pf_alloc(&(ptr), (count))
    PF_ALLOC(s->pf_x, C * H);
    PF_ALLOC(s->pf_qkv, C * (size_t)(m.qdim + 2 * m.kvdim));
    PF_ALLOC(s->pf_att, C * (size_t)m.qdim);
    PF_ALLOC(s->pf_gu, C * 2 * (size_t)m.d.ffn);
    PF_ALLOC(s->pf_tmp, C * H);
    PF_ALLOC(s->pf_xn, C * ldx);
    PF_ALLOC(s->pf_tok, C);
    const size_t part_cap = 3 * C * std::max(H, (size_t)(m.qdim + 2 * m.kvdim));
    PF_ALLOC(s->pf_part, part_cap);
    // widest GEMM input: hidden (q/k/v, gate/up), q_dim (output projection) or ffn (down)
    const size_t kmax = ((size_t)std::max(std::max(m.d.hidden, m.d.ffn), m.qdim) + 7) / 8 * 8;
    PF_ALLOC(s->pf_xh, 2 * C * kmax + 2 * C * (kmax / 32 + 1));  // value planes, then group-sum planes
    PF_ALLOC(s->pf_xs, C);
    const size_t kvh = pf_kv_planes_halves(m.d.head_dim, m.d.n_kv_heads, s->max_seq);
    const int kvblk = (s->max_seq + 31) / 32;
    if (kvh > 0) {
        PF_ALLOC(s->pf_kvh, kvh);
        PF_ALLOC(s->pf_kvs, 2 * (size_t)m.d.n_kv_heads * kvblk);
    }
#undef PF_ALLOC
    if (e == hipSuccess) {
        s->pf_cap = cap;
        s->pf_ldx = (int)ldx;
        s->pf_part_cap = part_cap;
        s->pf_kvblk = kvh > 0 ? kvblk : 0;
    } else {
        prefill_release(s);
    }
    return e;
}

// A GEMM input computed inside the fp16 split: the RmsNorm of rows (NORM: x [T][K], weights w) or
// the gated activation (ACT: gu [T][2 K]), never written as f32 rows.
struct PfSrc {
    enum { NORM = 1, ACT = 2 };
    int kind;
    float* x;
    const float* w;
    float eps;
    int fn;       // NORM: 1 GemmaRmsNorm; ACT: 1 GELU, 0 SiLU
    int nsp = 0;  // NORM: K-split slices of x left in pf_part by the previous GEMM, added into x first
};

// y_i (+)= X W_i^T over the chunk's rows for the matrices w[0..n) (one launch when their layouts
// agree); X = pf_xn (row stride pf_ldx), the given rows, or the rows src computes. With pending and
// one launch for all the matrices, that launch leaves its K-split slices (laid out from y[0]) in
// pf_part for the next kernel (launch_pf_gemm's pending); with several launches, *pending is 0.
static hipError_t pf_gemm(fllm_seq* s, const char* name, const Tensor* const* w, float* const* y, int n, int ldy, int T,
                          bool add, const float* x = nullptr, int ldx = 0, const PfSrc* src = nullptr,
                          int* pending = nullptr) {
    PfGemm g{};
    g.x = x ? x : s->pf_xn;
    g.ldx = x ? ldx : s->pf_ldx;
    g.K = (int)w[0]->cols;
    g.T = T;
    g.add = add ? 1 : 0;
    g.part = s->pf_part;
    g.part_cap = s->pf_part_cap;
    // the input's fp16 hi / lo planes, once for all the launch's matrices
    g.ldh = (g.K + 7) / 8 * 8;
    g.xh = s->pf_xh;
    g.xs = s->pf_xs;
    if (src && src->kind == PfSrc::NORM) {
        g.x = src->x;
        g.ldx = g.K;
        STEP("pf_norm_split", (8.0 + 4.0 * src->nsp + (src->nsp > 0 ? 4.0 : 0.0)) * T * g.K + 4.0 * T * g.ldh,
             launch_pf_split_norm(src->x, T, g.K, src->w, src->eps, src->fn, s->pf_xh, g.ldh, s->pf_xs, s->st,
                                  s->pf_part, src->nsp));
    } else if (src && src->kind == PfSrc::ACT) {
        g.x = src->x;
        g.ldx = 2 * g.K;
        STEP("pf_act_split", 8.0 * T * g.K + 4.0 * T * g.ldh,
             launch_pf_split_act(src->x, T, g.K, src->fn, s->pf_xh, g.ldh, s->pf_xs, s->st));
    } else {
        STEP("pf_split", 4.0 * T * g.K + 4.0 * T * g.ldh,
             launch_pf_split(g.x, g.ldx, T, g.K, s->pf_xh, g.ldh, s->pf_xs, s->st));
    }
    double bytes = 0.0;
    for (int i = 0; i < n; i++) {
        // one launch per run of tile-interleaved matrices, or of GGUF-row matrices of one type (a run
        // of tile Q4_K matrices only takes their own fp16 form; a mixed run, the general one)
        const bool split = g.nseg > 0 && ((w[i]->layout == LAYOUT_TILES) != (g.seg[0].layout == LAYOUT_TILES) ||
                                          (w[i]->layout != LAYOUT_TILES && w[i]->type != g.seg[0].type));
        if (split) {
            STEP(name, bytes, launch_pf_gemm(g, s->m->ctx->n_cu, s->st));
            g.nseg = 0;
            bytes = 0.0;
            if (pending) *pending = 0;
            pending = nullptr;
        }
        PfSeg& sg = g.seg[g.nseg++];
        sg.w = w[i]->ptr; sg.type = w[i]->type; sg.layout = w[i]->layout; sg.N = (int)w[i]->rows;
        sg.y = y[i]; sg.ldy = ldy; sg.wexp = w[i]->wexp;
        bytes += (double)w[i]->bytes + 8.0 * T * (double)(w[i]->rows + w[i]->cols);
    }
    STEP(name, bytes, launch_pf_gemm(g, s->m->ctx->n_cu, s->st, pending));
    return hipSuccess;
}

// T prompt tokens (device copy in pf_tok) at positions pos0.. through every layer; leaves the
// residual stream of the T rows in pf_x and their K / V in the cache.
static hipError_t prefill_chunk(fllm_seq* s, int T, int pos0) {
    fllm_model* m = s->m;
    const fllm_model_desc& d = m->d;
    const bool gemma = d.arch == FLLM_ARCH_GEMMA2;
    const int H = d.hidden, qdim = m->qdim, kvdim = m->kvdim, F = d.ffn, ldx = s->pf_ldx;
    const float eps = gemma ? 1e-6f : d.norm_eps;
    const int nk = gemma ? 1 : 0;
    const int ldq = qdim + 2 * kvdim;
    const size_t layer_kv = (size_t)s->max_seq * kvdim;
    hipError_t e;
    // K-split slices of the residual stream pf_x left in pf_part by the o or down GEMM, added by the
    // next norm split (Llama-form layers whose norms go into the split)
    int pend_x = 0;
    STEP("pf_embed", 4.0 * T * H, launch_pf_embed(s->pf_tok, T, m->tok_embd.ptr, m->tok_embd.type, H, s->pf_x, s->st));
    for (int l = 0; l < d.n_layers; l++) {
        const Layer& L = m->layers[(size_t)l];
        float* kc = s->kc + (size_t)l * layer_kv;
        float* vc = s->vc + (size_t)l * layer_kv;
        // the norms and the activation go into the split of the GEMM input (rows up to 20480)
        const bool fuse_h = pf_split_src_ok(H), fuse_f = pf_split_src_ok(F);
        const bool defer_x = fuse_h && !gemma;
        if (!fuse_h) STEP("pf_norm", 8.0 * T * H, launch_pf_norm(s->pf_x, T, H, L.attn_norm, eps, nk, s->pf_xn, ldx, s->st));
        int pend_qkv = 0;
        {
            const Tensor* w[3] = {&L.q, &L.k, &L.v};
            float* y[3] = {s->pf_qkv, s->pf_qkv + qdim, s->pf_qkv + qdim + kvdim};
            const PfSrc src{PfSrc::NORM, s->pf_x, L.attn_norm, eps, nk, pend_x};
            pend_x = 0;
            if ((e = pf_gemm(s, "pf_qkv", w, y, 3, ldq, T, false, nullptr, 0, fuse_h ? &src : nullptr, &pend_qkv)) !=
                hipSuccess)
                return e;
        }
        STEP("pf_qkv_post", (8.0 + 4.0 * pend_qkv) * T * ldq,
             launch_pf_qkv_post(s->pf_qkv, ldq, T, pos0, L.bq, L.bk, L.bv, s->rope, d.n_heads, d.n_kv_heads, d.head_dim,
                                kc, vc, s->st, s->pf_part, pend_qkv));
        PfAttn at{};
        at.q = s->pf_qkv; at.ldq = ldq; at.kc = kc; at.vc = vc; at.out = s->pf_att;
        at.T = T; at.pos0 = pos0; at.nh = d.n_heads; at.nkv = d.n_kv_heads; at.hd = d.head_dim; at.kvdim = kvdim;
        at.window = layer_window(d, l); at.scale = d.attn_scale; at.softcap = gemma ? d.attn_softcap : 0.0f;
        at.part = s->pf_part; at.part_cap = s->pf_part_cap; at.n_cu = s->m->ctx->n_cu;
        at.kvh = s->pf_kvh; at.kvs = s->pf_kvs; at.nblk = s->pf_kvblk;
        STEP("pf_attention", 8.0 * (double)kvdim * (pos0 + T) + 8.0 * T * qdim, launch_pf_attn(at, s->st));
        {
            const Tensor* w[1] = {&L.o};
            float* y[1] = {gemma ? s->pf_tmp : s->pf_x};
            // Gemma-2: the slices of tmp go into the post-norm
            int pend_t = 0;
            if ((e = pf_gemm(s, "pf_o", w, y, 1, H, T, !gemma, s->pf_att, qdim, nullptr,
                             defer_x ? &pend_x : (gemma ? &pend_t : nullptr))) != hipSuccess)
                return e;
            if (gemma)
                STEP("pf_postnorm", (12.0 + 4.0 * pend_t + (pend_t > 0 ? 4.0 : 0.0)) * T * H,
                     launch_pf_postnorm_add(s->pf_tmp, T, H, L.post_attn, s->pf_x, s->st, s->pf_part, pend_t));
        }
        if (!fuse_h) STEP("pf_norm", 8.0 * T * H, launch_pf_norm(s->pf_x, T, H, L.ffn_norm, eps, nk, s->pf_xn, ldx, s->st));
        {
            const Tensor* w[2] = {&L.gate, &L.up};
            float* y[2] = {s->pf_gu, s->pf_gu + F};
            const PfSrc src{PfSrc::NORM, s->pf_x, L.ffn_norm, eps, nk, pend_x};
            pend_x = 0;
            if ((e = pf_gemm(s, "pf_gate_up", w, y, 2, 2 * F, T, false, nullptr, 0, fuse_h ? &src : nullptr)) !=
                hipSuccess)
                return e;
        }
        if (!fuse_f) STEP("pf_act", 12.0 * T * F, launch_pf_act(s->pf_gu, T, F, gemma ? 1 : 0, s->pf_xn, ldx, s->st));
        {
            const Tensor* w[1] = {&L.down};
            float* y[1] = {gemma ? s->pf_tmp : s->pf_x};
            const PfSrc src{PfSrc::ACT, s->pf_gu, nullptr, 0.0f, gemma ? 1 : 0};
            // the last layer's sum is complete when the chunk ends; Gemma-2's goes into the post-norm
            int pend_t = 0;
            if ((e = pf_gemm(s, "pf_down", w, y, 1, H, T, !gemma, nullptr, 0, fuse_f ? &src : nullptr,
                             defer_x && l + 1 < d.n_layers ? &pend_x : (gemma ? &pend_t : nullptr))) != hipSuccess)
                return e;
            if (gemma)
                STEP("pf_postnorm", (12.0 + 4.0 * pend_t + (pend_t > 0 ? 4.0 : 0.0)) * T * H,
                     launch_pf_postnorm_add(s->pf_tmp, T, H, L.post_ffn, s->pf_x, s->st, s->pf_part, pend_t));
        }
    }
    return hipSuccess;
}

extern "C" int32_t fllm_prefill(fllm_seq* s, const int32_t* tokens, int32_t n, int32_t pos0) {
    NOT_NULL(s);
    if (n < 0) return fail(FLLM_E_ARG_RANGE, "n must be >= 0");
    if (n > 0) NOT_NULL(tokens);
    NOT_DISPOSED(s->m);
    APPEND_ORDER_OK(s);
    const fllm_model_desc& d = s->m->d;
    // The batched path runs when the positions continue the cache (the case of a prompt); with
    // debug capture, a single token, or positions that rewrite earlier slots it is n Forward calls.
    const bool batched = n >= 2 && pos0 == s->cur_len && !s->debug && prefill_batched_ok(s);
    // The checks of n Forward calls, before anything runs, on both paths: a prompt with an invalid
    // token or more positions than the cache has left is rejected with the cache unchanged (each
    // Forward appends one position). The per-token fllm_forward keeps the reference's
    // evict-then-throw at a full cache; a prompt does not start that way part-done.
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= d.vocab)
            return fail(FLLM_E_ARG_RANGE, "Token id %d is outside the valid vocabulary range [0, %d].", tokens[i],
                        d.vocab - 1);
    if ((int64_t)s->cur_len + n > s->max_seq)
        return fail(FLLM_E_ARG_RANGE, "KV cache full (%d positions)", s->max_seq);
    if (!batched) {
        for (int i = 0; i < n; i++) {
            int32_t rc = fllm_forward(s, tokens[i], pos0 + i);
            if (rc) return rc;
        }
        return FLLM_OK;
    }
    HIP_TRY(hipSetDevice(s->m->ctx->device));
    hipError_t e = prefill_alloc(s, n);
    if (e != hipSuccess) return fail(FLLM_E_OOM, "prefill scratch: %s", hipGetErrorString(e));
    // tokens per pass: the chunk, within the rows the scratch holds
    const int pass = std::min(prefill_pass(s), s->pf_cap);
    int done = 0;
    while (done < n) {
        const int T = n - done < pass ? n - done : pass;
        e = hipMemcpyAsync(s->pf_tok, tokens + done, sizeof(int32_t) * (size_t)T, hipMemcpyHostToDevice, s->st);
        if (e == hipSuccess) e = prefill_chunk(s, T, pos0 + done);
        if (e == hipSuccess) e = prof_collect(s);
        // the host buffer of the token ids is reused by the next chunk
        if (e == hipSuccess) e = hipStreamSynchronize(s->st);
        if (e != hipSuccess) return fail(FLLM_E_DEVICE, "prefill: %s", hipGetErrorString(e));
        done += T;
        s->cur_len = pos0 + done;
    }
    // the last token's logits and greedy token, with the step parameters of its Forward call
    const int T_last = n - ((n - 1) / pass) * pass;
    e = hipMemcpyAsync(s->x, s->pf_x + (size_t)(T_last - 1) * d.hidden, sizeof(float) * (size_t)d.hidden,
                       hipMemcpyDeviceToDevice, s->st);
    if (e == hipSuccess) e = launch_set_params(s->params, tokens[n - 1], pos0 + n - 1, pos0 + n - 1, s->st);
    if (e == hipSuccess) e = head_generic(s);
    if (e == hipSuccess) e = prof_collect(s);
    if (e != hipSuccess) return fail(FLLM_E_DEVICE, "prefill head: %s", hipGetErrorString(e));
    s->argmax_valid = true;
    return FLLM_OK;
}

extern "C" int32_t fllm_logits_copy(fllm_seq* s, float* dst, int64_t n) {
    NOT_NULL(s);
    NOT_NULL(dst);
    int V = s->m->d.vocab;
    if (n < V) return fail(FLLM_E_ARG, "destination must hold %d floats", V);
    HIP_TRY(hipMemcpyAsync(dst, s->logits, sizeof(float) * (size_t)V, hipMemcpyDeviceToHost, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    return FLLM_OK;
}

extern "C" int32_t fllm_logits_write(fllm_seq* s, const float* src, int64_t n) {
    NOT_NULL(s);
    NOT_NULL(src);
    int V = s->m->d.vocab;
    if (n != V) return fail(FLLM_E_ARG, "source must hold exactly %d floats", V);
    HIP_TRY(hipMemcpyAsync(s->logits, src, sizeof(float) * (size_t)V, hipMemcpyHostToDevice, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    s->argmax_valid = false;
    return FLLM_OK;
}

static const int kPinCand = 256;  // candidates the pinned block holds

// the sequence's pinned result block: [0] count or token, [16, 16 + kPinCand) ids, then kPinCand values
static hipError_t seq_pin(fllm_seq* s) {
    if (s->pin) return hipSuccess;
    return hipHostMalloc((void**)&s->pin, sizeof(int32_t) * (16 + 2 * (size_t)kPinCand), hipHostMallocDefault);
}

extern "C" int32_t fllm_sample_greedy(fllm_seq* s, int32_t* out_token) {
    NOT_NULL(s);
    NOT_NULL(out_token);
    // the decode step already reduced its logits to the greedy token; recompute only after the
    // logits were changed on the host or by the top-k sampler
    if (!s->argmax_valid) HIP_TRY(launch_argmax(s->logits, s->m->d.vocab, s->params, nullptr, 0, s->st));
    s->argmax_valid = true;
    if (seq_pin(s) == hipSuccess) {
        HIP_TRY(hipMemcpyAsync(s->pin, (const uint8_t*)s->params + offsetof(StepParams, argmax), sizeof(int32_t),
                               hipMemcpyDeviceToHost, s->st));
        HIP_TRY(hipStreamSynchronize(s->st));
        *out_token = s->pin[0];
        return FLLM_OK;
    }
    StepParams hp;
    HIP_TRY(hipMemcpyAsync(&hp, s->params, sizeof(hp), hipMemcpyDeviceToHost, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    *out_token = hp.argmax;
    return FLLM_OK;
}

extern "C" int32_t fllm_sample_topk(fllm_seq* s, float inv_temp, int32_t k, int32_t* ids, float* vals, int32_t cap,
                                    int32_t* n_out) {
    NOT_NULL(s);
    NOT_NULL(n_out);
    if (k < 1) return fail(FLLM_E_ARG_RANGE, "k must be at least 1.");
    // 1/Temperature of SamplerPipeline (SamplerPipeline.cs:67-70): finite and >= 0 (an infinite
    // temperature scales every logit to zero)
    if (!(inv_temp >= 0.0f) || isinf(inv_temp)) return fail(FLLM_E_ARG_RANGE, "inv_temp must be finite and >= 0.");
    if (cap > 0) { NOT_NULL(ids); NOT_NULL(vals); }
    int V = s->m->d.vocab;
    if (V > SAMPLE_MAX_VOCAB) return fail(FLLM_E_NOT_SUPPORTED, "device top-k handles vocabularies up to %d", SAMPLE_MAX_VOCAB);
    int dcap = cap < s->topk_cap ? cap : s->topk_cap;
    HIP_TRY(launch_topk(s->logits, V, inv_temp, k, dcap, s->topk_ids, s->topk_vals, s->topk_count, s->topk_sc, s->st));
    if (inv_temp != 1.0f) s->argmax_valid = false;
    // one round trip for the usual case: the count and the first candidates (as many as k, at
    // least 64, at most cap) come back together, through the pinned block when they fit in it;
    // only more survivors than that need a second copy
    int cnt = 0;
    int first = k < 64 ? 64 : k;
    first = first < dcap ? first : dcap;
    const bool pinned = first <= kPinCand && seq_pin(s) == hipSuccess;
    if (pinned) {
        HIP_TRY(hipMemcpyAsync(s->pin, s->topk_count, sizeof(int), hipMemcpyDeviceToHost, s->st));
        if (first > 0) {
            HIP_TRY(hipMemcpyAsync(s->pin + 16, s->topk_ids, sizeof(int) * (size_t)first, hipMemcpyDeviceToHost, s->st));
            HIP_TRY(hipMemcpyAsync(s->pin + 16 + kPinCand, s->topk_vals, sizeof(float) * (size_t)first,
                                   hipMemcpyDeviceToHost, s->st));
        }
        HIP_TRY(hipStreamSynchronize(s->st));
        cnt = s->pin[0];
        // the caller receives at most the survivors (fewer than `first` when fewer survive)
        const int got = cnt < first ? (cnt > 0 ? cnt : 0) : first;
        if (got > 0) {
            memcpy(ids, s->pin + 16, sizeof(int) * (size_t)got);
            memcpy(vals, s->pin + 16 + kPinCand, sizeof(float) * (size_t)got);
        }
    } else {
        HIP_TRY(hipMemcpyAsync(&cnt, s->topk_count, sizeof(int), hipMemcpyDeviceToHost, s->st));
        if (first > 0) {
            HIP_TRY(hipMemcpyAsync(ids, s->topk_ids, sizeof(int) * (size_t)first, hipMemcpyDeviceToHost, s->st));
            HIP_TRY(hipMemcpyAsync(vals, s->topk_vals, sizeof(float) * (size_t)first, hipMemcpyDeviceToHost, s->st));
        }
        HIP_TRY(hipStreamSynchronize(s->st));
    }
    *n_out = cnt;
    if (cnt > cap) return fail(FLLM_E_ARG, "%d candidates survive top-%d, capacity %d", cnt, k, cap);
    if (cnt > first) {
        size_t rest = (size_t)(cnt - first);
        HIP_TRY(hipMemcpyAsync(ids + first, s->topk_ids + first, sizeof(int) * rest, hipMemcpyDeviceToHost, s->st));
        HIP_TRY(hipMemcpyAsync(vals + first, s->topk_vals + first, sizeof(float) * rest, hipMemcpyDeviceToHost, s->st));
        HIP_TRY(hipStreamSynchronize(s->st));
    }
    return FLLM_OK;
}

extern "C" int32_t fllm_logits_penalize(fllm_seq* s, const int32_t* ids, int32_t n_ids, float penalty) {
    NOT_NULL(s);
    if (n_ids < 0) return fail(FLLM_E_ARG_RANGE, "n_ids must be >= 0");
    if (n_ids > 0) NOT_NULL(ids);
    if (!(penalty > 0.0f)) return fail(FLLM_E_ARG_RANGE, "Penalty must be greater than zero.");
    if (penalty == 1.0f || n_ids == 0) return FLLM_OK;  // every logit unchanged
    if (n_ids > s->pen_cap) {
        int cap = n_ids > 4096 ? n_ids : 4096;
        HIP_TRY(hipStreamSynchronize(s->st));
        int* p = nullptr;
        HIP_TRY(hipMalloc((void**)&p, sizeof(int) * (size_t)cap));
        if (s->pen_ids) {
            for (auto& a : s->allocs)
                if (a == (void*)s->pen_ids) a = (void*)p;
            hipFree(s->pen_ids);
        } else {
            s->allocs.push_back(p);
        }
        s->pen_ids = p;
        s->pen_cap = cap;
    }
    HIP_TRY(hipMemcpyAsync(s->pen_ids, ids, sizeof(int32_t) * (size_t)n_ids, hipMemcpyHostToDevice, s->st));
    HIP_TRY(launch_rep_penalty(s->logits, s->m->d.vocab, s->pen_ids, n_ids, penalty, s->pen_counts, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));  // the host's id array may be reused once this returns
    s->argmax_valid = false;
    return FLLM_OK;
}

extern "C" int32_t fllm_sample_nucleus(fllm_seq* s, float inv_temp, float top_p, float u, int32_t* out_token) {
    NOT_NULL(s);
    NOT_NULL(out_token);
    if (!(top_p > 0.0f && top_p <= 1.0f)) return fail(FLLM_E_ARG_RANGE, "topP must be in (0, 1].");
    if (!(u >= 0.0f && u < 1.0f)) return fail(FLLM_E_ARG_RANGE, "u must be in [0, 1).");
    if (!(inv_temp >= 0.0f) || isinf(inv_temp)) return fail(FLLM_E_ARG_RANGE, "inv_temp must be finite and >= 0.");
    int V = s->m->d.vocab;
    if (V > SAMPLE_MAX_VOCAB) return fail(FLLM_E_NOT_SUPPORTED, "device nucleus sampling handles vocabularies up to %d", SAMPLE_MAX_VOCAB);
    HIP_TRY(launch_sample_nucleus(s->logits, V, inv_temp, top_p, u, s->probs, s->samp_token, s->nuc_sc, s->st));
    if (inv_temp != 1.0f) s->argmax_valid = false;
    int tok = 0;
    if (seq_pin(s) == hipSuccess) {
        HIP_TRY(hipMemcpyAsync(s->pin, s->samp_token, sizeof(int), hipMemcpyDeviceToHost, s->st));
        HIP_TRY(hipStreamSynchronize(s->st));
        tok = s->pin[0];
    } else {
        HIP_TRY(hipMemcpyAsync(&tok, s->samp_token, sizeof(int), hipMemcpyDeviceToHost, s->st));
        HIP_TRY(hipStreamSynchronize(s->st));
    }
    *out_token = tok;
    return FLLM_OK;
}

extern "C" int32_t fllm_probs_copy(fllm_seq* s, float* dst, int64_t n) {
    NOT_NULL(s);
    NOT_NULL(dst);
    int V = s->m->d.vocab;
    if (n < V) return fail(FLLM_E_ARG, "destination must hold %d floats", V);
    HIP_TRY(hipMemcpyAsync(dst, s->probs, sizeof(float) * (size_t)V, hipMemcpyDeviceToHost, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    return FLLM_OK;
}

extern "C" int32_t fllm_debug_hidden(fllm_seq* s, int32_t layer, float* dst, int64_t n) {
    NOT_NULL(s);
    NOT_NULL(dst);
    const fllm_model_desc& d = s->m->d;
    if (!s->debug) return fail(FLLM_E_INVALID_OP, "debug capture is off (fllm_seq_set_debug)");
    if (layer < 0 || layer > d.n_layers) return fail(FLLM_E_ARG_RANGE, "layer %d outside [0, %d]", layer, d.n_layers);
    if (n < d.hidden) return fail(FLLM_E_ARG, "destination must hold %d floats", d.hidden);
    HIP_TRY(hipMemcpyAsync(dst, s->hidden_dbg + (size_t)layer * d.hidden, sizeof(float) * (size_t)d.hidden,
                           hipMemcpyDeviceToHost, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    return FLLM_OK;
}

extern "C" int32_t fllm_kv_read(fllm_seq* s, int32_t layer, int32_t kind, float* dst, int64_t n) {
    NOT_NULL(s);
    NOT_NULL(dst);
    const fllm_model_desc& d = s->m->d;
    if (layer < 0 || layer >= d.n_layers) return fail(FLLM_E_ARG_RANGE, "Layer index must be in [0, %d].", d.n_layers - 1);
    if (kind != 0 && kind != 1) return fail(FLLM_E_ARG_RANGE, "kind must be 0 (keys) or 1 (values)");
    int64_t cnt = (int64_t)kv_effective(s, layer) * s->m->kvdim;
    if (n < cnt) return fail(FLLM_E_ARG, "destination must hold %lld floats", (long long)cnt);
    if (cnt == 0) return FLLM_OK;
    const float* src = (kind == 0 ? s->kc : s->vc) + (size_t)layer * s->max_seq * s->m->kvdim;
    HIP_TRY(hipMemcpyAsync(dst, src, sizeof(float) * (size_t)cnt, hipMemcpyDeviceToHost, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_set_profile(fllm_seq* s, int32_t enable) {
    NOT_NULL(s);
    s->profile = enable != 0;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_profile_count(fllm_seq* s, int32_t* n) {
    NOT_NULL(s);
    NOT_NULL(n);
    *n = (int32_t)s->agg_order.size();
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_profile_entry(fllm_seq* s, int32_t i, char* name, int32_t name_cap, int64_t* launches,
                                          double* total_ms, double* total_bytes) {
    NOT_NULL(s);
    if (i < 0 || i >= (int32_t)s->agg_order.size()) return fail(FLLM_E_ARG_RANGE, "entry %d out of range", i);
    const std::string& nm = s->agg_order[(size_t)i];
    const ProfAgg& a = s->agg[nm];
    if (name && name_cap > 0) {
        snprintf(name, (size_t)name_cap, "%s", nm.c_str());
    }
    if (launches) *launches = a.launches;
    if (total_ms) *total_ms = a.ms;
    if (total_bytes) *total_bytes = a.bytes;
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_profile_reset(fllm_seq* s) {
    NOT_NULL(s);
    s->agg.clear();
    s->agg_order.clear();
    s->pending.clear();
    s->launch_names.clear();
    return FLLM_OK;
}

extern "C" int32_t fllm_seq_profile_launch(fllm_seq* s, int32_t i, char* name, int32_t name_cap) {
    NOT_NULL(s);
    NOT_NULL(name);
    if (i < 0 || i >= (int32_t)s->launch_names.size()) return fail(FLLM_E_ARG_RANGE, "launch %d out of range", i);
    if (name_cap > 0) snprintf(name, (size_t)name_cap, "%s", s->launch_names[(size_t)i].c_str());
    return FLLM_OK;
}
