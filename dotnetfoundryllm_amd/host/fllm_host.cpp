// fllm_host.cpp — the host side above the C ABI (include/fllm_host.h): GGUF reader and the
// loader's upload seam, XoshiroRandom + SamplerPipeline over the device sampler, the token
// loop of LlamaLanguageModel.GenerateAsync, and the seeded synthetic tensor generator.
// Plain C++17; talks to the device only through include/fllm.h.
#include "../../include/fllm_host.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <vector>

// =====================================================================================
// errors
// =====================================================================================
static thread_local std::string g_herr;

static int32_t hfail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_herr = buf;
    return code;
}

// Propagates a device-library failure, keeping its message.
static int32_t dfail(int32_t code) {
    g_herr = fllm_last_error();
    return code;
}

extern "C" FLLM_API const char* fllmh_last_error(void) { return g_herr.c_str(); }

// =====================================================================================
// half / bfloat16 rounding
// =====================================================================================
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

extern "C" uint16_t fllmh_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (ex == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t half = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return (uint16_t)half;
}

extern "C" uint16_t fllmh_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7FFFu + lsb;
    return (uint16_t)(x >> 16);
}

// =====================================================================================
// synthetic tensors
// =====================================================================================
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

namespace {
struct Rng {
    uint64_t s;
    uint64_t next() { s += 0x9e3779b97f4a7c15ULL; return mix64(s); }
    double uni() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
    float uni_f(float a, float b) { return (float)(a + (b - a) * uni()); }
    double normal() {
        double u1 = 1.0 - uni(), u2 = uni();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};
}  // namespace

static Rng block_rng(uint64_t seed, uint64_t tid, uint64_t blk) {
    Rng r;
    r.s = mix64(seed ^ mix64(tid * 0xD1B54A32D192ED03ULL + 1) ^ mix64(blk * 0x8CB92BA72F3D8DD7ULL + 2));
    return r;
}

static void put16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

static void fill_bytes(Rng& r, uint8_t* p, int n) {
    for (int i = 0; i < n; i += 8) {
        uint64_t v = r.next();
        for (int j = 0; j < 8 && i + j < n; j++) p[i + j] = (uint8_t)(v >> (8 * j));
    }
}

// Inverse of Dequantizer.DecodeKScaleMin (Dequantizer.cs:506-521).
static void pack_kscale_min(const int* sc, const int* mn, uint8_t* p) {
    for (int g = 0; g < 4; g++) {
        p[g] = (uint8_t)((sc[g] & 63) | ((sc[g + 4] >> 4) << 6));
        p[g + 4] = (uint8_t)((mn[g] & 63) | ((mn[g + 4] >> 4) << 6));
    }
    for (int g = 4; g < 8; g++) p[g + 4] = (uint8_t)((sc[g] & 15) | ((mn[g] & 15) << 4));
}

static int block_geom(int type, int& bb, int& be) {
    switch (type) {
        case FLLM_TYPE_F32: bb = 4 * 256; be = 256; return 0;
        case FLLM_TYPE_F16: case FLLM_TYPE_BF16: bb = 2 * 256; be = 256; return 0;
        case FLLM_TYPE_Q4_0: bb = 18; be = 32; return 0;
        case FLLM_TYPE_Q8_0: bb = 34; be = 32; return 0;
        case FLLM_TYPE_Q4_K: bb = 144; be = 256; return 0;
        case FLLM_TYPE_Q5_K: bb = 176; be = 256; return 0;
        case FLLM_TYPE_Q6_K: bb = 210; be = 256; return 0;
        case FLLM_TYPE_Q8_K: bb = 292; be = 256; return 0;
        default: return -1;
    }
}

static void synth_block(int type, Rng& r, int32_t dist, float p0, float p1, uint8_t* o, int64_t elems_here) {
    switch (type) {
        case FLLM_TYPE_F32: case FLLM_TYPE_F16: case FLLM_TYPE_BF16:
            for (int64_t i = 0; i < elems_here; i++) {
                float v = dist == 0 ? (float)(p0 + p1 * r.normal()) : dist == 1 ? p0 : r.uni_f(p0, p1);
                if (type == FLLM_TYPE_F32) memcpy(o + 4 * i, &v, 4);
                else if (type == FLLM_TYPE_F16) put16(o + 2 * i, fllmh_f32_to_f16(v));
                else put16(o + 2 * i, fllmh_f32_to_bf16(v));
            }
            break;
        case FLLM_TYPE_Q4_K: case FLLM_TYPE_Q5_K: {
            put16(o, fllmh_f32_to_f16(r.uni_f(p0, p1)));
            put16(o + 2, fllmh_f32_to_f16(r.uni_f(p0, p1)));
            int sc[8], mn[8];
            uint64_t v = r.next(), v2 = r.next();
            for (int g = 0; g < 8; g++) {
                sc[g] = (int)((v >> (6 * g)) & 63);
                mn[g] = (int)((v2 >> (6 * g)) & 63);
            }
            pack_kscale_min(sc, mn, o + 4);
            fill_bytes(r, o + 16, type == FLLM_TYPE_Q4_K ? 128 : 160);
            break;
        }
        case FLLM_TYPE_Q6_K: {
            fill_bytes(r, o, 192);
            for (int i = 0; i < 16; i++) o[192 + i] = (uint8_t)(r.next() & 63);
            put16(o + 208, fllmh_f32_to_f16(r.uni_f(p0, p1)));
            break;
        }
        case FLLM_TYPE_Q8_0: {
            put16(o, fllmh_f32_to_f16(r.uni_f(p0, p1)));
            for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)(int8_t)((int)(r.next() % 255u) - 127);
            break;
        }
        case FLLM_TYPE_Q4_0: {
            put16(o, fllmh_f32_to_f16(r.uni_f(p0, p1)));
            fill_bytes(r, o + 2, 16);
            break;
        }
        case FLLM_TYPE_Q8_K: {
            float d = r.uni_f(p0, p1);
            memcpy(o, &d, 4);
            for (int i = 0; i < 256; i++) o[4 + i] = (uint8_t)(int8_t)((int)(r.next() % 255u) - 127);
            for (int b = 0; b < 16; b++) {
                int s = 0;
                for (int i = 0; i < 16; i++) s += (int8_t)o[4 + 16 * b + i];
                put16(o + 260 + 2 * b, (uint16_t)(int16_t)s);
            }
            break;
        }
    }
}

extern "C" int32_t fllmh_synth_tensor(int32_t type, uint64_t seed, uint64_t tensor_id, int64_t n_elems, int32_t dist,
                                      float p0, float p1, void* dst, uint64_t dst_bytes, int32_t threads) {
    int bb, be;
    if (block_geom(type, bb, be) != 0) return hfail(FLLM_E_NOT_SUPPORTED, "type %d not supported", type);
    if (!dst) return hfail(FLLM_E_NULL, "dst must not be null");
    bool flt = type == FLLM_TYPE_F32 || type == FLLM_TYPE_F16 || type == FLLM_TYPE_BF16;
    if (!flt && n_elems % be != 0) return hfail(FLLM_E_ARG, "%lld elements is not a whole number of blocks", (long long)n_elems);
    int esz = type == FLLM_TYPE_F32 ? 4 : 2;
    uint64_t need = flt ? (uint64_t)n_elems * esz : (uint64_t)(n_elems / be) * bb;
    if (dst_bytes != need) return hfail(FLLM_E_ARG, "dst holds %llu bytes, %llu needed", (unsigned long long)dst_bytes, (unsigned long long)need);
    int64_t nblk = (n_elems + be - 1) / be;
    int nt = threads;
    if (nt <= 0) {  // default: the hardware threads, at most 16 (one GPU's share of a host)
        nt = (int)std::thread::hardware_concurrency();
        if (nt > 16) nt = 16;
    }
    if (nt < 1) nt = 1;
    if (nblk < 4096) nt = 1;
    uint8_t* out = (uint8_t*)dst;
    auto work = [&](int64_t b0, int64_t b1) {
        for (int64_t b = b0; b < b1; b++) {
            Rng r = block_rng(seed, tensor_id, (uint64_t)b);
            int64_t here = std::min<int64_t>(be, n_elems - b * be);
            synth_block(type, r, dist, p0, p1, out + (flt ? (uint64_t)b * be * esz : (uint64_t)b * bb), here);
        }
    };
    if (nt == 1) {
        work(0, nblk);
    } else {
        std::vector<std::thread> th;
        int64_t per = (nblk + nt - 1) / nt;
        for (int t = 0; t < nt; t++) {
            int64_t b0 = t * per, b1 = std::min<int64_t>(nblk, b0 + per);
            if (b0 < b1) th.emplace_back(work, b0, b1);
        }
        for (auto& t : th) t.join();
    }
    return FLLM_OK;
}

extern "C" int32_t fllmh_synth_tokens(uint64_t seed, uint64_t stream, int32_t vocab, int32_t* dst, int32_t n) {
    if (vocab <= 0) return hfail(FLLM_E_ARG_RANGE, "vocab must be positive");
    if (n > 0 && !dst) return hfail(FLLM_E_NULL, "dst must not be null");
    Rng r = block_rng(seed, 0x70C3E5ULL ^ stream, 0);
    for (int i = 0; i < n; i++) dst[i] = (int32_t)(r.next() % (uint64_t)vocab);
    return FLLM_OK;
}

// =====================================================================================
// GGUF reader (GgufReader.cs:37-93 / :95-167)
// =====================================================================================
namespace {
enum GType { U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32 = 6, BOOL = 7, STR = 8, ARR = 9, U64 = 10, I64 = 11, F64 = 12 };

struct GVal {
    uint32_t type = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    float f32 = 0;
    bool has_f32 = false;
    std::string s;
    uint64_t arr_len = 0;
};

struct GTensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
    int64_t elems() const { int64_t c = 1; for (auto d : dims) c *= (int64_t)d; return c; }
};

struct Cursor {
    const uint8_t* p;
    uint64_t n, pos = 0;
    bool ok = true;
    bool need(uint64_t k) { if (k > n - pos) { ok = false; return false; } return true; }  // pos <= n
    uint64_t rd(int bytes) {
        if (!need((uint64_t)bytes)) return 0;
        uint64_t v = 0;
        for (int b = 0; b < bytes; b++) v |= (uint64_t)p[pos + b] << (8 * b);
        pos += (uint64_t)bytes;
        return v;
    }
    std::string str() {
        uint64_t len = rd(8);
        if (!ok || !need(len)) return std::string();
        std::string s((const char*)p + pos, (size_t)len);
        pos += len;
        return s;
    }
};

struct GFile {
    uint32_t version = 0;
    std::map<std::string, GVal> meta;
    std::vector<GTensor> tensors;
    std::map<std::string, size_t> index;
    uint64_t data_start = 0;
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    int fd = -1;
    void* map = nullptr;
    ~GFile() {
        if (map && map != MAP_FAILED) munmap(map, (size_t)size);
        if (fd >= 0) close(fd);
    }
};
}  // namespace

static bool read_scalar(Cursor& c, uint32_t t, GVal& v) {
    v.type = t;
    switch (t) {
        case U8: v.u = c.rd(1); break;
        case I8: v.i = (int8_t)c.rd(1); break;
        case U16: v.u = c.rd(2); break;
        case I16: v.i = (int16_t)c.rd(2); break;
        case U32: v.u = c.rd(4); break;
        case I32: v.i = (int32_t)c.rd(4); break;
        case F32: { uint32_t b = (uint32_t)c.rd(4); memcpy(&v.f32, &b, 4); v.has_f32 = true; break; }
        case BOOL: v.u = c.rd(1) != 0; break;
        case STR: v.s = c.str(); break;
        case U64: v.u = c.rd(8); break;
        case I64: v.i = (int64_t)c.rd(8); break;
        case F64: { uint64_t b = c.rd(8); memcpy(&v.f, &b, 8); break; }
        default: return false;
    }
    return c.ok;
}

static int32_t open_gguf(const char* path, GFile& g) {
    if (!path || !*path) return hfail(FLLM_E_ARG, "path must not be empty");
    g.fd = open(path, O_RDONLY);
    if (g.fd < 0) return hfail(FLLM_E_MODEL_LOAD, "Failed to read GGUF file: cannot open %s", path);
    struct stat st;
    if (fstat(g.fd, &st) != 0 || st.st_size <= 0) return hfail(FLLM_E_MODEL_LOAD, "GGUF file is empty.");
    g.size = (uint64_t)st.st_size;
    g.map = mmap(nullptr, (size_t)g.size, PROT_READ, MAP_PRIVATE, g.fd, 0);
    if (g.map == MAP_FAILED) return hfail(FLLM_E_MODEL_LOAD, "Failed to read GGUF file: mmap failed");
    g.base = (const uint8_t*)g.map;
    Cursor c{g.base, g.size};
    if (g.size < 4 || memcmp(g.base, "GGUF", 4) != 0) return hfail(FLLM_E_MODEL_LOAD, "Not a GGUF file: invalid magic bytes.");
    c.pos = 4;
    g.version = (uint32_t)c.rd(4);
    if (g.version != 2 && g.version != 3) return hfail(FLLM_E_MODEL_LOAD, "Unsupported GGUF version %u. Expected 2 or 3.", g.version);
    uint64_t n_tensors = c.rd(8), n_kv = c.rd(8);
    for (uint64_t i = 0; i < n_kv && c.ok; i++) {
        std::string key = c.str();
        uint32_t t = (uint32_t)c.rd(4);
        GVal v;
        if (t == ARR) {
            uint32_t et = (uint32_t)c.rd(4);
            uint64_t cnt = g.version >= 3 ? c.rd(8) : c.rd(4);
            v.type = ARR;
            v.arr_len = cnt;
            for (uint64_t j = 0; j < cnt && c.ok; j++) {
                GVal e;
                if (!read_scalar(c, et, e)) {
                    if (!c.ok) break;
                    return hfail(FLLM_E_MODEL_LOAD, "Failed to read GGUF file: bad array element type %u", et);
                }
            }
        } else if (!read_scalar(c, t, v)) {
            if (!c.ok) break;
            return hfail(FLLM_E_MODEL_LOAD, "Failed to read GGUF file: Unknown GGUF metadata value type: %u", t);
        }
        g.meta[key] = v;
    }
    if (!c.ok) return hfail(FLLM_E_MODEL_LOAD, "Failed to read GGUF file: truncated metadata");
    for (uint64_t i = 0; i < n_tensors && c.ok; i++) {
        GTensor t;
        t.name = c.str();
        uint32_t nd = (uint32_t)c.rd(4);
        for (uint32_t d = 0; d < nd && c.ok; d++) t.dims.push_back(c.rd(8));
        t.type = (uint32_t)c.rd(4);
        t.offset = c.rd(8);
        g.index[t.name] = g.tensors.size();
        g.tensors.push_back(t);
    }
    if (!c.ok) return hfail(FLLM_E_MODEL_LOAD, "Failed to read GGUF file: truncated header");
    uint64_t align = 32;  // GgufReader.cs:11, :78-87
    auto it = g.meta.find("general.alignment");
    if (it != g.meta.end() && (it->second.type == U32 || it->second.type == U64) && it->second.u > 0) align = it->second.u;
    g.data_start = (c.pos + align - 1) / align * align;
    return FLLM_OK;
}

// Metadata helpers with GgufModelLoader's defaults (GgufModelLoader.cs:436-478).
static std::string get_str(const GFile& g, const std::string& k, const std::string& def) {
    auto it = g.meta.find(k);
    return (it != g.meta.end() && it->second.type == STR) ? it->second.s : def;
}
static uint64_t get_uint(const GFile& g, const std::string& k, uint64_t def, bool arr_len = false) {
    auto it = g.meta.find(k);
    if (it == g.meta.end()) return def;
    const GVal& v = it->second;
    if (arr_len && v.type == ARR) return v.arr_len;
    switch (v.type) {
        case U8: case U16: case U32: case U64: return v.u;
        case I32: case I64: return (uint64_t)v.i;
        default: return def;
    }
}
static float get_float(const GFile& g, const std::string& k, float def) {
    auto it = g.meta.find(k);
    return (it != g.meta.end() && it->second.has_f32) ? it->second.f32 : def;
}
static bool ieq(const std::string& a, const char* b) {
    size_t n = strlen(b);
    if (a.size() != n) return false;
    for (size_t i = 0; i < n; i++)
        if (tolower((unsigned char)a[i]) != tolower((unsigned char)b[i])) return false;
    return true;
}

// GgufModelLoader.Build -> BuildConfig / BuildGemma2 (GgufModelLoader.cs:89-102, :213-241, :296-322).
static int32_t build_desc(const GFile& g, fllmh_model_info* info) {
    fllm_model_desc d{};
    std::string arch = get_str(g, "general.architecture", "llama");
    std::string p;
    if (arch == "llama" || arch == "llama3" || arch == "llama4") d.arch = FLLM_ARCH_LLAMA;
    else if (arch == "mistral") d.arch = FLLM_ARCH_MISTRAL;
    else if (arch == "gemma" || arch == "gemma2") d.arch = FLLM_ARCH_GEMMA2;
    else if (arch == "qwen2") d.arch = FLLM_ARCH_QWEN2;
    else return hfail(FLLM_E_NOT_SUPPORTED, "Architecture '%s' is not supported. Supported: llama, mistral, gemma2, qwen2.", arch.c_str());
    if (d.arch == FLLM_ARCH_GEMMA2) p = g.meta.count("gemma2.block_count") ? "gemma2" : "gemma";
    else p = arch;
    d.n_layers = (int32_t)get_uint(g, p + ".block_count", 0);
    d.hidden = (int32_t)get_uint(g, p + ".embedding_length", 0);
    d.ffn = (int32_t)get_uint(g, p + ".feed_forward_length", 0);
    d.n_heads = (int32_t)get_uint(g, p + ".attention.head_count", 0);
    d.n_kv_heads = (int32_t)get_uint(g, p + ".attention.head_count_kv", get_uint(g, p + ".attention.head_count", 0));
    d.max_ctx = (int32_t)get_uint(g, p + ".context_length", 4096);
    d.vocab = (int32_t)get_uint(g, p + ".vocab_size", get_uint(g, "tokenizer.ggml.tokens", 32000, true));
    d.rope_base = get_float(g, p + ".rope.freq_base", 10000.0f);
    d.rope_scale = get_float(g, p + ".rope.scaling.factor", get_float(g, p + ".rope.freq_scale", 1.0f));
    std::string rtype = get_str(g, p + ".rope.scaling.type", "none");
    d.rope_scaled = (ieq(rtype, "linear") || ieq(rtype, "yarn")) ? 1 : 0;
    d.sliding_window = 0x7FFFFFFF;
    if (d.n_heads <= 0) return hfail(FLLM_E_MODEL_LOAD, "attention.head_count missing or zero");
    if (d.arch == FLLM_ARCH_GEMMA2) {
        int hdo = (int)get_uint(g, p + ".attention.key_length", 0);
        d.head_dim = hdo > 0 ? hdo : d.hidden / d.n_heads;
        d.sliding_window = (int32_t)get_uint(g, p + ".attention.sliding_window", 0x7FFFFFFFull);
        d.attn_softcap = get_float(g, p + ".attn_logit_softcapping", 0.0f);
        d.final_softcap = get_float(g, p + ".final_logit_softcapping", 0.0f);
        d.attn_scale = get_float(g, p + ".attention.query_pre_attn_scalar", 1.0f / sqrtf((float)d.head_dim));
        d.norm_eps = 1e-6f;  // GemmaRmsNorm, TensorOperations.cs:93
    } else {
        d.head_dim = d.hidden / d.n_heads;  // LlamaConfig.cs:27
        d.attn_scale = 1.0f / sqrtf((float)d.head_dim);
        d.norm_eps = 1e-5f;  // RmsNorm default, never read from GGUF (TensorOperations.cs:42)
        if (d.arch == FLLM_ARCH_MISTRAL)
            d.sliding_window = (int32_t)get_uint(g, "mistral.attention.sliding_window", 0x7FFFFFFFull);
    }
    info->desc = d;
    info->bos_token_id = (int32_t)get_uint(g, "tokenizer.ggml.bos_token_id", 1);
    info->eos_token_id = (int32_t)get_uint(g, "tokenizer.ggml.eos_token_id", 2);
    info->gguf_version = (int32_t)g.version;
    info->n_tensors = (int32_t)g.tensors.size();
    info->data_offset = g.data_start;
    return FLLM_OK;
}

extern "C" int32_t fllmh_read_gguf_info(const char* path, fllmh_model_info* info) {
    if (!info) return hfail(FLLM_E_NULL, "info must not be null");
    GFile g;
    int32_t rc = open_gguf(path, g);
    if (rc) return rc;
    return build_desc(g, info);
}

// GgufFile.ComputeByteSize (GgufFile.cs:99-122).
static bool tensor_bytes(const GTensor& t, uint64_t& out) {
    int64_t e = t.elems();
    switch (t.type) {
        case 0: out = (uint64_t)e * 4; return true;
        case 1: case 30: out = (uint64_t)e * 2; return true;
        case 2: out = (uint64_t)(e / 32) * 18; return true;
        case 3: out = (uint64_t)(e / 32) * 20; return true;
        case 6: out = (uint64_t)(e / 32) * 22; return true;
        case 7: out = (uint64_t)(e / 32) * 24; return true;
        case 8: out = (uint64_t)(e / 32) * 34; return true;
        case 9: out = (uint64_t)(e / 32) * 36; return true;
        case 12: out = (uint64_t)(e / 256) * 144; return true;
        case 13: out = (uint64_t)(e / 256) * 176; return true;
        case 14: out = (uint64_t)(e / 256) * 210; return true;
        case 15: out = (uint64_t)(e / 256) * 292; return true;
        default: return false;
    }
}

extern "C" int32_t fllmh_load_gguf(fllm_ctx* ctx, const char* path, fllm_model** model, fllmh_model_info* info) {
    if (!ctx) return hfail(FLLM_E_NULL, "ctx must not be null");
    if (!model) return hfail(FLLM_E_NULL, "model must not be null");
    *model = nullptr;
    fllmh_model_info local;
    if (!info) info = &local;
    GFile g;
    int32_t rc = open_gguf(path, g);
    if (rc) return rc;
    rc = build_desc(g, info);
    if (rc) return rc;
    fllm_model* m = nullptr;
    rc = fllm_model_create(ctx, &info->desc, &m);
    if (rc) return dfail(rc);
    // Tensor names read by LoadWeights / LoadQwen2Weights / LoadGemma2Weights.
    struct Want { std::string name; int slot; int layer; bool required; };
    std::vector<Want> want;
    const fllm_model_desc& d = info->desc;
    want.push_back({"token_embd.weight", FLLM_SLOT_TOKEN_EMBD, 0, true});
    want.push_back({"output_norm.weight", FLLM_SLOT_OUTPUT_NORM, 0, true});
    want.push_back({"output.weight", FLLM_SLOT_OUTPUT, 0, false});
    for (int l = 0; l < d.n_layers; l++) {
        std::string b = "blk." + std::to_string(l) + ".";
        want.push_back({b + "attn_norm.weight", FLLM_SLOT_ATTN_NORM, l, true});
        want.push_back({b + "attn_q.weight", FLLM_SLOT_ATTN_Q, l, true});
        want.push_back({b + "attn_k.weight", FLLM_SLOT_ATTN_K, l, true});
        want.push_back({b + "attn_v.weight", FLLM_SLOT_ATTN_V, l, true});
        want.push_back({b + "attn_output.weight", FLLM_SLOT_ATTN_OUTPUT, l, true});
        want.push_back({b + "ffn_norm.weight", FLLM_SLOT_FFN_NORM, l, true});
        want.push_back({b + "ffn_gate.weight", FLLM_SLOT_FFN_GATE, l, true});
        want.push_back({b + "ffn_up.weight", FLLM_SLOT_FFN_UP, l, true});
        want.push_back({b + "ffn_down.weight", FLLM_SLOT_FFN_DOWN, l, true});
        if (d.arch == FLLM_ARCH_QWEN2) {
            want.push_back({b + "attn_q.bias", FLLM_SLOT_ATTN_Q_BIAS, l, true});
            want.push_back({b + "attn_k.bias", FLLM_SLOT_ATTN_K_BIAS, l, true});
            want.push_back({b + "attn_v.bias", FLLM_SLOT_ATTN_V_BIAS, l, true});
        }
        if (d.arch == FLLM_ARCH_GEMMA2) {
            want.push_back({b + "post_attn_norm.weight", FLLM_SLOT_POST_ATTN_NORM, l, true});
            want.push_back({b + "post_ffn_norm.weight", FLLM_SLOT_POST_FFN_NORM, l, true});
        }
    }
    for (const Want& w : want) {
        auto it = g.index.find(w.name);
        if (it == g.index.end()) {
            if (!w.required) continue;
            fllm_model_destroy(m);
            return hfail(FLLM_E_INVALID_OP, "Required tensor '%s' not found in GGUF file.", w.name.c_str());
        }
        const GTensor& t = g.tensors[it->second];
        uint64_t nb;
        if (!tensor_bytes(t, nb)) {
            fllm_model_destroy(m);
            return hfail(FLLM_E_NOT_SUPPORTED, "Cannot compute byte size for tensor type %u.", t.type);
        }
        uint64_t off = g.data_start + t.offset;
        if (off > g.size || nb > g.size - off) {
            fllm_model_destroy(m);
            return hfail(FLLM_E_MODEL_LOAD, "tensor '%s' extends past the end of the file", w.name.c_str());
        }
        rc = fllm_model_upload(m, w.slot, w.layer, (int32_t)t.type, g.base + off, nb);
        if (rc) {
            int32_t code = dfail(rc);
            g_herr = w.name + ": " + g_herr;
            fllm_model_destroy(m);
            return code;
        }
    }
    rc = fllm_model_finalize(m);
    if (rc) { int32_t code = dfail(rc); fllm_model_destroy(m); return code; }
    *model = m;
    return FLLM_OK;
}

// =====================================================================================
// XoshiroRandom (XoshiroRandom.cs:4-49)
// =====================================================================================
static uint64_t splitmix_step(uint64_t* x) {
    *x += 0x9e3779b97f4a7c15ULL;
    return mix64(*x);
}
static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

extern "C" void fllmh_xoshiro_init(fllmh_xoshiro* r, uint64_t seed) {
    r->s0 = splitmix_step(&seed);
    r->s1 = splitmix_step(&seed);
    r->s2 = splitmix_step(&seed);
    r->s3 = splitmix_step(&seed);
}
extern "C" uint64_t fllmh_xoshiro_next(fllmh_xoshiro* r) {
    uint64_t result = rotl(r->s1 * 5, 7) * 9;
    uint64_t t = r->s1 << 17;
    r->s2 ^= r->s0;
    r->s3 ^= r->s1;
    r->s1 ^= r->s2;
    r->s0 ^= r->s3;
    r->s2 ^= t;
    r->s3 = rotl(r->s3, 45);
    return result;
}
extern "C" float fllmh_xoshiro_next_float(fllmh_xoshiro* r) {
    return (float)((double)(fllmh_xoshiro_next(r) >> 11) * (1.0 / 9007199254740992.0));
}

// =====================================================================================
// SamplerPipeline (SamplerPipeline.cs:14-89) over the device sampler
// =====================================================================================
struct fllmh_sampler {
    float temperature;
    int top_k;
    float top_p;
    fllmh_xoshiro rng;
    std::vector<float> buf;
    std::vector<int32_t> ids;
};

extern "C" int32_t fllmh_sampler_create(float temperature, int32_t top_k, float top_p, uint64_t seed, fllmh_sampler** out) {
    if (!out) return hfail(FLLM_E_NULL, "out must not be null");
    *out = nullptr;
    if (!(temperature >= 0.0f)) return hfail(FLLM_E_ARG_RANGE, "Temperature must be >= 0.");
    if (!(top_p > 0.0f && top_p <= 1.0f)) return hfail(FLLM_E_ARG_RANGE, "topP must be in (0, 1].");
    fllmh_sampler* s = new fllmh_sampler();
    s->temperature = temperature;
    s->top_k = top_k;
    s->top_p = top_p;
    if (seed == 0) seed = (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count();
    fllmh_xoshiro_init(&s->rng, seed);
    *out = s;
    return FLLM_OK;
}

extern "C" int32_t fllmh_sampler_destroy(fllmh_sampler* s) {
    delete s;
    return FLLM_OK;
}

// Softmax (TensorOperations.cs:23-39) over values already holding -inf for filtered entries.
static void softmax_inplace(float* x, int n) {
    if (n <= 0) return;
    float mx = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    for (int i = 0; i < n; i++) x[i] = std::exp(x[i] + (-mx));
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += x[i];
    if (sum != 0.0f) for (int i = 0; i < n; i++) x[i] = x[i] / sum;
}

// TopPSampler.ApplyTopP (TopPSampler.cs:39-89) on probabilities.
static void apply_top_p(float* probs, int n, float p) {
    if (p >= 1.0f) return;
    std::vector<int> idx((size_t)n);
    for (int i = 0; i < n; i++) idx[(size_t)i] = i;
    std::vector<float> cp(probs, probs + n);
    std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return cp[(size_t)a] > cp[(size_t)b]; });
    float cum = 0.0f;
    bool reached = false;
    for (int r = 0; r < n; r++) {
        if (reached) probs[idx[(size_t)r]] = 0.0f;
        else { cum += probs[idx[(size_t)r]]; if (cum >= p) reached = true; }
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += probs[i];
    if (sum > 0.0f) for (int i = 0; i < n; i++) probs[i] = probs[i] / sum;
}

// TemperatureSampler.SampleFromProbabilities (TemperatureSampler.cs:53-70) over (index, prob)
// pairs in ascending index order; entries not listed have probability 0.
static int32_t sample_cdf(fllmh_xoshiro* r, const int32_t* idx, const float* probs, int n, int vocab) {
    float u = fllmh_xoshiro_next_float(r);
    float cum = 0.0f;
    for (int i = 0; i < n; i++) {
        cum += probs[i];
        if (u < cum) return idx ? idx[i] : i;
    }
    for (int i = n - 1; i >= 0; i--)
        if (probs[i] > 0.0f) return idx ? idx[i] : i;
    return vocab - 1;
}

// k-th largest (TopKSampler.PartialSortDescending semantics: exact order statistic).
static float kth_largest(const float* x, int n, int k) {
    std::vector<float> c(x, x + n);
    std::nth_element(c.begin(), c.begin() + (k - 1), c.end(), [](float a, float b) { return a > b; });
    return c[(size_t)(k - 1)];
}

extern "C" int32_t fllmh_sampler_sample_host(fllmh_sampler* s, float* logits, int32_t n, int32_t* out_token) {
    if (!s || !logits || !out_token) return hfail(FLLM_E_NULL, "arguments must not be null");
    if (n <= 0) return hfail(FLLM_E_ARG, "Span must not be empty.");
    if (s->temperature == 0.0f) {  // ArgMax: first maximum, NaN first, +0 over -0
        int best = 0;
        for (int i = 0; i < n; i++) {
            if (std::isnan(logits[i])) { best = i; break; }
            float v = logits[i], b = logits[best];
            if (v > b || (v == b && v == 0.0f && !std::signbit(v) && std::signbit(b))) best = i;
        }
        *out_token = best;
        return FLLM_OK;
    }
    if (s->temperature != 1.0f) {
        float inv = 1.0f / s->temperature;
        for (int i = 0; i < n; i++) logits[i] = logits[i] * inv;
    }
    if (s->top_k > 0 && s->top_k < n) {
        float th = kth_largest(logits, n, s->top_k);
        for (int i = 0; i < n; i++)
            if (logits[i] < th) logits[i] = -INFINITY;
    }
    softmax_inplace(logits, n);
    apply_top_p(logits, n, s->top_p);
    *out_token = sample_cdf(&s->rng, nullptr, logits, n, n);
    return FLLM_OK;
}

static int32_t seq_vocab(fllm_seq* seq, int32_t* V) {
    fllm_model* m = nullptr;
    int32_t rc = fllm_seq_get_model(seq, &m);
    if (rc) return dfail(rc);
    fllm_model_desc d;
    rc = fllm_model_get_desc(m, &d);
    if (rc) return dfail(rc);
    *V = d.vocab;
    return FLLM_OK;
}

extern "C" int32_t fllmh_sampler_sample(fllmh_sampler* s, fllm_seq* seq, int32_t* out_token) {
    if (!s || !seq || !out_token) return hfail(FLLM_E_NULL, "arguments must not be null");
    if (s->temperature == 0.0f) {  // SamplerPipeline.cs:61-64: greedy on the device
        int32_t rc = fllm_sample_greedy(seq, out_token);
        return rc ? dfail(rc) : FLLM_OK;
    }
    int32_t V = 0;
    int32_t rc = seq_vocab(seq, &V);
    if (rc) return rc;
    if (V > 262144) {  // beyond the device samplers' one-workgroup limit: the pipeline on the host
        s->buf.resize((size_t)V);
        rc = fllm_logits_copy(seq, s->buf.data(), V);
        if (rc) return dfail(rc);
        return fllmh_sampler_sample_host(s, s->buf.data(), V, out_token);
    }
    if (s->top_k > 0 && s->top_k < V) {
        // stages 1-2 on the device (scale, top-k with ties kept), stages 3-5 on the survivors:
        // every filtered logit is -inf, so its probability is exactly 0 and the CDF walk in
        // index order over the survivors equals the walk over the whole vocabulary.
        float inv = s->temperature != 1.0f ? 1.0f / s->temperature : 1.0f;
        int cap = std::max(s->top_k * 4, 1024);
        s->ids.resize((size_t)cap);
        s->buf.resize((size_t)cap);
        int32_t cnt = 0;
        rc = fllm_sample_topk(seq, inv, s->top_k, s->ids.data(), s->buf.data(), cap, &cnt);
        if (rc == FLLM_E_ARG && cnt > cap) {  // more ties than room: the logits are scaled now
            cap = cnt;
            s->ids.resize((size_t)cap);
            s->buf.resize((size_t)cap);
            rc = fllm_sample_topk(seq, 1.0f, s->top_k, s->ids.data(), s->buf.data(), cap, &cnt);
        }
        if (rc) return dfail(rc);
        softmax_inplace(s->buf.data(), cnt);
        apply_top_p(s->buf.data(), cnt, s->top_p);
        *out_token = sample_cdf(&s->rng, s->ids.data(), s->buf.data(), cnt, V);
        return FLLM_OK;
    }
    // no top-k: stages 1 and 3-5 over the whole vocabulary on the device (no logits copy); the
    // draw's u comes from this pipeline's generator, one NextFloat per token as in the reference
    float inv = s->temperature != 1.0f ? 1.0f / s->temperature : 1.0f;
    float u = fllmh_xoshiro_next_float(&s->rng);
    rc = fllm_sample_nucleus(seq, inv, s->top_p, u, out_token);
    return rc ? dfail(rc) : FLLM_OK;
}

// =====================================================================================
// token loop (LlamaLanguageModel.GenerateAsync, LlamaLanguageModel.cs:100-331)
// =====================================================================================
extern "C" int32_t fllmh_generate(fllm_seq* seq, const int32_t* prompt, int32_t n_prompt, int32_t max_tokens,
                                  fllmh_sampler* sampler, int32_t eos_token_id, int32_t bos_token_id,
                                  float repetition_penalty, int32_t* out_tokens, fllmh_generate_stats* stats) {
    if (!seq || !sampler) return hfail(FLLM_E_NULL, "seq and sampler must not be null");
    if (n_prompt < 0 || max_tokens < 0) return hfail(FLLM_E_ARG_RANGE, "counts must be >= 0");
    if (n_prompt > 0 && !prompt) return hfail(FLLM_E_NULL, "prompt must not be null");
    if (max_tokens > 0 && !out_tokens) return hfail(FLLM_E_NULL, "out_tokens must not be null");
    using clk = std::chrono::steady_clock;
    int32_t rc = fllm_seq_reset(seq);
    if (rc) return dfail(rc);
    auto t0 = clk::now();
    int position = 0;
    if (n_prompt > 1) {  // the n-1 prefill Forward calls (:133-137) as one batched prefill
        rc = fllm_prefill(seq, prompt, n_prompt - 1, 0);
        if (rc) return dfail(rc);
        position = n_prompt - 1;
    }
    rc = fllm_seq_sync(seq);
    if (rc) return dfail(rc);
    auto t1 = clk::now();
    int next = n_prompt > 0 ? prompt[n_prompt - 1] : bos_token_id;  // :152
    int generated = 0;
    int finish = 0;
    for (int step = 0; step < max_tokens; step++) {  // :162-293
        rc = fllm_forward(seq, next, position++);
        if (rc) return dfail(rc);
        if (repetition_penalty != 1.0f && generated > 0) {
            // ApplyRepetitionPenalty (:183-186, 357-373) over the generated ids, on the device logits
            rc = fllm_logits_penalize(seq, out_tokens, generated, repetition_penalty);
            if (rc) return dfail(rc);
        }
        rc = fllmh_sampler_sample(sampler, seq, &next);
        if (rc) return rc;
        out_tokens[generated++] = next;
        if (eos_token_id >= 0 && next == eos_token_id) { finish = 1; break; }
    }
    rc = fllm_seq_sync(seq);
    if (rc) return dfail(rc);
    auto t2 = clk::now();
    if (stats) {
        stats->prompt_tokens = n_prompt;
        stats->completion_tokens = generated;
        stats->prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        stats->decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
        stats->tokens_per_second = stats->decode_ms > 0 ? generated / (stats->decode_ms / 1000.0) : 0.0;
        stats->finish_reason = finish;
    }
    return FLLM_OK;
}
