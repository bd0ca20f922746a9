// load_check.cpp — the GGUF loader (dotnetfoundryllm_amd/host/fllm_host.cpp: open_gguf,
// fllmh_load_gguf) and the upload staging (dotnetfoundryllm_amd/csrc/staging.hpp) on the CPU, over a
// stand-in device (hip_stub.hpp), built for the address + undefined-behaviour sanitizers and for the
// thread sanitizer (Makefile beside this file).
//
// The stand-in's fllm_model_upload runs the device library's sequence (csrc/api.hip): an allocation
// with 256 bytes of slack, the staged copy, the slack cleared, the stream synchronized; then it
// checks that the "device" bytes equal the caller's and that the slack is zero, and keeps a hash per
// tensor. The run over one GGUF file:
//   cold   the file's pages written out and dropped from the page cache, then loaded;
//   warm   loaded again from the page cache; the same tensors, sizes and hashes as cold;
//   shared two host threads load it at once into two models on one context (one staging pair);
//   errors a file cut inside its header, one cut inside its tensor data, one with a bad magic and a
//          missing path each fail with FLLM_E_MODEL_LOAD and load nothing.
// Usage: load_check <file.gguf> <scratch dir>. Exit 0 when every step holds.
#include "hip_stub.hpp"
#include "../../dotnetfoundryllm_amd/csrc/staging.hpp"
#include "../../include/fllm_host.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <string>
#include <thread>
#include <vector>

using fllm::Staging;

// ---- the stand-in device library (the symbols fllm_host.cpp binds) ----------------------------
static thread_local std::string g_err;
static int32_t fail(int32_t code, const std::string& msg) {
    g_err = msg;
    return code;
}

struct fllm_ctx {
    hipStream_t st = nullptr;
    Staging stage;
};

struct Upload {
    int slot, layer, type;
    uint64_t nbytes, hash;
};

struct fllm_model {
    fllm_ctx* ctx = nullptr;
    fllm_model_desc d{};
    std::vector<Upload> ups;
    bool finalized = false;
};

static const uint64_t kPad = 256;
static std::atomic<int> g_live_models{0};

// FNV-1a over 8-byte words (the tail zero-padded)
static uint64_t fnv1a(const uint8_t* p, size_t n) {
    uint64_t h = 1469598103934665603ULL;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        memcpy(&w, p + i, 8);
        h = (h ^ w) * 1099511628211ULL;
    }
    if (i < n) {
        uint64_t w = 0;
        memcpy(&w, p + i, n - i);
        h = (h ^ w) * 1099511628211ULL;
    }
    return h;
}

extern "C" const char* fllm_last_error(void) { return g_err.c_str(); }

extern "C" int32_t fllm_ctx_create(int32_t, fllm_ctx** out) {
    if (!out) return fail(FLLM_E_NULL, "out must not be null");
    fllm_ctx* c = new fllm_ctx();
    hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking);
    *out = c;
    return FLLM_OK;
}

extern "C" int32_t fllm_ctx_destroy(fllm_ctx* c) {
    if (!c) return FLLM_OK;
    hipStreamSynchronize(c->st);
    fllm::staging_free(c->stage);
    hipStreamDestroy(c->st);
    delete c;
    return FLLM_OK;
}

extern "C" int32_t fllm_model_create(fllm_ctx* ctx, const fllm_model_desc* d, fllm_model** out) {
    if (!ctx || !d || !out) return fail(FLLM_E_NULL, "null argument");
    if (d->n_layers <= 0 || d->hidden <= 0 || d->vocab <= 0) return fail(FLLM_E_ARG, "bad description");
    fllm_model* m = new fllm_model();
    m->ctx = ctx;
    m->d = *d;
    g_live_models++;
    *out = m;
    return FLLM_OK;
}

extern "C" int32_t fllm_model_upload(fllm_model* m, int32_t slot, int32_t layer, int32_t type, const void* bytes,
                                     uint64_t nbytes) {
    if (!m || !bytes) return fail(FLLM_E_NULL, "null argument");
    if (m->finalized) return fail(FLLM_E_INVALID_OP, "model already finalized");
    if (slot >= 10 && (layer < 0 || layer >= m->d.n_layers)) return fail(FLLM_E_ARG_RANGE, "layer out of range");
    if (nbytes == 0) return fail(FLLM_E_ARG, "empty tensor");
    hipStream_t st = m->ctx->st;
    uint8_t* dev = nullptr;
    if (hipMalloc(&dev, nbytes + kPad) != hipSuccess) return fail(FLLM_E_OOM, "allocation failed");
    memset(dev + nbytes, 0xA5, kPad);  // the slack as a fresh allocation may hold it
    hipError_t e = fllm::staged_upload(m->ctx->stage, st, dev, (const uint8_t*)bytes, nbytes);
    if (e == hipSuccess) e = hipMemsetAsync(dev + nbytes, 0, kPad, st);
    hipStreamSynchronize(st);
    if (e != hipSuccess) {
        hipFree(dev);
        return fail(FLLM_E_DEVICE, "upload failed");
    }
    std::string why;
    if (memcmp(dev, bytes, nbytes) != 0) why = "device bytes differ from the source";
    for (uint64_t i = 0; i < kPad && why.empty(); i++)
        if (dev[nbytes + i] != 0) why = "slack not cleared";
    const uint64_t h = fnv1a(dev, nbytes);
    hipFree(dev);
    if (!why.empty()) return fail(FLLM_E_DEVICE, why);
    m->ups.push_back({slot, layer, type, nbytes, h});
    return FLLM_OK;
}

extern "C" int32_t fllm_model_finalize(fllm_model* m) {
    if (!m) return fail(FLLM_E_NULL, "null model");
    m->finalized = true;
    return FLLM_OK;
}

extern "C" int32_t fllm_model_destroy(fllm_model* m) {
    if (!m) return FLLM_OK;
    g_live_models--;
    delete m;
    return FLLM_OK;
}

extern "C" int32_t fllm_model_get_desc(fllm_model* m, fllm_model_desc* out) {
    if (!m || !out) return fail(FLLM_E_NULL, "null argument");
    *out = m->d;
    return FLLM_OK;
}

// the decode entry points the token loop binds: not part of this check
static int32_t no_device() { return fail(FLLM_E_NOT_SUPPORTED, "no device in the loader check"); }
extern "C" int32_t fllm_seq_reset(fllm_seq*) { return no_device(); }
extern "C" int32_t fllm_seq_get_model(fllm_seq*, fllm_model**) { return no_device(); }
extern "C" int32_t fllm_forward(fllm_seq*, int32_t, int32_t) { return no_device(); }
extern "C" int32_t fllm_prefill(fllm_seq*, const int32_t*, int32_t, int32_t) { return no_device(); }
extern "C" int32_t fllm_seq_sync(fllm_seq*) { return no_device(); }
extern "C" int32_t fllm_logits_copy(fllm_seq*, float*, int64_t) { return no_device(); }
extern "C" int32_t fllm_sample_greedy(fllm_seq*, int32_t*) { return no_device(); }
extern "C" int32_t fllm_sample_topk(fllm_seq*, float, int32_t, int32_t*, float*, int32_t, int32_t*) { return no_device(); }
extern "C" int32_t fllm_logits_penalize(fllm_seq*, const int32_t*, int32_t, float) { return no_device(); }
extern "C" int32_t fllm_sample_nucleus(fllm_seq*, float, float, float, int32_t*) { return no_device(); }

// ---- the check ---------------------------------------------------------------------------------
static std::atomic<int> g_failures{0};  // (the two loading threads may report)
#define CHECK(cond, ...)                    \
    do {                                    \
        if (!(cond)) {                      \
            fprintf(stderr, "FAIL: " __VA_ARGS__); \
            fprintf(stderr, "\n");          \
            g_failures++;                   \
        }                                   \
    } while (0)

static double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

static void drop_page_cache(const char* path) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) return;
    fsync(fd);
    posix_fadvise(fd, 0, 0, POSIX_FADV_DONTNEED);
    close(fd);
}

// loads path; returns the uploads (empty on failure, with the status in *rc)
static std::vector<Upload> load(fllm_ctx* ctx, const char* path, int32_t* rc, fllmh_model_info* info = nullptr) {
    fllm_model* m = nullptr;
    fllmh_model_info local;
    *rc = fllmh_load_gguf(ctx, path, &m, info ? info : &local);
    std::vector<Upload> ups;
    if (*rc == FLLM_OK) {
        ups = m->ups;
        fllm_model_destroy(m);
    } else {
        CHECK(m == nullptr, "a failed load returned a model");
    }
    return ups;
}

static bool same(const std::vector<Upload>& a, const std::vector<Upload>& b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); i++)
        if (a[i].slot != b[i].slot || a[i].layer != b[i].layer || a[i].type != b[i].type ||
            a[i].nbytes != b[i].nbytes || a[i].hash != b[i].hash)
            return false;
    return true;
}

// writes the first n bytes of src (then `tail` if given) to dst
static bool write_prefix(const char* src, const std::string& dst, uint64_t n, const char* head = nullptr) {
    int in = open(src, O_RDONLY);
    int out = open(dst.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0600);
    bool ok = in >= 0 && out >= 0;
    std::vector<char> buf(1 << 20);
    uint64_t done = 0;
    while (ok && done < n) {
        ssize_t r = read(in, buf.data(), (size_t)std::min<uint64_t>(buf.size(), n - done));
        if (r <= 0) break;
        if (done == 0 && head) memcpy(buf.data(), head, strlen(head));
        ok = write(out, buf.data(), (size_t)r) == r;
        done += (uint64_t)r;
    }
    if (in >= 0) close(in);
    if (out >= 0) close(out);
    return ok && done == n;
}

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <file.gguf> <scratch dir>\n", argv[0]);
        return 2;
    }
    const char* path = argv[1];
    const std::string dir = argv[2];
    struct stat st;
    if (stat(path, &st) != 0) {
        fprintf(stderr, "cannot stat %s\n", path);
        return 2;
    }
    const uint64_t size = (uint64_t)st.st_size;
    fllm_ctx* ctx = nullptr;
    fllm_ctx_create(0, &ctx);

    int32_t rc;
    fllmh_model_info info{};
    drop_page_cache(path);
    double t = now_s();
    std::vector<Upload> cold = load(ctx, path, &rc, &info);
    const double cold_s = now_s() - t;
    CHECK(rc == FLLM_OK, "cold load: %d %s", rc, fllmh_last_error());
    uint64_t bytes = 0, big = 0;
    for (const Upload& u : cold) {
        bytes += u.nbytes;
        big += u.nbytes > Staging::kChunk;
    }
    printf("cold: %zu tensors, %llu bytes (%llu over one staging chunk), %.2f s\n", cold.size(),
           (unsigned long long)bytes, (unsigned long long)big, cold_s);

    t = now_s();
    std::vector<Upload> warm = load(ctx, path, &rc);
    printf("warm: %.2f s\n", now_s() - t);
    CHECK(rc == FLLM_OK && same(cold, warm), "warm load differs from cold (rc %d)", rc);

    std::vector<Upload> a, b;
    int32_t ra = 0, rb = 0;
    std::thread ta([&] { a = load(ctx, path, &ra); });
    std::thread tb([&] { b = load(ctx, path, &rb); });
    ta.join();
    tb.join();
    CHECK(ra == FLLM_OK && rb == FLLM_OK && same(cold, a) && same(cold, b), "concurrent loads differ (%d, %d)", ra, rb);
    printf("shared context, two threads: %s\n", same(cold, a) && same(cold, b) ? "same tensors" : "differ");

    struct Bad { std::string name; uint64_t n; const char* head; };
    const uint64_t data_cut = info.data_offset + (size - info.data_offset) / 2;
    const Bad bad[] = {{"cut_header.gguf", std::min<uint64_t>(size, 100), nullptr},
                       {"cut_data.gguf", data_cut, nullptr},
                       {"bad_magic.gguf", std::min<uint64_t>(size, 4096), "GGUX"}};
    for (const Bad& x : bad) {
        const std::string p = dir + "/" + x.name;
        CHECK(write_prefix(path, p, x.n, x.head), "writing %s", p.c_str());
        std::vector<Upload> u = load(ctx, p.c_str(), &rc);
        CHECK(rc == FLLM_E_MODEL_LOAD && u.empty(), "%s: status %d (%s)", x.name.c_str(), rc, fllmh_last_error());
        printf("%s: %d %s\n", x.name.c_str(), rc, fllmh_last_error());
        unlink(p.c_str());
    }
    std::vector<Upload> u = load(ctx, (dir + "/missing.gguf").c_str(), &rc);
    CHECK(rc == FLLM_E_MODEL_LOAD && u.empty(), "missing file: status %d", rc);

    fllm_ctx_destroy(ctx);
    CHECK(g_live_models.load() == 0, "%d models not destroyed", g_live_models.load());
    printf("%s\n", g_failures.load() ? "FAILED" : "load check ok");
    return g_failures.load() ? 1 : 0;
}
