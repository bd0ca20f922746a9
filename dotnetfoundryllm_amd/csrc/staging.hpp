// staging.hpp — host-to-device upload of caller memory through a pair of pinned staging buffers.
//
// Plain host C++ over the HIP runtime API. The includer declares that API first: the library
// includes <hip/hip_runtime.h>; the loader's sanitizer harness (tests/sanitize) a CPU stand-in whose
// copies run on a thread of their own, so that the address, undefined-behaviour and thread
// sanitizers see this code, the GGUF loader above it and the copies' ordering.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace fllm {

// The host copies chunk i of the source into buffer i % 2 (with several threads for a large chunk)
// while the DMA engine moves chunk i - 1 out of the other buffer, so a pageable source (a mapped
// GGUF file) streams at the rate of the slower of the two instead of their sum. Every byte of the
// caller's memory is read by the host: no device copy reads it, so the caller may free or unmap it
// as soon as the upload returns, and the runtime never pins or stages pages of it.
struct Staging {
    static constexpr size_t kChunk = 32u << 20;
    static constexpr size_t kPerThread = 4u << 20;  // at least this many bytes per copying thread
    uint8_t* buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    std::mutex mu;  // one upload at a time fills the pair (uploads from several host threads)
};

// Allocates the pinned pair and its events (once).
inline hipError_t staging_init(Staging& S) {
    for (int b = 0; b < 2; b++) {
        if (!S.buf[b]) {
            hipError_t e = hipHostMalloc((void**)&S.buf[b], Staging::kChunk, hipHostMallocDefault);
            if (e != hipSuccess) { S.buf[b] = nullptr; return e; }
        }
        if (!S.done[b]) {
            hipError_t e = hipEventCreateWithFlags(&S.done[b], hipEventDisableTiming);
            if (e != hipSuccess) { S.done[b] = nullptr; return e; }
        }
    }
    return hipSuccess;
}

// Frees the pair; the stream that used it has been synchronized.
inline void staging_free(Staging& S) {
    for (int b = 0; b < 2; b++) {
        if (S.done[b]) hipEventDestroy(S.done[b]);
        if (S.buf[b]) hipHostFree(S.buf[b]);
        S.done[b] = nullptr;
        S.buf[b] = nullptr;
    }
}

// Copies n bytes at src (host memory of any kind) to dst (device) on stream st. Returns when the
// last chunk's copy has been enqueued: src may be reused then, dst is complete when st reaches that
// point. On an error return, copies already enqueued may still be running: synchronize st before
// freeing dst.
inline hipError_t staged_upload(Staging& S, hipStream_t st, uint8_t* dst, const uint8_t* src, size_t n) {
    std::lock_guard<std::mutex> lock(S.mu);
    hipError_t e = staging_init(S);
    if (e != hipSuccess) return e;
    const unsigned hw = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    size_t off = 0;
    for (int i = 0; off < n; i++) {
        const int b = i & 1;
        const size_t len = std::min(Staging::kChunk, n - off);
        e = hipEventSynchronize(S.done[b]);  // the copy out of this buffer two chunks ago
        if (e != hipSuccess) return e;
        uint8_t* stage = S.buf[b];
        const uint8_t* from = src + off;
        const unsigned nthr = (unsigned)std::min<size_t>(hw, (len + Staging::kPerThread - 1) / Staging::kPerThread);
        const size_t part = (len + nthr - 1) / nthr;
        std::vector<std::thread> pool;
        for (unsigned t = 1; t < nthr && t * part < len; t++)
            pool.emplace_back([=] { memcpy(stage + t * part, from + t * part, std::min(part, len - t * part)); });
        memcpy(stage, from, std::min(part, len));
        for (auto& th : pool) th.join();
        e = hipMemcpyAsync(dst + off, stage, len, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(S.done[b], st);
        if (e != hipSuccess) return e;
        off += len;
    }
    return hipSuccess;
}

}  // namespace fllm
