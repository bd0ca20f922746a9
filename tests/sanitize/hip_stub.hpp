// hip_stub.hpp — a CPU stand-in for the part of the HIP runtime API that the upload staging
// (dotnetfoundryllm_amd/csrc/staging.hpp) and the loader harness use. Device memory is host memory;
// each stream runs its copies, fills and event records in order on a thread of its own, so a copy
// that the host has enqueued runs concurrently with what the host does next, as a DMA engine's
// would. FLLM_STUB_DMA_DELAY_US delays every stream operation by that many microseconds, which
// widens the window in which a missing wait would let the host touch a buffer a copy still reads.
#pragma once

#include <chrono>
#include <condition_variable>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <functional>
#include <mutex>
#include <thread>

enum hipError_t { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorOutOfMemory = 2 };
enum hipMemcpyKind { hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2 };
enum { hipHostMallocDefault = 0, hipEventDisableTiming = 2, hipStreamNonBlocking = 1 };

inline const char* hipGetErrorString(hipError_t e) {
    return e == hipSuccess ? "hipSuccess" : e == hipErrorOutOfMemory ? "hipErrorOutOfMemory" : "hipErrorInvalidValue";
}

struct StubStream {
    std::mutex mu;
    std::condition_variable cv;
    std::deque<std::function<void()>> q;
    uint64_t enqueued = 0, finished = 0;
    bool stop = false;
    unsigned delay_us = 0;
    std::thread worker;
    StubStream() {
        const char* d = getenv("FLLM_STUB_DMA_DELAY_US");
        delay_us = d ? (unsigned)atoi(d) : 0;
        worker = std::thread([this] { run(); });
    }
    ~StubStream() {
        {
            std::lock_guard<std::mutex> l(mu);
            stop = true;
        }
        cv.notify_all();
        worker.join();
    }
    void run() {
        for (;;) {
            std::function<void()> op;
            {
                std::unique_lock<std::mutex> l(mu);
                cv.wait(l, [this] { return stop || !q.empty(); });
                if (q.empty()) return;
                op = std::move(q.front());
                q.pop_front();
            }
            if (delay_us) std::this_thread::sleep_for(std::chrono::microseconds(delay_us));
            op();
            {
                std::lock_guard<std::mutex> l(mu);
                finished++;
            }
            cv.notify_all();
        }
    }
    void push(std::function<void()> op) {
        {
            std::lock_guard<std::mutex> l(mu);
            q.push_back(std::move(op));
            enqueued++;
        }
        cv.notify_all();
    }
    void sync() {
        std::unique_lock<std::mutex> l(mu);
        const uint64_t want = enqueued;
        cv.wait(l, [&] { return finished >= want; });
    }
};
typedef StubStream* hipStream_t;

struct StubEvent {
    std::mutex mu;
    std::condition_variable cv;
    uint64_t recorded = 0, reached = 0;
};
typedef StubEvent* hipEvent_t;

inline hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) { *s = new StubStream(); return hipSuccess; }
inline hipError_t hipStreamDestroy(hipStream_t s) { delete s; return hipSuccess; }
inline hipError_t hipStreamSynchronize(hipStream_t s) { s->sync(); return hipSuccess; }

inline hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
    *p = aligned_alloc(4096, (n + 4095) / 4096 * 4096);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipHostFree(void* p) { free(p); return hipSuccess; }
inline hipError_t hipMalloc(void** p, size_t n) {
    *p = malloc(n ? n : 1);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
template <typename T>
inline hipError_t hipMalloc(T** p, size_t n) { return hipMalloc((void**)p, n); }
inline hipError_t hipFree(void* p) { free(p); return hipSuccess; }

inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) { *e = new StubEvent(); return hipSuccess; }
inline hipError_t hipEventDestroy(hipEvent_t e) { delete e; return hipSuccess; }
inline hipError_t hipEventRecord(hipEvent_t e, hipStream_t s) {
    uint64_t ticket;
    {
        std::lock_guard<std::mutex> l(e->mu);
        ticket = ++e->recorded;
    }
    s->push([e, ticket] {
        {
            std::lock_guard<std::mutex> l(e->mu);
            if (ticket > e->reached) e->reached = ticket;
        }
        e->cv.notify_all();
    });
    return hipSuccess;
}
// waits for the last record enqueued before the call (returns at once for an event never recorded)
inline hipError_t hipEventSynchronize(hipEvent_t e) {
    std::unique_lock<std::mutex> l(e->mu);
    const uint64_t want = e->recorded;
    e->cv.wait(l, [&] { return e->reached >= want; });
    return hipSuccess;
}

inline hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind, hipStream_t s) {
    if (n && (!dst || !src)) return hipErrorInvalidValue;
    s->push([dst, src, n] { memcpy(dst, src, n); });
    return hipSuccess;
}
inline hipError_t hipMemsetAsync(void* dst, int v, size_t n, hipStream_t s) {
    if (n && !dst) return hipErrorInvalidValue;
    s->push([dst, v, n] { memset(dst, v, n); });
    return hipSuccess;
}
