// common.hpp — shared definitions for the gfx950 decode library (device + host side).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fllm.h"

namespace fllm {

// ---- GGML block geometry (Dequantizer.cs:21-43; GgufFile.ComputeByteSize GgufFile.cs:99-122)
struct TypeInfo {
    int block_bytes;
    int block_elems;
};

__host__ __device__ inline bool type_supported(int t) {
    return t == FLLM_TYPE_F32 || t == FLLM_TYPE_F16 || t == FLLM_TYPE_BF16 || t == FLLM_TYPE_Q4_0 ||
           t == FLLM_TYPE_Q8_0 || t == FLLM_TYPE_Q4_K || t == FLLM_TYPE_Q5_K || t == FLLM_TYPE_Q6_K ||
           t == FLLM_TYPE_Q8_K;
}

__host__ __device__ inline TypeInfo type_info(int t) {
    switch (t) {
        case FLLM_TYPE_F32: return {4, 1};
        case FLLM_TYPE_F16: return {2, 1};
        case FLLM_TYPE_BF16: return {2, 1};
        case FLLM_TYPE_Q4_0: return {18, 32};
        case FLLM_TYPE_Q8_0: return {34, 32};
        case FLLM_TYPE_Q4_K: return {144, 256};
        case FLLM_TYPE_Q5_K: return {176, 256};
        case FLLM_TYPE_Q6_K: return {210, 256};
        case FLLM_TYPE_Q8_K: return {292, 256};
        default: return {0, 0};
    }
}

// Bytes occupied by n elements of type t (n must be a whole number of blocks).
__host__ __device__ inline uint64_t type_bytes(int t, int64_t n) {
    TypeInfo ti = type_info(t);
    if (ti.block_elems == 0) return 0;
    return (uint64_t)(n / ti.block_elems) * (uint64_t)ti.block_bytes;
}

// ---- exact scalar conversions (Dequantizer.HalfToFloat / BFloat16ToFloat, Dequantizer.cs:49-59)
__host__ __device__ inline float bits_f32(uint32_t u) {
#ifdef __HIP_DEVICE_COMPILE__
    return __uint_as_float(u);
#else
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
#endif
}

// Integer-exact binary16 -> binary32 (keeps NaN payloads, independent of FP modes).
__host__ __device__ inline float half_exact(uint32_t h) {
    uint32_t sign = (h >> 15) << 31;
    uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (ex == 0) {
        float v = (float)man * 5.9604644775390625e-08f;  // man * 2^-24, exact
        return sign ? -v : v;
    }
    if (ex == 31) return bits_f32(sign | 0x7F800000u | (man << 13));
    return bits_f32(sign | ((ex + 112u) << 23) | (man << 13));
}

__host__ __device__ inline float bf16_exact(uint32_t b) { return bits_f32(b << 16); }

// DecodeKScaleMin (Dequantizer.cs:506-521) over the 12 packed scale bytes.
__host__ __device__ inline void kscale_min(const uint8_t* p, int g, int& sc, int& mn) {
    if (g < 4) {
        sc = p[g] & 0x3F;
        mn = p[g + 4] & 0x3F;
    } else {
        int i = g - 4;
        sc = (p[g + 4] & 0x0F) | ((p[i] >> 6) << 4);
        mn = (p[g + 4] >> 4) | ((p[i + 4] >> 6) << 4);
    }
}

// Q4_K in the matrix-core tile layout: each 8-byte half of a group's 16 qs bytes is stored as its
// bytes 0, 2, 4, 6, 1, 3, 5, 7 (so one dword holds the half's elements 4 by, 4 by + 1 and the other
// 4 by + 2, 4 by + 3, by = 0 .. 3: the activation table's order). q4t_src_byte(j): the group byte
// stored at position j; q4t_pos(b): the position of group byte b.
__host__ __device__ __forceinline__ int q4t_src_byte(int j) {
    const int p = j & 7;
    return (j & 8) + (p < 4 ? 2 * p : 2 * (p - 4) + 1);
}
__host__ __device__ __forceinline__ int q4t_pos(int b) {
    const int o = b & 7;
    return (b & 8) + ((o & 1) ? 4 + (o >> 1) : (o >> 1));
}

// FFN activation: 0 = SiLU, x * Sigmoid(x) (TensorOperations.cs:57-87); 1 = GELU, tanh form
// (TensorOperations.cs:110-117)
__device__ __forceinline__ float act_fn(float g, int act) {
    if (act == 0) {
        float sig = 1.0f / (1.0f + expf(-g));
        return g * sig;
    }
    return 0.5f * g * (1.0f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g)));
}

}  // namespace fllm
