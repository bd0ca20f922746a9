// actab.hpp — the quantized activation table shared by the matrix-core GEMV (its input) and the
// kernels that produce GEMV inputs (residual and GLU epilogues, the attention merge).
//
// Per chunk of 256 elements: 48 uint4 digit entries [step][quarter][digit], then (after all chunks'
// digit entries) 8 float4 group stats per chunk. Each 16-element half of a 32-element group is
// quantized on its own: X = rint(v * 65536 * 127 / amax), split into signed base-256 digits
// X = 65536 b2 + 256 b1 + b0 (digit 0 = b2). Stats of group g: {scale of half 0, scale of half 1,
// sum of half 0, sum of half 1}, scale = amax / 127, sums over the unquantized values. A lane of
// quarter Q covers groups Q and Q+4 of a chunk: step s is half s&1 of group Q + 4*(s>>1). Inside a
// step's 16-byte entry, byte `by` of dword j holds element 4*by + j of the half.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fllm {

constexpr int MF_TAB_ENTRIES = 56;  // uint4 entries of the activation table per chunk

__host__ __device__ __forceinline__ int atab_index(int b, int s, int q, int d) { return ((b * 4 + s) * 4 + q) * 3 + d; }

// signed base-256 digits of X = 65536 b2 + 256 b1 + b0
__device__ __forceinline__ void digits3(int X, int& b2, int& b1, int& b0) {
    b0 = (int)(int8_t)(X & 0xFF);
    const int x1 = (X - b0) >> 8;
    b1 = (int)(int8_t)(x1 & 0xFF);
    b2 = (x1 - b1) >> 8;
}

// scale and its inverse for a half whose largest magnitude is amax (both 0 for an all-zero half)
__device__ __forceinline__ void half_scale(float amax, float& sc, float& inv) {
    sc = 0.0f;
    inv = 0.0f;
    if (amax > 0.0f) { sc = amax / 127.0f; inv = 127.0f / amax; }
}

__device__ __forceinline__ int quant_x(float v, float inv) { return (int)rintf(v * inv * 65536.0f); }

// position of element e (0 .. n-1, n a multiple of 256) in the table: entry of digit 0 of its step
// and quarter, its byte inside that entry, and its 32-element group's stats entry and half
__device__ __forceinline__ void tab_pos(int e, int n, int& entry0, int& byte, int& stat, int& half) {
    const int h16 = e >> 4, g32 = h16 >> 1, b = g32 >> 3, gg = g32 & 7;
    half = h16 & 1;
    entry0 = atab_index(b, 2 * (gg >> 2) + half, gg & 3, 0);
    const int e16 = e & 15;
    byte = 4 * (e16 & 3) + (e16 >> 2);
    stat = (n / 256) * 48 + 8 * b + gg;
}

}  // namespace fllm
