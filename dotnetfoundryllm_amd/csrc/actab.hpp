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

// The digits of four quantized values packed one byte per value: byte k of the returned dwords
// comes from x_k. With X = 65536 b2 + 256 b1 + b0 and every digit in [-128, 127] (quant_x gives
// |X| <= 127 * 65536),
// b1 = floor((X + 128) / 256) and b2 = floor((X + 32896) / 65536), so b0 is byte 0 of X, b1 byte 1
// of X + 128 and b2 byte 2 of X + 32896 (the bytes digits3 would give, without its shifts and
// masks). d2 / d1 / d0: the dwords of b2 / b1 / b0.
__device__ __forceinline__ uint32_t byte_k_of4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t k) {
    const uint32_t sel = 0x0c0c0000u | ((4u + k) << 8) | k;  // {a_k, b_k, 0, 0} (0x0c selects zero)
    const uint32_t lo = __builtin_amdgcn_perm(b, a, sel), hi = __builtin_amdgcn_perm(d, c, sel);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);  // {lo_0, lo_1, hi_0, hi_1}
}
__device__ __forceinline__ void digits3_pack4(int x0, int x1, int x2, int x3, uint32_t& d2, uint32_t& d1,
                                              uint32_t& d0) {
    d2 = byte_k_of4((uint32_t)(x0 + 32896), (uint32_t)(x1 + 32896), (uint32_t)(x2 + 32896), (uint32_t)(x3 + 32896), 2);
    d1 = byte_k_of4((uint32_t)(x0 + 128), (uint32_t)(x1 + 128), (uint32_t)(x2 + 128), (uint32_t)(x3 + 128), 1);
    d0 = byte_k_of4((uint32_t)x0, (uint32_t)x1, (uint32_t)x2, (uint32_t)x3, 0);
}

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
