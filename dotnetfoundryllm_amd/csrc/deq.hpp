// deq.hpp — exact device dequantization of one element of a quantized GGUF block stream
// (Dequantizer.cs:155-456). Shared by the element-wise kernels and the fused GEMV prologue.
#pragma once

#include "common.hpp"

namespace fllm {

__device__ __forceinline__ uint32_t deq_ld_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
__device__ __forceinline__ uint32_t deq_ld_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Quantized types only (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K); returns 0 for anything else.
__device__ __forceinline__ float deq_elem_q(int type, const uint8_t* w, int64_t e) {
    switch (type) {
        case FLLM_TYPE_Q4_0: {  // Dequantizer.cs:172-184
            const uint8_t* p = w + (e >> 5) * 18;
            int j = (int)(e & 31);
            float d = half_exact(deq_ld_u16(p));
            uint32_t qs = p[2 + (j & 15)];
            int q = j < 16 ? (int)(qs & 0x0F) : (int)(qs >> 4);
            return (float)(q - 8) * d;
        }
        case FLLM_TYPE_Q8_0: {  // Dequantizer.cs:220-229
            const uint8_t* p = w + (e >> 5) * 34;
            float d = half_exact(deq_ld_u16(p));
            return (float)(int8_t)p[2 + (e & 31)] * d;
        }
        case FLLM_TYPE_Q4_K: {  // Dequantizer.cs:268-292
            const uint8_t* p = w + (e >> 8) * 144;
            int i = (int)(e & 255), g = i >> 5, ii = i & 31;
            float d = half_exact(deq_ld_u16(p)), dmin = half_exact(deq_ld_u16(p + 2));
            int sc, mn;
            kscale_min(p + 4, g, sc, mn);
            float dg = d * (float)sc;
            float mg = dmin * (float)mn;
            uint32_t packed = p[16 + g * 16 + (ii >> 1)];
            int q = (ii & 1) == 0 ? (int)(packed & 0x0F) : (int)(packed >> 4);
            return dg * (float)q - mg;
        }
        case FLLM_TYPE_Q5_K: {  // Dequantizer.cs:333-366
            const uint8_t* p = w + (e >> 8) * 176;
            int t = (int)(e & 255), g = t >> 5;
            float d = half_exact(deq_ld_u16(p)), dmin = half_exact(deq_ld_u16(p + 2));
            int sc, mn;
            kscale_min(p + 4, g, sc, mn);
            float dg = d * (float)sc;
            float mg = dmin * (float)mn;
            uint32_t pl = p[48 + (t >> 1)];
            int lo = (t & 1) == 0 ? (int)(pl & 0x0F) : (int)(pl >> 4);
            int hi = (p[16 + (t >> 3)] >> (t & 7)) & 1;
            int q = (hi << 4) | lo;
            return dg * (float)q - mg;
        }
        case FLLM_TYPE_Q6_K: {  // Dequantizer.cs:395-416
            const uint8_t* p = w + (e >> 8) * 210;
            int i = (int)(e & 255);
            uint32_t qlb = p[i >> 1];
            int low = (i & 1) == 0 ? (int)(qlb & 0x0F) : (int)(qlb >> 4);
            int high = (p[128 + (i >> 2)] >> ((i & 3) * 2)) & 3;
            int q = ((high << 4) | low) - 32;
            int scale = (int8_t)p[192 + (i >> 4)];
            float d = half_exact(deq_ld_u16(p + 208));
            return d * (float)scale * (float)q;
        }
        case FLLM_TYPE_Q8_K: {  // Dequantizer.cs:444-455
            const uint8_t* p = w + (e >> 8) * 292;
            float d = bits_f32(deq_ld_u32(p));
            return (float)(int8_t)p[4 + (e & 255)] * d;
        }
        default: return 0.0f;
    }
}

// Any supported type (F32, F16, BF16 and the quantized ones).
__device__ __forceinline__ float deq_elem(int type, const uint8_t* w, int64_t e) {
    switch (type) {
        case FLLM_TYPE_F32: return bits_f32(deq_ld_u32(w + e * 4));
        case FLLM_TYPE_F16: return half_exact(deq_ld_u16(w + e * 2));
        case FLLM_TYPE_BF16: return bf16_exact(deq_ld_u16(w + e * 2));
        default: return deq_elem_q(type, w, e);
    }
}

}  // namespace fllm
