// byhip_kernels.h - device helpers shared by the kernels of libbybyhip.so (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "byhip.h"

namespace byhip {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i8v __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 bits_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint16_t h_bits(_Float16 v) { return __builtin_bit_cast(uint16_t, v); }
__device__ __forceinline__ _Float16 bits_h(uint16_t v) { return __builtin_bit_cast(_Float16, v); }

// Sum over the 64 lanes of a wave (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// binary32 -> bfloat16 bits, round to nearest even; NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Output element store by dtype (BYHIP_F32 / BYHIP_F16 / BYHIP_BF16).
template <int YT>
__device__ __forceinline__ void store_y(void* y, size_t idx, float v) {
    if constexpr (YT == BYHIP_F32) {
        static_cast<float*>(y)[idx] = v;
    } else if constexpr (YT == BYHIP_F16) {
        static_cast<_Float16*>(y)[idx] = (_Float16)v;
    } else {
        static_cast<uint16_t*>(y)[idx] = f32_to_bf16_bits(v);
    }
}

}  // namespace byhip
