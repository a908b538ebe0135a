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

// DPP lane exchange within rows of 16 lanes (row_shr / quad_perm / mirror controls).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_rows(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes of a wave, all in DPP: rows of 16 lanes first (quad swaps, half-row and row
// mirrors), then row_bcast:15 adds row 0 into row 1 and row 2 into row 3, and row_bcast:31 adds
// rows 0-1 into rows 2-3. The total is valid in lane 63.
__device__ __forceinline__ float wave_sum_lane63(float v) {
    v += dpp<0xB1>(v);           // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);           // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);          // row_half_mirror
    v += dpp<0x140>(v);          // row_mirror
    v += dpp_rows<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_rows<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Sum over the 64 lanes of a wave; the total is valid in lane 0 only. Within each row of 16 lanes
// the sum is formed with DPP (quad_perm swaps, then half-row and row mirrors), then the four row
// sums are read from lanes 0, 16, 32, 48.
__device__ __forceinline__ float wave_sum_lane0(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Power-of-two exponent t that brings a magnitude `mx` (>= 0) into [2^14, 2^15) as mx * 2^t when mx
// is a normal fp32 value (subnormals land below, inf and NaN stay what they are): the shift that
// maps a chunk of fp32 activations onto fp16's range before it is split into fp16 hi + lo terms.
__device__ __forceinline__ int fp16_range_shift(float mx) {
    return 141 - (int)((__builtin_bit_cast(uint32_t, mx) >> 23) & 0xFFu);
}

// Buffer resource over `bytes` bytes at `p`: raw buffer loads take 32-bit offsets and return 0 for
// any offset past the end (hardware range check), so edge tiles need no clamps.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOutOfRange = 0xFFFFFFF0u;  // an offset every resource rejects
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(rsrc_t r, uint32_t off) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load2(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// binary32 -> bfloat16 bits, round to nearest even; a NaN keeps its sign and top payload bits and
// becomes quiet ((bits >> 16) | 0x40). gfx950 converts in hardware (v_cvt_pk_bf16_f32, two values
// per instruction); on the MI355X it gives exactly that integer formula on every bit pattern tried
// (specials, ties, subnormals and a million random patterns, during development), and the parity
// tests check the bf16 outputs against the formula.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
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

// LDS pointer type of the direct global-to-LDS loads (buffer_load ... lds).
typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from a buffer straight into LDS: lane l writes dst + 16 l. Completion counts in
// vmcnt like any buffer load.
__device__ __forceinline__ void lds_dma16(rsrc_t r, void* dst, uint32_t voffset, uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, voffset, soffset, 0, 0);
}

// s_waitcnt with vmcnt = N and lgkmcnt / expcnt left open (gfx9 encoding: vmcnt[3:0] and
// vmcnt[5:4] at bits 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

}  // namespace byhip
