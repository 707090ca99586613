// qsf_device.h - device-side helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qsf {

// IEEE binary16 bits -> fp32 with the hardware converter (v_cvt_f32_f16).
// Exact for every finite half (subnormals included: fp16 denormals are on);
// a NaN comes back quiet, which is the one difference from the bit-level
// decoder of src/quant.c:11-39.
__device__ __forceinline__ float f16_lo(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFFu));
}
__device__ __forceinline__ float f16_hi(uint32_t v) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}
__device__ __forceinline__ float f16_bits(uint16_t v) {
    return (float)__builtin_bit_cast(_Float16, v);
}

// Signed 4-bit x signed 4-bit dot of 8 nibble pairs, accumulated in int32
// (v_dot8_i32_i4).
__device__ __forceinline__ int sdot8(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot8((int)a, (int)b, c, false);
}

// Butterfly sum over groups of `width` consecutive lanes (power of two).
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ int wave_or_i(int v) {
    for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, 64);
    return v;
}

}  // namespace qsf
