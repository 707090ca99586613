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

// Byte j of block b of row `row` of a tensor in fragment order (the tile
// layout of qk_frag_offset in qsf_hip_internal.h): tile (row / 16, b / 4) of
// 64 * bb bytes, lane 16 (b % 4) + row % 16, 16-byte planes then a tail
// plane of bb % 16 bytes a lane.
__device__ __forceinline__ size_t frag_off(size_t row, int b, int j, int nq, int bb) {
    const size_t tile = (row >> 4) * (size_t)nq + (size_t)(b >> 2);
    const int lane = (b & 3) * 16 + (int)(row & 15);
    const int k = bb >> 4;
    const size_t base = tile * 64 * (size_t)bb;
    return j < 16 * k ? base + (size_t)(j >> 4) * 1024 + (size_t)lane * 16 + (size_t)(j & 15)
                      : base + (size_t)k * 1024 + (size_t)lane * (size_t)(bb & 15) + (size_t)(j - 16 * k);
}

// Byte j of block b of a row of nb blocks of bs codes in row-plane order
// (the layout of qk_plane_offset in qsf_hip_internal.h), from the row's
// first byte.  Blocks of up to 64 codes: 16-byte planes of nb blocks, then a
// tail plane of bb % 16 bytes a block.  Larger blocks: the meta dwords, then
// the same planes over 64-code parts.
__device__ __forceinline__ uint32_t plane_off(int b, int j, int nb, int bb, int bs) {
    if (bs <= 64) {
        const int k = bb >> 4;
        return j < 16 * k ? (uint32_t)(j >> 4) * (uint32_t)nb * 16u + (uint32_t)b * 16u + (uint32_t)(j & 15)
                          : (uint32_t)k * (uint32_t)nb * 16u + (uint32_t)b * (uint32_t)(bb & 15) +
                                (uint32_t)(j - 16 * k);
    }
    if (j < 4) return (uint32_t)b * 4u + (uint32_t)j;
    const int P = bs >> 6, cwb = (bb - 4) / P, k = cwb >> 4;
    const uint32_t np = (uint32_t)nb * (uint32_t)P, u = (uint32_t)b * (uint32_t)P + (uint32_t)((j - 4) / cwb);
    const int c = (j - 4) % cwb;
    return c < 16 * k ? (uint32_t)nb * 4u + (uint32_t)(c >> 4) * np * 16u + u * 16u + (uint32_t)(c & 15)
                      : (uint32_t)nb * 4u + (uint32_t)k * np * 16u + u * (uint32_t)(cwb & 15) + (uint32_t)(c - 16 * k);
}

// Signed 4-bit x signed 4-bit dot of 8 nibble pairs, accumulated in int32
// (v_dot8_i32_i4).
__device__ __forceinline__ int sdot8(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot8((int)a, (int)b, c, false);
}
// The same with a zero accumulator, as the three-operand v_dot8_i32_i4 with
// an inline-constant 0: for sdot8(a, b, 0) the compiler materialises the
// zero with a v_mov and uses the two-address v_dot8c form.
__device__ __forceinline__ int sdot8_z(uint32_t a, uint32_t b) {
    int r;
    asm("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// fp32 multiply, add and subtract, each rounded on its own to nearest even,
// as the reference's scalar C code performs them.  HIP's __fmul_rn and
// __fadd_rn are plain operators, which the compiler's default contraction
// mode may fuse into an FMA once inlined; these carry the contraction pragma
// at the operation itself, so they stay separate wherever they are inlined.
// (fmaf and __builtin_fmaf remain single-rounding FMAs.)
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

// act(g) * u with QSFActivation act: 2 SiLU, 0/1 GELU (tanh form), else
// ReLU (src/kernels_scalar.c:129-147, src/engine.c:1128-1140).  Every
// operation is rounded on its own (no contraction into FMAs), so the
// act-mul kernel and the gate/up GEMV's fused epilogue give the same bits.
__device__ __forceinline__ float act_mul(int act, float g, float u) {
    float x = g;
    if (act == 2) {
        x = __fdiv_rn(x, add_rn(1.0f, expf(-x)));
    } else if (act == 0 || act == 1) {
        const float inner = mul_rn(0.7978845608f, add_rn(x, mul_rn(mul_rn(mul_rn(0.044715f, x), x), x)));
        x = mul_rn(mul_rn(0.5f, x), add_rn(1.0f, tanhf(inner)));
    } else if (x < 0.0f) {
        x = 0.0f;
    }
    return mul_rn(x, u);
}

// Sum over the workgroup (blockDim.x a multiple of 64, <= 1024); every
// thread gets the total.  `red` holds one float per wave.  The norm launches
// and the GEMV's fused norm prologue both reduce through this, so equal
// thread counts give equal sums.
__device__ __forceinline__ float wg_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    __syncthreads();                       // `red` free from any earlier use
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < nw; w++) t += red[w];
    return t;
}

// Butterfly sum over groups of `width` consecutive lanes (power of two).
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
// Sum over groups of `width` consecutive lanes (power of two, <= 64) with
// DPP; the group's total lands in its last lane (others hold partials).
__device__ __forceinline__ float group_sum_last(float v, int width) {
#define QSF_DPPF(x, ctrl, rmask) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (x)), (ctrl), (rmask), 0xF, false))
    if (width >= 2) v += QSF_DPPF(v, 0xB1, 0xF);     // quad_perm [1,0,3,2]
    if (width >= 4) v += QSF_DPPF(v, 0x4E, 0xF);     // quad_perm [2,3,0,1]
    if (width >= 8) v += QSF_DPPF(v, 0x141, 0xF);    // row_half_mirror
    if (width >= 16) v += QSF_DPPF(v, 0x140, 0xF);   // row_mirror
    if (width >= 32) v += QSF_DPPF(v, 0x142, 0xA);   // row_bcast15 into rows 1, 3
    if (width >= 64) v += QSF_DPPF(v, 0x143, 0xC);   // row_bcast31 into rows 2, 3
#undef QSF_DPPF
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
