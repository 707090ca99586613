// gemv_decode.hip - batch-1 decode GEMV over QSF 2/3/4-bit blocks on gfx950.
//
// Replaces the fused dequant->dot loops of src/kernels_scalar.c:16-109 and the
// outlier matvec of src/quant.c:387-495 (CPU twins: src/kernels_avx2.c:77-549).
// The QSF block bytes are read as they are on disk:
//   [fp16 scale][fp16 zero | reserved][packed codes]   (src/quant.c:87-177)
//
// Arithmetic.  Per block the reference computes sum_k (s*q_k + z) * x_k.  Here
//   sum_k (s*q_k + z) x_k = s * sum_k q_k x_k + z * sum_k x_k
// and the code/activation products are done exactly in integers: each block
// of x becomes block-fixed-point integers X_k = x_k*2^sh (|X| <= 2^XB,
// XB = 22 bits, 20 for 3-bit) split into six signed base-16 digits.  The
// GEMV multiplies raw code nibbles by digit nibbles with v_dot8_i32_i4 (8
// exact products per instruction), recombines the digits per block in two
// exact int32 groups (digits 0-2 and 3-5), converts each exactly to fp32,
// joins them and adds s * sum q X + z' * sum X into an fp32 row sum (the
// block's meta holds the power-of-two rescale).  The roundings are x -> X
// (at most 2^-(XB+1) of the block's max |x|) and those of fp32 arithmetic on
// block partial sums, the same order as the reference's own fp32
// accumulation; for normal-distributed x the result sits within about 1e-6
// relative L2 of the fp64 value, an order inside the 1e-5 bar.
//
// Code unpacking is pure masking, chosen so each nibble holds one signed
// 4-bit value that the digit tables pair with the right x:
//   4-bit asym : q ^ 0x8 = q - 8 (two's complement); zero term z + 8s
//   4-bit sym  : raw nibble, already the two's-complement code the scalar
//                reference decodes (src/quant.c:166-174)
//   2-bit      : even crumbs (w & 0x33333333), odd crumbs ((w>>2) & 0x33333333)
//   3-bit      : every nibble of the bitstream holds the high part of one code
//                and the low part of the next; two masked copies (A, and B
//                shifted right by one) carry them, with digit tables scaled by
//                powers of two so that sum = S_A + S_B/4 exactly.
//
// Launch.  1024-thread workgroups on a 2-D grid: blockIdx.y picks the
// matrix of a group (gate/up share one launch and one x), blockIdx.x a run
// of tpw R-row tiles, about one workgroup per CU in total.  Each workgroup
// first turns x into digits in LDS itself (no separate launch; a v_perm
// nibble transpose builds the digit words), then its 16 waves walk their
// tiles.  Within a tile, lane l of a row group handles blocks l, l+LPG, ...
// so each lane reads whole blocks (dword loads from 4-byte aligned blocks,
// 32-bit offsets) and reuses its block's digits (odd LDS stride:
// conflict-free) for R rows.  Weight loads are issued straight-line, D
// blocks ahead, with no loads or stores inside conditionals (the compiler's
// wait counts stay exact); row sums go to an LDS stash and are stored at the
// end.  A fused CSR pass adds the fp16 outliers of each tile's rows; partial
// sums are reduced with DPP.
#include "qsf_device.h"
#include "qsf_hip_internal.h"

#include <hip/hip_ext.h>

#include <utility>

namespace {

constexpr int ND = 6;                  // balanced base-16 digits per multiplier
constexpr int ND_LO = 3;               // digits 0-2 and 3-5 are recombined separately
constexpr uint32_t DIGIT_BIAS = 0x888888u;   // 8 * (16^6 - 1) / 15
constexpr int WAVES = 16;              // waves per GEMV workgroup
constexpr int MAXT = 4;                // tiles per wave (compile-time bound)
// Main kernel with the digits in registers: one-row tiles, up to 8 a wave.
constexpr int tiles_per_wave(bool dreg) { return dreg ? 8 : MAXT; }
constexpr int kLdsBudget = 64 * 1024;  // block digits + meta held at once
constexpr size_t kLdsLimit = 160 * 1024; // cap on a GEMV workgroup's dynamic LDS (gfx950 LDS)

constexpr int pow2ceil(int v) { return v <= 1 ? 1 : 2 * pow2ceil((v + 1) / 2); }

// 4-byte alignment is all global dwordx4 loads need; x may be any float*
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef f32x4 f32x4_a4 __attribute__((aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));

template <int FMT, int BS>
struct Fmt {
    static constexpr int BITS = FMT == QK_FMT_2 ? 2 : (FMT == QK_FMT_3 ? 3 : 4);
    static constexpr int CW = BS * BITS / 32;                       // code dwords / block
    static constexpr int NC = (FMT == QK_FMT_2 || FMT == QK_FMT_3) ? 2 : 1;  // masked copies
    static constexpr int NA = FMT == QK_FMT_3 ? 2 : 1;              // accumulator sets
    static constexpr int BB = 4 + 4 * CW;                           // block bytes
    static constexpr int DW = CW * NC * ND;                         // digit dwords / block
    // LDS stride of a block's digits: a whole number of 16-byte quads, odd,
    // so that lanes reading consecutive blocks with ds_read_b128 hit
    // distinct banks
    static constexpr int DWS = (DW / 4) % 2 ? DW : DW + 4;
    static_assert(DW % 4 == 0, "digit words come in quads");
    // x-prep lanes per block and x values per lane: 2/4-bit, one code dword
    // a lane (its 16 or 8 codes); 3-bit, two lanes for each three code
    // dwords (32 codes, whose slots then map to fixed columns and shifts),
    // one masked copy each
    static constexpr int LPB = FMT == QK_FMT_3 ? 2 * CW / 3 : pow2ceil(CW);
    static constexpr int NX = FMT == QK_FMT_3 ? 32 : NC * 8;
    // |X| <= 2^XB.  Digit multipliers M = X * 2^shift (shift <= 2 for 3-bit)
    // must lie in the 6-digit balanced range [-0x888888, 0x777777].  A
    // digit sum over a block is at most 8 * 8 * BS <= 2^14 in magnitude, so
    // each 3-digit group sum stays below 273 * 2^14 < 2^23: exact in fp32.
    static constexpr int XB = FMT == QK_FMT_3 ? 20 : 22;
};

// 3-bit masks for code dword w with w % 3 == k.  Nibble g = 8w + i has
// delta = g mod 3 = (2k + i) mod 3; A keeps the bits of the first code in the
// nibble, B' (after >> 1) the bits of the second.
__host__ __device__ constexpr uint32_t f3_mask(int k, int which) {
    uint32_t m = 0;
    for (int i = 0; i < 8; i++) {
        int d = (2 * k + i) % 3;
        uint32_t v = which == 0 ? (d == 0 ? 7u : (d == 1 ? 3u : 1u))
                                : (d == 0 ? 4u : (d == 1 ? 6u : 7u));
        m |= v << (4 * i);
    }
    return m;
}

template <int FMT, int WI>
__device__ __forceinline__ uint32_t extract(uint32_t w, int c) {
    if constexpr (FMT == QK_FMT_4) return w ^ 0x88888888u;
    else if constexpr (FMT == QK_FMT_4SYM) return w;
    else if constexpr (FMT == QK_FMT_2) return c == 0 ? (w & 0x33333333u) : ((w >> 2) & 0x33333333u);
    else return c == 0 ? (w & f3_mask(WI % 3, 0)) : ((w >> 1) & f3_mask(WI % 3, 1));
}

// Code index (within the block) and power-of-two scale of the x multiplier
// paired with nibble m of copy c of code dword w.
template <int FMT>
__device__ __forceinline__ void slot_code(int w, int c, int m, int& code, int& shift) {
    if constexpr (FMT == QK_FMT_2) { code = 16 * w + 2 * m + c; shift = 0; }
    else if constexpr (FMT == QK_FMT_3) {
        int g = 8 * w + m;
        code = (4 * g) / 3 + c;
        shift = g % 3;
    } else { code = 8 * w + m; shift = 0; }
}

// Eight 24-bit biased multipliers U[m] -> six digit words: nibble m of
// word d = nibble d of U[m], re-biased to two's complement (n - 8).
__device__ __forceinline__ void digit_words(const uint32_t (&U)[8], uint32_t (&out)[ND]) {
    uint32_t P[4], Q[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        // byte k of P[j]: digit 2k of U[2j] | digit 2k of U[2j+1] << 4; Q: digit 2k+1
        P[j] = (U[2 * j] & 0x0F0F0F0Fu) | ((U[2 * j + 1] & 0x0F0F0F0Fu) << 4);
        Q[j] = ((U[2 * j] >> 4) & 0x0F0F0F0Fu) | (U[2 * j + 1] & 0xF0F0F0F0u);
    }
    // 4x4 byte transposes (v_perm_b32: selector byte 0-3 = src1 byte, 4-7 = src0 byte)
    const uint32_t pa0 = __builtin_amdgcn_perm(P[1], P[0], 0x05010400u);
    const uint32_t pa1 = __builtin_amdgcn_perm(P[1], P[0], 0x07030602u);
    const uint32_t pb0 = __builtin_amdgcn_perm(P[3], P[2], 0x05010400u);
    const uint32_t pb1 = __builtin_amdgcn_perm(P[3], P[2], 0x07030602u);
    const uint32_t qa0 = __builtin_amdgcn_perm(Q[1], Q[0], 0x05010400u);
    const uint32_t qa1 = __builtin_amdgcn_perm(Q[1], Q[0], 0x07030602u);
    const uint32_t qb0 = __builtin_amdgcn_perm(Q[3], Q[2], 0x05010400u);
    const uint32_t qb1 = __builtin_amdgcn_perm(Q[3], Q[2], 0x07030602u);
    out[0] = __builtin_amdgcn_perm(pb0, pa0, 0x05040100u) ^ 0x88888888u;
    out[2] = __builtin_amdgcn_perm(pb0, pa0, 0x07060302u) ^ 0x88888888u;
    out[4] = __builtin_amdgcn_perm(pb1, pa1, 0x05040100u) ^ 0x88888888u;
    out[1] = __builtin_amdgcn_perm(qb0, qa0, 0x05040100u) ^ 0x88888888u;
    out[3] = __builtin_amdgcn_perm(qb0, qa0, 0x07060302u) ^ 0x88888888u;
    out[5] = __builtin_amdgcn_perm(qb1, qa1, 0x05040100u) ^ 0x88888888u;
    (void)pb1;
}

// x preparation for one block b by a group of LPB lanes (lane w owns code
// dword w): block max, shift, X, digit words into dst[(w*NC + c)*ND + d], and
// from lane 0 the block meta {f = 2^-sh, sum_k X_k * f}.  All lanes of the
// group must call it together (group shuffles).
// Split in a load half and a compute half so callers can issue the x loads
// before other vector-memory traffic (loads return in issue order).
template <int FMT, int BS, bool V4 = false>
__device__ __forceinline__ void prep_load(const float* __restrict__ x, int cols, int b, bool live,
                                          int w, float (&xv)[Fmt<FMT, BS>::NX]) {
    using F = Fmt<FMT, BS>;
    constexpr int NX = F::NX;
    const bool lane_live = live && w < (FMT == QK_FMT_3 ? F::LPB : F::CW);
    const int col0 = b * BS + (FMT == QK_FMT_3 ? w >> 1 : w) * NX;
    if constexpr (!V4) {
        // any cols: the lane's NX consecutive x values (16-B vector loads
        // when in range and aligned), 2/4-bit re-ordered to slot order
        float xr[NX];
        const bool full = lane_live && col0 + NX <= cols &&
                          ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
        if (full) {
            const float4* x4 = reinterpret_cast<const float4*>(x + col0);
#pragma unroll
            for (int k = 0; k < NX / 4; k++) {
                const float4 v = x4[k];
                xr[4 * k] = v.x; xr[4 * k + 1] = v.y; xr[4 * k + 2] = v.z; xr[4 * k + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < NX; k++) {
                const int col = col0 + k;
                const float v = x[min(max(col, 0), cols - 1)];
                xr[k] = (lane_live && col < cols) ? v : 0.0f;
            }
        }
#pragma unroll
        for (int s = 0; s < NX; s++) {
            if constexpr (FMT == QK_FMT_3) {
                xv[s] = xr[s];
            } else {
                int code, shift;
                slot_code<FMT>(0, s / 8, s % 8, code, shift);
                xv[s] = xr[code];
            }
        }
    } else {
        // cols >= 4: only the loads -- the lane's NX consecutive x values as
        // dwordx4 (4-byte alignment suffices) at clamped addresses, raw into
        // xv; prep_settle() fixes them up once they are needed, so nothing
        // here waits for them
#pragma unroll
        for (int k = 0; k < NX / 4; k++) {
            const f32x4 v = *reinterpret_cast<const f32x4_a4*>(x + min(col0 + 4 * k, cols - 4));
            xv[4 * k] = v.x; xv[4 * k + 1] = v.y; xv[4 * k + 2] = v.z; xv[4 * k + 3] = v.w;
        }
    }
}

// Re-index chunks loaded at base = min(col0 + 4k, cols - 4): column c sits at
// c - base when c < cols; columns past the end and dead lanes read zero.
template <int NCH, int N>
__device__ __forceinline__ void settle_chunks(float (&xv)[N], int col0, int cols, bool lane_live) {
    static_assert(4 * NCH <= N, "chunks past the array");
#pragma unroll
    for (int k = 0; k < NCH; k++) {
        const int base = min(col0 + 4 * k, cols - 4);
        const float v0 = xv[4 * k], v1 = xv[4 * k + 1], v2 = xv[4 * k + 2], v3 = xv[4 * k + 3];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = col0 + 4 * k + i, at = c - base;
            const float v = at == 0 ? v0 : (at == 1 ? v1 : (at == 2 ? v2 : v3));
            xv[4 * k + i] = (lane_live && c < cols) ? v : 0.0f;
        }
    }
}

// Second half of a V4 prep_load: zero what lies past the last column or
// belongs to no block, re-index a clamped 2/4-bit chunk (chunk k was read at
// base = min(col0 + 4k, cols - 4); column c sits at c - base when c < cols)
// and put 2/4-bit values in slot order.
template <int FMT, int BS>
__device__ __forceinline__ void prep_settle(int b, bool live, int w, int cols,
                                            float (&xv)[Fmt<FMT, BS>::NX]) {
    using F = Fmt<FMT, BS>;
    constexpr int NX = F::NX;
    const bool lane_live = live && w < (FMT == QK_FMT_3 ? F::LPB : F::CW);
    const int col0 = b * BS + (FMT == QK_FMT_3 ? w >> 1 : w) * NX;
    if (!lane_live || col0 + NX > cols) settle_chunks<NX / 4>(xv, col0, cols, lane_live);
    if constexpr (FMT != QK_FMT_3) {
        float xr[NX];
#pragma unroll
        for (int s = 0; s < NX; s++) xr[s] = xv[s];
#pragma unroll
        for (int s = 0; s < NX; s++) {
            int code, shift;
            slot_code<FMT>(0, s / 8, s % 8, code, shift);
            xv[s] = xr[code];
        }
    }
}

// Block meta: f = 2^-sh (exact) and sx = f * sum_k X_k (rounded once), fp32.
// xs (optional): the lane's x values copied to LDS (columns < cols).
// op over aligned groups of W lanes (power of two, <= 64) with the result
// in every lane of the group: quad_perm exchanges within quads, then
// row_half_mirror (lane i <-> 7 - i) and row_mirror (i <-> 15 - i) pair each
// lane with one of the other half of its group; groups wider than a 16-lane
// row finish with one shuffle per doubling.  DPP instead of __shfl_xor: no
// LDS crossbar round trip per step.  Every lane of the wave must be active.
template <int W, typename OP>
__device__ __forceinline__ int group_allreduce(int v, OP op) {
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "power-of-two groups within a wave");
    if constexpr (W >= 2) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
    if constexpr (W >= 4) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
    if constexpr (W >= 8) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
    if constexpr (W >= 16) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
    if constexpr (W >= 32) v = op(v, __shfl_xor(v, 16, 64));
    if constexpr (W >= 64) v = op(v, __shfl_xor(v, 32, 64));
    return v;
}

template <int FMT, int BS>
__device__ __forceinline__ void prep_finish(const float (&xv)[Fmt<FMT, BS>::NX], int b,
                                            bool live, int w, uint32_t* dst, float2* meta,
                                            float* xs = nullptr, int cols = 0) {
    using F = Fmt<FMT, BS>;
    constexpr int NX = F::NX;
    const bool lane_live = live && w < (FMT == QK_FMT_3 ? F::LPB : F::CW);
    const int xg = FMT == QK_FMT_3 ? w >> 1 : w;         // the lane's group of NX x values
    if (xs && lane_live && (FMT != QK_FMT_3 || (w & 1) == 0)) {
        // the lane's NX consecutive columns from b*BS + NX*xg (zero past
        // cols, as the copy must hold there), in column order as 16-byte
        // LDS stores
        constexpr auto slot_of = [](int k) {
            return FMT == QK_FMT_2 ? (k & 1) * 8 + (k >> 1) : k;   // 3-bit: column order
        };
        f32x4* d4 = reinterpret_cast<f32x4*>(xs + b * BS + NX * xg);
#pragma unroll
        for (int q = 0; q < NX / 4; q++)
            d4[q] = f32x4{xv[slot_of(4 * q)], xv[slot_of(4 * q + 1)], xv[slot_of(4 * q + 2)],
                          xv[slot_of(4 * q + 3)]};
    }
    // block max of |x| as fp32 bits (non-negative floats order like their
    // bits; Inf and NaN give bits >= 0x7F800000): one integer max over the group
    uint32_t amax_u = 0;
#pragma unroll
    for (int s = 0; s < NX; s++) amax_u = max(amax_u, __builtin_bit_cast(uint32_t, xv[s]) & 0x7FFFFFFFu);
    const int amax_b = group_allreduce<F::LPB>((int)amax_u, [](int u, int v) { return max(u, v); });
    const bool bad = amax_b >= 0x7F800000;
    const float amax = __builtin_bit_cast(float, amax_b);
    int sh = 0;
    if (!bad && amax > 0.0f) {
        sh = F::XB - 1 - ilogbf(amax);                 // amax * 2^sh < 2^XB
        sh = sh > 126 ? 126 : sh;                      // f = 2^-sh stays a normal fp32
    }
    // X = rint(x * 2^sh) once per x value, biased: |x * 2^sh| < 2^XB <= 2^22,
    // so x * 2^sh + 1.5 * 2^23 (one rounding, to nearest even, as rintf)
    // is the integer 1.5 * 2^23 + X, whose bits are 0x4B400000 + X.  A block
    // with Inf or NaN gets NaN meta, which makes its digits irrelevant.
    const float scale = ldexpf(1.0f, sh);
    uint32_t U0[NX];
    uint32_t bsum = 0;
#pragma unroll
    for (int s = 0; s < NX; s++) {
        const uint32_t bits = __builtin_bit_cast(uint32_t, fmaf(xv[s], scale, 12582912.0f));
        U0[s] = bits - (0x4B400000u - DIGIT_BIAS);     // X + DIGIT_BIAS
        bsum += bits;
    }
    // every code counted once; |block total| <= BS * 2^XB <= 2^29: exact in
    // int32 (the sum of biased bits wraps back to it)
    // (3-bit: the two lanes of a group hold the same values; one counts them)
    int sum = bad || (FMT == QK_FMT_3 && (w & 1)) ? 0 : (int)(bsum - (uint32_t)NX * 0x4B400000u);
    sum = group_allreduce<F::LPB>(sum, [](int u, int v) { return u + v; });
    const double dsum = (double)sum;
    if (lane_live) {
        if constexpr (FMT == QK_FMT_3) {
            // code dwords 3*xg .. 3*xg+2, masked copy c = w % 2 of each: the
            // multiplier of slot (c, m) of dword v is X[code] * 2^shift,
            // where copy 1 pairs with the code after copy 0's
            const int c = w & 1;
#pragma unroll
            for (int v = 0; v < 3; v++) {
                uint32_t u8[8], dw[ND];
#pragma unroll
                for (int m = 0; m < 8; m++) {
                    int code, shift;
                    slot_code<FMT>(v, 0, m, code, shift);
                    const uint32_t xu = c ? U0[code + 1] : U0[code];
                    // X * 2^shift + DIGIT_BIAS
                    u8[m] = (xu << shift) + (DIGIT_BIAS - (DIGIT_BIAS << shift));
                }
                digit_words(u8, dw);
#pragma unroll
                for (int d = 0; d < ND; d++) dst[((3 * xg + v) * F::NC + c) * ND + d] = dw[d];
            }
        } else {
            // code dword w, both masked copies (one for 4-bit)
#pragma unroll
            for (int c = 0; c < F::NC; c++) {
                uint32_t u8[8], dw[ND];
#pragma unroll
                for (int m = 0; m < 8; m++) u8[m] = U0[c * 8 + m];   // X + DIGIT_BIAS
                digit_words(u8, dw);
#pragma unroll
                for (int d = 0; d < ND; d++) dst[(w * F::NC + c) * ND + d] = dw[d];
            }
        }
    }
    if (live && w == 0) {
        // f exact; sx = f * sum X rounded once (the fp64 product is exact)
        const float f = bad ? __builtin_nanf("") : ldexpf(1.0f, -sh);
        *meta = make_float2(f, (float)(dsum * ldexp(1.0, -sh)));
    }
}

template <int FMT, int BS>
__device__ __forceinline__ void prep_block(const float* __restrict__ x, int cols, int b, bool live,
                                           int w, uint32_t* dst, float2* meta,
                                           float* xs = nullptr) {
    float xv[Fmt<FMT, BS>::NX];
    prep_load<FMT, BS>(x, cols, b, live, w, xv);
    prep_finish<FMT, BS>(xv, b, live, w, dst, meta, xs, cols);
}

// Stand-alone x preparation (prepared mode): 256 threads, 256/LPB blocks each.
// With `xcopy` it also writes fp32 x there (nb*BS floats, zero past cols for
// 2/4-bit), which lets x come from host-mapped memory in one read.
template <int FMT, int BS>
__global__ __launch_bounds__(256) void xprep_kernel(const float* __restrict__ x, int cols, int nb,
                                                    uint32_t* __restrict__ xq,
                                                    float2* __restrict__ xmeta,
                                                    float* __restrict__ xcopy) {
    using F = Fmt<FMT, BS>;
    const int b = blockIdx.x * (256 / F::LPB) + threadIdx.x / F::LPB;
    const bool live = b < nb;
    const int bb = live ? b : 0;
    prep_block<FMT, BS>(x, cols, b, live, threadIdx.x & (F::LPB - 1), xq + (size_t)bb * F::DWS,
                        xmeta + bb, xcopy);
}

// Prepared digits at ws, block meta after them at the next 256-byte boundary.
template <int FMT, int BS>
__host__ __device__ inline float2* xmeta_in(void* ws, int nb) {
    const size_t dig = (size_t)nb * Fmt<FMT, BS>::DWS * 4;
    return (float2*)((uint8_t*)ws + ((dig + 255) & ~(size_t)255));
}

// Group sum over `lpg` lanes (power of two) with DPP; the total is valid in
// the group's last lane (all lanes for lpg <= 16).
__device__ __forceinline__ float group_reduce(float v, int lpg) {
    if (lpg == 64) return qsf::group_sum_last(v, 64);
    return qsf::group_sum_last(v, lpg);
}

template <int CTRL, int BANK>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, BANK, false));
}
#undef QSF_DPP

struct GemvArgs {
    const uint8_t* w[QK_MAX_GROUP];
    float* y[QK_MAX_GROUP];
    const uint32_t* rp[QK_MAX_GROUP];   // outlier CSR row pointers (rows + 1), or null
    const uint32_t* oe[QK_MAX_GROUP];   // packed entries col | fp16 << 16 (cols <= 65536)
    const uint32_t* oc[QK_MAX_GROUP];   // else split entries: columns ...
    const uint16_t* ov[QK_MAX_GROUP];   // ... and fp16 values
    int rows[QK_MAX_GROUP];
    int tile0[QK_MAX_GROUP + 1];   // prefix sums of tiles (R * 64/lpg rows each)
    int nent[QK_MAX_GROUP];             // outlier entries kept per matrix
    // main kernel: matrix blockIdx.y, all its fields in one record (read at
    // an address known when the wave starts, in one batch of scalar loads)
    struct Mat {
        const uint8_t* w;
        float* y;
        const uint32_t* rp;                 // null: no outliers
        const uint32_t* oe;                 // packed entries
        int rows, nent, tiles, pad;
    } mat[QK_MAX_GROUP];
    int n, cols, nb, lpg, lpg_log2, chunk, tpw;
    int xs_off;                    // LDS dword offset of fp32 x (main kernel)
    int st_off, st_wave;           // LDS dword offset / floats per wave of the result stash
    int pr_off;                    // one block a lane, one-row tiles, 64-lane groups: LDS dword
                                   // offset of each wave's [MT][64] lane partials, or 0
    uint32_t row_bytes;            // SPLIT kernels: bytes a stored row
    int lsplit;                    // SPLIT: log2(stored block size / BS)
    const uint32_t* xq;            // prepared digits (stride DWS), or null: prepare here
    const float2* xmeta;
    const float* x;
    // paired rows (row 2i gate_i, row 2i+1 up_i; two-row tiles, one matrix):
    // 1 + the activation, and y[i] = act(gate_i x) * (up_i x); 0: plain rows
    int act1;
    // NORM kernels: x is a residual increment.  r = res_in + x (workgroup
    // (0, 0) stores it to res_out and the NaN check to *bad), and the rows
    // multiply rms_norm(r) * nw, kept in LDS
    const float* res_in;
    float* res_out;
    const float* nw;
    int* bad;
    float eps;
};

// NORM kernels: elements of x a thread holds in the norm prologue
constexpr int kNormPerThread = 8;


// Main-kernel limits: x as XV (1 or kXvMax) float4 a thread, prepared digits
// as at most DV dwordx4 a thread, one block meta a thread.
constexpr int kXvMax = 4;              // cols <= 4 * kXvMax * 1024
constexpr int DV = 4;                  // nb * DWS <= 4 * DV * 1024 dwords
constexpr int kMainMaxNb = WAVES * 64;

// fp16 value and column of outlier entry e of matrix m (packed or split table).
__device__ __forceinline__ void entry_at(const GemvArgs& a, int m, uint32_t e, uint32_t& col,
                                         uint32_t& val) {
    if (a.oe[m] != nullptr) {
        const uint32_t u = a.oe[m][e];
        col = u & 0xFFFFu;
        val = u >> 16;
    } else {
        col = a.oc[m][e];
        val = a.ov[m][e];
    }
}

// Weights of one block for the R rows of a tile (row offsets in roff).
template <int FMT, int BS, int R, bool SPLIT = false>
__device__ __forceinline__ void load_block(const uint8_t* __restrict__ w, const uint32_t (&roff)[R],
                                           int b, uint32_t (&wv)[R][1 + Fmt<FMT, BS>::CW],
                                           int lsplit, int nb) {
    using F = Fmt<FMT, BS>;
    if constexpr (SPLIT) {
        // b is 64-code part b of the row (nb parts with data), part
        // b % 2^lsplit of stored block b >> lsplit; row-plane order (blocks
        // of 128 or 256 codes): the stored block's meta dword in the meta
        // plane, then the part's CW code dwords, its quads at 16 b in the
        // 16-byte planes over the row's parts (every part of every stored
        // block, so a partial last block counts whole) and the rest at
        // 4 (CW % 4) b in the tail plane
        constexpr int NQ = F::CW / 4, NT = F::CW % 4;
        const uint32_t nst = ((uint32_t)nb + (1u << lsplit) - 1u) >> lsplit;   // stored blocks a row
        const uint32_t ps = (nst << lsplit) * 16u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            wv[r][0] = __builtin_nontemporal_load(
                reinterpret_cast<const uint32_t*>(w + (roff[r] + 4u * (uint32_t)(b >> lsplit))));
            const uint32_t o = roff[r] + 4u * nst + (uint32_t)b * 16u;
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                const u32x4 v = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4_a4*>(w + (o + (uint32_t)q * ps)));
                wv[r][1 + 4 * q] = v.x;
                wv[r][2 + 4 * q] = v.y;
                wv[r][3 + 4 * q] = v.z;
                wv[r][4 + 4 * q] = v.w;
            }
            if constexpr (NT > 0) {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(
                    w + (roff[r] + 4u * nst + (uint32_t)NQ * ps + (uint32_t)b * (4u * NT)));
#pragma unroll
                for (int i = 0; i < NT; i++) wv[r][1 + 4 * NQ + i] = __builtin_nontemporal_load(p + i);
            }
        }
        return;
    }
    if constexpr (BS <= 64) {
        // row-plane order (tensors of blocks of at most 64 codes): dwords
        // 4i..4i+3 of block b at 16 b in plane i (nb x 16 bytes), the last
        // NW % 4 dwords at 4 (NW % 4) b in the tail plane after the planes.
        // The lanes of a row group read consecutive blocks, so each 16-byte
        // load instruction covers aligned, contiguous memory.
        constexpr int NW = 1 + F::CW, NQ = NW / 4, NT = NW % 4;
        const uint32_t ps = (uint32_t)nb * 16u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t o = roff[r] + (uint32_t)b * 16u;
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                const u32x4 v = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4_a4*>(w + (o + (uint32_t)q * ps)));
                wv[r][4 * q] = v.x;
                wv[r][4 * q + 1] = v.y;
                wv[r][4 * q + 2] = v.z;
                wv[r][4 * q + 3] = v.w;
            }
            if constexpr (NT > 0) {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(
                    w + (roff[r] + (uint32_t)NQ * ps + (uint32_t)b * (4u * NT)));
#pragma unroll
                for (int i = 0; i < NT; i++) wv[r][4 * NQ + i] = __builtin_nontemporal_load(p + i);
            }
        }
    } else {
        // blocks of 128 or 256 codes read whole (the table slots and prepared
        // x), from row-plane order: block b's meta dword at 4 b, then each of its
        // P 64-code parts u = b P + p as in the split read above
        constexpr int P = BS / 64, CWP = F::CW / P, NQ = CWP / 4, NT = CWP % 4;
        const uint32_t np = (uint32_t)nb * P, ps = np * 16u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            wv[r][0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(w + (roff[r] + 4u * (uint32_t)b)));
#pragma unroll
            for (int p = 0; p < P; p++) {
                const uint32_t u = (uint32_t)b * P + (uint32_t)p;
                const uint32_t o = roff[r] + 4u * (uint32_t)nb + u * 16u;
#pragma unroll
                for (int q = 0; q < NQ; q++) {
                    const u32x4 v = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4_a4*>(w + (o + (uint32_t)q * ps)));
                    wv[r][1 + p * CWP + 4 * q] = v.x;
                    wv[r][2 + p * CWP + 4 * q] = v.y;
                    wv[r][3 + p * CWP + 4 * q] = v.z;
                    wv[r][4 + p * CWP + 4 * q] = v.w;
                }
                if constexpr (NT > 0) {
                    const uint32_t* t = reinterpret_cast<const uint32_t*>(
                        w + (roff[r] + 4u * (uint32_t)nb + (uint32_t)NQ * ps + u * (4u * NT)));
#pragma unroll
                    for (int i = 0; i < NT; i++) wv[r][1 + p * CWP + 4 * NQ + i] = __builtin_nontemporal_load(t + i);
                }
            }
        }
    }
}

// Dequant-dot of one block for R rows: rs[r] += s*sum(q*x) + z*sum(x).  The
// digit sums are exact integers; each 3-digit group (< 2^23) converts to fp32
// exactly and the two join with one rounding, so the block's one rounding
// beyond x -> X is that of fp32 arithmetic on its partial sums.
// `dg` is the block's digit words: an LDS pointer, or the lane's own copy in
// registers (an array indexed with constants only).
template <int FMT, int BS, int R, typename DG>
__device__ __forceinline__ void compute_block(const uint32_t (&wv)[R][1 + Fmt<FMT, BS>::CW],
                                              const DG& dg, float2 xm, float (&rs)[R]) {
    using F = Fmt<FMT, BS>;
    int acc[R][F::NA][ND];
    auto step = [&](auto wic) __attribute__((always_inline)) {
        constexpr int wi = decltype(wic)::value;
        uint32_t dd[F::NC][ND];
#pragma unroll
        for (int c = 0; c < F::NC; c++)
#pragma unroll
            for (int d = 0; d < ND; d++) dd[c][d] = dg[(wi * F::NC + c) * ND + d];
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int c = 0; c < F::NC; c++) {
                const uint32_t nib = extract<FMT, wi>(wv[r][1 + wi], c);
                const int s = F::NA == 2 ? c : 0;
                const bool first = wi == 0 && (F::NA == 2 || c == 0);
#pragma unroll
                for (int d = 0; d < ND; d++)
                    acc[r][s][d] = first ? qsf::sdot8_z(nib, dd[c][d])
                                         : qsf::sdot8(nib, dd[c][d], acc[r][s][d]);
            }
        }
    };
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (step(std::integral_constant<int, I>{}), ...);
    }(std::make_integer_sequence<int, F::CW>{});

#pragma unroll
    for (int r = 0; r < R; r++) {
        float sf = 0.0f;
#pragma unroll
        for (int s = 0; s < F::NA; s++) {
            uint32_t lo = (uint32_t)acc[r][s][ND_LO - 1];
#pragma unroll
            for (int d = ND_LO - 2; d >= 0; d--) lo = (lo << 4) + (uint32_t)acc[r][s][d];
            uint32_t hi = (uint32_t)acc[r][s][ND - 1];
#pragma unroll
            for (int d = ND - 2; d >= ND_LO; d--) hi = (hi << 4) + (uint32_t)acc[r][s][d];
            const float v = fmaf((float)(int)hi, 4096.0f, (float)(int)lo);
            sf = s == 0 ? v : fmaf(0.25f, v, sf);
        }
        const float sc = qsf::f16_lo(wv[r][0]);
        rs[r] = fmaf(sc, sf * xm.x, rs[r]);                // sf * 2^-sh is exact
        if constexpr (FMT != QK_FMT_4SYM) {
            float z = qsf::f16_hi(wv[r][0]);
            if constexpr (FMT == QK_FMT_4) z = fmaf(8.0f, sc, z);
            rs[r] = fmaf(z, xm.y, rs[r]);
        }
    }
}

// Stage block digits + meta for blocks [c0, c1) in LDS: prepare them from x
// here, or copy the ones a stand-alone x-prep launch left in global memory.
template <int FMT, int BS>
__device__ __forceinline__ void stage_x(const GemvArgs& a, int c0, int c1, uint32_t* dig,
                                        float2* meta) {
    using F = Fmt<FMT, BS>;
    if (a.xq) {
        for (int i = threadIdx.x; i < (c1 - c0) * F::DWS; i += WAVES * 64)
            dig[i] = a.xq[(size_t)c0 * F::DWS + i];
        for (int i = threadIdx.x; i < c1 - c0; i += WAVES * 64) meta[i] = a.xmeta[c0 + i];
    } else {
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        for (int base = c0; base < c1; base += WAVES * 64 / F::LPB) {
            if (base + wave * (64 / F::LPB) >= c1) break;      // whole wave past the end
            const int b = base + threadIdx.x / F::LPB;
            const bool live = b < c1;
            const int bb = live ? b : c0;
            prep_block<FMT, BS>(a.x, a.cols, b, live, threadIdx.x & (F::LPB - 1),
                                dig + (bb - c0) * F::DWS, meta + (bb - c0));
        }
    }
}

// Tile t -> matrix m and first row of this lane's row group.
__device__ __forceinline__ void tile_of(const GemvArgs& a, int t, int rows_per_tile, int grp, int R,
                                        int& m, int& row0) {
    m = 0;
    while (m + 1 < a.n && t >= a.tile0[m + 1]) m++;
    row0 = (t - a.tile0[m]) * rows_per_tile + grp * R;
}

// Fused sparse pass (fp16 outliers of the tile's rows, src/quant.c:481-494),
// group reduction and store of one finished tile (chunked path).
template <int R>
__device__ __forceinline__ void flush_tile(const GemvArgs& a, int m, int row0, int lig, int lpg,
                                           float (&rs)[R]) {
    const int rows = a.rows[m];
    const uint32_t* rp = a.rp[m];
    if (rp) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
            if (row < rows) {
                const uint32_t e1 = rp[row + 1];
                for (uint32_t e = rp[row] + lig; e < e1; e += lpg) {
                    uint32_t col, val;
                    entry_at(a, m, e, col, val);
                    rs[r] = fmaf(qsf::f16_bits(val), a.x[col], rs[r]);
                }
            }
        }
    }
    float* __restrict__ y = a.y[m];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = group_reduce(rs[r], lpg);
        if (lig == lpg - 1 && row0 + r < rows) y[row0 + r] = v;
        rs[r] = 0.0f;
    }
}

// Main path: block digits, block meta and fp32 x of a whole row fit in LDS.
// A wave's work is the list of (tile, block) items, the same count for every
// lane; weights are loaded D items ahead into a ring of register sets.
//
// Vector-memory loads return in issue order and s_waitcnt counts them, and
// the compiler can only place tight waits across a straight-line load
// sequence: a load or store issued on some paths but not on others, between a
// load and its use, makes the wait for that load conservative (in practice,
// wait for everything in flight).  So every load up to the end of the item
// loop is issued unconditionally -- past a wave's last item at its last
// tile's row starts, for absent outlier tables at the group's own row -- and
// no global store happens before the end: finished rows park their sums in
// LDS.  The setup avoids chains of dependent scalar loads (kernel-argument
// arrays are read with static indices) and integer divisions, since every
// such step waits behind the weight stream once it is in flight.
// A wave64 memory instruction occupies the CU's address unit for about 16
// clocks whatever its width, and at the start every wave of the CU queues
// there: the prologue keeps the count of vector loads low (one CSR-bound load
// a lane, one first-entry load a tile).
// Issue order: outlier row pointers; in the prep waves the x of the first
// two passes; the first weight item; the prep waves' digit arithmetic and
// later passes; prepared digits and x; the first outlier entries of each
// tile; the barrier; the rest of the first D weight items; then the item loop
// (the first entries join the row sums before the one reduction a row), the
// remaining outlier entries and the stores.
template <int FMT, int BS, int R, int D, bool OUT, bool PREP, bool DREG, bool SPLIT = false,
          bool NORM = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs a) {
    constexpr int XV = kXvMax;
    constexpr int MT = tiles_per_wave(DREG);
    using F = Fmt<FMT, BS>;
    using WV = uint32_t[R][1 + F::CW];
    constexpr int NT = WAVES * 64;
    extern __shared__ __align__(16) uint32_t lds[];
    float2* meta = reinterpret_cast<float2*>(lds);            // nb x 8 B (+ pad to 16 B)
    uint32_t* dig = lds + ((2 * a.nb + 3) & ~3);              // nb x DWS dwords (+ pad to 4)
    float* xs = reinterpret_cast<float*>(lds + a.xs_off);     // nb*BS floats, zero past cols
    // wave index made provably uniform: tile -> matrix lookups then stay in
    // scalar registers (kernel arguments via s_load, no vector-memory waits)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lgl = a.lpg_log2, lpg = 1 << lgl;
    const int grp = lane >> lgl, lig = lane & (lpg - 1);
    const int rpt = R << (6 - lgl);                           // rows per tile
    // the workgroup's matrix: blockIdx.y (a workgroup never spans two)
    const GemvArgs::Mat& M = a.mat[blockIdx.y];
    const uint8_t* const W = M.w;
    float* const Y = M.y;
    const uint32_t* const RP = M.rp;                          // null: no outliers
    const uint32_t* const OE = M.oe;
    const int rows = M.rows;
    const uint32_t last = (uint32_t)max(M.nent - 1, 0);
    const int wgm = (int)blockIdx.x;                          // workgroup within the matrix
    const int mtiles = M.tiles;
    const int tw = wgm * a.tpw + wave;                        // this wave's first tile
    const int t_end = min(mtiles, wgm * a.tpw + a.tpw);
    const int nt = tw < t_end ? min(MT, (t_end - tw + WAVES - 1) / WAVES) : 0;
    const int ipt = (a.nb + lpg - 1) >> lgl;                  // items per tile
    const int ni = nt * ipt;
    const int tl = nt > 0 ? tw : 0;                           // tile the loads are anchored on
    const int ntl = nt > 0 ? nt : 1;
    const uint32_t row_bytes = SPLIT ? a.row_bytes : (uint32_t)a.nb * F::BB;

    // first row of the lane's group in tile j (clamped to the wave's last)
    auto row_of = [&](int j) __attribute__((always_inline)) {
        return (tl + WAVES * min(j, ntl - 1)) * rpt + grp * R;
    };
    // first dwords of the group's first row in tile j: what a load reads
    // where an outlier table is absent
    auto own_of = [&](int j) __attribute__((always_inline)) {
        return reinterpret_cast<const uint32_t*>(W + (size_t)min(row_of(j), rows - 1) * row_bytes);
    };

    // issue cursor: tile ij, step iq; row offsets of that tile, clamped to
    // the last row in bytes (the tile's first row times row_bytes is
    // wave-uniform, the group's row within the tile a per-lane constant: no
    // vector multiply a tile; the host keeps (rows + 128) * row_bytes within
    // 32 bits)
    int ij = 0, iq = 0;
    uint32_t ioff[R];
    uint32_t goff = (uint32_t)(grp * R) * row_bytes;
    asm volatile("" : "+v"(goff));   // opaque: else folded back into (row + grp R) * row_bytes
    const uint32_t olim = (uint32_t)max(rows - 1, 0) * row_bytes;
    auto at_tile = [&](int j) __attribute__((always_inline)) {
        const uint32_t base = (uint32_t)((tl + WAVES * min(j, ntl - 1)) * rpt) * row_bytes + goff;
#pragma unroll
        for (int r = 0; r < R; r++) ioff[r] = min(base + (uint32_t)r * row_bytes, olim);
    };
    at_tile(0);
    // The matrix record is materialised here, with the other arguments, in
    // one scalar round trip; left to the scheduler its loads sink behind the
    // x loads and cost a second round trip before the first weight load.
    asm volatile("" ::"s"(W), "s"(RP), "s"(OE), "s"(last), "s"(a.x), "s"(a.cols), "s"(a.xq));
    __builtin_amdgcn_sched_barrier(0);
    // next item's weights; past the last item, the last tile's row starts
    auto issue = [&](WV& wv) __attribute__((always_inline)) {
        const int b = ij < nt ? min(lig + (iq << lgl), a.nb - 1) : 0;
        load_block<FMT, BS, R, SPLIT>(W, ioff, b, wv, a.lsplit, a.nb);
        if (++iq == ipt) {
            iq = 0;
            ++ij;
            at_tile(min(ij, ntl - 1));
        }
    };

    // 1. CSR bounds of the wave's rows, one load a lane: lane lig < NBND of
    //    a row group loads bound lig of its group (tile lig / (R+1), row
    //    lig % (R+1)); the host sends row groups of fewer lanes to the chunked
    //    kernel.  Matrices without outliers read their own row.
    uint32_t rpl = 0;
    if constexpr (OUT) {
        const bool has = RP != nullptr;
        const int bj = min(lig / (R + 1), MT - 1), br = lig % (R + 1);
        const uint32_t* rp = has ? RP : own_of(bj);
        rpl = rp[has ? min(row_of(bj) + br, rows) : min(br, (int)F::BB / 4 - 1)];
    }

    // 1b. NORM: the residual add and the RMS norm of src/engine.c:1174-1187
    //    and 940-948 / 805-815 ahead of the matvec, as residual_norm_kernel
    //    computes them (same thread count, elements and order, so the same
    //    bits): every workgroup loads res_in, x and the norm weights, issues
    //    its first weight item behind them (3-bit: after the digits, as
    //    without the norm; issued here it held the norm's arithmetic back
    //    behind the CU's weight loads, 3.2 us more a 7B layer step),
    //    reduces, and leaves the normed x in LDS (xs), where the preparation
    //    reads it.  Workgroup (0, 0)
    //    stores the residual and the NaN check.  Only the passes that hold
    //    elements load (a wave-uniform guard; every such load comes before
    //    the weight item, so the waits stay exact); a pass's lanes past the
    //    end re-read their own first element.
    static_assert(!NORM || (!OUT && !PREP && WAVES * 64 == 1024), "NORM: one-launch, no outliers");
    const float* xsrc = a.x;
    uint32_t wv[D][R][1 + F::CW];
    if constexpr (NORM) {
        constexpr int KN = kNormPerThread;
        const int t_id = (int)threadIdx.x, n = a.cols;
        float nr[KN], nx[KN], nwv[KN];
#pragma unroll
        for (int k = 0; k < KN; k++) {
            nr[k] = nx[k] = nwv[k] = 0.f;
            if (k * NT < n) {
                const int i = t_id + k * NT < n ? t_id + k * NT : min(t_id, n - 1);
                nr[k] = a.res_in[i];
                nx[k] = a.x[i];
                nwv[k] = a.nw[i];
            }
        }
        if constexpr (FMT != QK_FMT_3) issue(wv[0]);
        float acc = 0.f;
        int first = n;
#pragma unroll
        for (int k = 0; k < KN; k++) {
            const int i = t_id + k * NT;
            const float r = qsf::add_rn(nr[k], nx[k]);
            nr[k] = r;
            if (i < n) {
                if ((r != r || r > 1e30f || r < -1e30f) && i < first) first = i;
                acc = fmaf(r, r, acc);
            }
        }
        float* red = reinterpret_cast<float*>(lds + a.st_off);
        const float ss = qsf::wg_sum(acc, red);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(qsf::add_rn(__fdiv_rn(ss, (float)n), a.eps)));
        if (blockIdx.x == 0 && blockIdx.y == 0) {
#pragma unroll
            for (int k = 0; k < KN; k++)
                if (t_id + k * NT < n) a.res_out[t_id + k * NT] = nr[k];
            if (a.bad) {
                for (int off = 32; off > 0; off >>= 1) first = min(first, __shfl_xor(first, off, 64));
                int* ired = reinterpret_cast<int*>(red);
                __syncthreads();                      // every wave past wg_sum's reads of red
                if (lane == 0) ired[wave] = first;
                __syncthreads();
                if (t_id == 0) {
                    int f = n;
                    for (int w = 0; w < WAVES; w++) f = min(f, ired[w]);
                    *a.bad = f < n ? f : -1;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < KN; k++)
            if (t_id + k * NT < n) xs[t_id + k * NT] = qsf::mul_rn(qsf::mul_rn(nr[k], inv), nwv[k]);
        __syncthreads();
        xsrc = xs;
    }

    // 2. Preparing here: the prep waves load the x of their first two passes
    //    of blocks, issue their first weight item, and then turn x into
    //    digits in LDS.  The x loads go ahead of every weight load of the
    //    wave (queued behind weights, x arrives late and holds the barrier),
    //    while the digit arithmetic overlaps the wave's own first item as
    //    well as the other waves' weight stream (measured: config 0 5.25 ->
    //    5.04 us, config 1 12.7 -> 12.45 us against digits before the first
    //    item).  Prepared digits: digits and meta, and for the
    //    outliers x, as whole float4s (the host guarantees cols >= 4) plus
    //    the cols % 4 tail (threads 0-2).  Loads past the end re-read the
    //    thread's own first element (never one address for the whole chip:
    //    that serialises on one L2 channel).
    constexpr int PASS = NT / F::LPB;                         // blocks per prep pass
    const int t_id = (int)threadIdx.x;
    const int pw = t_id & (F::LPB - 1), pb = t_id / F::LPB;
    const bool prep_wave = !PREP && wave * (64 / F::LPB) < a.nb;
    float* xcopy = OUT ? xs : nullptr;
    if constexpr (!PREP) {
        // 2/4-bit: the first two passes load their x together (the second
        // pass is the 7B down projection's: 172 4-bit blocks); 3-bit: one
        // pass covers 256 or more blocks, loaded ahead.  Passes past those,
        // for still wider rows, run one after another.
        constexpr int NX = F::NX;
        constexpr int AHEAD = FMT == QK_FMT_3 ? 1 : 2;
        const int pb1 = pb + PASS;
        const bool two = AHEAD == 2 && prep_wave && PASS + wave * (64 / F::LPB) < a.nb;
        float xv0[NX], xv1[AHEAD == 2 ? NX : 1];
        // 3-bit: the prep waves' digit arithmetic (the heaviest prep) comes
        // before their first weight item, whose issue can stall for a
        // microsecond behind the other waves' loads; the other waves issue
        // theirs at once.  2/4-bit: the first item goes first (measured:
        // config 0 5.25 -> 5.04 us, config 1 12.7 -> 12.45 us).
        constexpr bool kItemFirst = FMT != QK_FMT_3;
        if (prep_wave) prep_load<FMT, BS, true>(xsrc, a.cols, pb, pb < a.nb, pw, xv0);
        if constexpr (AHEAD == 2)
            if (two) prep_load<FMT, BS, true>(xsrc, a.cols, pb1, pb1 < a.nb, pw, xv1);
        if constexpr (kItemFirst && !NORM) issue(wv[0]);     // 3. the first weight item
        if (prep_wave) {
            const int b0 = pb < a.nb ? pb : 0;
            prep_settle<FMT, BS>(pb, pb < a.nb, pw, a.cols, xv0);
            prep_finish<FMT, BS>(xv0, pb, pb < a.nb, pw, dig + b0 * F::DWS, meta + b0, xcopy, a.cols);
        }
        if constexpr (!kItemFirst) issue(wv[0]);
        if constexpr (AHEAD == 2) {
            if (two) {
                const int b1 = pb1 < a.nb ? pb1 : 0;
                prep_settle<FMT, BS>(pb1, pb1 < a.nb, pw, a.cols, xv1);
                prep_finish<FMT, BS>(xv1, pb1, pb1 < a.nb, pw, dig + b1 * F::DWS, meta + b1, xcopy,
                                     a.cols);
            }
        }
        for (int base = AHEAD * PASS; base < a.nb; base += PASS) {
            if (base + wave * (64 / F::LPB) >= a.nb) break;     // whole wave past the end
            const int b = base + pb;
            const bool live = b < a.nb;
            const int bb = live ? b : 0;
            prep_block<FMT, BS>(xsrc, a.cols, b, live, pw, dig + bb * F::DWS, meta + bb, xcopy);
        }
    }
    constexpr bool XS = PREP && OUT;
    const int nf = a.cols >> 2;
    f32x4 xr[XV];
    float xt = 0.0f;
    if constexpr (XS) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const int f = t_id + i * NT;
            xr[i] = *reinterpret_cast<const f32x4_a4*>(a.x + 4 * (f < nf ? f : min(t_id, nf - 1)));
        }
        xt = a.x[t_id < 3 ? min(4 * nf + t_id, a.cols - 1) : min(t_id, a.cols - 1)];
    }
    const int nq = (a.nb * F::DWS + 3) >> 2;                  // dwordx4 of prepared digits
    u32x4 qr[DV];
    float2 mr;
    if constexpr (PREP) {
#pragma unroll
        for (int i = 0; i < DV; i++) {
            const int q = t_id + i * NT;
            qr[i] = reinterpret_cast<const u32x4*>(a.xq)[q < nq ? q : min(t_id, nq - 1)];
        }
        mr = a.xmeta[t_id < a.nb ? t_id : min(t_id & 63, a.nb - 1)];
    }

    // 3. the first weight item (issued in step 2 unless prepared).  The rest
    //    of the first D follow the barrier: once the memory system pushes
    //    back, each load waits at issue for earlier data to return, and a
    //    wave that queued all of its items before it would hold the barrier
    //    (and every wave's first item) until the stream had nearly drained.
    if constexpr (PREP) issue(wv[0]);

    // 4. LDS: prepared digits, meta and x as loaded.
    if constexpr (PREP) {
        if constexpr (XS) {
#pragma unroll
            for (int i = 0; i < XV; i++) {
                const int f = t_id + i * NT;
                if (f < nf) *reinterpret_cast<f32x4*>(xs + 4 * f) = xr[i];
            }
            if (t_id < a.cols - 4 * nf) xs[4 * nf + t_id] = xt;   // cols % 4 tail
        }
#pragma unroll
        for (int i = 0; i < DV; i++) {
            const int q = t_id + i * NT;
            if (q < nq) reinterpret_cast<u32x4*>(dig)[q] = qr[i];
        }
        if (t_id < a.nb) meta[t_id] = mr;
    }
    // 5. CSR bounds to every lane of the group (ds_bpermute), then the first
    //    outlier entries of each tile, one per lane: a tile's R rows own the
    //    contiguous entries [rpv[j][0], rpv[j][R]).  Issued before the
    //    barrier: the bounds (loaded first thing) are back by then, and the
    //    entries, first used at the wave's first tile end, queue ahead of the
    //    rest of its weights instead of behind them (config 1 12.64 ->
    //    11.98 us against issuing them after the barrier).
    //    Only what the item loop needs stays live: the entries, a mask of
    //    the row each lane's first entry belongs to (bit J*R + r), and
    //    whether any tile has entries past its first lpg.  The bounds
    //    themselves (R+1 registers a tile) held through the loop cost
    //    config 1 about 0.5 us; step 8 rebuilds them when it has work.
    uint32_t e0[MT];
    uint32_t omask = 0;
    bool orest = false;
    static_assert(MT * R <= 32, "one mask bit a tile row");
    if constexpr (OUT) {
        const int gl = lane & ~(lpg - 1);                     // group's first lane
        const bool pk = OE != nullptr;
        bool more = false;
#pragma unroll
        for (int j = 0; j < MT; j++) {
            uint32_t rb[R + 1];
#pragma unroll
            for (int r = 0; r <= R; r++) rb[r] = __shfl(rpl, gl + j * (R + 1) + r);
            const uint32_t* oe = pk ? OE : own_of(j);
            const uint32_t idx = rb[0] + lig;
            e0[j] = oe[pk ? min(idx, last) : 0u];
#pragma unroll
            for (int r = 0; r < R; r++)
                if (pk && idx >= rb[r] && idx < rb[r + 1]) omask |= 1u << (j * R + r);
            more |= j < nt && pk && idx + lpg < rb[R];
        }
        orest = __any(more);
    }

    __syncthreads();

    // (outlier kernels: only the items the wave has.  Measured with the
    // guard: config 1 10.83 -> 10.59 us, although its waves all have more
    // than D items, so the difference is in the generated code; in the
    // 3-bit kernels the same guard cost 0.9 us, so they issue all D.)
#pragma unroll
    for (int k = 1; k < D; k++)
        if (!OUT || k < ni) issue(wv[k]);

    // 6. Digits in registers: with one block a lane (nb <= lpg) the lane's
    //    block is the same in every item, so its digit words and meta are read
    //    from LDS once (idle lanes past nb read block nb - 1).
    constexpr int NDG = DREG ? F::CW * F::NC * ND : 1;
    uint32_t dreg[NDG];
    float2 mreg = make_float2(0.0f, 0.0f);
    if constexpr (DREG) {
        const uint32_t* dp = dig + min(lig, a.nb - 1) * F::DWS;
#pragma unroll
        for (int i = 0; i < NDG; i++) dreg[i] = dp[i];
        mreg = meta[min(lig, a.nb - 1)];
    }

    // 7. item loop.  At a tile's end the first outlier entry of each row joins
    //    the lane sums (src/quant.c:481-494, value * x[col]), the row is
    //    reduced once and its sum parked in the stash.
    float* stash = reinterpret_cast<float*>(lds + a.st_off) + wave * a.st_wave;
    float rs[R];
#pragma unroll
    for (int r = 0; r < R; r++) rs[r] = 0.0f;
    int cj = 0, cq = 0;                                       // compute cursor
    // first outlier entries of the tile ending now.  Tiles end in order, so
    // its entry and mask bits are always at the front: consumed there, then
    // the rest shift down (a few moves, where a per-tile selection over a
    // runtime tile index cost a chain of branches: config 1 11.25 -> 10.74
    // us).  The lane's entry belongs to row r when mask bit r is set.
    auto first_entries = [&]() __attribute__((always_inline)) {
        const uint32_t e = e0[0], mb = omask & ((1u << R) - 1);
        const float p = qsf::f16_bits(e >> 16) * xs[mb ? e & 0xFFFFu : 0u];
#pragma unroll
        for (int r = 0; r < R; r++) rs[r] += (mb >> r) & 1u ? p : 0.0f;
#pragma unroll
        for (int j = 0; j + 1 < MT; j++) e0[j] = e0[j + 1];
        omask >>= R;
    };
    auto tile_end = [&]() __attribute__((always_inline)) {
        if constexpr (OUT) first_entries();
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = group_reduce(rs[r], lpg);
            rs[r] = 0.0f;
            if (lig == lpg - 1) stash[cj * rpt + grp * R + r] = v;
        }
    };
    auto compute = [&](const WV& w) __attribute__((always_inline)) {
        const int b = lig + (cq << lgl);
        if constexpr (DREG) {
            if (b < a.nb) compute_block<FMT, BS, R>(w, dreg, mreg, rs);
        } else {
            if (b < a.nb) compute_block<FMT, BS, R>(w, dig + b * F::DWS, meta[b], rs);
        }
        if (++cq == ipt) {
            tile_end();
            cq = 0;
            ++cj;
        }
    };
    // Blocks of D items.  Every block but the last refills each slot as it
    // frees it (items past the end: issue()'s broadcast loads, back long
    // before the end); the last block issues nothing, since a wave cannot
    // retire before its loads return.
    const int nblk = (ni + D - 1) / D;
    if constexpr (DREG) {
        // One block a lane (nb <= lpg): every item is a whole tile, and the
        // lane's block, hence its byte offset in a row, is the same in every
        // item.  Item k of a block of D items reads its tile's first outlier
        // entries from e0[k] and mask bits k*R..; the block then shifts them
        // down by D (a shift each item cost MT - 1 moves an item: config 1
        // 9.45-9.82 -> 9.26-9.32 us with this loop and the multiply-free row
        // offsets, on one box; runs of 2 D items with one shift were slower,
        // 10.0-10.2 us).
        const bool live = lig < a.nb;
        const int bl = min(lig, a.nb - 1);
        auto issue_d = [&](WV& wv) __attribute__((always_inline)) {
            load_block<FMT, BS, R, SPLIT>(W, ioff, bl, wv, a.lsplit, a.nb);
            ++ij;
            at_tile(min(ij, ntl - 1));
        };
        // Two or more tiles, one row each, in 64-lane groups: an item leaves
        // its lane partial in LDS (slot cj of the wave's [MT][64]), and the
        // rows are reduced together after the loop, with the pairings of
        // group_reduce (same bits), instead of a DPP reduction an item.
        // Outlier kernels only: config 1 (5-6 tiles a wave) 8.96-9.56 ->
        // 8.84-8.94 us; in the plain kernels the added code alone took
        // config 0 (one tile a wave, never this path) from 3.91-4.00 to
        // 4.01-4.09 us.
        float* const prs = reinterpret_cast<float*>(lds + a.pr_off) + wave * (MT * 64);
        const bool multi = OUT && R == 1 && a.pr_off > 0 && ni >= 2;
        auto item = [&](const WV& w, int k) __attribute__((always_inline)) {
            if (live) compute_block<FMT, BS, R>(w, dreg, mreg, rs);
            if constexpr (OUT) {
                const uint32_t e = e0[k], mb = (omask >> (k * R)) & ((1u << R) - 1);
                const float p = qsf::f16_bits(e >> 16) * xs[mb ? e & 0xFFFFu : 0u];
#pragma unroll
                for (int r = 0; r < R; r++) rs[r] += (mb >> r) & 1u ? p : 0.0f;
            }
            if (OUT && multi) {
                prs[cj * 64 + lane] = rs[0];
                rs[0] = 0.0f;
            } else {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const float v = group_reduce(rs[r], lpg);
                    rs[r] = 0.0f;
                    if (lig == lpg - 1) stash[cj * rpt + grp * R + r] = v;
                }
            }
            ++cj;
        };
        for (int q = 0; q + 1 < nblk; q++) {
#pragma unroll
            for (int k = 0; k < D; k++) {
                item(wv[k], k);
                issue_d(wv[k]);
            }
            if constexpr (OUT) {
#pragma unroll
                for (int j = 0; j + D < MT; j++) e0[j] = e0[j + D];
                omask >>= D * R;
            }
        }
        if (nblk > 0) {
#pragma unroll
            for (int k = 0; k < D; k++)
                if ((nblk - 1) * D + k < ni) item(wv[k], k);
        }
        if (OUT && multi) {
            // lane 8 s + p: slot s's lanes 8 p .. 8 p + 7, paired as
            // group_sum_last pairs lanes (l^1, l^2, the two quads), then
            // the eight partial sums across p (its 8-lane groups, 16-lane
            // rows 0+1 and 2+3, and the two pairs); slots past the wave's
            // tiles hold stale values and are not stored
            const int sl = lane >> 3, pp = lane & 7;
            const f32x4 v0 = *reinterpret_cast<const f32x4*>(prs + sl * 64 + 8 * pp);
            const f32x4 v1 = *reinterpret_cast<const f32x4*>(prs + sl * 64 + 8 * pp + 4);
            float tsum = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
            tsum += dpp_f<0xB1, 0xF>(tsum);                 // quad_perm [1,0,3,2]
            tsum += dpp_f<0x4E, 0xF>(tsum);                 // quad_perm [2,3,0,1]
            tsum += dpp_f<0x141, 0xF>(tsum);                // row_half_mirror
            if (pp == 0 && sl < nt) stash[sl] = tsum;
        }
    } else {
        for (int q = 0; q + 1 < nblk; q++) {
#pragma unroll
            for (int k = 0; k < D; k++) {
                compute(wv[k]);
                issue(wv[k]);
            }
        }
        if (nblk > 0) {
#pragma unroll
            for (int k = 0; k < D; k++)
                if ((nblk - 1) * D + k < ni) compute(wv[k]);
        }
    }

    // 8. remaining outlier entries of each tile, one per lane each step;
    //    every slot loads (clamped index, own row where absent)
    if constexpr (OUT) if (orest) {
        uint32_t rpv[MT][R + 1];
        const int gl = lane & ~(lpg - 1);
#pragma unroll
        for (int j = 0; j < MT; j++)
#pragma unroll
            for (int r = 0; r <= R; r++) rpv[j][r] = __shfl(rpl, gl + j * (R + 1) + r);
        float orem[MT][R];
#pragma unroll
        for (int j = 0; j < MT; j++)
#pragma unroll
            for (int r = 0; r < R; r++) orem[j][r] = 0.0f;
        bool any_rem = false;
        for (uint32_t k = 1;; k++) {
            bool ok[MT];
            bool more = false;
#pragma unroll
            for (int j = 0; j < MT; j++) {
                ok[j] = j < nt && OE != nullptr && rpv[j][0] + lig + (k << lgl) < rpv[j][R];
                more |= ok[j];
            }
            if (!__any(more)) break;
            any_rem = true;
            uint32_t eu[MT];
            const bool pk = OE != nullptr;
#pragma unroll
            for (int j = 0; j < MT; j++) {
                const uint32_t* oe = pk ? OE : own_of(j);
                eu[j] = oe[pk ? min(rpv[j][0] + lig + (k << lgl), last) : 0u];
            }
#pragma unroll
            for (int j = 0; j < MT; j++) {
                const uint32_t idx = rpv[j][0] + lig + (k << lgl);
                const uint32_t col = ok[j] ? eu[j] & 0xFFFFu : 0u;
                const float p = qsf::f16_bits(eu[j] >> 16) * xs[col];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const bool mine = ok[j] && idx >= rpv[j][r] && idx < rpv[j][r + 1];
                    orem[j][r] += mine ? p : 0.0f;
                }
            }
        }
        if (any_rem) {
#pragma unroll
            for (int j = 0; j < MT; j++)
                if (j < nt) {
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const float v = group_reduce(orem[j][r], lpg);
                        if (lig == lpg - 1) stash[j * rpt + grp * R + r] += v;
                    }
                }
        }
    }

    // 9. stores (paired rows: the gate/up activation product,
    //    src/engine.c:1128-1140, as the act-mul kernel computes it)
    if constexpr (R == 2) {
        if (a.act1) {
#pragma unroll
            for (int j = 0; j < MT; j++) {
                const int row0 = row_of(j);
                if (j < nt && lig == lpg - 1 && row0 < rows)
                    Y[row0 >> 1] = qsf::act_mul(a.act1 - 1, stash[j * rpt + grp * R], stash[j * rpt + grp * R + 1]);
            }
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < MT; j++) {
        if (j < nt) {
            const int row0 = row_of(j);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = row0 + r;
                if (lig == lpg - 1 && row < rows) Y[row] = stash[j * rpt + grp * R + r];
            }
        }
    }
}

// Fallback when the digits of a row do not fit in LDS: K in chunks, at most
// MAXT tiles a wave kept in registers across chunks, no prefetch.
template <int FMT, int BS, int R, bool SPLIT = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_chunked_kernel(GemvArgs a) {
    using F = Fmt<FMT, BS>;
    extern __shared__ __align__(16) uint32_t lds[];
    float2* meta = reinterpret_cast<float2*>(lds);
    uint32_t* dig = lds + 2 * a.chunk;
    // wave index made provably uniform: tile -> matrix lookups then stay in
    // scalar registers (kernel arguments via s_load, no vector-memory waits)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lpg = a.lpg, grp = lane / lpg, lig = lane & (lpg - 1);
    const int rows_per_tile = R * (64 / lpg);
    const int t_begin = blockIdx.x * a.tpw;
    const int t_end = min(a.tile0[a.n], t_begin + a.tpw);
    const uint32_t row_bytes = SPLIT ? a.row_bytes : (uint32_t)a.nb * F::BB;

    float rs[MAXT][R];
#pragma unroll
    for (int j = 0; j < MAXT; j++)
#pragma unroll
        for (int r = 0; r < R; r++) rs[j][r] = 0.0f;

    for (int c0 = 0; c0 < a.nb; c0 += a.chunk) {
        const int c1 = min(a.nb, c0 + a.chunk);
        __syncthreads();
        stage_x<FMT, BS>(a, c0, c1, dig, meta);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MAXT; j++) {
            const int t = t_begin + wave + WAVES * j;
            if (t >= t_end) break;
            int m, row0;
            tile_of(a, t, rows_per_tile, grp, R, m, row0);
            if (row0 >= a.rows[m]) continue;
            uint32_t roff[R];
#pragma unroll
            for (int r = 0; r < R; r++) roff[r] = (uint32_t)min(row0 + r, a.rows[m] - 1) * row_bytes;
            for (int b = c0 + lig; b < c1; b += lpg) {
                uint32_t wv[R][1 + F::CW];
                load_block<FMT, BS, R, SPLIT>(a.w[m], roff, b, wv, a.lsplit, a.nb);
                compute_block<FMT, BS, R>(wv, dig + (b - c0) * F::DWS, meta[b - c0], rs[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < MAXT; j++) {
        const int t = t_begin + wave + WAVES * j;
        if (t >= t_end) break;
        int m, row0;
        tile_of(a, t, rows_per_tile, grp, R, m, row0);
        flush_tile<R>(a, m, row0, lig, lpg, rs[j]);
    }
}

__global__ void fill_kernel(float* y, int n, float v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = v;
}

// n floats from `src` (host memory mapped into the device address space) to
// device memory: the table slots' x in one dispatch on their own queue, no
// copy engine.  Whole float4s where the tail allows, then single floats.
__global__ __launch_bounds__(256) void stage_kernel(float* __restrict__ dst,
                                                     const float* __restrict__ src, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int n4 = n >> 2;
    if (i < n4) {
        reinterpret_cast<float4*>(dst)[i] = reinterpret_cast<const float4*>(src)[i];
    } else if (4 * n4 + (i - n4) < n) {
        dst[4 * n4 + (i - n4)] = src[4 * n4 + (i - n4)];
    }
}

int num_cus() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    }
    return n;
}

template <int FMT, int BS>
size_t xprep_bytes_t(int cols) {
    using F = Fmt<FMT, BS>;
    size_t nb = (size_t)((cols + BS - 1) / BS);
    size_t dig = nb * F::DWS * 4;
    return ((dig + 255) & ~(size_t)255) + nb * sizeof(float2);
}

// Dynamic LDS a GEMV workgroup may use in total (digits, meta, staged x, stash).
size_t lds_limit() {
    static size_t v = 0;
    if (!v) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
            n > 0)
            v = (size_t)n;
        else
            v = 64 * 1024;
        v = v < kLdsLimit ? v : kLdsLimit;
    }
    return v;
}

// Launch a main-path instantiation, allowing it the device's full LDS once.
// Kernel timing (diagnostics): while on, timed launches (main-path GEMV,
// prefill) record an event pair at the kernel's own start and end
// (hipExtLaunchKernel), so the durations exclude launch gaps.  Not for use
// under graph capture.
struct KernelTiming {
    static constexpr int N = 4096;
    bool on = false;
    int used = 0;
    hipEvent_t ev[N][2] = {};
};
KernelTiming g_timing;

}  // namespace

extern "C" int qk_timing_pair(hipEvent_t* start, hipEvent_t* stop) {
    if (!g_timing.on || g_timing.used >= KernelTiming::N) return 0;
    hipEvent_t* p = g_timing.ev[g_timing.used];
    if (!p[0] && (hipEventCreate(&p[0]) != hipSuccess || hipEventCreate(&p[1]) != hipSuccess))
        return 0;
    g_timing.used++;
    *start = p[0];
    *stop = p[1];
    return 1;
}

namespace {

template <auto K>
void launch_main(dim3 g, dim3 b, size_t lds, hipStream_t s, const GemvArgs& a) {
    static bool allowed = false;
    if (!allowed) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(K),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_limit());
        allowed = true;
    }
    hipEvent_t e0, e1;
    if (qk_timing_pair(&e0, &e1))
        hipExtLaunchKernelGGL(K, g, b, (uint32_t)lds, s, e0, e1, 0, a);
    else
        hipLaunchKernelGGL(K, g, b, lds, s, a);
}

// rows per tile: up to 2 for 64-code-or-smaller blocks, else 1 (register
// budget); prefetch depth: about 48 registers of weights in flight per lane
template <int FMT, int BS>
constexpr int tile_rows() { return Fmt<FMT, BS>::CW <= 8 ? 2 : 1; }
// (one item for 3-bit 256-code blocks: 25 dwords a row plus two accumulator
// sets leave no room for a second set within 128 VGPRs)
// (outlier kernels keep ~20 more registers of CSR state, and their waves
// have few items: 24, so that a wave computes its first item after issuing
// the second rather than after issuing all of them)
template <int FMT, int BS, int R, bool OUT>
constexpr int prefetch_depth() {
    constexpr int per = R * (1 + Fmt<FMT, BS>::CW);
    constexpr int budget = OUT ? 24 : 48;
    if (FMT == QK_FMT_3 && Fmt<FMT, BS>::CW >= 24) return 1;
    if (OUT && per > 24) return 1;
    return budget / per < 2 ? 2 : (budget / per > 4 ? 4 : budget / per);
}

// The launch plan of a GEMV over n tensors sharing x: kernel arguments, grid,
// LDS and the kernel instantiation (kid).  A row's arithmetic (the order of
// its fp32 adds) follows from R, DREG, the row-group width lpg, the chunk
// and kid alone; qk_gemv_signature packs those.  Returns 1 when there is
// nothing to launch, a negative code when the group is not supported.
struct Plan {
    int kid;        // 0 chunked; 1-4 split view; 5-10 whole-row (launch_rt)
    int grid, ny;
    size_t lds;
};

template <int FMT, int BS, int R, bool DREG = false, bool SPLIT = false>
int plan_rt(const qsf_hip_tensor* const* t, int n, int cols, int mode, float* const* d_y,
            GemvArgs& a, Plan& p) {
    constexpr int MT = tiles_per_wave(DREG);
    using F = Fmt<FMT, BS>;
    const int nb = (cols + BS - 1) / BS;
    a = GemvArgs{};
    a.n = n;
    a.row_bytes = (uint32_t)((size_t)t[0]->nb * t[0]->block_bytes);
    a.lsplit = 0;
    while ((BS << a.lsplit) < t[0]->bs) a.lsplit++;
    a.cols = cols;
    a.nb = nb;
    int lpg = 1, lgl = 0;
    while (lpg < nb && lpg < 64) {
        lpg <<= 1;
        lgl++;
    }
    // Wider row groups (the lanes past a row's blocks idle) while the
    // matrices have fewer tiles than the chip has waves: a 4096-row matrix
    // of 32 blocks in 32-lane groups would fill half of it.
    for (;;) {
        long tl = 0;
        const long rpt = (long)R * (64 / lpg);
        for (int i = 0; i < n; i++) tl += (t[i]->rows + rpt - 1) / rpt;
        if (lpg >= 64 || tl >= (long)num_cus() * WAVES) break;
        lpg <<= 1;
        lgl++;
    }
    a.lpg = lpg;
    a.lpg_log2 = lgl;
    const int per_block = F::DWS * 4 + (int)sizeof(float2);
    a.chunk = nb < kLdsBudget / per_block ? nb : kLdsBudget / per_block;
    const int rows_per_tile = R * (64 / lpg);
    bool any_out = false, split = false;
    a.tile0[0] = 0;
    for (int i = 0; i < n; i++) {
        if ((size_t)(t[i]->rows + 128) * nb * F::BB > 0xFFFFFFF0ull) return -2;   // 32-bit offsets
        float* y = d_y ? d_y[i] : nullptr;
        a.w[i] = t[i]->d_blocks;
        a.y[i] = y;
        a.rp[i] = t[i]->d_row_ptr;
        a.oe[i] = t[i]->d_oent;
        a.oc[i] = t[i]->d_ocol;
        a.ov[i] = t[i]->d_oval;
        a.nent[i] = (int)t[i]->n_csr;
        a.rows[i] = t[i]->rows;
        a.mat[i] = {t[i]->d_blocks, y, t[i]->d_row_ptr, t[i]->d_oent, t[i]->rows,
                    (int)t[i]->n_csr, (t[i]->rows + rows_per_tile - 1) / rows_per_tile, 0};
        a.tile0[i + 1] = a.tile0[i] + a.mat[i].tiles;
        any_out |= t[i]->d_row_ptr != nullptr;
        split |= t[i]->d_row_ptr != nullptr && t[i]->d_oent == nullptr;
    }
    const int tiles = a.tile0[n];
    // one workgroup per CU (fewer for small problems); at most MAXT tiles a
    // wave here (the chunked kernel's bound; the main kernel may take up to
    // MT below, to fit its grid in one round)
    int grid = (tiles + WAVES - 1) / WAVES;
    grid = grid < num_cus() ? grid : num_cus();
    if (grid > 0 && (tiles + grid - 1) / grid > WAVES * MAXT)
        grid = (tiles + WAVES * MAXT - 1) / (WAVES * MAXT);
    a.tpw = grid > 0 ? (tiles + grid - 1) / grid : 0;
    const bool prepared = !(mode & QK_RUN_XPREP) || (mode & QK_RUN_STANDALONE_PREP);

    // Main kernel LDS: [meta: nb x 16 B][digits: nb x DWS dwords, padded to
    // 4][x: nb*BS floats][fp32 stash: a wave's tiles x rows_per_tile].  When
    // the stash would not fit, fewer tiles a workgroup.
    const size_t dig_dw = ((size_t)nb * F::DWS + 3) & ~(size_t)3;
    const size_t meta_dw = ((size_t)nb * 2 + 3) & ~(size_t)3;
    const size_t main_fixed = meta_dw * 4 + dig_dw * 4 + (size_t)nb * BS * 4;
    const size_t per_tile = (size_t)WAVES * rows_per_tile * sizeof(float);
    // (the main kernel reads packed outlier tables only)
    // (the main kernel's outlier pass gathers a row group's CSR bounds from
    // one load a lane: groups need MT * (R + 1) lanes)
    const bool whole = !split && (!any_out || lpg >= MT * (R + 1)) && cols >= 4 && cols <= 4 * kXvMax * WAVES * 64 && nb <= kMainMaxNb &&
                       (!prepared || dig_dw <= (size_t)4 * DV * WAVES * 64) &&
                       main_fixed + per_tile <= lds_limit();
    size_t lds = (size_t)a.chunk * per_block;                 // chunked kernel
    int most = 1 << 30;                                       // items a wave at most
    a.xs_off = 0;
    a.st_off = 0;
    a.st_wave = 0;
    if (tiles == 0) {
        p = {0, 0, 0, 0};
        return 1;
    }
    if (whole) {
        const size_t room = (lds_limit() - main_fixed) / per_tile;
        if ((size_t)a.tpw > WAVES * room) a.tpw = (int)(WAVES * room);
        // main kernel: workgroups (x, matrix y); a matrix with fewer tiles
        // than the largest leaves its last workgroups without tiles
        auto grid_of = [&](int tpw) {
            int g = 0;
            for (int i = 0; i < n; i++) {
                const int gi = (a.mat[i].tiles + tpw - 1) / tpw;
                g = gi > g ? gi : g;
            }
            return g;
        };
        // all workgroups in one round: a few past the CU count would run
        // after the rest and double the time
        const int tpw_max = WAVES * (int)(room < (size_t)MT ? room : (size_t)MT);
        while (grid_of(a.tpw) * n > num_cus() && a.tpw < tpw_max) a.tpw++;
        grid = grid_of(a.tpw);
        const int ntc = (a.tpw + WAVES - 1) / WAVES;
        most = ntc * ((nb + lpg - 1) / lpg);
        a.xs_off = (int)(meta_dw + dig_dw);
        a.st_off = a.xs_off + nb * BS;
        a.st_wave = ntc * rows_per_tile;
        lds = main_fixed + (size_t)ntc * per_tile;
        // one block a lane in 64-lane groups, two or more tiles a wave, the
        // outlier kernels: room for every wave's lane partials, one row a
        // slot, reduced once at the wave's end
        a.pr_off = 0;
        if (DREG && R == 1 && lpg == 64 && ntc >= 2 && any_out) {
            const size_t at = (lds + 15) & ~(size_t)15;
            const size_t pr = (size_t)WAVES * MT * 64 * sizeof(float);
            if (at + pr <= lds_limit()) {
                a.pr_off = (int)(at / 4);
                lds = at + pr;
            }
        }
    } else {
        grid = (tiles + a.tpw - 1) / a.tpw;
    }
    // only the 2-bit and 4-bit asymmetric formats have outlier variants
    constexpr bool kHasOut = FMT == QK_FMT_2 || FMT == QK_FMT_4;
    constexpr int D = DREG ? 2 : prefetch_depth<FMT, BS, R, false>();
    if (any_out && !kHasOut) return -2;
    int kid;
    if (!whole) kid = 0;
    else if (SPLIT && prepared) kid = any_out ? 11 : 12;
    else if (SPLIT) kid = any_out ? 1 : most <= 1 ? 2 : (D > 2 && most <= 2) ? 3 : 4;
    else if (prepared && any_out) kid = 5;
    else if (prepared) kid = 6;
    else if (any_out) kid = 7;
    else if (most <= 1) kid = 8;
    else if (D > 2 && most <= 2) kid = 9;
    else kid = 10;
    p = {kid, grid, whole ? n : 1, lds};
    return 0;
}

// Paired-rows request of the calling thread for the launch being planned
// (qk_gemv_pair_act sets it around its one call): 1 + activation, or 0.
thread_local int tl_pair_act1 = 0;
// set by qk_gemv_group_norm / qk_gemv_pair_act_norm for the call's launches
thread_local const qk_norm_args* tl_norm = nullptr;

template <int FMT, int BS, int R, bool DREG = false, bool SPLIT = false>
int launch_rt(const qsf_hip_tensor* const* t, int n, int cols, const float* d_x,
              float* const* d_y, void* d_ws, int mode, hipStream_t s) {
    // SPLIT: the stored blocks are t[0]->bs codes, read as parts of BS, x
    // prepared here or (QK_RUN_GEMV) by qk_xprep, per part either way
    if (SPLIT && ((mode != QK_RUN_BOTH && mode != QK_RUN_GEMV) || t[0]->bs <= BS)) return -2;
    using F = Fmt<FMT, BS>;
    const int nb = (cols + BS - 1) / BS;
    // prepared digits and block meta (QK_RUN_XPREP / a prepared run only)
    uint32_t* xq = (uint32_t*)d_ws;
    float2* xmeta = d_ws ? xmeta_in<FMT, BS>(d_ws, nb) : nullptr;
    if (!d_ws && (mode != QK_RUN_BOTH)) return -2;
    if ((mode & QK_RUN_XPREP) && (!(mode & QK_RUN_GEMV) || (mode & QK_RUN_STANDALONE_PREP)))
        hipLaunchKernelGGL((xprep_kernel<FMT, BS>), dim3((nb + 256 / F::LPB - 1) / (256 / F::LPB)),
                           dim3(256), 0, s, d_x, cols, nb, xq, xmeta, (float*)nullptr);
    if (!(mode & QK_RUN_GEMV)) return hipGetLastError() == hipSuccess ? 0 : -1;

    GemvArgs a;
    Plan p;
    const int rc = plan_rt<FMT, BS, R, DREG, SPLIT>(t, n, cols, mode, d_y, a, p);
    if (rc) return rc < 0 ? rc : 0;
    // paired rows: the whole-row kernel with two-row tiles only (a tile's
    // two rows, a gate row and its up row, end in the same lane's stash)
    a.act1 = tl_pair_act1;
    if (a.act1 && (R != 2 || DREG || p.kid == 0 || n != 1 || t[0]->d_row_ptr)) return -2;
    const bool prepared = !(mode & QK_RUN_XPREP) || (mode & QK_RUN_STANDALONE_PREP);
    a.xq = prepared ? xq : nullptr;
    a.xmeta = xmeta;
    a.x = d_x;
    // fused residual + norm: the one-launch whole-row kernel without
    // outliers; any other plan is refused (never run without the norm)
    const qk_norm_args* const nm = tl_norm;
    a.res_in = nm ? nm->res_in : nullptr;
    a.res_out = nm ? nm->res_out : nullptr;
    a.nw = nm ? nm->w : nullptr;
    a.bad = nm ? nm->bad : nullptr;
    a.eps = nm ? nm->eps : 0.f;
    if (nm && (prepared || !(p.kid == 2 || p.kid == 3 || p.kid == 4 || p.kid >= 8) ||
               cols > kNormPerThread * WAVES * 64))
        return -2;

    constexpr bool kHasOut = FMT == QK_FMT_2 || FMT == QK_FMT_4;
    // one item a wave at most (a 4096-row matrix of up to 64 blocks): one
    // item in flight.  A second would only re-read a row for nothing, and
    // its wave could not retire before that load returned (4096x4096 4-bit
    // 5.05 -> 4.70 us, 3-bit 6.85 -> 6.44 us).  Likewise at most two items
    // keep two in flight (3-bit q/k/v 9.3 -> 9.0 us, down 12.86 -> 12.72).
    // digits in registers: small items, two in flight, so that a wave
    // alternates issue and compute
    constexpr int D = DREG ? 2 : prefetch_depth<FMT, BS, R, false>();
    constexpr int DO = DREG ? 2 : prefetch_depth<FMT, BS, R, kHasOut>();
    const dim3 g(p.grid, p.ny), b(WAVES * 64);
    if (nm) {
        if constexpr (SPLIT) {
            switch (p.kid) {
            case 2: launch_main<gemv_kernel<FMT, BS, R, 1, false, false, DREG, true, true>>(g, b, p.lds, s, a); break;
            case 3: launch_main<gemv_kernel<FMT, BS, R, (D > 2 ? 2 : D), false, false, DREG, true, true>>(g, b, p.lds, s, a); break;
            default: launch_main<gemv_kernel<FMT, BS, R, D, false, false, DREG, true, true>>(g, b, p.lds, s, a); break;
            }
        } else {
            switch (p.kid) {
            case 8: launch_main<gemv_kernel<FMT, BS, R, 1, false, false, DREG, false, true>>(g, b, p.lds, s, a); break;
            case 9: launch_main<gemv_kernel<FMT, BS, R, (D > 2 ? 2 : D), false, false, DREG, false, true>>(g, b, p.lds, s, a); break;
            default: launch_main<gemv_kernel<FMT, BS, R, D, false, false, DREG, false, true>>(g, b, p.lds, s, a); break;
            }
        }
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if constexpr (SPLIT) {
        // x prepared in the workgroups (1-4) or read as qk_xprep's digits of
        // the parts (11, 12); the chunked kernel prepares its own
        switch (p.kid) {
        case 0: hipLaunchKernelGGL((gemv_chunked_kernel<FMT, BS, R, true>), g, b, p.lds, s, a); break;
        case 11: launch_main<gemv_kernel<FMT, BS, R, DO, kHasOut, true, DREG, true>>(g, b, p.lds, s, a); break;
        case 12: launch_main<gemv_kernel<FMT, BS, R, D, false, true, DREG, true>>(g, b, p.lds, s, a); break;
        case 1: launch_main<gemv_kernel<FMT, BS, R, DO, kHasOut, false, DREG, true>>(g, b, p.lds, s, a); break;
        case 2: launch_main<gemv_kernel<FMT, BS, R, 1, false, false, DREG, true>>(g, b, p.lds, s, a); break;
        case 3: launch_main<gemv_kernel<FMT, BS, R, (D > 2 ? 2 : D), false, false, DREG, true>>(g, b, p.lds, s, a); break;
        default: launch_main<gemv_kernel<FMT, BS, R, D, false, false, DREG, true>>(g, b, p.lds, s, a); break;
        }
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    switch (p.kid) {
    case 0: hipLaunchKernelGGL((gemv_chunked_kernel<FMT, BS, R>), g, b, p.lds, s, a); break;
    case 5: launch_main<gemv_kernel<FMT, BS, R, DO, kHasOut, true, DREG>>(g, b, p.lds, s, a); break;
    case 6: launch_main<gemv_kernel<FMT, BS, R, D, false, true, DREG>>(g, b, p.lds, s, a); break;
    case 7: launch_main<gemv_kernel<FMT, BS, R, DO, kHasOut, false, DREG>>(g, b, p.lds, s, a); break;
    case 8: launch_main<gemv_kernel<FMT, BS, R, 1, false, false, DREG>>(g, b, p.lds, s, a); break;
    case 9: launch_main<gemv_kernel<FMT, BS, R, (D > 2 ? 2 : D), false, false, DREG>>(g, b, p.lds, s, a); break;
    default: launch_main<gemv_kernel<FMT, BS, R, D, false, false, DREG>>(g, b, p.lds, s, a); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int FMT, int BS, int R, bool DREG, bool SPLIT>
uint64_t sig_rt(const qsf_hip_tensor* const* t, int n, int cols, int mode) {
    GemvArgs a;
    Plan p;
    if (SPLIT && ((mode != QK_RUN_BOTH && mode != QK_RUN_GEMV) || t[0]->bs <= BS)) return 0;
    if (plan_rt<FMT, BS, R, DREG, SPLIT>(t, n, cols, mode, nullptr, a, p) < 0) return 0;
    return 1ull | (uint64_t)R << 1 | (uint64_t)DREG << 3 | (uint64_t)SPLIT << 4 |
           (uint64_t)(mode & 7) << 5 | (uint64_t)a.lpg << 8 | (uint64_t)p.kid << 16 |
           (uint64_t)a.chunk << 24 | (uint64_t)BS << 48;
}

// Tiles: 0 = one-row tiles with the digits in registers (a row is one block
// a lane and the lane's digit words fit in 48 registers: 2- and 4-bit blocks
// of <= 64 codes; not the 4-bit 64-code outlier kernel, whose CSR state on
// top spills), 1 = one-row tiles, 2 = two-row tiles.  Two-row tiles halve
// the digit reads a row, one-row tiles double the parallelism: one row when
// two-row tiles would leave waves of the chip without a tile (a 4096-row
// matrix fills half of it).
template <int FMT, int BS>
int pick_tiles(const qsf_hip_tensor* const* t, int n, int cols) {
    constexpr bool kDreg = FMT != QK_FMT_3 && Fmt<FMT, BS>::CW * Fmt<FMT, BS>::NC * ND <= 48;
    if constexpr (kDreg) {
        bool out = false;
        for (int i = 0; i < n; i++) out |= t[i]->d_row_ptr != nullptr;
        if ((cols + BS - 1) / BS <= 64 && !(out && FMT == QK_FMT_4 && BS == 64)) return 0;
    }
    if constexpr (tile_rows<FMT, BS>() == 1) {
        return 1;
    } else {
        const int nb = (cols + BS - 1) / BS;
        int lpg = 1;
        while (lpg < nb && lpg < 64) lpg <<= 1;
        const long rpt2 = 2L * (64 / lpg);
        long tiles2 = 0;
        for (int i = 0; i < n; i++) tiles2 += (t[i]->rows + rpt2 - 1) / rpt2;
        return tiles2 < (long)num_cus() * WAVES ? 1 : 2;
    }
}

template <int FMT, int BS, bool SPLIT = false>
int launch_t(const qsf_hip_tensor* const* t, int n, int cols, const float* d_x,
             float* const* d_y, void* d_ws, int mode, hipStream_t s) {
    constexpr bool kDreg = FMT != QK_FMT_3 && Fmt<FMT, BS>::CW * Fmt<FMT, BS>::NC * ND <= 48;
    if (tl_pair_act1) {
        // paired rows take two-row tiles whatever the row count
        if constexpr (tile_rows<FMT, BS>() == 2)
            return launch_rt<FMT, BS, 2, false, SPLIT>(t, n, cols, d_x, d_y, d_ws, mode, s);
        return -2;
    }
    const int k = pick_tiles<FMT, BS>(t, n, cols);
    if constexpr (kDreg)
        if (k == 0) return launch_rt<FMT, BS, 1, true, SPLIT>(t, n, cols, d_x, d_y, d_ws, mode, s);
    if constexpr (tile_rows<FMT, BS>() == 2)
        if (k == 2) return launch_rt<FMT, BS, 2, false, SPLIT>(t, n, cols, d_x, d_y, d_ws, mode, s);
    return launch_rt<FMT, BS, 1, false, SPLIT>(t, n, cols, d_x, d_y, d_ws, mode, s);
}

template <int FMT, int BS, bool SPLIT = false>
uint64_t sig_t(const qsf_hip_tensor* const* t, int n, int cols, int mode) {
    constexpr bool kDreg = FMT != QK_FMT_3 && Fmt<FMT, BS>::CW * Fmt<FMT, BS>::NC * ND <= 48;
    const int k = pick_tiles<FMT, BS>(t, n, cols);
    if constexpr (kDreg)
        if (k == 0) return sig_rt<FMT, BS, 1, true, SPLIT>(t, n, cols, mode);
    if constexpr (tile_rows<FMT, BS>() == 2)
        if (k == 2) return sig_rt<FMT, BS, 2, false, SPLIT>(t, n, cols, mode);
    return sig_rt<FMT, BS, 1, false, SPLIT>(t, n, cols, mode);
}

template <int FMT>
int launch_bs(int bs, const qsf_hip_tensor* const* t, int n, int cols, const float* x,
              float* const* y, void* ws, int mode, hipStream_t s) {
    switch (bs) {
    case 32: return launch_t<FMT, 32>(t, n, cols, x, y, ws, mode, s);
    case 64: return launch_t<FMT, 64>(t, n, cols, x, y, ws, mode, s);
    case 128: return launch_t<FMT, 128>(t, n, cols, x, y, ws, mode, s);
    case 256: return launch_t<FMT, 256>(t, n, cols, x, y, ws, mode, s);
    default: return -2;
    }
}

int launch_fmt(int fmt, int bs, const qsf_hip_tensor* const* t, int n, int cols, const float* x,
               float* const* y, void* ws, int mode, hipStream_t s) {
    switch (fmt) {
    case QK_FMT_2: return launch_bs<QK_FMT_2>(bs, t, n, cols, x, y, ws, mode, s);
    case QK_FMT_3: return launch_bs<QK_FMT_3>(bs, t, n, cols, x, y, ws, mode, s);
    case QK_FMT_4: return launch_bs<QK_FMT_4>(bs, t, n, cols, x, y, ws, mode, s);
    case QK_FMT_4SYM: return launch_bs<QK_FMT_4SYM>(bs, t, n, cols, x, y, ws, mode, s);
    default: return -2;
    }
}

template <int FMT>
size_t bytes_bs(int bs, int cols) {
    switch (bs) {
    case 32: return xprep_bytes_t<FMT, 32>(cols);
    case 64: return xprep_bytes_t<FMT, 64>(cols);
    case 128: return xprep_bytes_t<FMT, 128>(cols);
    case 256: return xprep_bytes_t<FMT, 256>(cols);
    default: return 0;
    }
}

// ---------------------------------------------------------------------------
// Bit-exact unpack check.  One thread per block; codes are rebuilt from the
// very masked copies and (code, shift) slot map the GEMV feeds to v_dot8, by
// evaluating the GEMV's sum with a one-hot x: 4*code = sum over the code's
// slots of nibble * 2^shift * (copy B ? 1 : 4).
template <int FMT, int BS>
__global__ void unpack_kernel(const uint8_t* __restrict__ blocks, int nblocks,
                              int8_t* __restrict__ codes, uint32_t* __restrict__ meta,
                              float* __restrict__ deq) {
    using F = Fmt<FMT, BS>;
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(blocks + (size_t)b * F::BB);
    int v4[BS];
#pragma unroll
    for (int k = 0; k < BS; k++) v4[k] = 0;
    auto one = [&](auto wic) {
        constexpr int wi = decltype(wic)::value;
        const uint32_t w = p[1 + wi];
#pragma unroll
        for (int c = 0; c < F::NC; c++) {
            const uint32_t nib = extract<FMT, wi>(w, c);
#pragma unroll
            for (int m = 0; m < 8; m++) {
                int code, shift;
                slot_code<FMT>(wi, c, m, code, shift);
                int val = (int)((nib >> (4 * m)) & 15u);
                val = val >= 8 ? val - 16 : val;           // signed nibble, as v_dot8 reads it
                const int weight = (F::NA == 2 && c == 1) ? 1 : 4;
                v4[code] += val * (1 << shift) * weight;
            }
        }
    };
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (one(std::integral_constant<int, I>{}), ...);
    }(std::make_integer_sequence<int, F::CW>{});
    const uint32_t m0 = p[0];
    const float sc = qsf::f16_lo(m0), z = qsf::f16_hi(m0);
#pragma unroll
    for (int k = 0; k < BS; k++) {
        int q = v4[k] / 4;
        if constexpr (FMT == QK_FMT_4) q += 8;            // undo the ^0x8 centring
        if (codes) codes[(size_t)b * BS + k] = (int8_t)q;
        if (deq) {
            const float prod = qsf::mul_rn(sc, (float)q);
            deq[(size_t)b * BS + k] = FMT == QK_FMT_4SYM ? prod : qsf::add_rn(prod, z);
        }
    }
    if (meta) meta[b] = m0;
}

template <int FMT>
int unpack_bs(int bs, const uint8_t* blk, int n, int8_t* c, uint32_t* m, float* d, hipStream_t s) {
    const dim3 g((n + 63) / 64), t(64);
    switch (bs) {
    case 32: hipLaunchKernelGGL((unpack_kernel<FMT, 32>), g, t, 0, s, blk, n, c, m, d); break;
    case 64: hipLaunchKernelGGL((unpack_kernel<FMT, 64>), g, t, 0, s, blk, n, c, m, d); break;
    case 128: hipLaunchKernelGGL((unpack_kernel<FMT, 128>), g, t, 0, s, blk, n, c, m, d); break;
    case 256: hipLaunchKernelGGL((unpack_kernel<FMT, 256>), g, t, 0, s, blk, n, c, m, d); break;
    default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int FMT>
uint64_t sig_bs(int bs, const qsf_hip_tensor* const* t, int n, int cols, int mode) {
    switch (bs) {
    case 32: return sig_t<FMT, 32>(t, n, cols, mode);
    case 64: return sig_t<FMT, 64>(t, n, cols, mode);
    case 128: return sig_t<FMT, 128>(t, n, cols, mode);
    case 256: return sig_t<FMT, 256>(t, n, cols, mode);
    default: return 0;
    }
}

}  // namespace

// Prepared x of blocks of 128 or 256 codes comes per 64-code part, the
// granularity the split GEMV reads them at (as the one-launch GEMV prepares
// them in its workgroups).
extern "C" size_t qk_xprep_bytes(int fmt, int bs, int cols) {
    if (bs == 128 || bs == 256) bs = 64;
    switch (fmt) {
    case QK_FMT_2: return bytes_bs<QK_FMT_2>(bs, cols);
    case QK_FMT_3: return bytes_bs<QK_FMT_3>(bs, cols);
    case QK_FMT_4: return bytes_bs<QK_FMT_4>(bs, cols);
    case QK_FMT_4SYM: return bytes_bs<QK_FMT_4SYM>(bs, cols);
    default: return 0;
    }
}

extern "C" int qk_xprep(int fmt, int bs, int cols, const float* d_x, void* d_ws, hipStream_t s) {
    if (cols <= 0) return 0;
    if (bs == 128 || bs == 256) bs = 64;
    return launch_fmt(fmt, bs, nullptr, 0, cols, d_x, nullptr, d_ws, QK_RUN_XPREP, s);
}

// Blocks of 128 or 256 codes are read as parts of 64, each part a block
// with the stored block's meta.  A 4096-row matrix of 32 blocks a row then
// uses every lane of its 64-lane row groups instead of half, and 86 blocks
// (11008 columns) 172 of 192 lanes instead of 86 of 128; on config 2's
// 3-bit block-128 layer every launch got faster (q/k/v 9.91 -> 9.53 us, o
// 6.48 -> 5.32, gate/up 14.26 -> 13.69, down 12.69 -> 11.92), so the view
// is taken whatever the row count, which also keeps a grouped launch's
// results equal to its single launches'.  Prepared x (qk_xprep) comes per
// part too, so the prepared GEMV takes the same view.
template <int FMT>
int launch_split(const qsf_hip_tensor* const* t, int n, int cols, const float* x, float* const* y,
                 void* ws, int mode, hipStream_t s) {
    return launch_t<FMT, 64, true>(t, n, cols, x, y, ws, mode, s);
}

extern "C" int qk_gemv_group(const qsf_hip_tensor* const* t, int n, const float* d_x,
                             float* const* d_y, void* d_ws, int mode, hipStream_t s) {
    if (n <= 0 || n > QK_MAX_GROUP) return -2;
    const int fmt = t[0]->fmt, bs = t[0]->bs, cols = t[0]->cols;
    for (int i = 1; i < n; i++)
        if (t[i]->fmt != fmt || t[i]->bs != bs || t[i]->cols != cols) return -2;
    if (cols <= 0) {
        // the scalar reference writes out[r] = 0 for every row
        for (int i = 0; i < n; i++)
            if (t[i]->rows > 0)
                hipLaunchKernelGGL(fill_kernel, dim3((t[i]->rows + 255) / 256), dim3(256), 0, s,
                                   d_y[i], t[i]->rows, 0.0f);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    // tensors in fragment order take the matrix-core kernel (from the fp32 x
    // in every mode) and nothing else
    bool frag = false, disk = false;
    for (int i = 0; i < n; i++) (t[i]->frag ? frag : disk) = true;
    if (frag) return disk ? -2 : qk_gemv_mfma(t, n, d_x, d_y, tl_pair_act1, tl_norm, s);
    if ((mode == QK_RUN_BOTH || mode == QK_RUN_GEMV) && (bs == 128 || bs == 256)) {
        switch (fmt) {
        case QK_FMT_2: return launch_split<QK_FMT_2>(t, n, cols, d_x, d_y, d_ws, mode, s);
        case QK_FMT_3: return launch_split<QK_FMT_3>(t, n, cols, d_x, d_y, d_ws, mode, s);
        case QK_FMT_4: return launch_split<QK_FMT_4>(t, n, cols, d_x, d_y, d_ws, mode, s);
        case QK_FMT_4SYM: return launch_split<QK_FMT_4SYM>(t, n, cols, d_x, d_y, d_ws, mode, s);
        default: return -2;
        }
    }
    return launch_fmt(fmt, bs, t, n, cols, d_x, d_y, d_ws, mode, s);
}

extern "C" int qk_gemv_pair_act(const qsf_hip_tensor* t, const float* d_x, float* d_y, int act,
                                hipStream_t s) {
    if (!t || t->rows % 2 || t->cols <= 0 || t->fmt < 0 || act < 0) return -2;
    tl_pair_act1 = act + 1;
    float* const y[1] = {d_y};
    const int rc = qk_gemv_group(&t, 1, d_x, y, nullptr, QK_RUN_BOTH, s);
    tl_pair_act1 = 0;
    return rc;
}

// The fused forms' checks: a norm needs its arguments, every matrix rows
// (a launch with no tiles would skip the residual store), and buffers that
// no workgroup writes while another still reads them.
static bool norm_ok(const qsf_hip_tensor* const* t, int n, const qk_norm_args* nm, const float* d_x,
                    float* const* d_y) {
    if (!nm || !nm->res_in || !nm->res_out || !nm->w || !d_x || n <= 0 || n > QK_MAX_GROUP) return false;
    if (nm->res_out == nm->res_in || nm->res_out == d_x) return false;
    for (int i = 0; i < n; i++) {
        if (!t[i] || t[i]->rows <= 0 || t[i]->cols <= 0 || t[i]->cols > kNormPerThread * WAVES * 64) return false;
        if (d_y[i] == nm->res_in || d_y[i] == nm->res_out || d_y[i] == d_x) return false;
    }
    return true;
}

extern "C" int qk_gemv_group_norm(const qsf_hip_tensor* const* t, int n, const qk_norm_args* nm,
                                  const float* d_x, float* const* d_y, hipStream_t s) {
    if (!norm_ok(t, n, nm, d_x, d_y)) return -2;
    tl_norm = nm;
    const int rc = qk_gemv_group(t, n, d_x, d_y, nullptr, QK_RUN_BOTH, s);
    tl_norm = nullptr;
    return rc;
}

extern "C" int qk_gemv_pair_act_norm(const qsf_hip_tensor* t, const qk_norm_args* nm, const float* d_x,
                                     float* d_y, int act, hipStream_t s) {
    float* const y[1] = {d_y};
    if (!norm_ok(&t, 1, nm, d_x, y)) return -2;
    tl_norm = nm;
    const int rc = qk_gemv_pair_act(t, d_x, d_y, act, s);
    tl_norm = nullptr;
    return rc;
}

extern "C" uint64_t qk_gemv_signature(const qsf_hip_tensor* const* t, int n, int mode) {
    if (n <= 0 || n > QK_MAX_GROUP) return 0;
    const int fmt = t[0]->fmt, bs = t[0]->bs, cols = t[0]->cols;
    for (int i = 1; i < n; i++)
        if (t[i]->fmt != fmt || t[i]->bs != bs || t[i]->cols != cols || t[i]->frag != t[0]->frag) return 0;
    if (cols <= 0) return 2;
    if (t[0]->frag) {
        // the matrix-core kernel: a row's arithmetic depends on its matrix
        // alone; groups mix no outlier and plain tables
        const bool o = t[0]->d_row_ptr != nullptr;
        for (int i = 1; i < n; i++)
            if ((t[i]->d_row_ptr != nullptr) != o) return 0;
        return 1ull | (1ull << 62) | (uint64_t)o << 1 | (uint64_t)fmt << 8 | (uint64_t)bs << 16;
    }
    if ((mode == QK_RUN_BOTH || mode == QK_RUN_GEMV) && (bs == 128 || bs == 256)) {
        switch (fmt) {
        case QK_FMT_2: return sig_t<QK_FMT_2, 64, true>(t, n, cols, mode);
        case QK_FMT_3: return sig_t<QK_FMT_3, 64, true>(t, n, cols, mode);
        case QK_FMT_4: return sig_t<QK_FMT_4, 64, true>(t, n, cols, mode);
        case QK_FMT_4SYM: return sig_t<QK_FMT_4SYM, 64, true>(t, n, cols, mode);
        default: return 0;
        }
    }
    switch (fmt) {
    case QK_FMT_2: return sig_bs<QK_FMT_2>(bs, t, n, cols, mode);
    case QK_FMT_3: return sig_bs<QK_FMT_3>(bs, t, n, cols, mode);
    case QK_FMT_4: return sig_bs<QK_FMT_4>(bs, t, n, cols, mode);
    case QK_FMT_4SYM: return sig_bs<QK_FMT_4SYM>(bs, t, n, cols, mode);
    default: return 0;
    }
}

template <int FMT, int BS>
int xstage_t(int cols, const float* x, float* d_xcopy, void* d_ws, hipStream_t s) {
    using F = Fmt<FMT, BS>;
    const int nb = (cols + BS - 1) / BS;
    hipLaunchKernelGGL((xprep_kernel<FMT, BS>), dim3((nb + 256 / F::LPB - 1) / (256 / F::LPB)),
                       dim3(256), 0, s, x, cols, nb, (uint32_t*)d_ws, xmeta_in<FMT, BS>(d_ws, nb),
                       d_xcopy);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int FMT>
int xstage_bs(int bs, int cols, const float* x, float* d_xcopy, void* d_ws, hipStream_t s) {
    switch (bs) {
    case 32: return xstage_t<FMT, 32>(cols, x, d_xcopy, d_ws, s);
    case 64: return xstage_t<FMT, 64>(cols, x, d_xcopy, d_ws, s);
    case 128: return xstage_t<FMT, 128>(cols, x, d_xcopy, d_ws, s);
    case 256: return xstage_t<FMT, 256>(cols, x, d_xcopy, d_ws, s);
    default: return -2;
    }
}

extern "C" int qk_xprep_stage(int fmt, int bs, int cols, const float* x, float* d_xcopy,
                              void* d_ws, hipStream_t s) {
    if (cols <= 0) return 0;
    if (bs == 128 || bs == 256) bs = 64;       // per 64-code part, as qk_xprep
    switch (fmt) {
    case QK_FMT_2: return xstage_bs<QK_FMT_2>(bs, cols, x, d_xcopy, d_ws, s);
    case QK_FMT_3: return xstage_bs<QK_FMT_3>(bs, cols, x, d_xcopy, d_ws, s);
    case QK_FMT_4: return xstage_bs<QK_FMT_4>(bs, cols, x, d_xcopy, d_ws, s);
    case QK_FMT_4SYM: return xstage_bs<QK_FMT_4SYM>(bs, cols, x, d_xcopy, d_ws, s);
    default: return -2;
    }
}

extern "C" int qk_stage_f32(float* d_dst, const float* src, int n, hipStream_t s) {
    if (n <= 0) return 0;
    if (((uintptr_t)d_dst | (uintptr_t)src) & 15) return -2;
    const int threads = (n >> 2) + 3;
    hipLaunchKernelGGL(stage_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, d_dst, src, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_unpack(int qt, const void* d_blocks, int nblocks, int bs, int8_t* d_codes,
                         uint32_t* d_meta, float* d_deq, hipStream_t s) {
    if (nblocks <= 0) return 0;
    const uint8_t* b = (const uint8_t*)d_blocks;
    switch (qt) {
    case QK_Q2: case QK_Q2SYM: case QK_Q2_OUTLIER:
        return unpack_bs<QK_FMT_2>(bs, b, nblocks, d_codes, d_meta, d_deq, s);
    case QK_Q3: return unpack_bs<QK_FMT_3>(bs, b, nblocks, d_codes, d_meta, d_deq, s);
    case QK_Q4SYM: return unpack_bs<QK_FMT_4SYM>(bs, b, nblocks, d_codes, d_meta, d_deq, s);
    default: return unpack_bs<QK_FMT_4>(bs, b, nblocks, d_codes, d_meta, d_deq, s);
    }
}

extern "C" int qk_timing(int enable) {
    g_timing.on = enable != 0;
    if (enable) g_timing.used = 0;
    return 0;
}

extern "C" int qk_timing_read(float* us, int max) {
    const int n = g_timing.used < max ? g_timing.used : max;
    for (int i = 0; i < n; i++) {
        float ms = 0.0f;
        if (hipEventSynchronize(g_timing.ev[i][1]) != hipSuccess ||
            hipEventElapsedTime(&ms, g_timing.ev[i][0], g_timing.ev[i][1]) != hipSuccess)
            return -1;
        us[i] = ms * 1000.0f;
    }
    return n;
}
