// gemv_decode.hip - batch-1 decode GEMV over QSF 2/3/4-bit blocks on gfx950.
//
// Replaces the fused dequant->dot loops of src/kernels_scalar.c:16-109 and the
// outlier matvec of src/quant.c:387-495 (CPU twins: src/kernels_avx2.c:77-549).
// The QSF block bytes are read as they are on disk:
//   [fp16 scale][fp16 zero | reserved][packed codes]   (src/quant.c:87-177)
//
// Arithmetic.  Per block the reference computes sum_k (s*q_k + z) * x_k.  Here
//   sum_k (s*q_k + z) x_k = s * sum_k q_k x_k + z * sum_k x_k
// and the code/activation products are done exactly in integers: the x-prep
// kernel turns each block of x into block-fixed-point integers X_k = x_k*2^sh
// (|X| <= 2^XB, XB = 24..26 bits) and splits every X into seven signed
// base-16 digits.  The GEMV multiplies raw code nibbles by digit nibbles with
// v_dot8_i32_i4 (8 products per instruction, exact int32), recombines the
// digits per block in two exact int32 groups (digits 0-3 and 4-6), joins them
// with one fp32 FMA and applies the fp16 scale/zero in fp32.  The rounding
// beyond fp32 accumulation is x -> X, at most 2^-(XB+1) of the block's max
// |x| -- finer than fp32 itself for the block's largest elements, so even a
// row whose result cancels 100x stays inside the 1e-5 bar against the strict
// scalar reference.
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
// Layout.  A wave owns R rows (x LG row groups when a row has < 64 blocks);
// lane l of a group handles blocks l, l+LPG, ...  of those rows, so each lane
// reads whole blocks (dword loads from 4-byte aligned blocks) and reuses its
// block's digits from LDS for R rows.  Partial sums are reduced with lane
// shuffles; a fused CSR pass adds the fp16 outliers of the wave's rows.
#include "qsf_device.h"
#include "qsf_hip_internal.h"

#include <utility>

namespace {

constexpr int ND = 7;                  // balanced base-16 digits per multiplier
constexpr int ND_LO = 4;               // digits 0-3 and 4-6 are recombined separately
constexpr uint32_t DIGIT_BIAS = 0x8888888u;  // 8 * (16^7 - 1) / 15


template <int FMT, int BS>
struct Fmt {
    static constexpr int BITS = FMT == QK_FMT_2 ? 2 : (FMT == QK_FMT_3 ? 3 : 4);
    static constexpr int CW = BS * BITS / 32;                       // code dwords / block
    static constexpr int NC = (FMT == QK_FMT_2 || FMT == QK_FMT_3) ? 2 : 1;  // masked copies
    static constexpr int NA = FMT == QK_FMT_3 ? 2 : 1;              // accumulator sets
    static constexpr int BB = 4 + 4 * CW;                           // block bytes
    static constexpr int DW = CW * NC * ND;                         // digit dwords / block
    static constexpr int DWS = (DW + 3) & ~3;                       // 16-B aligned stride
    // |X| <= 2^XB.  Digit multipliers M = X * 2^shift (shift <= 2 for 3-bit)
    // must lie in the 7-digit balanced range [-0x8888888, 0x7777777]; the
    // low-group sum is <= 8 * 34952 * BS and the high-group sum
    // <= 8 * (2^(XB+2)/65536 + 1) * BS, both far inside int32.
    static constexpr int XB = FMT == QK_FMT_3 ? 24 : 26;
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
        int delta = g % 3;
        code = (4 * g) / 3 + c;
        shift = delta;
    } else { code = 8 * w + m; shift = 0; }
}

// ---------------------------------------------------------------------------
// x preparation: one wave per block of x.
// Output per block b: Fmt::DW digit dwords (layout [w][c][digit]) and
// meta {f_b = 2^-sh, sum_k X_k * f_b}.
template <int FMT, int BS>
__global__ __launch_bounds__(256) void xprep_kernel(const float* __restrict__ x, int cols, int nb,
                                                    uint32_t* __restrict__ xq,
                                                    float2* __restrict__ xmeta) {
    using F = Fmt<FMT, BS>;
    constexpr int NSLOT = F::CW * F::NC * 8;
    __shared__ int xs[4][BS];
    __shared__ uint32_t us[4][NSLOT];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + wave;
    const bool live = b < nb;

    float v[(BS + 63) / 64];
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int j = 0; j < (BS + 63) / 64; j++) {
        int k = lane + 64 * j;
        int col = b * BS + k;
        float t = (live && k < BS && col < cols) ? x[col] : 0.0f;
        v[j] = t;
        if (!(fabsf(t) <= 3.402823466e38f)) bad = 1;   // Inf or NaN
        else amax = fmaxf(amax, fabsf(t));
    }
    amax = qsf::wave_max(amax);
    bad = qsf::wave_or_i(bad);
    int sh = 0;
    if (amax > 0.0f) {
        sh = F::XB - 1 - ilogbf(amax);                 // amax * 2^sh < 2^XB
        sh = sh > 126 ? 126 : (sh < -100 ? -100 : sh);
    }
    int sumx = 0;
#pragma unroll
    for (int j = 0; j < (BS + 63) / 64; j++) {
        int k = lane + 64 * j;
        if (k < BS) {
            int X = bad ? 0 : (int)rintf(ldexpf(v[j], sh));
            xs[wave][k] = X;
            sumx += X;
        }
    }
    sumx = qsf::wave_sum_i(sumx);
    __syncthreads();
    for (int s = lane; s < NSLOT; s += 64) {
        int w = s / (F::NC * 8), c = (s / 8) % F::NC, m = s % 8, code, shift;
        slot_code<FMT>(w, c, m, code, shift);
        int M = xs[wave][code] * (1 << shift);
        us[wave][s] = (uint32_t)(M + (int)DIGIT_BIAS);
    }
    __syncthreads();
    if (!live) return;
    for (int o = lane; o < F::DW; o += 64) {
        int wc = o / ND, d = o % ND;                  // wc = w * NC + c
        uint32_t out = 0;
#pragma unroll
        for (int m = 0; m < 8; m++) out |= ((us[wave][wc * 8 + m] >> (4 * d)) & 15u) << (4 * m);
        xq[(size_t)b * F::DWS + o] = out ^ 0x88888888u;  // nibble n-8 in two's complement
    }
    if (lane == 0) {
        float f = ldexpf(1.0f, -sh);
        if (bad) f = __builtin_nanf("");
        xmeta[b] = make_float2(f, (float)sumx * f);
    }
}

struct GemvArgs {
    const uint8_t* w[QK_MAX_GROUP];
    float* y[QK_MAX_GROUP];
    const uint32_t* rp[QK_MAX_GROUP];
    const uint32_t* oc[QK_MAX_GROUP];
    const uint16_t* ov[QK_MAX_GROUP];
    int rows[QK_MAX_GROUP];
    int tile0[QK_MAX_GROUP + 1];
    int n, cols, nb, lpg, chunk;
    const uint32_t* xq;
    const float2* xmeta;
    const float* x;
};

template <int FMT, int BS, int R, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(GemvArgs a) {
    using F = Fmt<FMT, BS>;
    extern __shared__ uint32_t lds[];
    const int tile = blockIdx.x;
    int m = 0;
    while (m + 1 < a.n && tile >= a.tile0[m + 1]) m++;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lpg = a.lpg, grp = lane / lpg, lig = lane % lpg;
    const int rows_per_wave = (64 / lpg) * R;
    const int row0 = (tile - a.tile0[m]) * WAVES * rows_per_wave + wave * rows_per_wave + grp * R;
    const int rows = a.rows[m];
    const uint8_t* __restrict__ wbase = a.w[m];
    const size_t row_bytes = (size_t)a.nb * F::BB;

    float rsum[R];
#pragma unroll
    for (int r = 0; r < R; r++) rsum[r] = 0.0f;

    for (int c0 = 0; c0 < a.nb; c0 += a.chunk) {
        const int c1 = min(a.nb, c0 + a.chunk);
        // stage this chunk's digits and block meta in LDS
        __syncthreads();
        {
            const uint4* src = reinterpret_cast<const uint4*>(a.xq + (size_t)c0 * F::DWS);
            uint4* dst = reinterpret_cast<uint4*>(lds);
            const int n4 = (c1 - c0) * F::DWS / 4;
            for (int i = threadIdx.x; i < n4; i += WAVES * 64) dst[i] = src[i];
            float2* mdst = reinterpret_cast<float2*>(lds + a.chunk * F::DWS);
            for (int i = threadIdx.x; i < c1 - c0; i += WAVES * 64) mdst[i] = a.xmeta[c0 + i];
        }
        __syncthreads();
        const float2* meta = reinterpret_cast<const float2*>(lds + a.chunk * F::DWS);

        for (int b = c0 + lig; b < c1; b += lpg) {
            uint32_t wv[R][1 + F::CW];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = row0 + r;
                if (row < rows) {
                    const uint32_t* p = reinterpret_cast<const uint32_t*>(
                        wbase + (size_t)row * row_bytes + (size_t)b * F::BB);
#pragma unroll
                    for (int i = 0; i < 1 + F::CW; i++) wv[r][i] = __builtin_nontemporal_load(p + i);
                } else {
#pragma unroll
                    for (int i = 0; i < 1 + F::CW; i++) wv[r][i] = 0u;
                }
            }
            const uint32_t* dg = lds + (size_t)(b - c0) * F::DWS;
            int acc[R][F::NA][ND];
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int s = 0; s < F::NA; s++)
#pragma unroll
                    for (int d = 0; d < ND; d++) acc[r][s][d] = 0;

            auto step = [&](auto wic) {
                constexpr int wi = decltype(wic)::value;
                uint32_t dig[F::NC][ND];
#pragma unroll
                for (int c = 0; c < F::NC; c++)
#pragma unroll
                    for (int d = 0; d < ND; d++) dig[c][d] = dg[(wi * F::NC + c) * ND + d];
#pragma unroll
                for (int r = 0; r < R; r++) {
#pragma unroll
                    for (int c = 0; c < F::NC; c++) {
                        const uint32_t nib = extract<FMT, wi>(wv[r][1 + wi], c);
                        const int s = F::NA == 2 ? c : 0;
#pragma unroll
                        for (int d = 0; d < ND; d++) acc[r][s][d] = qsf::sdot8(nib, dig[c][d], acc[r][s][d]);
                    }
                }
            };
            [&]<int... I>(std::integer_sequence<int, I...>) {
                (step(std::integral_constant<int, I>{}), ...);
            }(std::make_integer_sequence<int, F::CW>{});

            const float2 xm = meta[b - c0];
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
                    const float v = fmaf((float)(int)hi, 65536.0f, (float)(int)lo);
                    sf = s == 0 ? v : fmaf(0.25f, v, sf);
                }
                const float sc = qsf::f16_lo(wv[r][0]);
                const float coef = sc * xm.x;
                if constexpr (FMT == QK_FMT_4SYM) {
                    rsum[r] = fmaf(coef, sf, rsum[r]);
                } else {
                    float z = qsf::f16_hi(wv[r][0]);
                    if constexpr (FMT == QK_FMT_4) z = fmaf(8.0f, sc, z);
                    rsum[r] = fmaf(coef, sf, rsum[r]);
                    rsum[r] = fmaf(z, xm.y, rsum[r]);
                }
            }
        }
    }

    // fused sparse pass: fp16 outliers of this group's rows (src/quant.c:481-494)
    const uint32_t* rp = a.rp[m];
    if (rp) {
        const uint32_t* __restrict__ oc = a.oc[m];
        const uint16_t* __restrict__ ov = a.ov[m];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
            if (row < rows) {
                const uint32_t e1 = rp[row + 1];
                for (uint32_t j = rp[row] + lig; j < e1; j += lpg)
                    rsum[r] = fmaf(qsf::f16_bits(ov[j]), a.x[oc[j]], rsum[r]);
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; r++) rsum[r] = qsf::group_sum(rsum[r], lpg);
    // every lane of the group holds all R sums; lane (r mod LPG) stores row r
    float* __restrict__ y = a.y[m];
#pragma unroll
    for (int r = 0; r < R; r++)
        if (lig == (r & (lpg - 1)) && row0 + r < rows) y[row0 + r] = rsum[r];
}

__global__ void fill_kernel(float* y, int n, float v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = v;
}

constexpr int kLdsBudget = 64 * 1024;
constexpr int kR = 4;
constexpr int kWaves = 4;

template <int FMT, int BS>
size_t xprep_bytes_t(int cols) {
    using F = Fmt<FMT, BS>;
    size_t nb = (size_t)((cols + BS - 1) / BS);
    size_t dig = nb * F::DWS * 4;
    return ((dig + 255) & ~(size_t)255) + nb * sizeof(float2);
}

template <int FMT, int BS>
int launch_t(const qsf_hip_tensor* const* t, int n, int cols, const float* d_x,
             float* const* d_y, void* d_ws, int mode, hipStream_t s) {
    using F = Fmt<FMT, BS>;
    const int nb = (cols + BS - 1) / BS;
    uint32_t* xq = (uint32_t*)d_ws;
    size_t dig = (size_t)nb * F::DWS * 4;
    float2* xmeta = (float2*)((uint8_t*)d_ws + ((dig + 255) & ~(size_t)255));
    if (mode & QK_RUN_XPREP)
        hipLaunchKernelGGL((xprep_kernel<FMT, BS>), dim3((nb + 3) / 4), dim3(256), 0, s,
                           d_x, cols, nb, xq, xmeta);
    if (!(mode & QK_RUN_GEMV)) return hipGetLastError() == hipSuccess ? 0 : -1;

    GemvArgs a = {};
    a.n = n;
    a.cols = cols;
    a.nb = nb;
    int lpg = 1;
    while (lpg < nb && lpg < 64) lpg <<= 1;
    a.lpg = lpg;
    const int per_block = F::DWS * 4 + (int)sizeof(float2);
    a.chunk = nb < kLdsBudget / per_block ? nb : kLdsBudget / per_block;
    const int rows_per_wg = kWaves * (64 / lpg) * kR;
    a.tile0[0] = 0;
    for (int i = 0; i < n; i++) {
        a.w[i] = t[i]->d_blocks;
        a.y[i] = d_y[i];
        a.rp[i] = t[i]->d_row_ptr;
        a.oc[i] = t[i]->d_ocol;
        a.ov[i] = t[i]->d_oval;
        a.rows[i] = t[i]->rows;
        a.tile0[i + 1] = a.tile0[i] + (t[i]->rows + rows_per_wg - 1) / rows_per_wg;
    }
    a.xq = xq;
    a.xmeta = xmeta;
    a.x = d_x;
    const size_t lds = (size_t)a.chunk * per_block;
    if (a.tile0[n] > 0)
        hipLaunchKernelGGL((gemv_kernel<FMT, BS, kR, kWaves>), dim3(a.tile0[n]), dim3(kWaves * 64),
                           lds, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
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
            const float prod = __fmul_rn(sc, (float)q);
            deq[(size_t)b * BS + k] = FMT == QK_FMT_4SYM ? prod : __fadd_rn(prod, z);
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

}  // namespace

extern "C" size_t qk_xprep_bytes(int fmt, int bs, int cols) {
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
    return launch_fmt(fmt, bs, nullptr, 0, cols, d_x, nullptr, d_ws, QK_RUN_XPREP, s);
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
    return launch_fmt(fmt, bs, t, n, cols, d_x, d_y, d_ws, mode, s);
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
