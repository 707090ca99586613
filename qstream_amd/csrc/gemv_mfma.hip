// gemv_mfma.hip - batch-1 decode GEMV over QSF 2/3/4-bit blocks on the
// gfx950 matrix cores (v_mfma_i32_16x16x64_i8).
//
// Replaces the fused dequant->dot loops of src/kernels_scalar.c:16-109 and the
// outlier matvec of src/quant.c:387-495 for decode calls over tensors
// uploaded in fragment order (x fits the workgroup: cols <= 16384).  Each
// block keeps its QSF bytes, [fp16 scale][fp16 zero][packed codes]
// (src/quant.c:87-177); only the blocks' order in memory changes: a tile of
// 16 rows x 4 blocks is 64 blocks whose 16-byte pieces are interleaved in
// 1 KB planes (qk_frag_offset), so every load a wave issues covers 1 KB of
// contiguous memory.
//
// Arithmetic.  Per block, sum_k (s*q_k + z) x_k = s * sum_k q_k x_k + z * sum_k x_k.
// x becomes block-fixed-point integers X_k = rint(x_k * 2^sh), |X| < 2^XB
// (XB = 29; 25 for 3-bit codes, whose multipliers carry up to four more
// bits), each the sum of four balanced base-256 digits.  The codes, unpacked
// to int8 in registers, meet the digits on the int8 matrix core: the integer
// products and sums are exact.  The digit sums are joined in int32 pairs,
// converted and joined in fp32, then s * (. * 2^-sh) + z * (2^-sh sum X) per
// block.  Roundings: x -> X (at most 2^-(XB+1) of the block's max |x|) and
// fp32 arithmetic on block partial sums, the order of the reference's own
// fp32 accumulation.
//
// MFMA mapping.  One tile is 16 rows x 4 consecutive blocks.  Lane (n, g)
// (n = lane % 16, g = lane / 16) loads block g of row n (meta + code dwords,
// 16-byte pieces from the tile's planes).  MFMA j (one per 16 int8 code positions of
// a lane) takes as B the lane's own codes j, and as A the digits: A row
// m = 4g' + d holds digit d of block g' in the k positions of lane group g',
// zero in the other groups.  The product C[4g + d][n] is then block g's
// digit-d sum for row n, and it lands in lane (n, g), register d: each lane
// finishes its own block with the meta it loaded.  The A operands come from
// LDS (one 16-byte read a lane, the 48 lanes outside their group reading a
// zero region).
//
// Launch.  1024-thread workgroups, about one per CU.  A workgroup owns whole
// 16-row groups of one matrix (so every row's sum is finished in LDS), its
// 16 waves split the groups' tiles in quad-major order.  The workgroup loads
// x once, every thread a few columns (all of it ahead of any weights), each
// wave requests its first tile once x is in, and the 1024 threads turn x
// into digits in LDS together while those tiles stream; every wave then keeps
// D tiles in flight in a register ring.  The fp16 outliers of the
// workgroup's rows (CSR entries, contiguous) are requested after the
// weights, turned into products in LDS, and summed per row in the final pass.
#include "qsf_device.h"
#include "qsf_hip_internal.h"

#include <hip/hip_ext.h>

#include <type_traits>
#include <utility>

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef f32x4 f32x4_a4 __attribute__((aligned(4)));

constexpr int NT = 1024;                 // threads a workgroup
constexpr int NWAVE = NT / 64;
constexpr int kMaxCols = 16 * NT;        // columns (incl. quad padding) the x preparation covers
constexpr int kEntAhead = 4;             // outlier entries a thread requests ahead
constexpr size_t kLdsCap = 160 * 1024;

template <int FMT, int BS>
struct MF {
    static constexpr int BITS = FMT == QK_FMT_2 ? 2 : (FMT == QK_FMT_3 ? 3 : 4);
    static constexpr int CW = BS * BITS / 32;                  // code dwords a block
    static constexpr int NW = 1 + CW;                          // dwords a block
    static constexpr int BB = 4 * NW;                          // bytes a block
    // fragment order: 16-byte planes a block, bytes in the tail plane
    static constexpr int KP = BB / 16, TB = BB % 16;
    // MFMAs a tile: 16 int8 code positions a lane each
    static constexpr int NJ = FMT == QK_FMT_2 || FMT == QK_FMT_3 ? CW : CW / 2;
    static constexpr int XB = FMT == QK_FMT_3 ? 25 : 29;
    static constexpr int LPB1 = BS / 8;                        // x-group lanes a block (8 columns each)
    // ring slots a wave may hold: at most 48 registers of weights
    static constexpr int DMAX = 48 / NW < 1 ? 1 : (48 / NW > 8 ? 8 : 48 / NW);
    // the largest slot count instantiated (1, 2, 4, 8) within it
    static constexpr int DFIT = DMAX >= 8 ? 8 : DMAX >= 4 ? 4 : DMAX >= 2 ? 2 : 1;
    static_assert(BS % 32 == 0 && BS >= 32 && BS <= 256, "block sizes 32-256");
};

// 3-bit masks for code dword w with w % 3 == k.  Nibble g = 8w + i of the
// bitstream holds the bits of code floor(4g/3) from bit g % 3 up (copy A),
// then the low bits of the next code (copy B, read after >> 1).
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

// B operand of MFMA j: 16 int8 code values from the lane's block.
// Byte s of dword t holds:
//   2-bit : crumb 4s + t of code dword j           (code 16j + 4s + t)
//   4-bit : nibble 2s + (t & 1) of dword 2j + t/2  (code 16j + 8(t/2) + 2s + (t&1))
//   4sym  : the same, re-biased to 0..15 (n ^ 8; the zero term takes -8s)
//   3-bit : copy A (t < 2) / B (t >= 2) nibble 2s + (t & 1) of code dword j
template <int FMT, int BS, int J>
__device__ __forceinline__ i32x4 unpack_b(const uint32_t (&wv)[MF<FMT, BS>::NW]) {
    if constexpr (FMT == QK_FMT_2) {
        const uint32_t w = wv[1 + J];
        return i32x4{(int)(w & 0x03030303u), (int)((w >> 2) & 0x03030303u),
                     (int)((w >> 4) & 0x03030303u), (int)((w >> 6) & 0x03030303u)};
    } else if constexpr (FMT == QK_FMT_3) {
        const uint32_t w = wv[1 + J];
        constexpr uint32_t ma = f3_mask(J % 3, 0), mb = f3_mask(J % 3, 1);
        return i32x4{(int)(w & (ma & 0x0F0F0F0Fu)), (int)((w >> 4) & ((ma >> 4) & 0x0F0F0F0Fu)),
                     (int)((w >> 1) & (mb & 0x0F0F0F0Fu)), (int)((w >> 5) & ((mb >> 4) & 0x0F0F0F0Fu))};
    } else {
        constexpr uint32_t bias = FMT == QK_FMT_4SYM ? 0x88888888u : 0u;
        const uint32_t w0 = wv[1 + 2 * J] ^ bias, w1 = wv[2 + 2 * J] ^ bias;
        return i32x4{(int)(w0 & 0x0F0F0F0Fu), (int)((w0 >> 4) & 0x0F0F0F0Fu),
                     (int)(w1 & 0x0F0F0F0Fu), (int)((w1 >> 4) & 0x0F0F0F0Fu)};
    }
}

// Code index (within the block) and power-of-two multiplier shift of int8
// position p (byte p % 4 of dword p / 4) of MFMA j's B operand.  3-bit copy
// A positions carry 4x their weight so that the digit sums are 4x the block
// sum, exactly (f is stored as 2^-sh / 4).
template <int FMT>
__device__ __forceinline__ void pos_code(int j, int p, int& code, int& shift) {
    const int t = p >> 2, s = p & 3;
    if constexpr (FMT == QK_FMT_2) {
        code = 16 * j + 4 * s + t;
        shift = 0;
    } else if constexpr (FMT == QK_FMT_3) {
        const int c = t >> 1, m = 2 * s + (t & 1);
        const int gn = 8 * j + m;
        code = (4 * gn) / 3 + c;
        shift = gn % 3 + (c == 0 ? 2 : 0);
    } else {
        code = 16 * j + 8 * (t >> 1) + 2 * s + (t & 1);
        shift = 0;
    }
}

struct MfArgs {
    struct Mat {
        const uint8_t* w;
        float* y;
        const uint32_t* rp;        // outlier CSR row pointers (rows + 1), or null
        const uint32_t* oe;        // packed entries col | fp16 << 16
        int rows, nent, rgs, gpm;  // rows, entries, 16-row groups, workgroups
        int rq, rr;                // workgroup w takes rq + (w < rr) groups from w*rq + min(w, rr)
    } mat[QK_MAX_GROUP];
    const float* x;
    int n, cols, nb, nq;           // matrices, columns, blocks a row, 4-block quads a row
    uint32_t row_bytes;
    int nrg_max;                   // 16-row groups a workgroup at most
    int act1;                      // paired rows (gate 2i, up 2i+1): 1 + activation, else 0
    // LDS byte offsets
    int o_dig, o_zero, o_meta, o_xq, o_xs, o_stash, o_rp, o_prod;
    int prod_cap;                  // outlier products LDS holds
    // NORM kernels: x is a residual increment.  r = res_in + x (workgroup 0
    // stores it to res_out and the NaN check to *bad), and the rows multiply
    // rms_norm(r) * nw, computed by every workgroup into LDS
    const float* res_in;
    float* res_out;
    const float* nw;
    int* bad;
    float eps;
    int o_xn, o_red;
};

// NORM kernels: elements of x a thread holds in the norm prologue (the
// residual + norm launch's own count, so the sums match bit for bit)
constexpr int kNormPerThread = 8;

// op over aligned groups of W lanes (power of two, <= 16) with DPP; the
// result in every lane of the group.
template <int W, typename OP>
__device__ __forceinline__ int group_all(int v, OP op) {
    if constexpr (W >= 2) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
    if constexpr (W >= 4) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
    if constexpr (W >= 8) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
    if constexpr (W >= 16) v = op(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
    return v;
}

template <int FMT, int BS, int D, bool OUT, bool NORM>
__global__ __launch_bounds__(NT) void gemv_mfma_kernel(MfArgs a) {
    static_assert(!(OUT && NORM), "NORM: no outlier tables");
    using F = MF<FMT, BS>;
    constexpr int NW = F::NW, NJ = F::NJ, KP = F::KP, TB = F::TB;
    extern __shared__ __align__(16) uint8_t lds[];
    const int t = (int)threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int g = lane >> 4;

    // the workgroup's matrix (blockIdx.y) and 16-row groups [rg0, rg0 + nrg).
    // The record and the other arguments are materialised together, in one
    // scalar round trip ahead of the first load (a chain of dependent
    // argument loads costs a memory latency each before any weight moves).
    const MfArgs::Mat& M = a.mat[blockIdx.y];
    const int wgm = (int)blockIdx.x;
    asm volatile("" ::"s"(M.w), "s"(M.y), "s"(M.rows), "s"(M.gpm), "s"(M.rq), "s"(M.rr), "s"(a.x),
                 "s"(a.cols), "s"(a.nq), "s"(a.nb), "s"(a.o_dig), "s"(a.o_zero), "s"(a.o_meta), "s"(a.o_xq),
                 "s"(a.o_xs), "s"(a.o_stash), "s"(a.o_rp), "s"(a.o_prod), "s"(a.prod_cap), "s"(a.act1));
    if constexpr (OUT) asm volatile("" ::"s"(M.rp), "s"(M.oe), "s"(M.nent));
    if constexpr (NORM)
        asm volatile("" ::"s"(a.res_in), "s"(a.res_out), "s"(a.nw), "s"(a.bad), "s"(a.eps), "s"(a.o_xn),
                     "s"(a.o_red));
    if (wgm >= M.gpm) return;                                 // (whole workgroup)
    const int rg0 = wgm * M.rq + min(wgm, M.rr);
    const int nrg = M.rq + (wgm < M.rr ? 1 : 0);
    const int rows = M.rows, nb = a.nb, nq = a.nq;
    const uint8_t* __restrict__ W = M.w;
    const int row_a = rg0 * 16, row_b = min(row_a + nrg * 16, rows);

    // this wave's tiles: the workgroup's T = nrg * nq tiles in quad-major
    // order (u -> quad u / nrg, group u % nrg), contiguous runs a wave
    const int T = nrg * nq;
    const int u0 = (wave * T) / NWAVE, u1 = ((wave + 1) * T) / NWAVE;
    const int nmy = u1 - u0;
    uint32_t wv[D][NW];
    // slot k <- tile u (clamped into the wave's run: past its end a slot
    // re-reads the run's last tile, a cache hit, so every load is issued
    // unconditionally and the compiler's waits stay exact).  Lane L reads
    // its block's 16-byte pieces from planes 1 KB apart and its tail.
    auto issue = [&](int k, int u) __attribute__((always_inline)) {
        u = max(min(u, u1 - 1), 0);
        const int q = u / nrg, rl = u - q * nrg;
        const uint8_t* tp = W + (size_t)((rg0 + rl) * nq + q) * (64 * F::BB);
#pragma unroll
        for (int i = 0; i < KP; i++) {
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tp + i * 1024 + lane * 16));
            wv[k][4 * i] = v.x; wv[k][4 * i + 1] = v.y; wv[k][4 * i + 2] = v.z; wv[k][4 * i + 3] = v.w;
        }
        const uint32_t* tl = reinterpret_cast<const uint32_t*>(tp + KP * 1024 + lane * TB);
#pragma unroll
        for (int i = 0; i < TB / 4; i++) wv[k][4 * KP + i] = __builtin_nontemporal_load(tl + i);
    };

    // 2. x, cooperatively: in pass p thread t holds XPQ columns of block
    //    64 p + t / 16 (lane t % 16 of it), the layout the digit rows are
    //    built from; a workgroup covers 64 blocks a pass and every block in
    //    at most kMaxCols / (64 BS) passes (XC 4-vectors a thread in all).
    //    Issued ahead of every weight load (loads return in order, and x is
    //    waited for first); chunks of passes past the blocks re-read the
    //    thread's first (first-level cache hits: no branch, so the waits stay
    //    exact).  NORM: the residual, the increment and the norm weights of
    //    elements t + k * NT instead, as the residual + norm launch loads
    //    them (only the passes that hold elements load; past the end a
    //    thread re-reads its first).
    constexpr int XPQ = BS / 16;                              // x values a thread a pass
    constexpr int NPASS = kMaxCols / (64 * BS);               // passes at most
    const int nbp = 4 * nq;                                   // blocks incl. quad padding
    const int npass = (nbp + 63) >> 6;
    const int xl0 = (t >> 4) * BS + (t & 15) * XPQ;           // the thread's first column in pass 0
    f32x4 xc[NPASS][XPQ / 4];
    float nr[kNormPerThread], nx[kNormPerThread], nwv[kNormPerThread];
    if constexpr (NORM) {
        const int n = a.cols;
#pragma unroll
        for (int k = 0; k < kNormPerThread; k++) {
            nr[k] = nx[k] = nwv[k] = 0.f;
            if (k * NT < n) {
                const int i = t + k * NT < n ? t + k * NT : min(t, n - 1);
                nr[k] = a.res_in[i];
                nx[k] = a.x[i];
                nwv[k] = a.nw[i];
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < NPASS; p++)
#pragma unroll
            for (int k = 0; k < XPQ / 4; k++)
                xc[p][k] = *reinterpret_cast<const f32x4_a4*>(
                    a.x + min((p < npass ? p * 64 * BS : 0) + xl0 + 4 * k, a.cols - 4));
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2b. outliers: the workgroup's CSR bounds (its entries are contiguous),
    //     behind x: they come from HBM, and x, waited for first, must not
    //     wait for them
    uint32_t e0 = 0, e1 = 0, rpv = 0;
    if constexpr (OUT) {
        e0 = M.rp[row_a];
        e1 = M.rp[row_b];
        rpv = M.rp[min(row_a + t, row_b)];
    }
    __builtin_amdgcn_sched_barrier(0);
    // every wave's x requests ahead of any wave's weights: the CU issues
    // memory instructions oldest wave first, so without this the last waves'
    // x would queue behind the first waves' tiles
    if constexpr (!NORM) __syncthreads();

    // 3. the first tile's weights, once x is in (issued with x, the whole
    //    ring ahead of the digits measured slower); the other slots once the
    //    digits are built
    if constexpr (OUT) __builtin_amdgcn_s_waitcnt(0x0F73);   // vmcnt(3): x is in, the bounds may not be
    else if constexpr (!NORM) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x is in
    issue(0, u0);
    __builtin_amdgcn_sched_barrier(0);

    // 3b. NORM: the residual add and the RMS norm of src/engine.c:1174-1187
    //     and 940-948 / 805-815 as residual_norm_kernel computes them (same
    //     thread count, elements and order, so the same bits); the normed x
    //     goes to LDS, where the preparation reads it.  Workgroup (0, 0)
    //     stores the residual and the NaN check.
    if constexpr (NORM) {
        const int n = a.cols;
        float acc = 0.f;
        int first = n;
#pragma unroll
        for (int k = 0; k < kNormPerThread; k++) {
            const int i = t + k * NT;
            const float r = qsf::add_rn(nr[k], nx[k]);
            nr[k] = r;
            if (i < n) {
                if ((r != r || r > 1e30f || r < -1e30f) && i < first) first = i;
                acc = fmaf(r, r, acc);
            }
        }
        float* red = reinterpret_cast<float*>(lds + a.o_red);
        const float ss = qsf::wg_sum(acc, red);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(qsf::add_rn(__fdiv_rn(ss, (float)n), a.eps)));
        if (blockIdx.x == 0 && blockIdx.y == 0) {
#pragma unroll
            for (int k = 0; k < kNormPerThread; k++)
                if (t + k * NT < n) a.res_out[t + k * NT] = nr[k];
            if (a.bad) {
                for (int off = 32; off > 0; off >>= 1) first = min(first, __shfl_xor(first, off, 64));
                int* ired = reinterpret_cast<int*>(red);
                __syncthreads();                      // every wave past wg_sum's reads of red
                if (lane == 0) ired[wave] = first;
                __syncthreads();
                if (t == 0) {
                    int f = n;
                    for (int w = 0; w < NWAVE; w++) f = min(f, ired[w]);
                    *a.bad = f < n ? f : -1;
                }
            }
        }
        float* xn = reinterpret_cast<float*>(lds + a.o_xn);
#pragma unroll
        for (int k = 0; k < kNormPerThread; k++)
            if (t + k * NT < n) xn[t + k * NT] = qsf::mul_rn(qsf::mul_rn(nr[k], inv), nwv[k]);
        __syncthreads();
    }

    // 4. the digits, cooperatively.  Phase 1, a pass at a time: x -> X.  A
    //    thread's XPQ columns lie in block 64 p + t / 16; block max of |x| as
    //    bits (Inf/NaN above every finite value), shift, X = rint(x 2^sh)
    //    (exact: |x 2^sh| < 2^XB), block sum of X in two exact halves, meta
    //    {f, f sum X}.  Phase 2: one thread a (block, MFMA j, 4-position
    //    slice tq): the 4 multipliers of the slice, biased by 0x80808080 so
    //    that byte d is digit d + 128, byte-transposed into one dword of
    //    each digit row, re-biased to int8.
    float2* meta = reinterpret_cast<float2*>(lds + a.o_meta);
    int* xq = reinterpret_cast<int*>(lds + a.o_xq);
    float* xs = reinterpret_cast<float*>(lds + a.o_xs);
    uint8_t* dig = lds + a.o_dig;
#pragma unroll
    for (int p = 0; p < NPASS; p++) {
      if (p < npass) {                                        // (uniform)
        const int c0 = p * 64 * BS + xl0;
        float v8[XPQ];
        if constexpr (NORM) {
            const float* xn = reinterpret_cast<const float*>(lds + a.o_xn);
#pragma unroll
            for (int k = 0; k < XPQ; k++) v8[k] = c0 + k < a.cols ? xn[c0 + k] : 0.0f;
        } else {
#pragma unroll
            for (int k = 0; k < XPQ / 4; k++) {
                const f32x4 ch = xc[p][k];
                const int c = c0 + 4 * k;
                // in range: the chunk as read; straddling the last column: it
                // was read at cols - 4, so column c + i sits at i + sh; past it: 0
                const int sh = c - (a.cols - 4);
                const float n0 = sh == 1 ? ch.y : (sh == 2 ? ch.z : ch.w);
                const float n1 = sh == 1 ? ch.z : ch.w;
                const bool full = c + 4 <= a.cols;
                v8[4 * k] = full ? ch.x : (c < a.cols ? n0 : 0.0f);
                v8[4 * k + 1] = full ? ch.y : (c + 1 < a.cols ? n1 : 0.0f);
                v8[4 * k + 2] = full ? ch.z : (c + 2 < a.cols ? ch.w : 0.0f);
                v8[4 * k + 3] = full ? ch.w : 0.0f;
            }
        }
        uint32_t amax = 0;
#pragma unroll
        for (int k = 0; k < XPQ; k++) amax = max(amax, __builtin_bit_cast(uint32_t, v8[k]) & 0x7FFFFFFFu);
        const int amax_b = group_all<16>((int)amax, [](int u, int v) { return max(u, v); });
        const bool bad = amax_b >= 0x7F800000;
        int sh = 0;
        if (!bad && amax_b > 0) {
            sh = F::XB - 1 - ilogbf(__builtin_bit_cast(float, amax_b));
            sh = sh > 126 ? 126 : sh;
        }
        int X[XPQ];
        int hs = 0, ls = 0;
#pragma unroll
        for (int k = 0; k < XPQ; k++) {
            X[k] = bad ? 0 : (int)rintf(ldexpf(v8[k], sh));
            hs += X[k] >> 16;
            ls += X[k] & 0xFFFF;
        }
        hs = group_all<16>(hs, [](int u, int v) { return u + v; });
        ls = group_all<16>(ls, [](int u, int v) { return u + v; });
        if (c0 < nbp * BS) {
#pragma unroll
            for (int k = 0; k < XPQ / 4; k++) {
                reinterpret_cast<i32x4*>(xq + c0)[k] = i32x4{X[4 * k], X[4 * k + 1], X[4 * k + 2], X[4 * k + 3]};
                if constexpr (OUT)
                    reinterpret_cast<f32x4*>(xs + c0)[k] =
                        f32x4{v8[4 * k], v8[4 * k + 1], v8[4 * k + 2], v8[4 * k + 3]};
            }
            if ((t & 15) == 0) {
                const double tot = (double)hs * 65536.0 + (double)ls;           // exact
                const float f = bad ? __builtin_nanf("") : ldexpf(FMT == QK_FMT_3 ? 0.25f : 1.0f, -sh);
                meta[c0 / BS] = make_float2(f, bad ? 0.0f : (float)(tot * ldexp(1.0, -sh)));
            }
        }
      }
    }
    // the zero rows of the A operands
    if (t < NJ * 4) reinterpret_cast<u32x4*>(lds + a.o_zero)[t] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
    for (int idx = t; idx < nbp * NJ * 4; idx += NT) {
        const int tq = idx & 3, bj = idx >> 2;                // bj = block * NJ + j
        const int b = bj / NJ, j = bj - b * NJ;
        uint32_t V[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            int code, shift;
            pos_code<FMT>(j, 4 * tq + s4, code, shift);
            const uint32_t mlt = (uint32_t)xq[b * BS + code] << shift;
            V[s4] = (mlt + 0x80808080u) ^ 0x80808080u;
        }
        const uint32_t l01 = __builtin_amdgcn_perm(V[1], V[0], 0x05010400u);
        const uint32_t h01 = __builtin_amdgcn_perm(V[1], V[0], 0x07030602u);
        const uint32_t l23 = __builtin_amdgcn_perm(V[3], V[2], 0x05010400u);
        const uint32_t h23 = __builtin_amdgcn_perm(V[3], V[2], 0x07030602u);
        uint32_t* out = reinterpret_cast<uint32_t*>(dig + (size_t)(b * NJ + j) * 64) + tq;
        out[0] = __builtin_amdgcn_perm(l23, l01, 0x05040100u);
        out[4] = __builtin_amdgcn_perm(l23, l01, 0x07060302u);
        out[8] = __builtin_amdgcn_perm(h23, h01, 0x05040100u);
        out[12] = __builtin_amdgcn_perm(h23, h01, 0x07060302u);
    }
#pragma unroll
    for (int k = 1; k < D; k++) issue(k, u0 + k);
    __syncthreads();

    // 5. outlier entries of the workgroup's rows, kEntAhead a thread
    //    (clamped indices: always loaded, so the waits stay exact)
    uint32_t ent[kEntAhead];
    if constexpr (OUT) {
        const uint32_t last = (uint32_t)max(M.nent - 1, 0);
#pragma unroll
        for (int k = 0; k < kEntAhead; k++) ent[k] = M.oe[min(e0 + (uint32_t)(t + k * NT), last)];
    }

    // 6. tiles: NJ MFMA k-steps of int8 codes against digits, the block's
    //    scale/zero epilogue, the lane's block partial into the stash
    //    [group][quad][lane] (every slot written once).  A ring of D slots:
    //    a slot is refilled with the tile D ahead as soon as it is computed.
    const bool act = ((lane & 15) >> 2) == g;                 // A row 4g + d in group g
    const uint32_t a_lane = act ? (uint32_t)(g * NJ * 64 + (lane & 3) * 16) : (uint32_t)(a.o_zero - a.o_dig);
    float* stash = reinterpret_cast<float*>(lds + a.o_stash);
    auto compute = [&](int k, int u) __attribute__((always_inline)) {
        const int q = u / nrg, rl = u - q * nrg;
        const uint32_t aq = act ? (uint32_t)(4 * q * NJ * 64) : 0u;
        const uint8_t* ap = dig + a_lane + aq;
        i32x4 c = {0, 0, 0, 0};
        [&]<int... J>(std::integer_sequence<int, J...>) {
            ((c = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                  *reinterpret_cast<const i32x4*>(ap + J * 64), unpack_b<FMT, BS, J>(wv[k]), c, 0, 0, 0)),
             ...);
        }(std::make_integer_sequence<int, NJ>{});
        const uint32_t lo = (uint32_t)c[0] + ((uint32_t)c[1] << 8);
        const uint32_t hi = (uint32_t)c[2] + ((uint32_t)c[3] << 8);
        const float v = fmaf((float)(int)hi, 65536.0f, (float)(int)lo);
        const int blk = 4 * q + g;
        const float2 xm = meta[blk];
        const float sc = qsf::f16_lo(wv[k][0]);
        float z;
        if constexpr (FMT == QK_FMT_4SYM) z = -8.0f * sc;
        else z = qsf::f16_hi(wv[k][0]);
        const float pv = fmaf(z, xm.y, sc * (v * xm.x));
        stash[(rl * nq + q) * 64 + lane] = blk < nb ? pv : 0.0f;
    };
    const int nblk = (nmy + D - 1) / D;
    for (int bi = 0; bi + 1 < nblk; bi++) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            compute(k, u0 + bi * D + k);
            issue(k, u0 + (bi + 1) * D + k);
        }
    }
    if (nblk > 0) {
#pragma unroll
        for (int k = 0; k < D; k++)
            if ((nblk - 1) * D + k < nmy) compute(k, u0 + (nblk - 1) * D + k);
    }

    // 7. the workgroup's outlier entries into LDS in entry order (their
    //    products need every wave's x copy, so they wait for the barrier)
    uint32_t* oent = reinterpret_cast<uint32_t*>(lds + a.o_prod);
    if constexpr (OUT) {
#pragma unroll
        for (int k = 0; k < kEntAhead; k++) {
            const uint32_t e = e0 + (uint32_t)(t + k * NT);
            if (e < e1 && e - e0 < (uint32_t)a.prod_cap) oent[e - e0] = ent[k];
        }
        for (uint32_t e = e0 + (uint32_t)(t + kEntAhead * NT); e < e1 && e - e0 < (uint32_t)a.prod_cap; e += NT)
            oent[e - e0] = M.oe[e];
        if (t <= row_b - row_a) reinterpret_cast<uint32_t*>(lds + a.o_rp)[t] = rpv;
    }
    __syncthreads();

    // 8. rows: 4 lanes a row.  Lane g of a row sums its nq block partials
    //    of lane group g in quad order, then every 4th of its outlier
    //    products val * x[col] (src/quant.c:481-494), and two DPP steps join
    //    the lanes; the order depends on the row's shape and entries only.
    const int i4 = t & 3;
    const uint32_t* rpl = reinterpret_cast<const uint32_t*>(lds + a.o_rp);
    const int nrows = row_b - row_a;
    for (int r0 = 0; r0 < nrg * 16; r0 += NT / 4) {
        const int rr = r0 + (t >> 2);
        float v = 0.0f;
        if (rr < nrows) {
            const int rl = rr >> 4, n = rr & 15;
            const float* sp = stash + (rl * nq) * 64 + i4 * 16 + n;
#pragma unroll 8
            for (int q = 0; q < nq; q++) v += sp[q * 64];
            if constexpr (OUT) {
                // (clamped to the workgroup's entries: a global read never
                // depends on LDS contents alone)
                const uint32_t b0 = max(rpl[rr], e0), b1 = min(rpl[rr + 1], e1);
                for (uint32_t e = b0 + i4; e < b1; e += 4) {
                    const uint32_t u = e - e0 < (uint32_t)a.prod_cap ? oent[e - e0] : M.oe[e];
                    v += qsf::mul_rn(qsf::f16_bits((uint16_t)(u >> 16)), xs[u & 0xFFFFu]);
                }
            }
        }
        v = qsf::group_sum_last(v, 4);
        // paired rows: gate 2i, up 2i + 1 four lanes on (the same wave)
        const float up = __shfl_down(v, 4, 64);
        if (i4 == 3 && rr < nrows) {
            if (a.act1) {
                if ((rr & 1) == 0) M.y[(row_a + rr) >> 1] = qsf::act_mul(a.act1 - 1, v, up);
            } else {
                M.y[row_a + rr] = v;
            }
        }
    }
}

int num_cus_mf() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
    }
    return n;
}

size_t lds_cap_mf() {
    static size_t v = 0;
    if (!v) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && n > 0)
            v = (size_t)n;
        else
            v = 64 * 1024;
        v = v < kLdsCap ? v : kLdsCap;
    }
    return v;
}

// 0 off, 1 the 3-bit formats, 2 every format it covers
int g_mfma_on = 1;

// LDS layout of a launch (byte offsets in `a`); returns the bytes before
// the outlier products.
template <int FMT, int BS>
size_t lds_plan(MfArgs& a, int cols, int nrg_max, bool out, bool norm) {
    using F = MF<FMT, BS>;
    const int nbp = 4 * a.nq;
    auto al = [](size_t v) { return (v + 15) & ~(size_t)15; };
    size_t off = 0;
    a.o_dig = (int)off;   off += al((size_t)nbp * F::NJ * 64);
    a.o_zero = (int)off;  off += al((size_t)F::NJ * 64);
    a.o_meta = (int)off;  off += al((size_t)nbp * 8);
    a.o_xq = (int)off;    off += al((size_t)nbp * BS * 4);
    a.o_xs = (int)off;    off += out ? al((size_t)nbp * BS * 4) : 0;
    a.o_stash = (int)off; off += al((size_t)nrg_max * a.nq * 256);
    a.o_rp = (int)off;    off += out ? al((size_t)(nrg_max * 16 + 1) * 4) : 0;
    a.o_xn = (int)off;    off += norm ? al((size_t)cols * 4) : 0;
    a.o_red = (int)off;   off += norm ? al((size_t)NWAVE * 4) : 0;
    a.o_prod = (int)off;
    return off;
}

template <int FMT, int BS>
bool covers_mf(int cols, bool outliers) {
    const int nb = (cols + BS - 1) / BS, nq = (nb + 3) / 4;
    if (cols < 16 || 4 * nq * BS > kMaxCols) return false;
    MfArgs a{};
    a.nq = nq;
    // one 16-row group a workgroup: plain, with the norm, and with outliers
    // (the larger plan) where the tensor has an outlier table
    return lds_plan<FMT, BS>(a, cols, 1, false, false) <= lds_cap_mf() &&
           lds_plan<FMT, BS>(a, cols, 1, false, true) <= lds_cap_mf() &&
           (!outliers || lds_plan<FMT, BS>(a, cols, 1, true, false) + (size_t)NT * 4 <= lds_cap_mf());
}

template <int FMT, int BS>
int launch_mf(const qsf_hip_tensor* const* t, int n, int cols, const float* d_x, float* const* d_y,
              int act1, const qk_norm_args* nm, hipStream_t s) {
    using F = MF<FMT, BS>;
    const int nb = (cols + BS - 1) / BS, nq = (nb + 3) / 4;
    if (!covers_mf<FMT, BS>(cols, false)) return -2;
    MfArgs a{};
    a.x = d_x;
    a.n = n;
    a.cols = cols;
    a.nb = nb;
    a.nq = nq;
    a.act1 = act1;
    bool out = false;
    long total_rg = 0;
    for (int i = 0; i < n; i++) {
        if (!t[i]->frag || t[i]->frag_nq != nq) return -2;
        if (t[i]->d_row_ptr && (!t[i]->d_oent)) return -2;                // packed entries only
        if ((size_t)qk_frag_bytes(t[i]->rows, nb, F::BB) > ((size_t)1 << 40)) return -2;
        const bool o = t[i]->d_row_ptr && t[i]->n_csr > 0;
        if (i > 0 && o != out) return -2;        // outlier tables in all matrices or in none
        out = o;
        a.mat[i] = {t[i]->d_blocks, d_y[i], o ? t[i]->d_row_ptr : nullptr, o ? t[i]->d_oent : nullptr,
                    t[i]->rows, (int)t[i]->n_csr, (t[i]->rows + 15) / 16, 0, 0, 0};
        total_rg += a.mat[i].rgs;
    }
    if (act1 && (n != 1 || out)) return -2;
    if (nm && (out || cols > kNormPerThread * NT)) return -2;
    // 16-row groups a workgroup: with outliers one CSR bound a thread
    // (rows + 1 <= NT); the stash within LDS
    int nrg_fit = 1 << 20;
    if (out) nrg_fit = (NT - 1) / 16;
    {
        MfArgs b = a;
        const size_t fixed = lds_plan<FMT, BS>(b, cols, 0, out, nm != nullptr);
        const size_t room = lds_cap_mf() - (out ? (size_t)NT * 4 : 0);
        if (fixed >= room) return -2;
        const int by_lds = (int)((room - fixed) / ((size_t)nq * 256 + (out ? 64 : 0)));
        nrg_fit = by_lds < nrg_fit ? by_lds : nrg_fit;
    }
    if (nrg_fit < 1) return -2;
    // workgroups per matrix in proportion to its 16-row groups, about one a
    // CU in all; each takes whole groups, spread evenly
    const int cus = num_cus_mf();
    int g = 0, nrg_max = 0;
    for (int i = 0; i < n; i++) {
        const int rgs = a.mat[i].rgs;
        int gi = (int)((long)cus * rgs / (total_rg > 0 ? total_rg : 1));
        gi = gi < 1 ? 1 : gi;
        gi = gi > rgs ? rgs : gi;
        if ((rgs + gi - 1) / gi > nrg_fit) gi = (rgs + nrg_fit - 1) / nrg_fit;
        a.mat[i].gpm = gi;
        a.mat[i].rq = rgs / gi;
        a.mat[i].rr = rgs % gi;
        g = gi > g ? gi : g;
        const int mx = (rgs + gi - 1) / gi;
        nrg_max = mx > nrg_max ? mx : nrg_max;
    }
    if (g == 0) return 0;
    a.nrg_max = nrg_max;
    size_t off = lds_plan<FMT, BS>(a, cols, nrg_max, out, nm != nullptr);
    if (off > lds_cap_mf()) return -2;
    a.prod_cap = out ? (int)((lds_cap_mf() - off) / 4) : 0;
    if (out && a.prod_cap > kEntAhead * NT * 2) a.prod_cap = kEntAhead * NT * 2;
    if (out && a.prod_cap < NT) return -2;
    off += out ? (size_t)a.prod_cap * 4 : 0;
    if (nm) {
        a.res_in = nm->res_in;
        a.res_out = nm->res_out;
        a.nw = nm->w;
        a.bad = nm->bad;
        a.eps = nm->eps;
    }
    auto go = [&](auto kern) {
        static bool allowed = false;
        if (!allowed) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_cap_mf());
            allowed = true;
        }
        hipEvent_t e0, e1;
        if (qk_timing_pair(&e0, &e1))
            hipExtLaunchKernelGGL(kern, dim3(g, n), dim3(NT), (uint32_t)off, s, e0, e1, 0, a);
        else
            hipLaunchKernelGGL(kern, dim3(g, n), dim3(NT), off, s, a);
    };
    // ring depth: the slots a wave's tiles need, up to the format's budget
    const int per = (nrg_max * nq + NWAVE - 1) / NWAVE;
    auto go_d = [&](auto dc) {
        constexpr int DD = decltype(dc)::value < F::DFIT ? decltype(dc)::value : F::DFIT;
        if (out) go(gemv_mfma_kernel<FMT, BS, DD, true, false>);
        else if (nm) go(gemv_mfma_kernel<FMT, BS, DD, false, true>);
        else go(gemv_mfma_kernel<FMT, BS, DD, false, false>);
    };
    if (per <= 2) go_d(std::integral_constant<int, 2>{});
    else go_d(std::integral_constant<int, 4>{});
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int FMT>
int launch_mf_bs(int bs, const qsf_hip_tensor* const* t, int n, int cols, const float* x,
                 float* const* y, int act1, const qk_norm_args* nm, hipStream_t s) {
    // block sizes 64 (QStream's default) and 128
    switch (bs) {
    case 64: return launch_mf<FMT, 64>(t, n, cols, x, y, act1, nm, s);
    case 128: return launch_mf<FMT, 128>(t, n, cols, x, y, act1, nm, s);
    default: return -2;
    }
}

template <int FMT>
bool covers_bs(int bs, int cols, bool outliers) {
    switch (bs) {
    case 64: return covers_mf<FMT, 64>(cols, outliers);
    case 128: return covers_mf<FMT, 128>(cols, outliers);
    default: return false;
    }
}

}  // namespace

extern "C" int qk_mfma_layout(int fmt, int bs, int cols, int outliers) {
    switch (fmt) {
    case QK_FMT_2: return covers_bs<QK_FMT_2>(bs, cols, outliers != 0);
    case QK_FMT_3: return covers_bs<QK_FMT_3>(bs, cols, outliers != 0);
    case QK_FMT_4: return covers_bs<QK_FMT_4>(bs, cols, outliers != 0);
    case QK_FMT_4SYM: return covers_bs<QK_FMT_4SYM>(bs, cols, outliers != 0);
    default: return 0;
    }
}

// One-launch MFMA decode GEMV over n tensors in fragment order sharing x;
// -2 when the call is not covered.
extern "C" int qk_gemv_mfma(const qsf_hip_tensor* const* t, int n, const float* d_x, float* const* d_y,
                            int act1, const qk_norm_args* nm, hipStream_t s) {
    if (n <= 0 || n > QK_MAX_GROUP) return -2;
    const int fmt = t[0]->fmt, bs = t[0]->bs, cols = t[0]->cols;
    for (int i = 0; i < n; i++)
        if (t[i]->fmt != fmt || t[i]->bs != bs || t[i]->cols != cols || t[i]->rows <= 0 || !t[i]->frag) return -2;
    switch (fmt) {
    case QK_FMT_2: return launch_mf_bs<QK_FMT_2>(bs, t, n, cols, d_x, d_y, act1, nm, s);
    case QK_FMT_3: return launch_mf_bs<QK_FMT_3>(bs, t, n, cols, d_x, d_y, act1, nm, s);
    case QK_FMT_4: return launch_mf_bs<QK_FMT_4>(bs, t, n, cols, d_x, d_y, act1, nm, s);
    case QK_FMT_4SYM: return launch_mf_bs<QK_FMT_4SYM>(bs, t, n, cols, d_x, d_y, act1, nm, s);
    default: return -2;
    }
}

extern "C" int qk_gemv_mfma_enable(int on) {
    const int old = g_mfma_on;
    if (on >= 0) g_mfma_on = on > 2 ? 2 : on;
    return old;
}
