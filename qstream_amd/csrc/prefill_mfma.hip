// prefill_mfma.hip - batched prefill through the 4-bit QSF format on gfx950
// MFMA: Y[m][n] = sum_k float(x_bf16[m][k]) * w[n][k], M tokens at once.
//
// There is no reference kernel: the engine runs one matvec per token
// (src/engine.c:1289-1295), so the specification is M independent
// src/kernels_scalar.c:64-85 matvecs on float(bf16(x_m)), with
// w = s*q + z per block (src/quant.c:136-155).
//
// Arithmetic.  Nothing is rounded below fp32.  Per block b of a weight row,
//   sum_k (s q_k + z) x_k = s * (sum_k q_k x_k) + z * X_b,   X_b = sum_k x_k.
//  * The codes q (0..15) are exact bf16 integers, x is bf16, so every MFMA
//    product q*x is exact; v_mfma_f32_16x16x32_bf16 sums them in fp32.  The
//    sum restarts every 64 k (a "sub-block"; the scale is constant inside
//    one) and is folded into the output in fp32: out = fma(s, acc, out).
//  * The zero-point term sum_b z_b X_b is itself a small contraction over
//    the blocks.  It runs on the same MFMA as extra k-steps after the
//    codes, on exact bf16 splits: z = zh + zl (fp16 has 11 significant
//    bits, bf16 8, so the remainder has at most 3) and X_b = X1 + X2 + X3
//    (fp32 sum of the block, 24 bits in three 8-bit parts).  Each block
//    takes 8 extra k positions, {X1, X2, X3, X1, X2, 0, 0, 0} against
//    {zh, zh, zh, zl, zl, 0, 0, 0}: every product is exact and only
//    zl*X3 (2^-26 of z X_b) is left out.
// Against the scalar oracle this is at the level of fp32 accumulation
// order (about 1e-6 rel-L2), not of bf16 weights.
//
// Tiling.  One 512-thread workgroup per 256 (m) x 112 (n) tile of Y; at
// config-4 shape (M 512, N 14336) that is exactly one workgroup per CU.  K
// advances in stages of 128 (4 MFMA k-steps): first the code stages, then
// the zero-point stages (8 k positions per block, padded to an even stage
// count).  The waves split by role, one of each per SIMD, so the VALU work
// (code conversion, scale epilogue) and MFMAs overlap in the hardware:
//  * 4 producer waves write stage s+1's 112 x 128 B tile into LDS (bf16,
//    [112][128 + 8 pad], two buffers) with each column's sub-block scales,
//    while stage s is contracted; their loads run two stages ahead.  The
//    code stages read each block's meta dword for its scale and keep its
//    fp16 zero in an LDS stash [112][16 per zero-point stage], from which
//    the zero-point stages build their B tiles: every weight byte is
//    fetched once.  (With the zero-point stages first, reading the meta
//    from memory, they pulled every 64-byte line of the tile's rows through
//    the cache, and the code stages fetched them all again: 2x the weight
//    bytes.)  Rows of more than 448 blocks, too long for the stash, read the
//    meta dwords from memory again in the zero-point stages;
//  * 4 consumer waves each own 64 rows x 112 columns (4 x 7 MFMA tiles).
//    A fragments come from x repacked into fragment order (xpack_kernel:
//    one contiguous 1 KB load per fragment), one stage ahead in registers;
//    B fragments come from LDS one n-tile ahead.
// One barrier per stage.  Loads go through raw buffer descriptors: offsets
// past a tensor read zeros, so prefetches past the end need no clamps.
//
#include "qsf_device.h"
#include "qsf_hip_internal.h"

#include <hip/hip_ext.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 112;      // workgroup tile: 4 waves x 64 m, 7 x 16 n
constexpr int MT = 4, NT = 7;          // 16x16 MFMA tiles per wave
constexpr int SK = 128;                // k per stage (4 MFMA k-steps)
constexpr int PITCH = SK + 8;          // LDS row pitch of the B tile, bf16
constexpr int BUF = BN * PITCH;        // bf16 per B buffer
constexpr int SCN = 2 * BN;            // fp32 scales per buffer: [sub-block][column]
constexpr int EP_PITCH = BN + 4;       // LDS row pitch of the output staging tile, fp32
constexpr int EP_FLOATS = 4 * 64 * EP_PITCH;
constexpr int LDS_MAIN = 2 * BUF * 2 + 2 * SCN * 4;
constexpr int LDS_BYTES = LDS_MAIN > EP_FLOATS * 4 ? LDS_MAIN : EP_FLOATS * 4;
constexpr int ZK = 8;                  // zero-point k positions per block
// Zero stash: fp16 zeros [BN][16 sz] after the B buffers, in LDS left free
// up to 160 KB (the epilogue tile reuses it): rows of up to 448 blocks.
constexpr int ZP_MAX = 448;
constexpr int LDS_STASH = LDS_MAIN + BN * ZP_MAX * 2;
constexpr int LDS_TOTAL = LDS_STASH > LDS_BYTES ? LDS_STASH : LDS_BYTES;
static_assert(LDS_TOTAL <= 160 * 1024, "LDS of a CU");

__device__ __forceinline__ float bf16_f32(__bf16 v) {
    return __builtin_bit_cast(float, (uint32_t)__builtin_bit_cast(uint16_t, v) << 16);
}

// Round two fp32 to bf16 (round-to-nearest-even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x2 to_bf16x2(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_convertvector(v, bf16x2);
}

// Eight codes (one dword; code 2i is the low nibble of byte i, code 2i+1
// the high one) -> the integers 0..15 as exact bf16, in the k order
// {0, 2, 4, 6, 1, 3, 5, 7} (xpack_kernel orders x the same way).  A byte
// 0000qqqq read as OCP FP8 E4M3 is q * 2^-9 (subnormal for q < 8, exponent
// field 1 for q >= 8), so one v_cvt_scalef32_pk_bf16_fp8 with scale 2^9
// (only the scale's exponent is used) turns two nibble bytes into two exact
// bf16 integers: 7 VALU operations per 8 codes.
__device__ __forceinline__ bf16x8 codes8(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, false);   // codes 0, 2
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, true);    // codes 4, 6
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, false);   // codes 1, 3
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, true);    // codes 5, 7
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Eight bf16 of x in k order 0..7 -> the codes8 order {0, 2, 4, 6, 1, 3, 5, 7}.
__device__ __forceinline__ u32x4 x_order(u32x4 v) {
    return u32x4{__builtin_amdgcn_perm(v[1], v[0], 0x05040100u),   // x0, x2
                 __builtin_amdgcn_perm(v[3], v[2], 0x05040100u),   // x4, x6
                 __builtin_amdgcn_perm(v[1], v[0], 0x07060302u),   // x1, x3
                 __builtin_amdgcn_perm(v[3], v[2], 0x07060302u)};  // x5, x7
}

// Zero-point chunk of one block from its meta dword (fp16 scale | fp16 zero
// << 16): {zh, zh, zh, zl, zl, 0, 0, 0}, zh = bf16(z), zl = z - zh (exact).
__device__ __forceinline__ bf16x8 zchunk(uint32_t meta) {
    const float z = qsf::f16_hi(meta);
    const bf16x2 h = to_bf16x2(z, 0.f);
    const bf16x2 l = to_bf16x2(z - bf16_f32(h[0]), 0.f);
    const __bf16 zero = h[1];
    return bf16x8{h[0], h[0], h[0], l[0], l[0], zero, zero, zero};
}

struct PrefillArgs {
    const uint8_t* w;        // QSF 4-bit blocks, rows n, row stride nb*BB
    const u32x4* xp;         // [X parts | x] in A-fragment order (xpack_kernel)
    float* y;                // fp32 [m][n]
    int m, n, k, nb;
    int tiles_n;
    int sz, s;               // zero-point stages; all stages (both even)
    int zp;                  // zero stash entries a column (16 sz), or 0: zeros re-read from memory
    uint32_t w_bytes, xp_bytes;
    int nq;                  // FRAG: 4-block quads a row (the blocks are in fragment order)
};

// x bf16 [m][k] -> A-fragment order.  For each group of 16 rows, ksp_total
// k-steps of 64 chunks of 16 bytes; chunk l of k-step kk holds row
// 16 g + l%16:
//  * k-steps kk < kz: the zero-point part, one chunk per block
//    b = 4 kk + l/16: {X1, X2, X3, X1, X2, 0, 0, 0}, the bf16 split of the
//    block's fp32 sum X_b = X1 + X2 + X3 (exact);
//  * k-steps kz + kk: columns 32 kk + 8 (l/16)..+7 of x, in the k order
//    {0, 2, 4, 6, 1, 3, 5, 7} of the codes (codes8).
// Zeros past m, k and nb.  The GEMM then loads each fragment as one
// contiguous 1 KB read instead of 64 scattered 16-byte pieces.  One
// workgroup per (row group, 8 code k-steps) reads its 16 x 256 tile of x
// row-contiguously into LDS and writes it back in fragment order; the same
// workgroup sums the tile's blocks (256 / bs of each row) from LDS for the
// zero-point part.  Workgroup 0 of a row group also writes the zero chunks
// of the blocks past nb.  (Summing the blocks in workgroups of their own,
// which read x again from memory with 16-byte pieces scattered over rows,
// cost 3 us of config 4's 74 us step.)
constexpr int XP_PITCH = 256 + 8;      // LDS row pitch of the pack tile, bf16

// The zero-point chunk {X1, X2, X3, X1, X2, 0, 0, 0} of a block sum X
// (X = X1 + X2 + X3 exactly, each part bf16).
__device__ __forceinline__ u32x4 xchunk(float X) {
    const bf16x2 p1 = to_bf16x2(X, 0.f);
    const float r1 = X - bf16_f32(p1[0]);
    const bf16x2 p2 = to_bf16x2(r1, 0.f);
    const bf16x2 p3 = to_bf16x2(r1 - bf16_f32(p2[0]), 0.f);
    const __bf16 zero = p1[1];
    return __builtin_bit_cast(u32x4, bf16x8{p1[0], p2[0], p3[0], p1[0], p2[0], zero, zero, zero});
}

__global__ __launch_bounds__(256) void xpack_kernel(const uint16_t* __restrict__ x, u32x4* xp,
                                                   int m, int k, int ksp_total, int kz,
                                                   int bs, int nb) {
    __shared__ __align__(16) uint16_t tile[16 * XP_PITCH];
    const int g = blockIdx.y, t = threadIdx.x;
    const int kk0 = (int)blockIdx.x * 8;
    const int c = t & 31;                      // 16-byte chunk of a 256-wide row piece
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int r = (t >> 5) + 8 * h, row = g * 16 + r, col = kk0 * 32 + 8 * c;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < m && col < k) v = x_order(*reinterpret_cast<const u32x4*>(x + (size_t)row * k + col));
        *reinterpret_cast<u32x4*>(&tile[r * XP_PITCH + 8 * c]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int j = t + 256 * h, kk = j >> 6, l = j & 63;
        xp[((size_t)g * ksp_total + kz + kk0 + kk) * 64 + l] =
            *reinterpret_cast<const u32x4*>(&tile[(l & 15) * XP_PITCH + kk * 32 + 8 * (l >> 4)]);
    }
    // Zero-point part: thread (row r, tile block jb) sums its block's
    // elements in index order from the tile (a chunk's slots hold elements
    // {0, 2, 4, 6, 1, 3, 5, 7}: dword 0 = x0 | x2, 1 = x4 | x6, 2 = x1 | x3,
    // 3 = x5 | x7).  Rows past m and blocks past nb get zero chunks, and
    // workgroup 0 writes those of the blocks past nb that no tile holds.
    const int nbt = 256 / bs;                  // blocks of the tile a row
    if (t < 16 * nbt) {
        const int r = t & 15, jb = t >> 4;
        const int b = kk0 * 32 / bs + jb, row = g * 16 + r;
        const int cnt = row < m && b < nb ? min(bs, k - b * bs) : 0;   // a multiple of 8
        const uint16_t* src = &tile[r * XP_PITCH + jb * bs];
        float X = 0.f;
        for (int e = 0; e < cnt; e += 8) {
            const u32x4 q = *reinterpret_cast<const u32x4*>(src + e);
            X += __builtin_bit_cast(float, q[0] << 16);           // x0
            X += __builtin_bit_cast(float, q[2] << 16);           // x1
            X += __builtin_bit_cast(float, q[0] & 0xFFFF0000u);   // x2
            X += __builtin_bit_cast(float, q[2] & 0xFFFF0000u);   // x3
            X += __builtin_bit_cast(float, q[1] << 16);           // x4
            X += __builtin_bit_cast(float, q[3] << 16);           // x5
            X += __builtin_bit_cast(float, q[1] & 0xFFFF0000u);   // x6
            X += __builtin_bit_cast(float, q[3] & 0xFFFF0000u);   // x7
        }
        if (b < 4 * kz) xp[((size_t)g * ksp_total + (b >> 2)) * 64 + r + 16 * (b & 3)] = xchunk(X);
    }
    if (blockIdx.x == 0)
        for (int i = t; i < 16 * (4 * kz - nb); i += 256) {
            const int b = nb + (i >> 4), r = i & 15;
            xp[((size_t)g * ksp_total + (b >> 2)) * 64 + r + 16 * (b & 3)] = u32x4{0u, 0u, 0u, 0u};
        }
}

// Raw buffer descriptor (gfx9 family word 3): loads at offsets >= `bytes`
// return zero, so clamped-free prefetch past a tensor's end is safe.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Workgroup id -> (m tile, n tile).  Workgroups are dealt to the 8 XCDs
// round-robin; this numbering hands each XCD a contiguous run of tiles in
// column-major order, so the M tiles of one N tile run side by side on one
// XCD and the weight tile they share is fetched into that XCD's L2 once.
__device__ __forceinline__ void tile_of(int id, int nwg, int tiles_n, int& tm, int& tn) {
    const int q = nwg >> 3, r = nwg & 7, xcd = id & 7, slot = id >> 3;
    const int t = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
    const int tiles_m = nwg / tiles_n;
    tn = t / tiles_m;
    tm = t - tn * tiles_m;
}

// RAGGED: k is not a multiple of 2 SK, so code stages reach past the last
// column; their B items are zeroed (and x is zero there).
template <int BS, bool RAGGED, bool FRAG = false, bool PLANE = false>
__global__ __launch_bounds__(512) void prefill_kernel(PrefillArgs a) {
    constexpr int BB = 4 + BS / 2;             // block bytes
    // two B buffers and their scales during the main loop; the output
    // staging tile after it
    __shared__ __align__(16) uint8_t lds_raw[LDS_TOTAL];
    __bf16* const lds = reinterpret_cast<__bf16*>(lds_raw);
    float* const scl = reinterpret_cast<float*>(lds_raw + 2 * BUF * 2);
    uint16_t* const zst = reinterpret_cast<uint16_t*>(lds_raw + LDS_MAIN);
    const int ncode = a.s - a.sz;              // code stages 0..ncode-1, then the zero-point ones

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, a.tiles_n, tm, tn);
    const int n0 = tn * BN;

    if (wave >= 4) {
        // ---- producer waves: write stage s+1's B tile during stage s.
        // Item p < 2 BN: column p/2, k positions 64 (p%2)..+63 of the stage.
        //  * code stage c: one meta dword and two 16-byte code loads; the
        //    codes become 8 chunks of 8 bf16 integers, the scale goes to the
        //    stage's scale row (p%2 = the stage's 64-wide sub-block) and the
        //    zero to the stash;
        //  * zero-point stage z: the 8 blocks 16 z + 8 (p%2) + j of the
        //    column, one stashed zero (or meta dword) each -> one 16-byte
        //    chunk each.
        // Byte offsets in a row: the lane part is fixed, the stage part
        // uniform; columns past n read zeros.
        const uint32_t row_bytes = (uint32_t)a.nb * BB;
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);
        const int p = t - 256, col = p >> 1, h = p & 1;
        const bool active = p < 2 * BN;
        const uint32_t lane_meta = BS == 64 ? (uint32_t)h * BB : 0u;
        const uint32_t lane_code = lane_meta + 4 + (BS == 64 ? 0u : (uint32_t)h * 32);
        const uint32_t wv = (uint32_t)(n0 + col) * row_bytes;
        const int it_base = col * PITCH + 64 * h;
        // FRAG: block b of row n0 + col sits in tile (row / 16, b / 4) at
        // lane 16 (b % 4) + row % 16; its 16-byte planes are 1 KB apart, the
        // 4-byte tail plane after them (rows and blocks past the tensor read
        // zero or are masked below, as in on-disk order)
        constexpr int KP = BB / 16;            // 16-byte planes a block
        const uint32_t frow = (uint32_t)(n0 + col);
        auto fbase = [&](uint32_t b) __attribute__((always_inline)) {
            return (((frow >> 4) * (uint32_t)a.nq + (b >> 2)) * 64u) * (uint32_t)BB +
                   ((b & 3u) * 16u + (frow & 15u)) * 16u;
        };
        auto ftail = [&](uint32_t b) __attribute__((always_inline)) {
            return (((frow >> 4) * (uint32_t)a.nq + (b >> 2)) * 64u) * (uint32_t)BB + KP * 1024u +
                   ((b & 3u) * 16u + (frow & 15u)) * 4u;
        };
        auto load = [&](int s, u32x4 (&c)[2], uint32_t& meta) __attribute__((always_inline)) {
            if (s >= a.s || (s >= ncode && a.zp)) return;   // past the end; zeros from the stash
            if constexpr (FRAG) {
                static_assert(BS == 64 || BS == 128, "fragment order: blocks of 64 or 128");
                if (s >= ncode) {
                    const uint32_t b0 = (uint32_t)(16 * (s - ncode) + 8 * h);
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        c[j >> 2][j & 3] = __builtin_amdgcn_raw_buffer_load_b32(wr, fbase(b0 + j), 0, 0);
                    meta = 0;
                } else {
                    // the 32 code bytes from byte 4 + 32 (h or 0) of the block:
                    // dwords 1-3 of plane pa, plane pa + 1, dword 0 of plane
                    // pa + 2 (or of the tail plane)
                    const int sc = s;
                    const uint32_t b = BS == 64 ? (uint32_t)(2 * sc + h) : (uint32_t)sc;
                    const uint32_t pa = BS == 64 ? 0u : 2u * (uint32_t)h;
                    const uint32_t o = fbase(b);
                    const u32x4 pA = __builtin_amdgcn_raw_buffer_load_b128(wr, o + pa * 1024u, 0, 0);
                    const u32x4 pB = __builtin_amdgcn_raw_buffer_load_b128(wr, o + (pa + 1) * 1024u, 0, 0);
                    const uint32_t pC = pa + 2 < (uint32_t)KP
                                            ? __builtin_amdgcn_raw_buffer_load_b32(wr, o + (pa + 2) * 1024u, 0, 0)
                                            : __builtin_amdgcn_raw_buffer_load_b32(wr, ftail(b), 0, 0);
                    meta = pa == 0 ? pA.x : __builtin_amdgcn_raw_buffer_load_b32(wr, o, 0, 0);
                    c[0] = u32x4{pA.y, pA.z, pA.w, pB.x};
                    c[1] = u32x4{pB.y, pB.z, pB.w, pC};
                }
                return;
            }
            if constexpr (PLANE && BS > 64) {
                // row-plane order, blocks of 128 or 256: block b's meta dword
                // at 4 b, then 64-code part u's 32 code bytes at 16 u in the
                // two 16-byte planes over the row's np parts
                constexpr uint32_t P = BS / 64;
                const uint32_t np = (uint32_t)a.nb * P, cb = 4u * (uint32_t)a.nb;
                if (s >= ncode) {
                    const uint32_t b0 = (uint32_t)(16 * (s - ncode) + 8 * h);
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        c[j >> 2][j & 3] = __builtin_amdgcn_raw_buffer_load_b32(wr, wv + (b0 + j) * 4u, 0, 0);
                    meta = 0;
                } else {
                    const uint32_t b = BS == 128 ? (uint32_t)s : (uint32_t)s / 2;
                    const uint32_t u = b * P + (BS == 128 ? (uint32_t)h : 2u * ((uint32_t)s % 2) + (uint32_t)h);
                    meta = __builtin_amdgcn_raw_buffer_load_b32(wr, wv + 4u * b, 0, 0);
                    c[0] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + cb + u * 16u, 0, 0);
                    c[1] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + cb + np * 16u + u * 16u, 0, 0);
                }
                return;
            }
            if constexpr (PLANE && BS == 64) {
                // row-plane order, blocks of 64: block b's meta and first 12
                // code bytes at 16 b in plane 0, the next 16 at 16 b in plane
                // 1 (nb * 16 bytes on), the last 4 at 4 b in the tail plane
                const uint32_t ps = (uint32_t)a.nb * 16u;
                if (s >= ncode) {
                    const uint32_t b0 = (uint32_t)(16 * (s - ncode) + 8 * h);
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        c[j >> 2][j & 3] = __builtin_amdgcn_raw_buffer_load_b32(wr, wv + (b0 + j) * 16u, 0, 0);
                    meta = 0;
                } else {
                    const uint32_t b = (uint32_t)(2 * s + h);
                    const u32x4 pA = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + b * 16u, 0, 0);
                    const u32x4 pB = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + ps + b * 16u, 0, 0);
                    const uint32_t pC = __builtin_amdgcn_raw_buffer_load_b32(wr, wv + 2u * ps + b * 4u, 0, 0);
                    meta = pA.x;
                    c[0] = u32x4{pA.y, pA.z, pA.w, pB.x};
                    c[1] = u32x4{pB.y, pB.z, pB.w, pC};
                }
                return;
            }
            if (s >= ncode) {
                const uint32_t b0 = (uint32_t)(16 * (s - ncode) + 8 * h);
#pragma unroll
                for (int j = 0; j < 8; j++)
                    c[j >> 2][j & 3] = __builtin_amdgcn_raw_buffer_load_b32(wr, wv + (b0 + j) * BB, 0, 0);
                meta = 0;
            } else {
                const int sc = s;
                const uint32_t sm = BS <= SK ? (uint32_t)sc * (SK / BS) * BB : (uint32_t)(sc / (BS / SK)) * BB;
                const uint32_t so = BS <= SK ? sm : sm + (uint32_t)(sc % (BS / SK)) * (SK / 2);
                meta = __builtin_amdgcn_raw_buffer_load_b32(wr, wv + lane_meta + sm, 0, 0);
                c[0] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + lane_code + so, 0, 0);
                c[1] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + lane_code + so + 16, 0, 0);
            }
        };
        auto produce = [&](int s, const u32x4 (&c)[2], uint32_t meta, __bf16* buf, float* sc)
            __attribute__((always_inline)) {
            if (!active || s >= a.s) return;
            if (s >= ncode) {
                const int b0 = 16 * (s - ncode) + 8 * h;
                u32x4 zs = {0u, 0u, 0u, 0u};            // stashed zeros b0..b0+7
                if (a.zp) zs = *reinterpret_cast<const u32x4*>(zst + col * a.zp + b0);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int b = b0 + j;
                    const uint32_t m = a.zp ? (zs[j >> 1] >> (16 * (j & 1))) << 16 : c[j >> 2][j & 3];
                    bf16x8 v = zchunk(m);
                    if (b >= a.nb) v = bf16x8{};
                    *reinterpret_cast<bf16x8*>(buf + it_base + 8 * j) = v;
                }
            } else {
                // the block's zero into the stash, once a block
                const int zb = BS == 64 ? 2 * s + h : BS == 128 ? s : s >> 1;
                if (a.zp && zb < a.nb && (BS == 64 || (h == 0 && (BS == 128 || (s & 1) == 0))))
                    zst[col * a.zp + zb] = (uint16_t)(meta >> 16);
                const int k0 = s * SK + 64 * h;
                // a sub-block wholly past k has zero codes and x; a zero
                // scale keeps junk meta (Inf, NaN) out of the sum
                sc[h * BN + col] = RAGGED && k0 >= a.k ? 0.f : qsf::f16_lo(meta);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    bf16x8 v = codes8(c[j >> 2][j & 3]);
                    if (RAGGED && k0 + 8 * j >= a.k) v = bf16x8{};
                    *reinterpret_cast<bf16x8*>(buf + it_base + 8 * j) = v;
                }
            }
        };
        // loads double-buffered two stages ahead
        u32x4 ca[2], cb[2];
        uint32_t ma, mb;
        load(0, ca, ma);
        load(1, cb, mb);
        produce(0, ca, ma, lds, scl);
        load(2, ca, ma);
        __syncthreads();
        for (int s = 0; s < a.s; s += 2) {
            produce(s + 1, cb, mb, lds + BUF, scl + SCN);
            load(s + 3, cb, mb);
            __syncthreads();
            produce(s + 2, ca, ma, lds, scl);
            load(s + 4, ca, ma);
            __syncthreads();
        }
        __syncthreads();                           // the consumers' epilogue barrier
        return;
    }

    // ---- consumer waves: wave w owns rows m0..m0+63 and all 112 columns.
    const int l16 = lane & 15, g4 = lane >> 4;
    const int m0 = tm * BM + wave * 64;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xp, a.xp_bytes);
    // A fragment (rows m0 + 16 mt.., k-step kk): 1 KB at (group * ksp + kk)
    // KB of the packed x, 16 bytes per lane; groups past m read zeros
    const uint32_t ksp = 4u * (uint32_t)a.s;
    uint32_t xv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) xv[mt] = ((uint32_t)(m0 / 16 + mt) * ksp * 64u + lane) * 16u;
    // B fragment of n-tile nt, k-step ks: column 16 nt + l%16, k 32 ks + 8 (l/16)
    const int bf_base = l16 * PITCH + 8 * g4;

    // stage s's k-steps in the packed x: its zero-point part first, then x
    auto load_a = [&](int s, int ks, u32x4 (&A)[MT][4]) __attribute__((always_inline)) {
        const int xs = s < ncode ? s + a.sz : s - ncode;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            A[mt][ks] = __builtin_amdgcn_raw_buffer_load_b128(xr, xv[mt] + (uint32_t)(xs * 4 + ks) * 1024u, 0, 0);
    };
    auto load_b = [&](const __bf16* src, int nt, int ks) __attribute__((always_inline)) {
        return *reinterpret_cast<const bf16x8*>(src + bf_base + nt * 16 * PITCH + ks * 32);
    };
    f32x4 out[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) out[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 A[MT][4];
    bf16x8 b0, b1;                             // the next n-tile's two B fragments
    // Sums of the previous n-tile and their scale, folded into `out` while
    // the MFMAs of the current one run (the previous n-tile is always the
    // last one, NT-1, when the current one is the first of a sub-block).
    f32x4 accp[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) accp[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float scp = 0.f;

    // One stage.  ZS (zero-point stages): the MFMAs accumulate into the
    // outputs.  Code stages: per 64-wide sub-block j and n-tile, a fresh
    // two-MFMA sum per m-tile, folded in as out = fma(scale, sum, out) one
    // n-tile later.  The next n-tile's B fragments are read before the
    // current MFMAs; the last n-tile of a stage reads the next stage's first
    // ones after the stage barrier (the producers finish stage s+1's tile
    // before it, and no wave reads this stage's tile after it).
    auto stage = [&]<bool ZS>(int s, const __bf16* cur, const float* sc, const __bf16* nxt)
        __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            float scv[NT];
            if constexpr (!ZS) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) scv[nt] = sc[j * BN + nt * 16 + l16];
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const bf16x8 f0 = b0, f1 = b1;
                if (nt < NT - 1) {
                    b0 = load_b(cur, nt + 1, 2 * j);
                    b1 = load_b(cur, nt + 1, 2 * j + 1);
                } else if (j == 0) {
                    b0 = load_b(cur, 0, 2);
                    b1 = load_b(cur, 0, 3);
                } else {
                    __syncthreads();
                    b0 = load_b(nxt, 0, 0);
                    b1 = load_b(nxt, 0, 1);
                }
                const int pnt = nt == 0 ? NT - 1 : nt - 1;
                f32x4 acc[MT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const bf16x8 a0 = __builtin_bit_cast(bf16x8, A[mt][2 * j]);
                    if constexpr (ZS) {
                        out[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, f0, out[mt][nt], 0, 0, 0);
                    } else {
                        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, f0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            out[mt][pnt][i] = __builtin_fmaf(scp, accp[mt][i], out[mt][pnt][i]);
                    }
                }
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const bf16x8 a1 = __builtin_bit_cast(bf16x8, A[mt][2 * j + 1]);
                    if constexpr (ZS)
                        out[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, f1, out[mt][nt], 0, 0, 0);
                    else
                        accp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, f1, acc[mt], 0, 0, 0);
                }
                if constexpr (!ZS) {
                    scp = scv[nt];
                    // one n-tile per scheduling region: the B reads first,
                    // then each MFMA followed by two of the previous
                    // n-tile's folds, which the wave issues while the
                    // matrix core runs (in-order issue: a run of MFMAs
                    // would hold the folds back until the core drains)
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);      // DS reads
#pragma unroll
                    for (int i = 0; i < 2 * MT; i++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
                    }
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    // zero-point stages: the next n-tile's B reads ahead of
                    // this one's MFMAs too (left to the scheduler, they sank
                    // behind them, into one register set, and every n-tile
                    // waited for its reads)
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);      // DS reads
                    __builtin_amdgcn_sched_group_barrier(0x008, 2 * MT, 0); // MFMA
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            // this sub-block's A fragments are refilled with stage s+1's
            load_a(s + 1, 2 * j, A);
            load_a(s + 1, 2 * j + 1, A);
        }
    };
#pragma unroll
    for (int ks = 0; ks < 4; ks++) load_a(0, ks, A);
    __syncthreads();
    b0 = load_b(lds, 0, 0);
    b1 = load_b(lds, 0, 1);
    int s = 0;
    for (; s < ncode; s += 2) {
        stage.template operator()<false>(s, lds, scl, lds + BUF);
        stage.template operator()<false>(s + 1, lds + BUF, scl + SCN, lds);
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            out[mt][NT - 1][i] = __builtin_fmaf(scp, accp[mt][i], out[mt][NT - 1][i]);
    for (; s < a.s; s += 2) {
        stage.template operator()<true>(s, lds, scl, lds + BUF);
        stage.template operator()<true>(s + 1, lds + BUF, scl + SCN, lds);
    }

    // Epilogue: each wave stages its 64 x 112 fp32 tile in LDS (once every
    // wave is past its last B read) and writes whole row pieces with 16-byte
    // stores, instead of 4-byte stores scattered over four rows each.
    __syncthreads();
    float* ep = reinterpret_cast<float*>(lds_raw) + wave * 64 * EP_PITCH;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) ep[(mt * 16 + 4 * g4 + i) * EP_PITCH + nt * 16 + l16] = out[mt][nt][i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool vec = (a.n & 3) == 0;               // rows 16-byte aligned
#pragma unroll 4
    for (int c = lane; c < 64 * (BN / 4); c += 64) {
        const int r = c / (BN / 4), q = c - r * (BN / 4);
        const int m = m0 + r, n = n0 + 4 * q;
        if (m >= a.m || n >= a.n) continue;
        const f32x4 v = *reinterpret_cast<const f32x4*>(ep + r * EP_PITCH + 4 * q);
        float* dst = a.y + (size_t)m * a.n + n;
        if (vec) {
            *reinterpret_cast<f32x4*>(dst) = v;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (n + e < a.n) dst[e] = v[e];
        }
    }
}

template <auto K>
void launch(dim3 g, dim3 b, hipStream_t s, const PrefillArgs& a) {
    hipEvent_t e0, e1;
    if (qk_timing_pair(&e0, &e1))
        hipExtLaunchKernelGGL(K, g, b, 0, s, e0, e1, 0, a);
    else
        hipLaunchKernelGGL(K, g, b, 0, s, a);
}

// Stage counts of a (cols, block size) prefill: zero-point stages (8 k
// positions per block, rounded up to an even stage count) and code stages
// (cols rounded up to an even stage count).
struct Stages { int sz, sc; };
Stages stages_of(int cols, int bs) {
    const int nb = (cols + bs - 1) / bs;
    return {2 * ((ZK * nb + 2 * SK - 1) / (2 * SK)), 2 * ((cols + 2 * SK - 1) / (2 * SK))};
}

}  // namespace

// Packed-x layout of qk_prefill_4bit: ceil(m/16) row groups of 4 (sz + sc)
// k-steps of 1 KB.
extern "C" size_t qk_prefill_ws_bytes(int m, int cols, int bs) {
    if (m <= 0 || cols <= 0 || bs <= 0) return 0;
    const Stages st = stages_of(cols, bs);
    return (size_t)((m + 15) / 16) * (size_t)(4 * (st.sz + st.sc)) * 1024;
}

// x bf16 [m][cols] -> the packed activations (qk_prefill_ws_bytes) a
// prefill of any 4-bit tensor with these cols and block size reads.
extern "C" int qk_prefill_pack(const uint16_t* d_x_bf16, int m, int cols, int bs, void* d_ws, hipStream_t s) {
    if (m <= 0) return 0;
    if (cols < 32 || cols % 8 || !(bs == 64 || bs == 128 || bs == 256)) return -2;
    const Stages st = stages_of(cols, bs);
    const int ksp_total = 4 * (st.sz + st.sc), kz = 4 * st.sz, nb = (cols + bs - 1) / bs;
    if ((uint64_t)((m + BM - 1) / BM) * (BM / 16) * ksp_total * 1024 + 8 * 1024 >= (1ull << 32)) return -2;
    hipLaunchKernelGGL(xpack_kernel, dim3((ksp_total - kz) / 8, (m + 15) / 16), dim3(256), 0, s,
                       d_x_bf16, static_cast<u32x4*>(d_ws), m, cols, ksp_total, kz, bs, nb);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

namespace {
// 0 when qk_prefill_gemm takes (t, m): a 4-bit tensor without outliers and
// 32-bit byte offsets inside the weight payload (including the columns of
// the last tile past the end, and the zero-point stages' block reads up to
// 16 sz blocks a row) and the packed activations (including the row groups
// of the last tile and the prefetch past the last stage); else -2.
int gemm_check(const qsf_hip_tensor* t, int m) {
    if (t->fmt != QK_FMT_4 || t->n_outliers) return -2;
    if (m <= 0 || t->rows <= 0) return 0;
    if (t->cols < 32 || t->cols % 8) return -2;
    if (t->bs == 256 && t->frag) return -2;
    const int bb = 4 + t->bs / 2;
    const Stages st = stages_of(t->cols, t->bs);
    const int ksp_total = 4 * (st.sz + st.sc);
    const uint64_t row_bytes = (uint64_t)t->nb * bb;
    if ((uint64_t)(t->rows + BN) * row_bytes + (uint64_t)16 * st.sz * bb >= (1ull << 32) ||
        (uint64_t)((m + BM - 1) / BM) * (BM / 16) * ksp_total * 1024 + 8 * 1024 >= (1ull << 32))
        return -2;
    if (t->frag && (uint64_t)((t->rows + BN) / 16 + 1) * t->frag_nq * 64 * bb >= (1ull << 32)) return -2;
    return 0;
}
}  // namespace

// The GEMM over activations qk_prefill_pack wrote for m tokens.
extern "C" int qk_prefill_gemm(const qsf_hip_tensor* t, const void* d_ws, int m, float* d_y, hipStream_t s) {
    if (gemm_check(t, m)) return -2;
    if (m <= 0 || t->rows <= 0) return 0;
    const int bb = 4 + t->bs / 2;
    const Stages st = stages_of(t->cols, t->bs);
    const size_t xp_bytes = qk_prefill_ws_bytes(m, t->cols, t->bs);
    const int tiles_m = (m + BM - 1) / BM;
    const uint64_t row_bytes = (uint64_t)t->nb * bb;
    const int tiles_n = (t->rows + BN - 1) / BN;
    const bool ragged = t->cols % (2 * SK) != 0;
    const uint64_t w_bytes = t->frag ? (uint64_t)qk_frag_bytes(t->rows, t->nb, bb) : (uint64_t)t->rows * row_bytes;
    PrefillArgs a = {t->d_blocks, static_cast<const u32x4*>(d_ws), d_y, m, t->rows, t->cols, t->nb,
                     tiles_n, st.sz, st.sz + st.sc, 16 * st.sz <= ZP_MAX ? 16 * st.sz : 0,
                     (uint32_t)w_bytes, (uint32_t)xp_bytes, t->frag_nq};
    const dim3 grid(tiles_n * tiles_m), block(512);
#define QK_PREFILL_CASE(B, F, P)                                                \
    if (ragged) launch<prefill_kernel<B, true, F, P>>(grid, block, s, a);       \
    else launch<prefill_kernel<B, false, F, P>>(grid, block, s, a);
    switch (t->bs) {
    case 64:
        if (t->frag) { QK_PREFILL_CASE(64, true, false) } else { QK_PREFILL_CASE(64, false, true) }
        break;
    case 128:
        if (t->frag) { QK_PREFILL_CASE(128, true, false) } else { QK_PREFILL_CASE(128, false, true) }
        break;
    case 256:
        QK_PREFILL_CASE(256, false, true)
        break;
    default: return -2;
    }
#undef QK_PREFILL_CASE
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_prefill_4bit(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                               float* d_y, void* d_ws, hipStream_t s) {
    if (gemm_check(t, m)) return -2;
    if (m <= 0 || t->rows <= 0) return 0;
    const int r = qk_prefill_pack(d_x_bf16, m, t->cols, t->bs, d_ws, s);
    return r ? r : qk_prefill_gemm(t, d_ws, m, d_y, s);
}

// ---- allocation-free form -------------------------------------------------
// The packed activations live in one file-scope device array per GPU
// (QK_PREFILL_SCRATCH_BYTES; every GPU the library runs on holds it until the
// process ends).  In host code `scratch` names a host-side stand-in, so its
// device address is looked up once per device (with that device current)
// and only that address is ever passed to kernels.  xpack_kernel rewrites
// every byte the GEMM reads from it, so nothing needs clearing between
// calls; calls that overlap on one GPU race on it.
static __device__ __align__(256) uint8_t scratch[QK_PREFILL_SCRATCH_BYTES];
static void* g_scratch[QK_MAX_DEVICES];

extern "C" int qk_prefill_scratch_init(void) {
    int d = -1;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= QK_MAX_DEVICES) return -1;
    if (g_scratch[d]) return 0;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return -1;
    g_scratch[d] = p;
    return 0;
}

extern "C" int qk_prefill_4bit_noalloc(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                                       float* d_y, hipStream_t s) {
    if (qk_prefill_ws_bytes(m, t->cols, t->bs) > (size_t)QK_PREFILL_SCRATCH_BYTES) return -3;
    int d = -1;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= QK_MAX_DEVICES) return -1;
    if (!g_scratch[d] && qk_prefill_scratch_init() != 0) return -1;
    return qk_prefill_4bit(t, d_x_bf16, m, d_y, g_scratch[d], s);
}
