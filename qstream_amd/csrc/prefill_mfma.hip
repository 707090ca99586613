// prefill_mfma.hip - batched prefill through the 4-bit QSF format on gfx950
// MFMA: Y[m][n] = sum_k float(x_bf16[m][k]) * w[n][k], M tokens at once.
//
// There is no reference kernel: the engine runs one matvec per token
// (src/engine.c:1289-1295), so the specification is M independent
// src/kernels_scalar.c:64-85 matvecs on float(bf16(x_m)).  Here the weights
// are dequantised in registers, w = s*q + z (exact in fp32: s*q has at most
// 15 significant bits), rounded to bf16 (round-to-nearest-even,
// v_cvt_pk_bf16_f32) and contracted with v_mfma_f32_16x16x32_bf16 in fp32.
// The one rounding beyond fp32 accumulation is that of w to bf16.
//
// Tiling.  One 512-thread workgroup per 256 (m) x 112 (n) tile of Y; at
// config-4 shape (M 512, N 14336) that is exactly one workgroup per CU.  K
// advances in stages of 128 codes (4 MFMA k-steps).  The waves split by role,
// one of each per SIMD, so dequantisation (VALU) and MFMAs overlap in the
// hardware rather than in one instruction stream:
//  * 4 producer waves dequantise stage s+1's 112 x 128 codes into a bf16 LDS
//    tile ([112][128 + 8 pad], two buffers) while stage s is contracted;
//    codes are loaded two stages ahead;
//  * 4 consumer waves each own 64 rows x 112 columns (4 x 7 MFMA tiles, 112
//    fp32 accumulators per lane).  A fragments come from x repacked into
//    fragment order (xpack_kernel: one contiguous 1 KB load per fragment),
//    one stage ahead in registers; B fragments come from LDS one k-step
//    ahead.
// One barrier per stage.  Loads go through raw buffer descriptors: offsets
// past a tensor read zeros, so prefetches past the end need no clamps and
// all loads are issued unconditionally (exact compiler wait counts).
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
constexpr int EP_PITCH = BN + 4;       // LDS row pitch of the output staging tile, fp32
constexpr int EP_FLOATS = 4 * 64 * EP_PITCH;

// Eight codes (one dword, low nibble = even code) -> bf16(s*q + z) x 8.
__device__ __forceinline__ bf16x8 dequant8(uint32_t w, float s, float z) {
    // (byte extracts to float become v_cvt_f32_ubyte0..3)
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const float q[8] = {(float)(lo & 0xFFu),         (float)(hi & 0xFFu),
                        (float)((lo >> 8) & 0xFFu),  (float)((hi >> 8) & 0xFFu),
                        (float)((lo >> 16) & 0xFFu), (float)((hi >> 16) & 0xFFu),
                        (float)(lo >> 24),           (float)(hi >> 24)};
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const f32x2 v = {fmaf(s, q[j], z), fmaf(s, q[j + 1], z)};
        const bf16x2 b = __builtin_convertvector(v, bf16x2);
        r[j] = b[0];
        r[j + 1] = b[1];
    }
    return r;
}

// The same with one shift and one and-or per pair of codes: code q becomes
// the fp16 value 1 + q/16 (q in mantissa bits 6..9 of 1.0), and
// fma(16 s, 1 + q/16, c) with c = z - 16 s equals fp32(s q + z) exactly
// whenever c is exact in fp32 (the caller checks that per block).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// `one` is 0x3C003C00 (fp16 1.0 twice) held in a VGPR by the caller: with
// the mask in an SGPR the and-or is one v_and_or_b32 (a VOP3 reads at most
// one scalar operand here, and two literals would split it in two).
__device__ __forceinline__ bf16x8 dequant8_m16(uint32_t w, float s16, float c, uint32_t one) {
    const uint32_t h[4] = {((w << 6) & 0x03C003C0u) | one,   // codes 0, 4
                           ((w << 2) & 0x03C003C0u) | one,   // codes 1, 5
                           ((w >> 2) & 0x03C003C0u) | one,   // codes 2, 6
                           ((w >> 6) & 0x03C003C0u) | one};  // codes 3, 7
    float x[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const f16x2 p = __builtin_bit_cast(f16x2, h[j]);
        x[j] = (float)p[0];
        x[j + 4] = (float)p[1];
    }
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const f32x2 v = {fmaf(s16, x[j], c), fmaf(s16, x[j + 1], c)};
        const bf16x2 b = __builtin_convertvector(v, bf16x2);
        r[j] = b[0];
        r[j + 1] = b[1];
    }
    return r;
}

struct PrefillArgs {
    const uint8_t* w;        // QSF 4-bit blocks, rows n, row stride nb*BB
    const u32x4* xp;         // x in A-fragment order (xpack_kernel)
    float* y;                // fp32 [m][n]
    int m, n, k, nb;
    int tiles_n, pairs;      // n tiles; stage pairs (ceil(k / 2 SK))
    uint32_t w_bytes, xp_bytes;
};

// x bf16 [m][k] -> A-fragment order: for each group of 16 rows and each
// 32-wide k-step kk < ksp, 64 chunks of 16 bytes, chunk l holding row
// 16 g + l%16, columns 32 kk + 8 (l/16)..+7 (zero past m or k).  The GEMM
// then loads each fragment as one contiguous 1 KB read instead of 64
// scattered 16-byte pieces.  One workgroup per (row group, 8 k-steps): the
// 16 x 256 tile is read row-contiguously into LDS and written back in
// fragment order, both coalesced.
constexpr int XP_PITCH = 256 + 8;      // LDS row pitch of the pack tile, bf16
__global__ __launch_bounds__(256) void xpack_kernel(const uint16_t* __restrict__ x, u32x4* xp,
                                                   int m, int k, int ksp) {
    __shared__ __align__(16) uint16_t tile[16 * XP_PITCH];
    const int g = blockIdx.y, kk0 = blockIdx.x * 8, t = threadIdx.x;
    const int c = t & 31;                      // 16-byte chunk of a 256-wide row piece
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int r = (t >> 5) + 8 * h, row = g * 16 + r, col = kk0 * 32 + 8 * c;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < m && col < k) v = *reinterpret_cast<const u32x4*>(x + (size_t)row * k + col);
        *reinterpret_cast<u32x4*>(&tile[r * XP_PITCH + 8 * c]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int j = t + 256 * h, kk = j >> 6, l = j & 63;
        xp[((size_t)g * ksp + kk0 + kk) * 64 + l] =
            *reinterpret_cast<const u32x4*>(&tile[(l & 15) * XP_PITCH + kk * 32 + 8 * (l >> 4)]);
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
// XCD and the weight tile they share is fetched into that XCD's L2 once
// (measured: 72 MB fetched a launch at config 4 instead of 91 MB).
__device__ __forceinline__ void tile_of(int id, int nwg, int tiles_n, int& tm, int& tn) {
    const int q = nwg >> 3, r = nwg & 7, xcd = id & 7, slot = id >> 3;
    const int t = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
    const int tiles_m = nwg / tiles_n;
    tn = t / tiles_m;
    tm = t - tn * tiles_m;
}

// RAGGED: k is not a multiple of 2 SK, so stages reach past the last column;
// their B items and A fragments are zeroed.
template <int BS, bool RAGGED>
__global__ __launch_bounds__(512) void prefill_kernel(PrefillArgs a) {
    constexpr int BB = 4 + BS / 2;             // block bytes
    constexpr int BUF = BN * PITCH;            // bf16 per B buffer
    // two B buffers during the main loop; the output staging tile after it
    __shared__ __align__(16) __bf16 lds[2 * BUF > EP_FLOATS * 2 ? 2 * BUF : EP_FLOATS * 2];

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, a.tiles_n, tm, tn);
    const int n0 = tn * BN;
    const int S = 2 * a.pairs;                 // stages

    if (wave >= 4) {
        // ---- producer waves: dequantise stage s+1's B tile during stage s.
        // Item p < 2 BN: column p/2, codes 64 (p%2)..+63 of the stage, read
        // as one meta dword and two 16-byte loads; each becomes 8 LDS
        // writes of 8 bf16.  Byte offsets in a row: the lane part is fixed,
        // the stage part uniform; columns past n read zeros.
        const uint32_t row_bytes = (uint32_t)a.nb * BB;
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);
        const int p = t - 256, col = p >> 1, h = p & 1;
        const bool active = p < 2 * BN;
        // 64 codes (p%2) of the stage: block offset and the codes' offset in it
        const uint32_t lane_meta = BS == 64 ? (uint32_t)h * BB : 0u;
        const uint32_t lane_code = lane_meta + 4 + (BS == 64 ? 0u : (uint32_t)h * 32);
        const uint32_t wv = (uint32_t)(n0 + col) * row_bytes;
        const int it_base = col * PITCH + 64 * h;
        uint32_t one = 0x3C003C00u;
        asm volatile("" : "+v"(one));                // kept in a VGPR (see dequant8_m16)
        auto load_codes = [&](int s, u32x4 (&code)[2], uint32_t& meta) __attribute__((always_inline)) {
            const uint32_t sm = BS <= SK ? (uint32_t)s * (SK / BS) * BB : (uint32_t)(s / (BS / SK)) * BB;
            const uint32_t sc = BS <= SK ? sm : sm + (uint32_t)(s % (BS / SK)) * (SK / 2);
            meta = __builtin_amdgcn_raw_buffer_load_b32(wr, wv + lane_meta + sm, 0, 0);
            code[0] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + lane_code + sc, 0, 0);
            code[1] = __builtin_amdgcn_raw_buffer_load_b128(wr, wv + lane_code + sc + 16, 0, 0);
        };
        auto dequant = [&](int s, const u32x4 (&code)[2], uint32_t meta, __bf16* buf) __attribute__((always_inline)) {
            if (!active) return;
            const float sc = qsf::f16_lo(meta), zp = qsf::f16_hi(meta);
            // z - 16 s is exact in fp64 (fp16 operands); the short form
            // applies when it is also exact (and finite) in fp32
            const double cd = (double)zp - 16.0 * (double)sc;
            const float c = (float)cd;
            if (__builtin_isfinite(cd) && (double)c == cd) {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    bf16x8 v = dequant8_m16(code[j >> 2][j & 3], 16.0f * sc, c, one);
                    if (RAGGED && s * SK + 64 * h + 8 * j >= a.k) v = bf16x8{};
                    *reinterpret_cast<bf16x8*>(buf + it_base + 8 * j) = v;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    bf16x8 v = dequant8(code[j >> 2][j & 3], sc, zp);
                    if (RAGGED && s * SK + 64 * h + 8 * j >= a.k) v = bf16x8{};
                    *reinterpret_cast<bf16x8*>(buf + it_base + 8 * j) = v;
                }
            }
        };
        // codes double-buffered two stages ahead
        u32x4 ca[2], cb[2];
        uint32_t ma, mb;
        load_codes(0, ca, ma);
        load_codes(1, cb, mb);
        dequant(0, ca, ma, lds);
        load_codes(2, ca, ma);
        __syncthreads();
        for (int s = 0; s < S; s += 2) {
            dequant(s + 1, cb, mb, lds + BUF);
            load_codes(s + 3, cb, mb);
            __syncthreads();
            dequant(s + 2, ca, ma, lds);
            load_codes(s + 4, ca, ma);
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
    const uint32_t ksp = 8u * (uint32_t)a.pairs;
    uint32_t xv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) xv[mt] = ((uint32_t)(m0 / 16 + mt) * ksp * 64u + lane) * 16u;
    // B fragment of n-tile nt, k-step ks: column 16 nt + l%16, k 32 ks + 8 (l/16)
    const int bf_base = l16 * PITCH + 8 * g4;

    auto load_a = [&](int s, int ks, u32x4 (&A)[MT][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            A[mt][ks] = __builtin_amdgcn_raw_buffer_load_b128(xr, xv[mt] + (uint32_t)(s * 4 + ks) * 1024u, 0, 0);
    };
    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 A[MT][4];
    bf16x8 bf[NT];
    // k-step ks of a stage: for each n-tile, its 4 MFMAs, then that B
    // fragment register is refilled with the next k-step's (from `src`,
    // k-step kn); then the A fragments used are refilled with stage s+1's.
    auto kstep = [&](int s, int ks, const __bf16* src, int kn) __attribute__((always_inline)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, A[mt][ks]), bf[nt], acc[mt][nt], 0, 0, 0);
            bf[nt] = *reinterpret_cast<const bf16x8*>(src + bf_base + nt * 16 * PITCH + kn * 32);
        }
        load_a(s + 1, ks, A);
        // keep the machine scheduler from sliding these loads into the next
        // k-step
        __builtin_amdgcn_sched_barrier(0);
    };
    // The producers finish stage s+1's tile before the barrier inside stage
    // s, whose last k-step already reads its first fragments.
    auto stage = [&](int s, const __bf16* cur, const __bf16* nxt) __attribute__((always_inline)) {
        kstep(s, 0, cur, 1);
        kstep(s, 1, cur, 2);
        kstep(s, 2, cur, 3);
        __syncthreads();
        kstep(s, 3, nxt, 0);
        // the next stage's first fragments are loaded here, not re-read in
        // front of their MFMAs (which would expose the LDS latency per tile)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) asm volatile("" : "+v"(bf[nt]));
    };
#pragma unroll
    for (int ks = 0; ks < 4; ks++) load_a(0, ks, A);
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
        bf[nt] = *reinterpret_cast<const bf16x8*>(lds + bf_base + nt * 16 * PITCH);
    for (int s = 0; s < S; s += 2) {
        stage(s, lds, lds + BUF);
        stage(s + 1, lds + BUF, lds);
    }

    // Epilogue: each wave stages its 64 x 112 fp32 tile in LDS (once every
    // wave is past its last B read) and writes whole row pieces with 16-byte
    // stores, instead of 4-byte stores scattered over four rows each.
    __syncthreads();
    float* ep = reinterpret_cast<float*>(lds) + wave * 64 * EP_PITCH;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) ep[(mt * 16 + 4 * g4 + i) * EP_PITCH + nt * 16 + l16] = acc[mt][nt][i];
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

}  // namespace

// Packed-x layout of qk_prefill_4bit: ceil(m/16) row groups of ksp k-steps.
static int packed_ksp(int cols) { return 8 * ((cols + 2 * SK - 1) / (2 * SK)); }

extern "C" size_t qk_prefill_ws_bytes(int m, int cols) {
    if (m <= 0 || cols <= 0) return 0;
    return (size_t)((m + 15) / 16) * (size_t)packed_ksp(cols) * 1024;
}

extern "C" int qk_prefill_4bit(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                               float* d_y, void* d_ws, hipStream_t s) {
    if (t->fmt != QK_FMT_4 || t->n_outliers) return -2;
    if (m <= 0 || t->rows <= 0) return 0;
    if (t->cols < 32 || t->cols % 8) return -2;
    const int bb = 4 + t->bs / 2;
    const size_t xp_bytes = qk_prefill_ws_bytes(m, t->cols);
    // 32-bit byte offsets inside the weight payload (including the columns
    // of the last tile past the end) and the packed activations (including
    // the row groups of the last tile and the prefetch past the last stage)
    const int tiles_m = (m + BM - 1) / BM;
    if ((uint64_t)(t->rows + BN) * (uint64_t)t->nb * bb >= (1ull << 32) ||
        (uint64_t)tiles_m * (BM / 16) * packed_ksp(t->cols) * 1024 + 8 * 1024 >= (1ull << 32))
        return -2;
    const int tiles_n = (t->rows + BN - 1) / BN;
    const int pairs = (t->cols + 2 * SK - 1) / (2 * SK);
    const bool ragged = t->cols % (2 * SK) != 0;
    hipLaunchKernelGGL(xpack_kernel, dim3(packed_ksp(t->cols) / 8, (m + 15) / 16), dim3(256), 0, s,
                       d_x_bf16, static_cast<u32x4*>(d_ws), m, t->cols, packed_ksp(t->cols));
    PrefillArgs a = {t->d_blocks, static_cast<const u32x4*>(d_ws), d_y, m, t->rows, t->cols, t->nb,
                     tiles_n, pairs, (uint32_t)((uint64_t)t->rows * t->nb * bb), (uint32_t)xp_bytes};
    const dim3 grid(tiles_n * tiles_m), block(512);
#define QK_PREFILL_CASE(B)                                                   \
    case B:                                                                  \
        if (ragged) launch<prefill_kernel<B, true>>(grid, block, s, a);      \
        else launch<prefill_kernel<B, false>>(grid, block, s, a);            \
        break;
    switch (t->bs) {
        QK_PREFILL_CASE(64)
        QK_PREFILL_CASE(128)
        QK_PREFILL_CASE(256)
    default: return -2;
    }
#undef QK_PREFILL_CASE
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
