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
// Tiling.  One 256-thread workgroup per 256 (m) x 112 (n) tile of Y; at
// config-4 shape (M 512, N 14336) that is exactly one workgroup per CU.  Wave
// w owns rows 64w..64w+63 and all 112 columns: 4 x 7 MFMA tiles, 112 fp32
// accumulators per lane.  K advances in stages of 128 codes (4 MFMA
// k-steps):
//  * B (weights): the workgroup dequantises the stage's 112 x 128 codes once
//    into an LDS tile (bf16 [112][128 + 8 pad], two buffers), 7 items of 8
//    codes per thread, interleaved with the previous stage's MFMAs;
//  * A (activations): each wave's rows are private, so its fragments come
//    straight from global memory into registers, loaded two stages ahead.
// One barrier per stage.  All loads are issued unconditionally (clamped
// addresses) so the compiler's wait counts stay exact.
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
constexpr int NR = BN * (SK / 8) / 256;   // dequant items (8 codes) per thread per stage

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
// scattered 16-byte pieces.
__global__ __launch_bounds__(256) void xpack_kernel(const uint16_t* __restrict__ x, u32x4* xp,
                                                   int m, int k, int ksp, uint32_t chunks) {
    for (uint32_t c = blockIdx.x * 256u + threadIdx.x; c < chunks; c += gridDim.x * 256u) {
        const uint32_t l = c & 63u, f = c >> 6, kk = f % (uint32_t)ksp, g = f / (uint32_t)ksp;
        const int row = (int)(g * 16 + (l & 15u)), col = (int)(kk * 32 + 8 * (l >> 4));
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < m && col < k) v = *reinterpret_cast<const u32x4*>(x + (size_t)row * k + col);
        xp[c] = v;
    }
}

// Raw buffer descriptor (gfx9 family word 3): loads at offsets >= `bytes`
// return zero, so clamped-free prefetch past a tensor's end is safe.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Workgroup id -> (m tile, n tile).  Workgroups are dealt to the 8 XCDs
// round-robin; this numbering hands each XCD a contiguous run of tiles, so
// the XCDs that share an m tile share its activation rows in their own L2.
__device__ __forceinline__ void tile_of(int id, int nwg, int tiles_n, int& tm, int& tn) {
    const int q = nwg >> 3, r = nwg & 7, xcd = id & 7, slot = id >> 3;
    const int t = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
    tm = t / tiles_n;
    tn = t - tm * tiles_n;
}

// RAGGED: k is not a multiple of 2 SK, so stages reach past the last column;
// their B items and A fragments are zeroed.
template <int BS, bool RAGGED>
__global__ __launch_bounds__(512) void prefill_kernel(PrefillArgs a) {
    constexpr int BB = 4 + BS / 2;             // block bytes
    constexpr int BUF = BN * PITCH;            // bf16 per B buffer
    __shared__ __align__(16) __bf16 lds[2 * BUF];

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    int tm, tn;
    tile_of(blockIdx.x, gridDim.x, a.tiles_n, tm, tn);
    const int n0 = tn * BN;
    const int S = 2 * a.pairs;                 // stages

    if (wave >= 4) {
        // ---- producer waves: dequantise stage s+1's B tile during stage s.
        // Thread p converts dword d = p%16 of the stage's 16 code dwords
        // (128 codes) of columns p/16 + 16 r, r < NR.  Byte offsets in a
        // row: the lane part is fixed, the stage part uniform; columns past
        // n read zeros.
        const uint32_t row_bytes = (uint32_t)a.nb * BB;
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes);
        const int p = t - 256, d = p & 15, c0 = p >> 4;
        const uint32_t lane_meta = BS <= SK ? (uint32_t)(8 * d / BS) * BB : 0u;
        const uint32_t lane_code = lane_meta + 4 + 4 * (uint32_t)((8 * d % BS) / 8);
        const uint32_t wv = (uint32_t)(n0 + c0) * row_bytes;
        const int it_base = c0 * PITCH + 8 * d;
        auto load_codes = [&](int s, uint32_t (&code)[NR], uint32_t (&meta)[NR]) {
            const uint32_t sm = BS <= SK ? (uint32_t)s * (SK / BS) * BB : (uint32_t)(s / (BS / SK)) * BB;
            const uint32_t sc = BS <= SK ? sm : sm + (uint32_t)(s % (BS / SK)) * (SK / 2);
            const uint32_t mo = wv + lane_meta + sm, co = wv + lane_code + sc;
#pragma unroll
            for (int r = 0; r < NR; r++) {
                meta[r] = __builtin_amdgcn_raw_buffer_load_b32(wr, mo + 16 * r * row_bytes, 0, 0);
                code[r] = __builtin_amdgcn_raw_buffer_load_b32(wr, co + 16 * r * row_bytes, 0, 0);
            }
        };
        auto dequant = [&](int s, const uint32_t (&code)[NR], const uint32_t (&meta)[NR], __bf16* buf) {
            const bool zero = RAGGED && s * SK + 8 * d >= a.k;
#pragma unroll
            for (int r = 0; r < NR; r++) {
                bf16x8 v = dequant8(code[r], qsf::f16_lo(meta[r]), qsf::f16_hi(meta[r]));
                if (zero) v = bf16x8{};
                *reinterpret_cast<bf16x8*>(buf + it_base + 16 * r * PITCH) = v;
            }
        };
        // codes double-buffered two stages ahead
        uint32_t ca[NR], ma[NR], cb[NR], mb[NR];
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

#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int n = n0 + nt * 16 + l16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + mt * 16 + 4 * g4 + i;
                if (m < a.m && n < a.n) a.y[(size_t)m * a.n + n] = acc[mt][nt][i];
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
    {
        const uint32_t chunks = (uint32_t)(xp_bytes / 16);
        const int blocks = (int)((chunks + 255) / 256 < 4096 ? (chunks + 255) / 256 : 4096);
        hipLaunchKernelGGL(xpack_kernel, dim3(blocks), dim3(256), 0, s, d_x_bf16,
                           static_cast<u32x4*>(d_ws), m, t->cols, packed_ksp(t->cols), chunks);
    }
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
