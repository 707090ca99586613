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
// Tiling.  A 256-thread workgroup computes a 128 (m) x 64 (n) tile of Y over
// K in steps of one quant block (BS codes, BS/32 MFMA k-steps); wave w owns
// 64 m x 32 n = 4 x 2 MFMA tiles.  The x tile of the next block is loaded
// into registers while the current one is used from LDS (two LDS buffers,
// rows padded to 144 bytes against bank conflicts).  Each lane dequantises the
// B fragments it feeds to the MFMA straight from the packed block: one dword
// (8 codes) per n-tile and k-step, plus the block's scale/zero dword, loaded
// one block ahead.
//
// MFMA 16x16x32 operand layout (lane l): A row l%16, k 8*(l/16)..+7;
// B column l%16, same k; C column l%16, rows 4*(l/16)..+3.
#include "qsf_device.h"
#include "qsf_hip_internal.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 64;       // workgroup tile
constexpr int KB_PITCH = 72;           // LDS row pitch in bf16 (64 + 8 pad)

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
    const uint16_t* x;       // bf16 [m][k]
    float* y;                // fp32 [m][n]
    int m, n, k, nb;
};

template <int BS>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
    constexpr int BB = 4 + BS / 2;             // block bytes
    constexpr int KS = BS / 32;                // MFMA k-steps per block
    constexpr int KC = BS / 64 > 0 ? BS / 64 : 1;   // 64-wide x chunks per block
    __shared__ __align__(16) __bf16 xs[2][BM][KB_PITCH];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const uint32_t row_bytes = (uint32_t)a.nb * BB;
    const int l16 = lane & 15, g4 = lane >> 4;

    // this lane's two weight rows (clamped; stores are guarded)
    const uint8_t* wrow[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++)
        wrow[nt] = a.w + (size_t)min(n0 + wn * 32 + nt * 16 + l16, a.n - 1) * row_bytes;

    // x tile loader: thread t -> row t/2, 32 bf16 at column 32*(t%2) of a
    // 64-wide chunk; columns past k read as zero (their codes then add 0)
    const int xr = threadIdx.x >> 1, xc = (threadIdx.x & 1) * 32;
    const int xm = min(m0 + xr, a.m - 1);
    auto load_x = [&](int kb, int c, u32x4 (&v)[4]) {
        const int col = kb * BS + c * 64 + xc;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int cc = col + 8 * i;
            if (cc + 8 <= a.k) {
                v[i] = *reinterpret_cast<const u32x4*>(a.x + (size_t)xm * a.k + cc);
            } else {
                uint32_t e[4];
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const int c0 = cc + 2 * h;
                    const uint32_t lo = c0 < a.k ? a.x[(size_t)xm * a.k + c0] : 0u;
                    const uint32_t hi = c0 + 1 < a.k ? a.x[(size_t)xm * a.k + c0 + 1] : 0u;
                    e[h] = lo | hi << 16;
                }
                v[i] = u32x4{e[0], e[1], e[2], e[3]};
            }
        }
    };
    auto store_x = [&](int buf, const u32x4 (&v)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<u32x4*>(&xs[buf][xr][xc + 8 * i]) = v[i];
    };
    // weight dwords of block kb: meta per n-tile, codes per (n-tile, k-step)
    auto load_w = [&](int kb, uint32_t (&meta)[2], uint32_t (&code)[2][KS]) {
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(wrow[nt] + (uint32_t)kb * BB);
            meta[nt] = p[0];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) code[nt][ks] = p[1 + ks * 4 + g4];
        }
    };

    f32x4 acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    uint32_t meta[2], code[2][KS];
    load_w(0, meta, code);
    for (int kb = 0; kb < a.nb; kb++) {
        uint32_t meta_n[2], code_n[2][KS];
        load_w(min(kb + 1, a.nb - 1), meta_n, code_n);     // next block (last: again)
        float s[2], z[2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            s[nt] = qsf::f16_lo(meta[nt]);
            z[nt] = qsf::f16_hi(meta[nt]);
        }
#pragma unroll
        for (int c = 0; c < KC; c++) {
            // x chunk c of block kb into LDS (64 k wide)
            u32x4 v[4];
            load_x(kb, c, v);
            __syncthreads();                       // previous chunk fully read
            store_x(c & 1, v);
            __syncthreads();
            constexpr int KSC = BS >= 64 ? 2 : 1;  // k-steps in this chunk
#pragma unroll
            for (int kk = 0; kk < KSC; kk++) {
                const int ks = c * 2 + kk;
                bf16x8 bf[2];
#pragma unroll
                for (int nt = 0; nt < 2; nt++) bf[nt] = dequant8(code[nt][ks], s[nt], z[nt]);
#pragma unroll
                for (int mt = 0; mt < 4; mt++) {
                    const bf16x8 af = *reinterpret_cast<const bf16x8*>(
                        &xs[c & 1][wm * 64 + mt * 16 + l16][kk * 32 + 8 * g4]);
#pragma unroll
                    for (int nt = 0; nt < 2; nt++)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[nt], acc[mt][nt],
                                                                             0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            meta[nt] = meta_n[nt];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) code[nt][ks] = code_n[nt][ks];
        }
    }

#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int n = n0 + wn * 32 + nt * 16 + l16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + wm * 64 + mt * 16 + 4 * g4 + i;
                if (m < a.m && n < a.n) a.y[(size_t)m * a.n + n] = acc[mt][nt][i];
            }
        }
}

}  // namespace

extern "C" int qk_prefill_4bit(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                               float* d_y, hipStream_t s) {
    if (t->fmt != QK_FMT_4 || t->n_outliers) return -2;
    if (m <= 0 || t->rows <= 0) return 0;
    if (t->cols <= 0) return -2;
    PrefillArgs a = {t->d_blocks, d_x_bf16, d_y, m, t->rows, t->cols, t->nb};
    const dim3 grid((t->rows + BN - 1) / BN, (m + BM - 1) / BM), block(256);
    switch (t->bs) {
    case 64: hipLaunchKernelGGL(prefill_kernel<64>, grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL(prefill_kernel<128>, grid, block, 0, s, a); break;
    case 256: hipLaunchKernelGGL(prefill_kernel<256>, grid, block, 0, s, a); break;
    default: return -2;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
