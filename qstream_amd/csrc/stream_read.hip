// stream_read.hip - the measured ceilings the bench sets its kernels
// beside, diagnostics with no counterpart in the reference:
//  * the bare-read floor of a decode launch: one launch that streams the
//    device bytes of a step's tensors once and does nothing else, on the
//    same rotated bytes as the GEMV;
//  * the bf16 matrix-core peak: v_mfma_f32_16x16x32_bf16 (the prefill's
//    instruction) in independent chains on every SIMD, no memory traffic.
//
// Layout of the work: the ranges are cut into 16 KB chunks (256 threads x
// 4 x 16-byte nontemporal loads, each load covering 4 KB of contiguous
// memory across the workgroup), numbered across ranges in order; workgroup
// w takes chunks w, w + G, w + 2G, ... (G workgroups, a few per CU), so
// every CU streams from the start.  Loads past a range's end are clamped
// to its last 16 bytes (the ranges are 16-byte multiples).
#include <hip/hip_runtime.h>

#include "qsf_hip_internal.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int kChunk = kThreads * kUnroll * 16;
constexpr uint32_t kMagic = 0x5A17C0DEu;

struct ReadArgs {
    const uint8_t* p[QK_MAX_GROUP];
    uint64_t bytes[QK_MAX_GROUP];
    uint64_t chunk0[QK_MAX_GROUP + 1];   // first chunk of each range, and the total
    int n;
    uint32_t* sink;
};

__global__ __launch_bounds__(kThreads) void stream_read_kernel(ReadArgs a) {
    uint32_t acc = 0;
    const uint64_t total = a.chunk0[a.n];
    for (uint64_t c = blockIdx.x; c < total; c += gridDim.x) {
        int r = 0;
        while (r + 1 < a.n && c >= a.chunk0[r + 1]) r++;
        const uint64_t base = (c - a.chunk0[r]) * kChunk;
        const uint64_t last = a.bytes[r] - 16;
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            uint64_t off = base + (uint64_t)(u * kThreads + threadIdx.x) * 16;
            off = off < last ? off : last;
            v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.p[r] + off));
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == kMagic) *a.sink = acc;
}

// kMfmaChains independent accumulators a wave, each advanced `iters` times
// (operands from the thread id, so nothing folds); the sum of every
// accumulator is stored only if its bits equal a fixed constant.
constexpr int kMfmaChains = 8, kMfmaWgPerCu = 4;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// (four waves a SIMD, as launched: with the hint the accumulators stay in
// place in VGPRs; without it the compiler routed them through AGPR moves,
// 20-50 an iteration, and measured those instead of the matrix core)
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void mfma_peak_kernel(
    int iters, uint32_t* sink) {
    const float f = (float)(threadIdx.x & 7) * 0.125f;
    bf16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (__bf16)(f + (float)i);
        b[i] = (__bf16)(f - (float)i);
    }
    f32x4 c0 = {f, f, f, f}, c1 = c0 + 1.f, c2 = c0 + 2.f, c3 = c0 + 3.f, c4 = c0 + 4.f, c5 = c0 + 5.f,
          c6 = c0 + 6.f, c7 = c0 + 7.f;
    static_assert(kMfmaChains == 8, "eight chains");
    for (int it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c3, 0, 0, 0);
        c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c4, 0, 0, 0);
        c5 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c5, 0, 0, 0);
        c6 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c6, 0, 0, 0);
        c7 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c7, 0, 0, 0);
    }
    const f32x4 t = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
    const float sum = (t[0] + t[1]) + (t[2] + t[3]);
    if (__builtin_bit_cast(uint32_t, sum) == kMagic) *sink = 1u;
}

}  // namespace

extern "C" double qk_mfma_peak(int iters, uint32_t* sink, hipStream_t s) {
    if (iters <= 0 || !sink) return -2;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const unsigned g = (unsigned)cus * kMfmaWgPerCu;
    hipLaunchKernelGGL(mfma_peak_kernel, dim3(g), dim3(kThreads), 0, s, iters, sink);
    if (hipGetLastError() != hipSuccess) return -1;
    // FLOP of the launch: every wave's chains, 2 * 16 * 16 * 32 a MFMA
    return (double)g * (kThreads / 64) * (double)iters * kMfmaChains * 2.0 * 16 * 16 * 32;
}

extern "C" int qk_stream_read(const void* const* ptr, const size_t* bytes, int n, uint32_t* sink,
                              hipStream_t s) {
    if (n <= 0 || n > QK_MAX_GROUP || !sink) return -2;
    ReadArgs a{};
    a.n = n;
    a.sink = sink;
    uint64_t c = 0;
    for (int i = 0; i < n; i++) {
        if (!ptr[i] || bytes[i] < 16 || (bytes[i] & 15) || ((uintptr_t)ptr[i] & 15)) return -2;
        a.p[i] = static_cast<const uint8_t*>(ptr[i]);
        a.bytes[i] = bytes[i];
        a.chunk0[i] = c;
        c += (bytes[i] + kChunk - 1) / kChunk;
    }
    a.chunk0[n] = c;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const uint64_t want = (uint64_t)cus * 8;
    const unsigned g = (unsigned)(c < want ? c : want);
    hipLaunchKernelGGL(stream_read_kernel, dim3(g), dim3(kThreads), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
