// stream_read.hip - the bare-read floor of a decode launch: one launch that
// streams the device bytes of a step's tensors once and does nothing else.
// A diagnostic with no counterpart in the reference: the bench sets the
// GEMV's time beside it, on the same rotated bytes.
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

}  // namespace

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
