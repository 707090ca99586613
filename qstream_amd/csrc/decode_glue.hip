// decode_glue.hip - the per-layer work around the matvecs of a batch-1
// decode step, on gfx950, so a device-resident engine needs no host round
// trip between its projections (src/engine.c:709-1187):
//   RMS / layer norm          src/kernels_scalar.c:148-185 (engine.c:805-815)
//   RoPE                      apply_rope, src/engine.c:204-235
//   int8 KV-cache store       kv_cache_store, src/engine.c:240-300
//   attention over the cache  src/engine.c:879-923
//   activation x up           src/engine.c:1128-1140
//   residual add + NaN check  src/engine.c:1172-1187
//   embedding row             src/engine.c:709-765
// Where the reference's result is integer (int8 KV codes) or follows one
// fixed sequence of fp32 roundings (KV scales, embedding values, the
// residual add) the kernels use the same operations in the same order with
// explicitly rounded multiplies and adds, so they match bit for bit; sums
// the kernels spread over lanes differ only in fp32 rounding order.
#include "qsf_device.h"
#include "qsf_hip_internal.h"

namespace {

constexpr int NORM_THREADS = 1024;

__device__ __forceinline__ float block_sum(float v, float* red) { return qsf::wg_sum(v, red); }

// RMS norm (LAYER = false) or layer norm over one vector of `dim` floats,
// one workgroup.  Output rounding order as src/kernels_scalar.c:148-185:
// (x * inv) * w, and (x - mean) * inv_std * w + b.
template <bool LAYER>
__global__ __launch_bounds__(NORM_THREADS) void norm_kernel(const float* __restrict__ in, float* out,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ b, int dim,
                                                            float eps) {
    __shared__ float red[NORM_THREADS / 64];
    if (!LAYER) {
        float ss = 0.f;
        for (int i = threadIdx.x; i < dim; i += blockDim.x) ss = fmaf(in[i], in[i], ss);
        ss = block_sum(ss, red);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(qsf::add_rn(__fdiv_rn(ss, (float)dim), eps)));
        for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = qsf::mul_rn(qsf::mul_rn(in[i], inv), w[i]);
    } else {
        float s = 0.f;
        for (int i = threadIdx.x; i < dim; i += blockDim.x) s += in[i];
        const float mean = __fdiv_rn(block_sum(s, red), (float)dim);
        float v = 0.f;
        for (int i = threadIdx.x; i < dim; i += blockDim.x) {
            const float d = in[i] - mean;
            v = fmaf(d, d, v);
        }
        const float var = __fdiv_rn(block_sum(v, red), (float)dim);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(qsf::add_rn(var, eps)));
        for (int i = threadIdx.x; i < dim; i += blockDim.x) {
            float o = qsf::mul_rn(qsf::mul_rn(qsf::sub_rn(in[i], mean), inv), w[i]);
            if (b) o = qsf::add_rn(o, b[i]);
            out[i] = o;
        }
    }
}

// RoPE: one thread per (head, pair).  freq[j] = 1 / powf(theta, 2j/hd) is
// computed by the host C library once (qsf_hip_rope_create), so every
// angle position * freq matches the reference's; the angle is reduced in
// double as there, then rotated in fp32.
__global__ __launch_bounds__(256) void rope_kernel(float* q, float* k, const float* __restrict__ freq,
                                                   int head_dim, int nq_pairs, int nk_pairs,
                                                   int position) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nq_pairs + nk_pairs) return;
    float* v = t < nq_pairs ? q + 2 * t : k + 2 * (t - nq_pairs);
    const int j = (t < nq_pairs ? t : t - nq_pairs) % (head_dim / 2);
    double ang = (double)position * (double)freq[j];
    ang = fmod(ang, 2.0 * 3.14159265358979323846);
    const float c = cosf((float)ang), s = sinf((float)ang);
    const float a0 = v[0], a1 = v[1];
    v[0] = qsf::sub_rn(qsf::mul_rn(a0, c), qsf::mul_rn(a1, s));
    v[1] = qsf::add_rn(qsf::mul_rn(a0, s), qsf::mul_rn(a1, c));
}

// int8 KV store: one wave per (kv head, K or V).  absmax, scale =
// amax / 127, codes = trunc(clamp(x * (127 / amax)) +- 0.5) with every
// operation rounded as in src/engine.c:252-296: bit-exact.
__global__ __launch_bounds__(64) void kv_store_kernel(int8_t* kc, int8_t* vc, float* ks, float* vs,
                                                      const float* __restrict__ k,
                                                      const float* __restrict__ v, int max_seq,
                                                      int head_dim, int position) {
    const int h = blockIdx.x >> 1, isv = blockIdx.x & 1, lane = threadIdx.x;
    const float* src = (isv ? v : k) + (size_t)h * head_dim;
    const size_t row = (size_t)h * max_seq + position;
    int8_t* dst = (isv ? vc : kc) + row * head_dim;
    float amax = 0.f;
    for (int i = lane; i < head_dim; i += 64) {
        const float a = src[i] < 0 ? -src[i] : src[i];
        amax = a > amax ? a : amax;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(amax, off, 64);
        amax = o > amax ? o : amax;
    }
    if (lane == 0) (isv ? vs : ks)[row] = __fdiv_rn(amax, 127.0f);
    if (amax > 1e-30f) {
        const float inv = __fdiv_rn(127.0f, amax);
        for (int i = lane; i < head_dim; i += 64) {
            float x = qsf::mul_rn(src[i], inv);
            if (x > 127.0f) x = 127.0f;
            if (x < -127.0f) x = -127.0f;
            dst[i] = (int8_t)(int)qsf::add_rn(x, x >= 0 ? 0.5f : -0.5f);
        }
    } else {
        for (int i = lane; i < head_dim; i += 64) dst[i] = 0;
    }
}

// Attention over positions 0..position, split over positions so a short
// decode step still fills the chip: workgroup (head, chunk) handles
// ATT_CHUNK positions and leaves its local max m, its sum l of
// exp(score - m) and its unnormalised output o[d] = sum exp(score - m) *
// v_scale * v[d] in the workspace; attention_combine_kernel rescales the
// chunks to the global max and normalises.  This is the reference's
// softmax(q . k * scale / sqrt(hd)) . v (src/engine.c:879-923), regrouped:
// the fp32 sums run in a different order.
constexpr int ATT_THREADS = 256;
constexpr int ATT_CHUNK = 128;
constexpr int ATT_MAX_SEQ = QK_ATT_MAX_SEQ;
typedef uint32_t att_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float sbyte(uint32_t w, int i) {
    return (float)(int8_t)(uint8_t)(w >> (8 * i));
}

__global__ __launch_bounds__(ATT_THREADS) void attention_part_kernel(
    const float* __restrict__ q, const int8_t* __restrict__ kc, const int8_t* __restrict__ vc,
    const float* __restrict__ ks, const float* __restrict__ vs, int max_seq, int groups,
    int head_dim, int seq, int nsplit, float* __restrict__ ws) {
    __shared__ float qs[256];
    __shared__ float ew[ATT_CHUNK];                      // exp(score - m) * v_scale per position
    __shared__ float parts[ATT_THREADS];
    __shared__ float red[ATT_THREADS / 64];
    const int h = blockIdx.x, chunk = blockIdx.y, kvh = h / groups, t = threadIdx.x;
    const int p0 = chunk * ATT_CHUNK, np = min(ATT_CHUNK, seq - p0);
    for (int d = t; d < head_dim; d += ATT_THREADS) qs[d] = q[(size_t)h * head_dim + d];
    __syncthreads();
    // scores: one thread per position; the row's int8 codes 16 at a time
    const float inv_sqrt_d = __fdiv_rn(1.0f, __fsqrt_rn((float)head_dim));
    float sc = -INFINITY;
    if (t < np) {
        const size_t row = (size_t)kvh * max_seq + p0 + t;
        const att_u32x4* kr = reinterpret_cast<const att_u32x4*>(kc + row * head_dim);
        const float kscale = ks[row];
        float dot = 0.f;
        for (int c = 0; c < head_dim / 16; c++) {
            const att_u32x4 w = kr[c];
#pragma unroll
            for (int j = 0; j < 16; j++)
                dot = fmaf(qs[16 * c + j], qsf::mul_rn(sbyte(w[j >> 2], j & 3), kscale), dot);
        }
        sc = qsf::mul_rn(dot, inv_sqrt_d);
    }
    float m = sc;
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float e = t < np ? expf(sc - m) : 0.f;
    if (t < np) ew[t] = qsf::mul_rn(e, vs[(size_t)kvh * max_seq + p0 + t]);
    const float l = block_sum(e, red);                   // also orders the ew writes
    // weighted V: thread (d, part) over positions part, part + P, ...
    const int P = ATT_THREADS / head_dim, d = t % head_dim, part = t / head_dim;
    float acc = 0.f;
    if (part < P) {
        const int8_t* vr = vc + ((size_t)kvh * max_seq + p0) * head_dim + d;
        for (int p = part; p < np; p += P) acc = fmaf(ew[p], (float)vr[(size_t)p * head_dim], acc);
    }
    parts[t] = acc;
    __syncthreads();
    float* rec = ws + ((size_t)h * nsplit + chunk) * (head_dim + 2);
    if (t < head_dim) {
        float o = 0.f;
        for (int i = 0; i < P; i++) o += parts[i * head_dim + t];
        rec[2 + t] = o;
    }
    if (t == 0) {
        rec[0] = m;
        rec[1] = l;
    }
}

// The same chunk result for head_dim = 16 HC in {64, 128, 256}, with every
// K and V byte of the chunk (and its scales) requested before any is used:
// the chunk arrives in one memory round trip instead of one a 16-byte K load
// and one a V position.  Two threads a position for the scores (half a row
// each); for the weighted V each thread keeps 16 output dims of the 16-byte
// pieces it loaded (ATT_THREADS % HC == 0, so always the same 16), summed
// over threads through LDS.  Positions past the chunk end load the last
// valid row and are masked.
template <int HC>
__global__ __launch_bounds__(ATT_THREADS) void attention_part_fast_kernel(
    const float* __restrict__ q, const int8_t* __restrict__ kc, const int8_t* __restrict__ vc,
    const float* __restrict__ ks, const float* __restrict__ vs, int max_seq, int groups, int seq,
    int nsplit, float* __restrict__ ws) {
    constexpr int HD = 16 * HC, KH = HC / 2, VJ = ATT_CHUNK * HC / ATT_THREADS;
    static_assert(HD <= ATT_THREADS && ATT_THREADS % HC == 0, "one q element a thread");
    __shared__ float qs[HD];
    __shared__ float ew[ATT_CHUNK];                      // exp(score - m) * v_scale per position
    __shared__ float red[ATT_THREADS / 64];
    __shared__ float part[ATT_THREADS][17];
    const int h = blockIdx.x, chunk = blockIdx.y, kvh = h / groups, t = threadIdx.x;
    const int p0 = chunk * ATT_CHUNK, np = min(ATT_CHUNK, seq - p0);
    const size_t row0 = (size_t)kvh * max_seq + p0;
    // 1. all loads
    const int kp = t >> 1, kh = t & 1;
    const int kpc = min(kp, np - 1);
    const att_u32x4* kr = reinterpret_cast<const att_u32x4*>(kc + (row0 + kpc) * HD) + kh * KH;
    att_u32x4 kv[KH];
#pragma unroll
    for (int j = 0; j < KH; j++) kv[j] = kr[j];
    const float kscale = ks[row0 + kpc];
    const float vscale = vs[row0 + kpc];
    const att_u32x4* vr = reinterpret_cast<const att_u32x4*>(vc + row0 * HD);
    att_u32x4 vv[VJ];
#pragma unroll
    for (int j = 0; j < VJ; j++) {
        const int i = t + ATT_THREADS * j;
        vv[j] = vr[min(i / HC, np - 1) * HC + i % HC];
    }
    if (t < HD) qs[t] = q[(size_t)h * HD + t];
    __syncthreads();
    // 2. scores and the chunk's softmax terms
    const float inv_sqrt_d = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < KH; j++)
#pragma unroll
        for (int b = 0; b < 16; b++)
            dot = fmaf(qs[16 * (kh * KH + j) + b], qsf::mul_rn(sbyte(kv[j][b >> 2], b & 3), kscale), dot);
    dot += __shfl_xor(dot, 1, 64);
    const bool mine = kh == 0 && kp < np;
    const float sc = kp < np ? qsf::mul_rn(dot, inv_sqrt_d) : -INFINITY;
    float m = sc;
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float e = mine ? expf(sc - m) : 0.f;
    if (mine) ew[kp] = qsf::mul_rn(e, vscale);
    const float l = block_sum(e, red);                   // also orders the ew writes
    // 3. weighted V: dims 16 (t % HC) .. +15 of the thread's pieces
    float acc[16];
#pragma unroll
    for (int b = 0; b < 16; b++) acc[b] = 0.f;
#pragma unroll
    for (int j = 0; j < VJ; j++) {
        const int p = (t + ATT_THREADS * j) / HC;
        const float w = p < np ? ew[p] : 0.f;
#pragma unroll
        for (int b = 0; b < 16; b++) acc[b] = fmaf(w, sbyte(vv[j][b >> 2], b & 3), acc[b]);
    }
#pragma unroll
    for (int b = 0; b < 16; b++) part[t][b] = acc[b];
    __syncthreads();
    float* rec = ws + ((size_t)h * nsplit + chunk) * (HD + 2);
    if (t < HD) {
        const int c = t >> 4, b = t & 15;
        float o = 0.f;
#pragma unroll
        for (int r = 0; r < ATT_THREADS / HC; r++) o += part[c + HC * r][b];
        rec[2 + t] = o;
    }
    if (t == 0) {
        rec[0] = m;
        rec[1] = l;
    }
}

__global__ __launch_bounds__(256) void attention_combine_kernel(const float* __restrict__ ws,
                                                                int head_dim, int nsplit,
                                                                float* __restrict__ out) {
    const int h = blockIdx.x, d = threadIdx.x;
    if (d >= head_dim) return;
    const float* base = ws + (size_t)h * nsplit * (head_dim + 2);
    float M = -INFINITY;
    for (int c = 0; c < nsplit; c++) M = fmaxf(M, base[(size_t)c * (head_dim + 2)]);
    float L = 0.f, O = 0.f;
    for (int c = 0; c < nsplit; c++) {
        const float* rec = base + (size_t)c * (head_dim + 2);
        const float f = expf(rec[0] - M);
        L = fmaf(f, rec[1], L);
        O = fmaf(f, rec[2 + d], O);
    }
    out[(size_t)h * head_dim + d] = __fdiv_rn(O, L);
}

// gate = act(gate) * up (QSFActivation: 2 SiLU, 0/1 GELU tanh form, else
// ReLU), src/kernels_scalar.c:129-147 and src/engine.c:1128-1140.
__global__ __launch_bounds__(256) void act_mul_kernel(float* gate, const float* __restrict__ up,
                                                      int n, int act) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    gate[i] = qsf::act_mul(act, gate[i], up[i]);
}

// res += x, then the first index whose value is NaN or beyond +-1e30 (or
// -1) into *bad when bad is given.  One workgroup: the minimum is reduced
// in LDS, so nothing has to be cleared before the launch.
__global__ __launch_bounds__(1024) void residual_kernel(float* res, const float* __restrict__ x, int n,
                                                        int* bad) {
    __shared__ int red[1024 / 64];
    int first = n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float r = qsf::add_rn(res[i], x[i]);
        res[i] = r;
        if ((r != r || r > 1e30f || r < -1e30f) && i < first) first = i;
    }
    if (!bad) return;
    for (int off = 32; off > 0; off >>= 1) first = min(first, __shfl_xor(first, off, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = first;
    __syncthreads();
    if (threadIdx.x == 0) {
        int f = n;
        for (int w = 0; w < (int)(blockDim.x >> 6); w++) f = min(f, red[w]);
        *bad = f < n ? f : -1;
    }
}

// Residual add + NaN check, then the next norm of the updated residual, in
// one workgroup: the engine's sequence res += x (src/engine.c:937 / 1174),
// check (1176-1187), norm (940-948 / 805-815).  Each thread walks the same
// elements as residual_kernel and norm_kernel, so the results equal those
// two launches bit for bit.
template <bool LAYER>
__global__ __launch_bounds__(NORM_THREADS) void residual_norm_kernel(
    float* res, const float* __restrict__ x, int n, int* bad, const float* __restrict__ w,
    const float* __restrict__ b, float eps, float* out) {
    __shared__ int ired[NORM_THREADS / 64];
    __shared__ float red[NORM_THREADS / 64];
    int first = n;
    float acc = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float r = qsf::add_rn(res[i], x[i]);
        res[i] = r;
        if ((r != r || r > 1e30f || r < -1e30f) && i < first) first = i;
        acc = LAYER ? acc + r : fmaf(r, r, acc);
    }
    if (bad) {
        for (int off = 32; off > 0; off >>= 1) first = min(first, __shfl_xor(first, off, 64));
        if ((threadIdx.x & 63) == 0) ired[threadIdx.x >> 6] = first;
        __syncthreads();
        if (threadIdx.x == 0) {
            int f = n;
            for (int wv = 0; wv < (int)(blockDim.x >> 6); wv++) f = min(f, ired[wv]);
            *bad = f < n ? f : -1;
        }
    }
    if (!LAYER) {
        const float ss = block_sum(acc, red);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(qsf::add_rn(__fdiv_rn(ss, (float)n), eps)));
        for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = qsf::mul_rn(qsf::mul_rn(res[i], inv), w[i]);
    } else {
        const float mean = __fdiv_rn(block_sum(acc, red), (float)n);
        float v = 0.f;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const float d = res[i] - mean;
            v = fmaf(d, d, v);
        }
        const float var = __fdiv_rn(block_sum(v, red), (float)n);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(qsf::add_rn(var, eps)));
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            float o = qsf::mul_rn(qsf::mul_rn(qsf::sub_rn(res[i], mean), inv), w[i]);
            if (b) o = qsf::add_rn(o, b[i]);
            out[i] = o;
        }
    }
}

// RoPE of q and k and the int8 KV store of k (rotated) and v in one launch:
// one wave per q head (rotate), per kv head's k (rotate, then store) and
// per kv head's v (store).  The rotation is rope_kernel's arithmetic and the
// store kv_store_kernel's, so q, k and the cache rows equal the two
// launches bit for bit (absmax and the per-element codes do not depend on
// the order elements are visited).  head_dim <= 256: two pairs a lane.
__device__ __forceinline__ void rope_pair(float& a0, float& a1, const float* __restrict__ freq, int j,
                                          int position) {
    double ang = (double)position * (double)freq[j];
    ang = fmod(ang, 2.0 * 3.14159265358979323846);
    const float c = cosf((float)ang), sn = sinf((float)ang);
    const float x0 = a0, x1 = a1;
    a0 = qsf::sub_rn(qsf::mul_rn(x0, c), qsf::mul_rn(x1, sn));
    a1 = qsf::add_rn(qsf::mul_rn(x0, sn), qsf::mul_rn(x1, c));
}

__device__ __forceinline__ int8_t kv_code(float x, float inv) {
    x = qsf::mul_rn(x, inv);
    if (x > 127.0f) x = 127.0f;
    if (x < -127.0f) x = -127.0f;
    return (int8_t)(int)qsf::add_rn(x, x >= 0 ? 0.5f : -0.5f);
}

__global__ __launch_bounds__(64) void rope_kv_kernel(float* q, float* k, const float* __restrict__ v,
                                                     const float* __restrict__ freq, int head_dim,
                                                     int n_heads, int position, int8_t* kc, int8_t* vc,
                                                     float* ks, float* vs, int max_seq) {
    const int lane = threadIdx.x, hp = head_dim / 2;
    if ((int)blockIdx.x < n_heads) {
        float* qh = q + (size_t)blockIdx.x * head_dim;
        for (int j = lane; j < hp; j += 64) rope_pair(qh[2 * j], qh[2 * j + 1], freq, j, position);
        return;
    }
    const int idx = (int)blockIdx.x - n_heads, h = idx >> 1, isv = idx & 1;
    const size_t row = (size_t)h * max_seq + position;
    float val[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
    const float* src = (isv ? v : k) + (size_t)h * head_dim;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int j = lane + 64 * u;
        if (j < hp) {
            val[u][0] = src[2 * j];
            val[u][1] = src[2 * j + 1];
            if (!isv) {
                rope_pair(val[u][0], val[u][1], freq, j, position);
                float* kh = k + (size_t)h * head_dim;
                kh[2 * j] = val[u][0];
                kh[2 * j + 1] = val[u][1];
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float a = val[u][e] < 0 ? -val[u][e] : val[u][e];
            amax = a > amax ? a : amax;
        }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(amax, off, 64);
        amax = o > amax ? o : amax;
    }
    if (lane == 0) (isv ? vs : ks)[row] = __fdiv_rn(amax, 127.0f);
    int8_t* dst = (isv ? vc : kc) + row * head_dim;
    const bool live = amax > 1e-30f;
    const float inv = live ? __fdiv_rn(127.0f, amax) : 0.f;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int j = lane + 64 * u;
        if (j < hp) {
            dst[2 * j] = live ? kv_code(val[u][0], inv) : (int8_t)0;
            dst[2 * j + 1] = live ? kv_code(val[u][1], inv) : (int8_t)0;
        }
    }
}

// RoPE + int8 KV store + the chunk pass of attention in one launch, for
// head_dim = 16 HC in {64, 128, 256}: the cache rows, scales and chunk
// records of rope_kv_kernel followed by attention_part_fast_kernel, bit for
// bit.  Every workgroup (head, chunk) rotates its head's q itself, into LDS.
// The position being decoded lies in the last chunk: its workgroups rotate
// the new k and quantise k and v with the KV store's arithmetic, and use
// those codes for that row instead of reading the cache; the first head of
// each KV group also stores them, with the scales.  No other workgroup
// needs that row, so the store orders with nothing.  q and k stay as they
// were: several workgroups read each of them, so none may rotate them in
// place.
template <int HC>
__global__ __launch_bounds__(ATT_THREADS) void rope_attention_part_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ freq, int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq, int groups,
    int position, int nsplit, float* __restrict__ ws) {
    constexpr int HD = 16 * HC, KH = HC / 2, VJ = ATT_CHUNK * HC / ATT_THREADS, HP = HD / 2;
    static_assert(HD <= ATT_THREADS && ATT_THREADS % HC == 0 && HP <= 128, "one q pair a thread");
    __shared__ float qs[HD];
    __shared__ float ew[ATT_CHUNK];                      // exp(score - m) * v_scale per position
    __shared__ float red[ATT_THREADS / 64];
    __shared__ float part[ATT_THREADS][17];
    __shared__ __align__(16) int8_t newc[2][HD];         // the new row's K and V codes
    __shared__ float news[2];                            // and their scales
    const int h = blockIdx.x, chunk = blockIdx.y, kvh = h / groups, t = threadIdx.x;
    const int p0 = chunk * ATT_CHUNK, np = min(ATT_CHUNK, position + 1 - p0);
    const bool last = chunk == nsplit - 1;               // holds the new row, np - 1
    const size_t row0 = (size_t)kvh * max_seq + p0;
    // 1. all loads.  In the last chunk only the rows before the new one:
    //    its own slot loads the row before it and is replaced below, and
    //    when the new row starts the chunk nothing is loaded (no workgroup
    //    reads the row the first head of the group is storing).
    const int kp = t >> 1, kh = t & 1;
    const int nold = last ? np - 1 : np;                 // rows already in the cache
    const int kpc = min(kp, max(nold, 1) - 1);
    att_u32x4 kv[KH], vv[VJ];
    float kscale = 0.f, vscale = 0.f;
    if (nold > 0) {                                      // (uniform)
        const att_u32x4* kr = reinterpret_cast<const att_u32x4*>(kc + (row0 + kpc) * HD) + kh * KH;
#pragma unroll
        for (int j = 0; j < KH; j++) kv[j] = kr[j];
        kscale = ks[row0 + kpc];
        vscale = vs[row0 + kpc];
        const att_u32x4* vr = reinterpret_cast<const att_u32x4*>(vc + row0 * HD);
#pragma unroll
        for (int j = 0; j < VJ; j++) {
            const int i = t + ATT_THREADS * j;
            vv[j] = vr[min(i / HC, nold - 1) * HC + i % HC];
        }
    } else {
#pragma unroll
        for (int j = 0; j < KH; j++) kv[j] = att_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < VJ; j++) vv[j] = att_u32x4{0u, 0u, 0u, 0u};
    }
    // q pair t of the head, and in the last chunk k and v pair t
    float q0 = 0.f, q1 = 0.f, nk[2] = {0.f, 0.f}, nv[2] = {0.f, 0.f};
    if (t < HP) {
        q0 = q[(size_t)h * HD + 2 * t];
        q1 = q[(size_t)h * HD + 2 * t + 1];
        if (last) {
            nk[0] = k[(size_t)kvh * HD + 2 * t];
            nk[1] = k[(size_t)kvh * HD + 2 * t + 1];
            nv[0] = v[(size_t)kvh * HD + 2 * t];
            nv[1] = v[(size_t)kvh * HD + 2 * t + 1];
        }
        rope_pair(q0, q1, freq, t, position);
        qs[2 * t] = q0;
        qs[2 * t + 1] = q1;
    }
    if (last) {
        if (t < HP) rope_pair(nk[0], nk[1], freq, t, position);
        // absmax as the KV store takes it (NaN compares false and drops out)
        float ak = 0.f, av = 0.f;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const float a = nk[e] < 0 ? -nk[e] : nk[e], b = nv[e] < 0 ? -nv[e] : nv[e];
            ak = a > ak ? a : ak;
            av = b > av ? b : av;
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float ok = __shfl_xor(ak, off, 64), ov = __shfl_xor(av, off, 64);
            ak = ok > ak ? ok : ak;
            av = ov > av ? ov : av;
        }
        if (HP > 64) {                                   // pairs in waves 0 and 1
            if (t == 0 || t == 64) {
                red[t >> 5] = ak;
                red[(t >> 5) + 1] = av;
            }
            __syncthreads();
            ak = red[2] > red[0] ? red[2] : red[0];
            av = red[3] > red[1] ? red[3] : red[1];
        }
        const bool lk = ak > 1e-30f, lv = av > 1e-30f;
        const float ik = lk ? __fdiv_rn(127.0f, ak) : 0.f, iv = lv ? __fdiv_rn(127.0f, av) : 0.f;
        const bool store = h % groups == 0;
        const size_t row = (size_t)kvh * max_seq + position;
        if (t < HP) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int8_t ck = lk ? kv_code(nk[e], ik) : (int8_t)0, cv = lv ? kv_code(nv[e], iv) : (int8_t)0;
                newc[0][2 * t + e] = ck;
                newc[1][2 * t + e] = cv;
                if (store) {
                    kc[row * HD + 2 * t + e] = ck;
                    vc[row * HD + 2 * t + e] = cv;
                }
            }
        }
        if (t == 0) {
            news[0] = __fdiv_rn(ak, 127.0f);
            news[1] = __fdiv_rn(av, 127.0f);
            if (store) {
                ks[row] = news[0];
                vs[row] = news[1];
            }
        }
    }
    __syncthreads();
    if (last) {                                          // the new row in place of the loaded one
        if (kp == np - 1) {
            const att_u32x4* nkr = reinterpret_cast<const att_u32x4*>(newc[0]) + kh * KH;
#pragma unroll
            for (int j = 0; j < KH; j++) kv[j] = nkr[j];
            kscale = news[0];
            vscale = news[1];
        }
#pragma unroll
        for (int j = 0; j < VJ; j++) {
            const int i = t + ATT_THREADS * j;
            if (i / HC == np - 1) vv[j] = reinterpret_cast<const att_u32x4*>(newc[1])[i % HC];
        }
    }
    // 2. scores and the chunk's softmax terms, as attention_part_fast_kernel
    const float inv_sqrt_d = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < KH; j++)
#pragma unroll
        for (int b = 0; b < 16; b++)
            dot = fmaf(qs[16 * (kh * KH + j) + b], qsf::mul_rn(sbyte(kv[j][b >> 2], b & 3), kscale), dot);
    dot += __shfl_xor(dot, 1, 64);
    const bool mine = kh == 0 && kp < np;
    const float sc = kp < np ? qsf::mul_rn(dot, inv_sqrt_d) : -INFINITY;
    float m = sc;
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((t & 63) == 0) red[t >> 6] = m;                  // red's absmax use ended at the barrier
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float e = mine ? expf(sc - m) : 0.f;
    if (mine) ew[kp] = qsf::mul_rn(e, vscale);
    const float l = block_sum(e, red);                   // also orders the ew writes
    // 3. weighted V
    float acc[16];
#pragma unroll
    for (int b = 0; b < 16; b++) acc[b] = 0.f;
#pragma unroll
    for (int j = 0; j < VJ; j++) {
        const int p = (t + ATT_THREADS * j) / HC;
        const float w = p < np ? ew[p] : 0.f;
#pragma unroll
        for (int b = 0; b < 16; b++) acc[b] = fmaf(w, sbyte(vv[j][b >> 2], b & 3), acc[b]);
    }
#pragma unroll
    for (int b = 0; b < 16; b++) part[t][b] = acc[b];
    __syncthreads();
    float* rec = ws + ((size_t)h * nsplit + chunk) * (HD + 2);
    if (t < HD) {
        const int c = t >> 4, b = t & 15;
        float o = 0.f;
#pragma unroll
        for (int r = 0; r < ATT_THREADS / HC; r++) o += part[c + HC * r][b];
        rec[2 + t] = o;
    }
    if (t == 0) {
        rec[0] = m;
        rec[1] = l;
    }
}

// One row of a blockwise table: value i = scale * q + zero (4-bit sym:
// scale * q), each product and sum rounded as in src/quant.c:95-177.
__global__ __launch_bounds__(256) void embed_row_kernel(const uint8_t* __restrict__ blocks, int fmt,
                                                        int bs, int bb, int hd, float* out,
                                                        int frag_row, int nq, int plane, int nb) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hd) return;
    // byte j of the value's block: on-disk or row-plane order (`blocks` is
    // the row), or fragment order (`blocks` is the tensor, frag_row the row)
    const int b = i / bs;
    auto byte_at = [&](int j) -> unsigned {
        return frag_row >= 0 ? blocks[qsf::frag_off((size_t)frag_row, b, j, nq, bb)]
               : plane       ? blocks[qsf::plane_off(b, j, nb, bb, bs)]
                             : blocks[(size_t)b * bb + j];
    };
    const uint32_t meta = byte_at(0) | (byte_at(1) << 8) | (byte_at(2) << 16) | (byte_at(3) << 24);
    const int k = i % bs;
    unsigned c;
    if (fmt == QK_FMT_2) {
        c = (byte_at(4 + (k >> 2)) >> ((k & 3) * 2)) & 3u;
    } else if (fmt == QK_FMT_3) {
        const int bit = 3 * k, byte = bit >> 3, off = bit & 7;
        unsigned v = byte_at(4 + byte) >> off;
        if (off > 5) v |= byte_at(4 + byte + 1) << (8 - off);
        c = v & 7u;
    } else {
        c = (byte_at(4 + (k >> 1)) >> ((k & 1) * 4)) & 15u;
    }
    const float s = qsf::f16_lo(meta);
    if (fmt == QK_FMT_4SYM) {
        out[i] = qsf::mul_rn(s, (float)(c >= 8u ? (int)c - 16 : (int)c));
    } else {
        out[i] = qsf::add_rn(qsf::mul_rn(s, (float)c), qsf::f16_hi(meta));
    }
}

__global__ __launch_bounds__(256) void embed_row_fp16_kernel(const uint16_t* __restrict__ row, int hd,
                                                             float* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < hd) out[i] = qsf::f16_bits(row[i]);
}

}  // namespace

extern "C" int qk_norm(const float* in, float* out, const float* w, const float* b, int dim,
                       float eps, int layer, hipStream_t s) {
    if (dim <= 0) return 0;
    if (layer)
        hipLaunchKernelGGL(norm_kernel<true>, dim3(1), dim3(NORM_THREADS), 0, s, in, out, w, b, dim, eps);
    else
        hipLaunchKernelGGL(norm_kernel<false>, dim3(1), dim3(NORM_THREADS), 0, s, in, out, w, b, dim, eps);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_rope(float* q, float* k, const float* freq, int head_dim, int n_heads,
                       int n_kv, int position, hipStream_t s) {
    const int nq = n_heads * head_dim / 2, nk = n_kv * head_dim / 2;
    if (nq + nk == 0) return 0;
    hipLaunchKernelGGL(rope_kernel, dim3((nq + nk + 255) / 256), dim3(256), 0, s, q, k, freq, head_dim,
                       nq, nk, position);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_kv_store(int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq, int n_kv,
                           int head_dim, int position, const float* k, const float* v,
                           hipStream_t s) {
    if (n_kv <= 0) return 0;
    hipLaunchKernelGGL(kv_store_kernel, dim3(2 * n_kv), dim3(64), 0, s, kc, vc, ks, vs, k, v, max_seq,
                       head_dim, position);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" size_t qk_attention_ws_bytes(int n_heads, int head_dim, int position) {
    const int nsplit = (position + 1 + ATT_CHUNK - 1) / ATT_CHUNK;
    return sizeof(float) * (size_t)n_heads * nsplit * (head_dim + 2);
}

extern "C" int qk_attention(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                            const float* vs, int max_seq, int n_heads, int n_kv, int head_dim,
                            int position, float* out, void* ws, hipStream_t s) {
    const int seq = position + 1;
    if (head_dim > ATT_THREADS || head_dim % 16 || seq > ATT_MAX_SEQ || n_kv <= 0 ||
        n_heads % n_kv)
        return -2;
    const int nsplit = (seq + ATT_CHUNK - 1) / ATT_CHUNK;
    const dim3 grid(n_heads, nsplit), block(ATT_THREADS);
    const int groups = n_heads / n_kv;
    float* part = (float*)ws;
    switch (head_dim) {
    case 64:
        hipLaunchKernelGGL(attention_part_fast_kernel<4>, grid, block, 0, s, q, kc, vc, ks, vs, max_seq,
                           groups, seq, nsplit, part);
        break;
    case 128:
        hipLaunchKernelGGL(attention_part_fast_kernel<8>, grid, block, 0, s, q, kc, vc, ks, vs, max_seq,
                           groups, seq, nsplit, part);
        break;
    case 256:
        hipLaunchKernelGGL(attention_part_fast_kernel<16>, grid, block, 0, s, q, kc, vc, ks, vs, max_seq,
                           groups, seq, nsplit, part);
        break;
    default:
        hipLaunchKernelGGL(attention_part_kernel, grid, block, 0, s, q, kc, vc, ks, vs, max_seq, groups,
                           head_dim, seq, nsplit, part);
    }
    hipLaunchKernelGGL(attention_combine_kernel, dim3(n_heads), dim3(256), 0, s, (const float*)ws,
                       head_dim, nsplit, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_act_mul(float* gate, const float* up, int n, int act, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(act_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, gate, up, n, act);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_residual(float* res, const float* x, int n, int* bad, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(residual_kernel, dim3(1), dim3(1024), 0, s, res, x, n, bad);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_residual_norm(float* res, const float* x, int n, int* bad, const float* w,
                                const float* b, float eps, int layer, float* out, hipStream_t s) {
    if (n <= 0) return 0;
    if (layer)
        hipLaunchKernelGGL(residual_norm_kernel<true>, dim3(1), dim3(NORM_THREADS), 0, s, res, x, n, bad, w,
                           b, eps, out);
    else
        hipLaunchKernelGGL(residual_norm_kernel<false>, dim3(1), dim3(NORM_THREADS), 0, s, res, x, n, bad,
                           w, b, eps, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_rope_kv_store(float* q, float* k, const float* v, const float* freq, int head_dim,
                                int n_heads, int n_kv, int position, int8_t* kc, int8_t* vc, float* ks,
                                float* vs, int max_seq, hipStream_t s) {
    if (head_dim <= 0 || head_dim > 256 || (head_dim & 1) || n_kv <= 0 || position < 0 ||
        position >= max_seq)
        return -2;
    hipLaunchKernelGGL(rope_kv_kernel, dim3(n_heads + 2 * n_kv), dim3(64), 0, s, q, k, v, freq, head_dim,
                       n_heads, position, kc, vc, ks, vs, max_seq);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_rope_kv_attention(float* q, float* k, const float* v, const float* freq, int head_dim,
                                    int n_heads, int n_kv, int position, int8_t* kc, int8_t* vc, float* ks,
                                    float* vs, int max_seq, float* out, void* ws, hipStream_t s) {
    const int seq = position + 1;
    if (head_dim <= 0 || head_dim > 256 || head_dim % 16 || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv ||
        position < 0 || position >= max_seq || seq > ATT_MAX_SEQ)
        return -2;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) {
        const int rc = qk_rope_kv_store(q, k, v, freq, head_dim, n_heads, n_kv, position, kc, vc, ks, vs,
                                        max_seq, s);
        return rc ? rc : qk_attention(q, kc, vc, ks, vs, max_seq, n_heads, n_kv, head_dim, position, out, ws, s);
    }
    const int nsplit = (seq + ATT_CHUNK - 1) / ATT_CHUNK, groups = n_heads / n_kv;
    const dim3 grid(n_heads, nsplit), block(ATT_THREADS);
    float* part = (float*)ws;
    if (head_dim == 64)
        hipLaunchKernelGGL(rope_attention_part_kernel<4>, grid, block, 0, s, q, k, v, freq, kc, vc, ks, vs,
                           max_seq, groups, position, nsplit, part);
    else if (head_dim == 128)
        hipLaunchKernelGGL(rope_attention_part_kernel<8>, grid, block, 0, s, q, k, v, freq, kc, vc, ks, vs,
                           max_seq, groups, position, nsplit, part);
    else
        hipLaunchKernelGGL(rope_attention_part_kernel<16>, grid, block, 0, s, q, k, v, freq, kc, vc, ks, vs,
                           max_seq, groups, position, nsplit, part);
    hipLaunchKernelGGL(attention_combine_kernel, dim3(n_heads), dim3(256), 0, s, (const float*)ws, head_dim,
                       nsplit, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_embed_row(const qsf_hip_tensor* t, int token, float* out, hipStream_t s) {
    if (t->fmt < 0 || token < 0 || token >= t->rows) return -2;
    if (t->cols <= 0) return 0;
    const uint8_t* row = t->frag ? t->d_blocks : t->d_blocks + (size_t)token * t->nb * t->block_bytes;
    hipLaunchKernelGGL(embed_row_kernel, dim3((t->cols + 255) / 256), dim3(256), 0, s, row, t->fmt, t->bs,
                       t->block_bytes, t->cols, out, t->frag ? token : -1, t->frag_nq, t->plane, t->nb);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int qk_embed_row_fp16(const uint16_t* table, int hd, int token, float* out,
                                 hipStream_t s) {
    if (hd <= 0) return 0;
    hipLaunchKernelGGL(embed_row_fp16_kernel, dim3((hd + 255) / 256), dim3(256), 0, s,
                       table + (size_t)token * hd, hd, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
