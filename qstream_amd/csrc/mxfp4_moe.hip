// mxfp4_moe.hip - MXFP4 expert matvec and the MoE FFN chain on gfx950.
//
// Format (quant type 11): codes plane [rows][nblk][16 B] (element 2j = low
// nibble of byte j, tools/convert_hf.py:1456-1495), then an E8M0 scales plane
// [rows][nblk]; value = E2M1(code) * 2^(E-127) (OCP MX v1.0).
//
// Decode: one lane per 32-element block, 16-B code load + 1 scale byte;
// v_cvt_scalef32_pk_f32_fp4 turns two E2M1 codes into two exact fp32 values,
// an fp32 FMA chain forms sum_k e2m1_k * x_k for the block, and the power of
// two scale is applied once per block.
//
// MoE (src/engine.c:951-1107): route (softmax over router logits, strict '>'
// top-K insertion, optional renormalisation) -> per selected expert gate/up
// GEMV + bias + activation * up -> down GEMV + bias -> weighted sum over the
// token's experts in rank order.  Expert weights are read once per step:
// tokens that pick the same expert are served by one owner slot.
#include "qsf_device.h"
#include "qsf_hip_internal.h"

namespace {

typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read once per step).
__device__ __forceinline__ uint4 ld_nt16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// E8M0 byte -> fp32 2^(e-127); 0 -> 2^-127 (subnormal); 0xFF -> NaN.
__device__ __forceinline__ float e8m0(uint32_t e) {
    uint32_t bits = e == 0 ? 0x00400000u : (e == 255 ? 0x7FC00000u : e << 23);
    return __builtin_bit_cast(float, bits);
}

// sum_{k<count} e2m1(code_k) * x[k] for one 32-element block.
__device__ __forceinline__ float block_dot(uint4 c, const float* __restrict__ x, int count) {
    float acc = 0.0f;
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    if (count >= 32) {
        const float4* x4 = reinterpret_cast<const float4*>(x);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 xa = x4[2 * i], xb = x4[2 * i + 1];
            f2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 0);
            f2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 1);
            f2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 2);
            f2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[i], 1.0f, 3);
            acc = fmaf(v0.x, xa.x, acc); acc = fmaf(v0.y, xa.y, acc);
            acc = fmaf(v1.x, xa.z, acc); acc = fmaf(v1.y, xa.w, acc);
            acc = fmaf(v2.x, xb.x, acc); acc = fmaf(v2.y, xb.y, acc);
            acc = fmaf(v3.x, xb.z, acc); acc = fmaf(v3.y, xb.w, acc);
        }
    } else {
        for (int k = 0; k < count; k++) {
            uint32_t nib = (w[k >> 3] >> (4 * (k & 7))) & 15u;
            f2 v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(nib, 1.0f, 0);
            acc = fmaf(v.x, x[k], acc);
        }
    }
    return acc;
}

// One MXFP4 matrix against up to 8 activation vectors (tokens).  XF(t)
// returns token t's activation pointer; loops over tokens are unrolled to 8
// with guards so every array index is a compile-time constant.
struct MxMat {
    const uint8_t* codes;
    const uint8_t* scales;
    int rows, cols, nb;
};

constexpr int R = 4;      // rows per lane group
constexpr int WAVES = 4;
constexpr int MAXT = 8;

template <typename XF>
__device__ __forceinline__ void mx_rows(const MxMat& j, int ntok, XF xf, int row0, int lig,
                                        int lpg, float (&rs)[R][MAXT]) {
    for (int b = lig; b < j.nb; b += lpg) {
        uint4 c[R];
        float s[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = row0 + r;
            if (row < j.rows) {
                c[r] = ld_nt16(j.codes + ((size_t)row * j.nb + b) * 16);
                s[r] = e8m0(j.scales[(size_t)row * j.nb + b]);
            } else {
                c[r] = make_uint4(0, 0, 0, 0);
                s[r] = 0.0f;
            }
        }
        const int count = min(32, j.cols - 32 * b);
#pragma unroll
        for (int t = 0; t < MAXT; t++) {
            if (t < ntok) {
                const float* xb = xf(t) + 32 * b;
#pragma unroll
                for (int r = 0; r < R; r++) rs[r][t] = fmaf(block_dot(c[r], xb, count), s[r], rs[r][t]);
            }
        }
    }
}

__device__ __forceinline__ int pick_lpg(int nb) {
    int lpg = 1;
    while (lpg < nb && lpg < 64) lpg <<= 1;
    return lpg;
}

__device__ __forceinline__ void zero_rs(float (&rs)[R][MAXT]) {
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < MAXT; t++) rs[r][t] = 0.0f;
}

// y[t][rows] = W x[t][cols], tokens contiguous.
__global__ __launch_bounds__(WAVES * 64) void mx_gemv_kernel(MxMat j, int ntok, const float* x,
                                                             float* y) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lpg = pick_lpg(j.nb), grp = lane / lpg, lig = lane % lpg;
    const int rows_per_wave = (64 / lpg) * R;
    const int row0 = blockIdx.x * WAVES * rows_per_wave + wave * rows_per_wave + grp * R;
    float rs[R][MAXT];
    zero_rs(rs);
    mx_rows(j, ntok, [&](int t) { return x + (size_t)t * j.cols; }, row0, lig, lpg, rs);
#pragma unroll
    for (int t = 0; t < MAXT; t++) {
        if (t < ntok) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float v = qsf::group_sum(rs[r][t], lpg);
                if (lig == (r & (lpg - 1)) && row0 + r < j.rows) y[(size_t)t * j.rows + row0 + r] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// MoE
typedef qk_mx_expert MxExpert;

constexpr int MAX_TOK = 8;
constexpr int MAX_K = 8;
constexpr int MAX_EXP = 256;

// Routing result shared by the three MoE kernels.
struct Route {
    int idx[MAX_TOK][MAX_K];
    float w[MAX_TOK][MAX_K];
    int owner[MAX_TOK * MAX_K];            // 1 if slot (t,k) is the first to pick its expert
    int ntl[MAX_TOK * MAX_K];              // tokens served by an owner slot
    int tl[MAX_TOK * MAX_K][MAX_TOK];      // their slot ids (t*K + k)
};

// softmax (src/kernels_scalar.c:187-214) + top-K (src/engine.c:987-1018)
__device__ void route_token(const float* __restrict__ logits, int n_exp, int k, int norm,
                            float* probs, int* idx, float* w) {
    float mx = logits[0];
    for (int i = 1; i < n_exp; i++) mx = logits[i] > mx ? logits[i] : mx;
    float sum = 0.0f;
    for (int i = 0; i < n_exp; i++) { probs[i] = expf(logits[i] - mx); sum += probs[i]; }
    if (sum < 1e-30f) {
        for (int i = 0; i < n_exp; i++) probs[i] = 1.0f / (float)n_exp;
    } else {
        const float inv = 1.0f / sum;
        for (int i = 0; i < n_exp; i++) probs[i] *= inv;
    }
    for (int i = 0; i < k; i++) { idx[i] = -1; w[i] = -1e30f; }
    for (int e = 0; e < n_exp; e++) {
        const float p = probs[e];
        for (int i = 0; i < k; i++) {
            if (p > w[i]) {
                for (int q = k - 1; q > i; q--) { w[q] = w[q - 1]; idx[q] = idx[q - 1]; }
                w[i] = p; idx[i] = e;
                break;
            }
        }
    }
    if (norm) {
        float s = 0.0f;
        for (int i = 0; i < k; i++) s += w[i];
        if (s > 0.0f) {
            const float inv = 1.0f / s;
            for (int i = 0; i < k; i++) w[i] *= inv;
        }
    }
}

// Every workgroup of the gate/up kernel computes the (tiny) routing itself;
// workgroup 0 also publishes it for the down and combine kernels.
__device__ void compute_route(const float* __restrict__ logits, int n_exp, int k, int norm,
                              int ntok, Route& rt, float* probs_lds) {
    if (threadIdx.x < ntok) {
        const int t = threadIdx.x;
        route_token(logits + (size_t)t * n_exp, n_exp, k, norm, probs_lds + t * n_exp,
                    rt.idx[t], rt.w[t]);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int ns = ntok * k;
        for (int s = 0; s < ns; s++) {
            const int e = rt.idx[s / k][s % k];
            int first = e >= 0;
            for (int q = 0; q < s && first; q++)
                if (rt.idx[q / k][q % k] == e) first = 0;
            rt.owner[s] = first;
            rt.ntl[s] = 0;
            if (first)
                for (int q = s; q < ns; q++)
                    if (rt.idx[q / k][q % k] == e) rt.tl[s][rt.ntl[s]++] = q;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ float act_fn(int act, float v) {
    if (act == 2) return v / (1.0f + expf(-v));                       // SiLU
    if (act == 0 || act == 1) {                                       // GELU (tanh)
        const float inner = 0.7978845608f * (v + 0.044715f * v * v * v);
        return 0.5f * v * (1.0f + tanhf(inner));
    }
    return v < 0.0f ? 0.0f : v;                                       // ReLU
}

struct MoeArgs {
    const MxExpert* experts;
    int n_exp, k, norm, act, hidden, eid, ntok;
    const float* x;        // [ntok][hidden]
    const float* logits;   // [ntok][n_exp]
    float* out;            // [ntok][hidden]
    Route* route;          // workspace
    float* h;              // [ntok*k][eid]   act(gate)*up
    float* d;              // [ntok*k][hidden] down outputs
    int tiles_gu, tiles_dn;
};

__global__ __launch_bounds__(WAVES * 64) void moe_gate_up_kernel(MoeArgs a) {
    __shared__ Route rt;
    __shared__ float probs[MAX_TOK * MAX_EXP];
    compute_route(a.logits, a.n_exp, a.k, a.norm, a.ntok, rt, probs);
    if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i < (int)(sizeof(Route) / 4); i += blockDim.x)
            reinterpret_cast<int*>(a.route)[i] = reinterpret_cast<const int*>(&rt)[i];
    }
    const int slot = blockIdx.x / a.tiles_gu, tile = blockIdx.x % a.tiles_gu;
    if (slot >= a.ntok * a.k || !rt.owner[slot]) return;
    const int e = rt.idx[slot / a.k][slot % a.k];
    const MxExpert ex = a.experts[e];
    const int nb = (a.hidden + 31) / 32;
    const MxMat g = {ex.gc, ex.gs, a.eid, a.hidden, nb};
    const MxMat u = {ex.uc, ex.us, a.eid, a.hidden, nb};
    const int ntl = rt.ntl[slot];
    const int* tl = rt.tl[slot];
    auto xf = [&](int t) { return a.x + (size_t)(tl[t] / a.k) * a.hidden; };
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lpg = pick_lpg(nb), grp = lane / lpg, lig = lane % lpg;
    const int rows_per_wave = (64 / lpg) * R;
    const int row0 = tile * WAVES * rows_per_wave + wave * rows_per_wave + grp * R;
    float rg[R][MAXT], ru[R][MAXT];
    zero_rs(rg);
    zero_rs(ru);
    mx_rows(g, ntl, xf, row0, lig, lpg, rg);
    mx_rows(u, ntl, xf, row0, lig, lpg, ru);
#pragma unroll
    for (int i = 0; i < MAXT; i++) {
        if (i < ntl) {
            const int s2 = tl[i];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float gv = qsf::group_sum(rg[r][i], lpg);
                const float uv = qsf::group_sum(ru[r][i], lpg);
                const int row = row0 + r;
                if (lig == (r & (lpg - 1)) && row < a.eid) {
                    float gg = gv, uu = uv;
                    if (ex.gb) gg += qsf::f16_bits(ex.gb[row]);
                    if (ex.ub) uu += qsf::f16_bits(ex.ub[row]);
                    a.h[(size_t)s2 * a.eid + row] = act_fn(a.act, gg) * uu;
                }
            }
        }
    }
}

__global__ __launch_bounds__(WAVES * 64) void moe_down_kernel(MoeArgs a) {
    const Route* rt = a.route;
    const int slot = blockIdx.x / a.tiles_dn, tile = blockIdx.x % a.tiles_dn;
    if (slot >= a.ntok * a.k || !rt->owner[slot]) return;
    const int e = rt->idx[slot / a.k][slot % a.k];
    const MxExpert ex = a.experts[e];
    const int nb = (a.eid + 31) / 32;
    const MxMat dm = {ex.dc, ex.ds, a.hidden, a.eid, nb};
    const int ntl = rt->ntl[slot];
    const int* tl = rt->tl[slot];
    auto xf = [&](int t) { return (const float*)(a.h + (size_t)tl[t] * a.eid); };
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lpg = pick_lpg(nb), grp = lane / lpg, lig = lane % lpg;
    const int rows_per_wave = (64 / lpg) * R;
    const int row0 = tile * WAVES * rows_per_wave + wave * rows_per_wave + grp * R;
    float rs[R][MAXT];
    zero_rs(rs);
    mx_rows(dm, ntl, xf, row0, lig, lpg, rs);
#pragma unroll
    for (int i = 0; i < MAXT; i++) {
        if (i < ntl) {
            float* y = a.d + (size_t)tl[i] * a.hidden;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float v = qsf::group_sum(rs[r][i], lpg);
                const int row = row0 + r;
                if (lig == (r & (lpg - 1)) && row < a.hidden)
                    y[row] = ex.db ? v + qsf::f16_bits(ex.db[row]) : v;
            }
        }
    }
}

// out[t] = sum over the token's experts, in rank order, of w * down
// (src/engine.c:1021, 1104-1106).
__global__ void moe_combine_kernel(MoeArgs a) {
    const Route& rt = *a.route;
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.hidden) return;
    float acc = 0.0f;
    for (int q = 0; q < a.k; q++) {
        if (rt.idx[t][q] < 0) continue;
        acc += rt.w[t][q] * a.d[(size_t)(t * a.k + q) * a.hidden + i];
    }
    a.out[(size_t)t * a.hidden + i] = acc;
}

}  // namespace

extern "C" int qk_mxfp4_gemv(const qsf_hip_tensor* t, const float* d_x, int ntok, float* d_y,
                             hipStream_t s) {
    if (ntok < 1 || ntok > MAXT) return -2;
    if (t->rows <= 0) return 0;
    if (t->cols % 4) return -2;   // float4 activation loads
    const MxMat j = {t->d_blocks, t->d_scales, t->rows, t->cols, t->nb};
    int lpg = 1;
    while (lpg < j.nb && lpg < 64) lpg <<= 1;
    const int rows_per_wg = WAVES * (64 / lpg) * R;
    hipLaunchKernelGGL(mx_gemv_kernel, dim3((t->rows + rows_per_wg - 1) / rows_per_wg),
                       dim3(WAVES * 64), 0, s, j, ntok, d_x, d_y);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" size_t qk_moe_ws_bytes(int n_exp, int k, int ntok, int hidden, int eid) {
    (void)n_exp;
    size_t r = (sizeof(Route) + 255) & ~(size_t)255;
    size_t h = ((size_t)ntok * k * eid * 4 + 255) & ~(size_t)255;
    size_t d = ((size_t)ntok * k * hidden * 4 + 255) & ~(size_t)255;
    return r + h + d;
}

extern "C" int qk_moe_launch(const qk_mx_expert* d_experts, int n_exp, int k, int norm, int act,
                             int hidden, int eid, int ntok, const float* d_x,
                             const float* d_logits, float* d_out, void* d_ws, hipStream_t s) {
    if (ntok < 1 || ntok > MAX_TOK || k < 1 || k > MAX_K || n_exp < 1 || n_exp > MAX_EXP ||
        hidden < 1 || eid < 1 || (hidden % 4) || (eid % 4))
        return -2;
    MoeArgs a = {};
    a.experts = d_experts;
    a.n_exp = n_exp; a.k = k; a.norm = norm; a.act = act;
    a.hidden = hidden; a.eid = eid; a.ntok = ntok;
    a.x = d_x; a.logits = d_logits; a.out = d_out;
    uint8_t* ws = (uint8_t*)d_ws;
    a.route = (Route*)ws;
    size_t r = (sizeof(Route) + 255) & ~(size_t)255;
    a.h = (float*)(ws + r);
    a.d = (float*)(ws + r + (((size_t)ntok * k * eid * 4 + 255) & ~(size_t)255));
    auto tiles = [](int rows, int cols) {
        int nb = (cols + 31) / 32, lpg = 1;
        while (lpg < nb && lpg < 64) lpg <<= 1;
        const int rpw = WAVES * (64 / lpg) * R;
        return (rows + rpw - 1) / rpw;
    };
    a.tiles_gu = tiles(eid, hidden);
    a.tiles_dn = tiles(hidden, eid);
    const int slots = ntok * k;
    hipLaunchKernelGGL(moe_gate_up_kernel, dim3(slots * a.tiles_gu), dim3(WAVES * 64), 0, s, a);
    hipLaunchKernelGGL(moe_down_kernel, dim3(slots * a.tiles_dn), dim3(WAVES * 64), 0, s, a);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((hidden + 255) / 256, ntok), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

