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

#include <hip/hip_ext.h>

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
            // (a select chain: a runtime index into w[] would put it in scratch)
            const uint32_t wk = k < 8 ? c.x : k < 16 ? c.y : k < 24 ? c.z : c.w;
            uint32_t nib = (wk >> (4 * (k & 7))) & 15u;
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
constexpr int MAX_SLOTS = MAX_TOK * MAX_K;     // slot s = t*K + rank; one lane each
static_assert(MAX_SLOTS <= 64 && MAX_TOK <= 32, "one wave routes every slot; token masks are 32-bit");

// A distinct expert and the slots that picked it, in slot order (a token
// picks an expert at most once, so at most MAX_TOK slots).
struct Work {
    int expert, n;
    int slot[MAX_TOK];
};
struct Route {
    int idx[MAX_SLOTS];        // expert of slot s (-1: none)
    float w[MAX_SLOTS];        // its routing weight
    int nwork;
    Work work[MAX_SLOTS];      // distinct experts in order of first pick
};


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
    float* h;              // [ntok*k][eid]   act(gate)*up per slot
    float* d;              // [ntok*k][hidden] down outputs per slot
};

// Routing of token t by one wave, into s_idx/s_w[t*K .. t*K+K-1]:
// softmax (src/kernels_scalar.c:187-214) and top-K (src/engine.c:987-1018).
// - max: the reference's running max from x[0] keeps the largest non-NaN
//   value (NaN never wins a '>') unless x[0] itself is NaN; a DPP max tree
//   over the non-NaN values is the same number.
// - sum: in index order as the reference adds, each lane running the same
//   sequential fp32 sum over the wave's exps in LDS (broadcast reads).
// - top-K as ranks: expert e takes place r = #{q : p_q > p_e, or p_q == p_e
//   and q < e} among those with p > -1e30 (NaN never qualifies), the order
//   the strict '>' insertion from a -1e30 start produces; each lane counts
//   its rank against every p in LDS.
// - optional renormalisation by the rank-ordered sum.
// sp: this wave's LDS scratch of MAX_EXP floats.  RJ experts per lane: 1 for
// up to 64 experts, else MAX_EXP / 64.
__device__ __forceinline__ float wave_max_dpp(float v) {
#define QSF_DPPM(x, ctrl, rmask) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -__builtin_inff()), \
                                                          __builtin_bit_cast(int, (x)), (ctrl), (rmask), 0xF, false))
    v = fmaxf(v, QSF_DPPM(v, 0xB1, 0xF));     // quad_perm [1,0,3,2]
    v = fmaxf(v, QSF_DPPM(v, 0x4E, 0xF));     // quad_perm [2,3,0,1]
    v = fmaxf(v, QSF_DPPM(v, 0x141, 0xF));    // row_half_mirror
    v = fmaxf(v, QSF_DPPM(v, 0x140, 0xF));    // row_mirror
    v = fmaxf(v, QSF_DPPM(v, 0x142, 0xA));    // row_bcast15
    v = fmaxf(v, QSF_DPPM(v, 0x143, 0xC));    // row_bcast31
#undef QSF_DPPM
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

template <int RJ>
__device__ void route_token(const float* __restrict__ lg, int n, int k, int norm, int t,
                            int* s_idx, float* s_w, float* sp) {
    const int lane = threadIdx.x & 63;
    if (lane < k) { s_idx[t * k + lane] = -1; s_w[t * k + lane] = -1e30f; }
    float v[RJ];
#pragma unroll
    for (int j = 0; j < RJ; j++) v[j] = lane + 64 * j < n ? lg[lane + 64 * j] : 0.0f;
    const float v0 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v[0])));
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < RJ; j++)
        if (lane + 64 * j < n) m = fmaxf(m, v[j]);          // fmaxf skips NaN
    const float mx = v0 != v0 ? v0 : wave_max_dpp(m);
#pragma unroll
    for (int j = 0; j < RJ; j++) {
        v[j] = expf(v[j] - mx);
        if (lane + 64 * j < n) sp[lane + 64 * j] = v[j];
    }
    __builtin_amdgcn_wave_barrier();
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += sp[i];
    const bool flat = sum < 1e-30f;
    const float inv = 1.0f / sum;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < RJ; j++) {
        v[j] = flat ? 1.0f / (float)n : v[j] * inv;
        if (lane + 64 * j < n) sp[lane + 64 * j] = v[j];
    }
    __builtin_amdgcn_wave_barrier();
    int rank[RJ];
#pragma unroll
    for (int j = 0; j < RJ; j++) rank[j] = 0;
    for (int q = 0; q < n; q++) {
        const float pq = sp[q];
#pragma unroll
        for (int j = 0; j < RJ; j++) {
            const int e = lane + 64 * j;
            rank[j] += pq > -1e30f && (pq > v[j] || (pq == v[j] && q < e)) ? 1 : 0;
        }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < RJ; j++) {
        const int e = lane + 64 * j;
        if (e < n && v[j] > -1e30f && rank[j] < k) { s_idx[t * k + rank[j]] = e; s_w[t * k + rank[j]] = v[j]; }
    }
    __builtin_amdgcn_wave_barrier();
    if (norm) {
        float ws = 0.0f;
        for (int i = 0; i < k; i++) ws += s_w[t * k + i];
        __builtin_amdgcn_wave_barrier();
        if (ws > 0.0f && lane < k) s_w[t * k + lane] *= 1.0f / ws;
    }
}

// The distinct experts of the routed slots, in order of first pick, each
// with the slots that picked it in slot order (wave 0, lane = slot, after
// every token is routed).  A token picks an expert at most once, so the mask
// of the tokens that picked expert e (an LDS OR, whatever the lane order)
// gives its slot count, its first slot and each slot's place in its list,
// all in one pass over the lanes.  s_tok, s_item: LDS, MAX_EXP each.
__device__ void build_work(const int* s_idx, int ns, int k, unsigned* s_tok, int* s_item, Route& rt) {
    const int lane = threadIdx.x & 63;
    const int e = lane < ns ? s_idx[lane] : -1;
    const int t = lane / k;
    if (e >= 0) s_tok[e] = 0u;
    __builtin_amdgcn_wave_barrier();
    if (e >= 0) atomicOr(&s_tok[e], 1u << t);
    __builtin_amdgcn_wave_barrier();
    const unsigned m = e >= 0 ? s_tok[e] : 0u;
    const bool first = e >= 0 && __builtin_ctz(m) == t;  // the earliest token's slot
    const uint64_t owners = __ballot(first);
    if (first) s_item[e] = __popcll(owners & ((1ull << lane) - 1));
    __builtin_amdgcn_wave_barrier();
    if (e >= 0) {
        Work& w = rt.work[s_item[e]];
        w.slot[__popc(m & ((1u << t) - 1))] = lane;
        if (first) {
            w.expert = e;
            w.n = __popc(m);
        }
    }
    if (lane == 0) rt.nwork = __popcll(owners);
}

// LDS pitch of one staged 32-element block, in floats: 4 floats of padding
// put the blocks that neighbouring lanes read 16 bytes apart in the banks
// (at a 128-byte pitch eight lanes of a 16-byte read hit the same banks).
constexpr int XBP = 36;

// Expert GEMV tile: NM matrices with the same shape ([rows][cols] MXFP4)
// against the inputs xs[i] (LDS, i < n) of one work item.  A 32-lane group
// owns MR consecutive rows; lane l reads blocks l, l+32, ... of each row, so
// a row's 16-byte code loads are contiguous across the group, and all NI
// blocks of a lane are loaded before stage() stages the inputs.  The codes
// stay in registers while a runtime loop walks the inputs; for each input
// the lane partial sums acc[m][r] go to done(i, acc).
// Rows per 32-lane group (rows per workgroup waves * 2 * MR): 1 for gate/up
// and down (about 64 registers, so many workgroups stay resident; two rows
// took 158-206), and 1 for the batch-1 fused down too, where a workgroup
// carries four experts' rows: 4-row workgroups make 720 of them at hidden
// 2880, three a CU, with more loads in flight than 240 of 12 rows (batch-1
// step 20.7 -> 20.0 us; 8-row workgroups 22.7 us).
constexpr int GU_MR = 1, DN_MR = 1, FD_MR = 1;
// Waves an expert workgroup: 8, so the 16 rows of a workgroup share one
// staging of its inputs (4-wave workgroups staged them for 8 rows).
constexpr int GU_WAVES = 8, DN_WAVES = 8;
// Inputs staged in LDS at a time: an expert averages one or two tokens, and
// LDS sized for the whole batch (8 tokens: 103 KB at hidden 2880) would hold
// a CU to one expert workgroup.
constexpr int TCH = 2;

template <int NM, int NI, int MR, typename PRE, typename STAGE, typename DONE>
__device__ __forceinline__ void mx_tile(const MxMat (&mat)[NM], const float* xs, int n, int row0,
                                        int lig, PRE pre, STAGE stage, DONE done) {
    // the first chunk's inputs into registers ahead of the code loads, so
    // they do not queue behind the weights
    pre();
    uint4 c[NI][NM][MR];
    float sc[NI][NM][MR];
#pragma unroll
    for (int it = 0; it < NI; it++) {
        const int b = min(lig + 32 * it, mat[0].nb - 1);
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < MR; r++) {
                const size_t at = (size_t)min(row0 + r, mat[m].rows - 1) * mat[m].nb + b;
                c[it][m][r] = ld_nt16(mat[m].codes + at * 16);
                sc[it][m][r] = e8m0(mat[m].scales[at]);
            }
    }
    // inputs TCH at a time (LDS for TCH inputs, not the batch): the first
    // chunk is written to LDS from the registers pre() filled
    stage(0, n < TCH ? n : TCH);
#pragma unroll 1
    for (int i = 0; i < n; i++) {
        if (i > 0 && i % TCH == 0) {
            __syncthreads();               // every wave done with the previous chunk
            stage(i, n - i < TCH ? n - i : TCH);
        }
        float acc[NM][MR];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < MR; r++) acc[m][r] = 0.0f;
#pragma unroll
        for (int it = 0; it < NI; it++) {
            const int b = lig + 32 * it;
            // inputs are zero-padded to whole blocks in LDS; lanes past the
            // last block add nothing
            const float4* x4 = reinterpret_cast<const float4*>(xs + (size_t)(i % TCH) * XBP * mat[0].nb +
                                                               XBP * min(b, mat[0].nb - 1));
            const bool live = b < mat[0].nb;
            float dot[NM][MR];
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < MR; r++) dot[m][r] = 0.0f;
            // one code word (8 elements) of every row at a time, so only
            // that word's values are live
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 xa = x4[2 * q], xc = x4[2 * q + 1];
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int r = 0; r < MR; r++) {
                        uint32_t w = q == 0 ? c[it][m][r].x : q == 1 ? c[it][m][r].y
                                   : q == 2 ? c[it][m][r].z : c[it][m][r].w;
                        // converted per input: hoisting the conversions out
                        // of the input loop would hold every row's 32 floats
                        asm volatile("" : "+v"(w));
                        const f2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
                        const f2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
                        const f2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
                        const f2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
                        float d = dot[m][r];
                        d = fmaf(v0.x, xa.x, d); d = fmaf(v0.y, xa.y, d);
                        d = fmaf(v1.x, xa.z, d); d = fmaf(v1.y, xa.w, d);
                        d = fmaf(v2.x, xc.x, d); d = fmaf(v2.y, xc.y, d);
                        d = fmaf(v3.x, xc.z, d); d = fmaf(v3.y, xc.w, d);
                        dot[m][r] = d;
                    }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < MR; r++) {
                    const float v = fmaf(dot[m][r], sc[it][m][r], acc[m][r]);
                    acc[m][r] = live ? v : acc[m][r];
                }
        }
        done(i, acc);
    }
}

// Stage a work item's input vectors (n rows of `cols` floats, row i at
// src(i)) into LDS as nb blocks of XBP floats, zero past cols.
template <typename SRC>
__device__ __forceinline__ void stage_inputs(float* xs, int n, int cols, int nb, SRC src) {
    for (int i = 0; i < n; i++) {
        const float4* s4 = reinterpret_cast<const float4*>(src(i));
        float* d = xs + (size_t)i * nb * XBP;
#pragma unroll 4
        for (int j = threadIdx.x; j < nb * 8; j += blockDim.x)
            *reinterpret_cast<float4*>(d + (j >> 3) * XBP + 4 * (j & 7)) =
                j < cols / 4 ? s4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// Inputs of the first chunk in registers: vectors i < n (n <= T) of cols
// <= 4096 floats over 512 threads, XR float4s a thread; put_inputs writes
// them in stage_inputs' LDS layout.
constexpr int XR = 2;
static_assert(GU_WAVES * 64 * XR * 4 >= 4096 && DN_WAVES * 64 * XR * 4 >= 4096,
              "one register chunk holds a 4096-float input");
template <int T, typename SRC>
__device__ __forceinline__ void load_inputs(float4 (&xr)[T][XR], int n, int cols, SRC src) {
#pragma unroll
    for (int i = 0; i < T; i++)
#pragma unroll
        for (int q = 0; q < XR; q++) {
            const int j = threadIdx.x + q * blockDim.x;
            xr[i][q] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < n && j < cols / 4) xr[i][q] = reinterpret_cast<const float4*>(src(i))[j];
        }
}
template <int T>
__device__ __forceinline__ void put_inputs(float* xs, const float4 (&xr)[T][XR], int n, int nb) {
#pragma unroll
    for (int i = 0; i < T; i++)
#pragma unroll
        for (int q = 0; q < XR; q++) {
            const int j = threadIdx.x + q * blockDim.x;
            if (i < n && j < nb * 8)
                *reinterpret_cast<float4*>(xs + (size_t)i * nb * XBP + (j >> 3) * XBP + 4 * (j & 7)) = xr[i][q];
        }
}

// Pointer fields [F0, F0 + NF) of every expert's table entry into LDS,
// tab[e * NF + f], by the threads from t0 up of a TB-thread workgroup: the
// loads into registers (table_load), then the LDS stores (table_store).
// Loaded at a kernel's start, beside the routing or the route record's
// reads (issued between the two calls, so that neither waits for the
// other), the entries a work item needs are an LDS read away once its
// expert is known, instead of one more memory round trip in front of the
// first weight load.  The caller synchronises the workgroup before reading.
static_assert(sizeof(MxExpert) == 9 * sizeof(void*), "expert table entry: nine pointers");
template <int NF, int TB, int T0>
constexpr int kTabPer = (MAX_EXP * NF + TB - T0 - 1) / (TB - T0);   // entries a thread
template <int F0, int NF, int TB, int T0>
__device__ __forceinline__ void table_load(const MxExpert* ex, int n_exp, uint64_t (&tv)[kTabPer<NF, TB, T0>]) {
    const uint64_t* src = reinterpret_cast<const uint64_t*>(ex);
#pragma unroll
    for (int j = 0; j < kTabPer<NF, TB, T0>; j++) {
        const int i = (int)threadIdx.x - T0 + j * (TB - T0);
        const int e = i / NF, f = i - e * NF;
        tv[j] = i >= 0 && i < n_exp * NF ? src[e * 9 + F0 + f] : 0ull;
    }
}
template <int NF, int TB, int T0>
__device__ __forceinline__ void table_store(int n_exp, const uint64_t (&tv)[kTabPer<NF, TB, T0>], uint64_t* tab) {
#pragma unroll
    for (int j = 0; j < kTabPer<NF, TB, T0>; j++) {
        const int i = (int)threadIdx.x - T0 + j * (TB - T0);
        if (i >= 0 && i < n_exp * NF) tab[i] = tv[j];
    }
}
template <typename T>
__device__ __forceinline__ T tab_ptr(const uint64_t* tab, int i) {
    return reinterpret_cast<T>(tab[i]);
}

// Routing once per step: one wave per token, then the distinct-expert list
// (one launch of MAX_TOK waves; the expert kernels read the result).
__global__ __launch_bounds__(MAX_TOK * 64) void moe_route_kernel(MoeArgs a) {
    __shared__ int s_idx[MAX_SLOTS];
    __shared__ float s_w[MAX_SLOTS];
    __shared__ float s_p[MAX_TOK][MAX_EXP];
    __shared__ unsigned s_tok[MAX_EXP];
    __shared__ int s_item[MAX_EXP];
    const int t = threadIdx.x >> 6;
    if (t < a.ntok) {
        const float* lg = a.logits + (size_t)t * a.n_exp;
        if (a.n_exp <= 64) route_token<1>(lg, a.n_exp, a.k, a.norm, t, s_idx, s_w, s_p[t]);
        else route_token<MAX_EXP / 64>(lg, a.n_exp, a.k, a.norm, t, s_idx, s_w, s_p[t]);
    }
    __syncthreads();
    if (t != 0) return;
    const int lane = threadIdx.x, ns = a.ntok * a.k;
    Route& rt = *a.route;
    if (lane < ns) {
        rt.idx[lane] = s_idx[lane];
        rt.w[lane] = s_w[lane];
    }
    build_work(s_idx, ns, a.k, s_tok, s_item, rt);
}

// Gate/up: workgroup (x, y) computes rows of row tile x of the gate and up
// matrices of distinct expert y for the tokens that picked it:
// h[slot] = act(gate + b) * (up + b).
// RT (one token): every workgroup routes the token itself (one wave; what
// the route kernel does) instead of waiting for a routing launch, and
// workgroup (0, 0) stores the result for the down kernel.
template <int NI, bool RT>
__global__ __launch_bounds__(GU_WAVES * 64) void moe_gate_up_kernel(MoeArgs a) {
    constexpr int MR = GU_MR;
    extern __shared__ __align__(16) float xs[];           // [n][hidden, padded], expert table
    float4 xr[TCH][XR];
    const Route* rtp = a.route;
    const int nb = (a.hidden + 31) / 32;
    // in-kernel routing: the expert table after the input (wave 0 routes,
    // the others load the table)
    uint64_t* tab = reinterpret_cast<uint64_t*>(xs + (size_t)nb * XBP);
    constexpr int T0 = 64;
    if constexpr (RT) {
        uint64_t tv[kTabPer<6, GU_WAVES * 64, T0>];
        // the one token's input does not depend on the routing: loaded first
        load_inputs<TCH>(xr, 1, a.hidden, [&](int) { return a.x; });
        table_load<0, 6, GU_WAVES * 64, T0>(a.experts, a.n_exp, tv);
        __shared__ int s_idx[MAX_K];
        __shared__ float s_w[MAX_K];
        __shared__ float s_p[MAX_EXP];
        __shared__ unsigned s_tok[MAX_EXP];
        __shared__ int s_item[MAX_EXP];
        __shared__ Route s_rt;
        if (threadIdx.x < 64) {
            if (a.n_exp <= 64) route_token<1>(a.logits, a.n_exp, a.k, a.norm, 0, s_idx, s_w, s_p);
            else route_token<MAX_EXP / 64>(a.logits, a.n_exp, a.k, a.norm, 0, s_idx, s_w, s_p);
            __builtin_amdgcn_wave_barrier();
            if ((int)threadIdx.x < a.k) {
                s_rt.idx[threadIdx.x] = s_idx[threadIdx.x];
                s_rt.w[threadIdx.x] = s_w[threadIdx.x];
            }
            build_work(s_idx, a.k, a.k, s_tok, s_item, s_rt);
        }
        table_store<6, GU_WAVES * 64, T0>(a.n_exp, tv, tab);
        __syncthreads();
        if (blockIdx.x == 0 && blockIdx.y == 0) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(&s_rt);
            uint32_t* dst = reinterpret_cast<uint32_t*>(a.route);
            for (int i = threadIdx.x; i < (int)(sizeof(Route) / 4); i += blockDim.x) dst[i] = src[i];
        }
        rtp = &s_rt;
    }
    if ((int)blockIdx.y >= rtp->nwork) return;
    const Work& wk = rtp->work[blockIdx.y];
    struct { const uint8_t *gc, *gs; const uint16_t* gb; const uint8_t *uc, *us; const uint16_t* ub; } ex;
    if constexpr (RT) {
        const uint64_t* te = tab + wk.expert * 6;
        ex = {tab_ptr<const uint8_t*>(te, 0), tab_ptr<const uint8_t*>(te, 1), tab_ptr<const uint16_t*>(te, 2),
              tab_ptr<const uint8_t*>(te, 3), tab_ptr<const uint8_t*>(te, 4), tab_ptr<const uint16_t*>(te, 5)};
    } else {
        // (many workgroup rounds: a table copy in each cost more than the
        // one dependent read it saves)
        const MxExpert& e = a.experts[wk.expert];
        ex = {e.gc, e.gs, e.gb, e.uc, e.us, e.ub};
    }
    const MxMat mat[2] = {{ex.gc, ex.gs, a.eid, a.hidden, nb}, {ex.uc, ex.us, a.eid, a.hidden, nb}};
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lig = lane & 31;
    const int row0 = blockIdx.x * (GU_WAVES * 2 * MR) + wave * 2 * MR + (lane >> 5) * MR;
    auto src = [&](int i) { return a.x + (size_t)(wk.slot[i] / a.k) * a.hidden; };
    auto pre = [&]() {
        if constexpr (!RT) load_inputs<TCH>(xr, wk.n, a.hidden, src);
    };
    auto stage = [&](int i0, int cnt) {
        if (i0 == 0) put_inputs<TCH>(xs, xr, cnt, nb);
        else stage_inputs(xs, cnt, a.hidden, nb, [&](int i) { return src(i0 + i); });
        __syncthreads();
    };
    mx_tile<2, NI, MR>(mat, xs, wk.n, row0, lig, pre, stage, [&](int i, const float (&acc)[2][MR]) {
        const int s2 = wk.slot[i];
#pragma unroll
        for (int r = 0; r < MR; r++) {
            const float gv = qsf::group_sum_last(acc[0][r], 32);
            const float uv = qsf::group_sum_last(acc[1][r], 32);
            const int row = row0 + r;
            if (lig == 31 && row < a.eid) {
                float gg = gv, uu = uv;
                if (ex.gb) gg += qsf::f16_bits(ex.gb[row]);
                if (ex.ub) uu += qsf::f16_bits(ex.ub[row]);
                a.h[(size_t)s2 * a.eid + row] = act_fn(a.act, gg) * uu;
            }
        }
    });
}

// Down: workgroup (x, y) computes rows of row tile x of expert y's down
// matrix for its slots, d[slot] = down h[slot] + b.
template <int NI>
__global__ __launch_bounds__(DN_WAVES * 64) void moe_down_kernel(MoeArgs a) {
    extern __shared__ __align__(16) float xs[];           // [n][eid, padded]
    if ((int)blockIdx.y >= a.route->nwork) return;
    const Work& wk = a.route->work[blockIdx.y];
    const int n = wk.n;
    const MxExpert ex = a.experts[wk.expert];
    const int nb = (a.eid + 31) / 32;
    const MxMat mat[1] = {{ex.dc, ex.ds, a.hidden, a.eid, nb}};
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lig = lane & 31;
    constexpr int MR = DN_MR;
    const int row0 = blockIdx.x * (DN_WAVES * 2 * MR) + wave * 2 * MR + (lane >> 5) * MR;
    auto src = [&](int i) { return (const float*)(a.h + (size_t)wk.slot[i] * a.eid); };
    float4 xr[TCH][XR];
    auto pre = [&]() { load_inputs<TCH>(xr, n, a.eid, src); };
    auto stage = [&](int i0, int cnt) {
        if (i0 == 0) put_inputs<TCH>(xs, xr, cnt, nb);
        else stage_inputs(xs, cnt, a.eid, nb, [&](int i) { return src(i0 + i); });
        __syncthreads();
    };
    mx_tile<1, NI, MR>(mat, xs, n, row0, lig, pre, stage, [&](int i, const float (&acc)[1][MR]) {
        float* y = a.d + (size_t)wk.slot[i] * a.hidden;
#pragma unroll
        for (int r = 0; r < MR; r++) {
            const float v = qsf::group_sum_last(acc[0][r], 32);
            const int row = row0 + r;
            if (lig == 31 && row < a.hidden) y[row] = ex.db ? v + qsf::f16_bits(ex.db[row]) : v;
        }
    });
}

// Down and combine in one launch for one token with at most FG experts
// (batch-1 decode).  The FG wave groups of a workgroup each take one expert
// (work item g = the token's rank g) over the workgroup's FROWS rows; the
// rows' sums meet in LDS and the workgroup adds them in rank order like the
// combine kernel below (src/engine.c:1021, 1104-1106).
constexpr int FG = 4;                      // wave groups: experts of the token
constexpr int FGW = 2;                     // waves a group (512 threads: 256 VGPRs a lane)
constexpr int FMR = FD_MR;                 // rows per 32-lane group
constexpr int FROWS = FGW * 2 * FMR;       // rows of a workgroup (4)
template <int NI>
__global__ __launch_bounds__(FG * FGW * 64) void moe_down_fused_kernel(MoeArgs a) {
    // [FG][eid, padded], then [FG][FROWS] row sums, then the expert table
    extern __shared__ __align__(16) float xs[];
    const Route& rt = *a.route;
    const int nb = (a.eid + 31) / 32;
    float* part = xs + (size_t)FG * nb * XBP;
    uint64_t* tab = reinterpret_cast<uint64_t*>(part + FG * FROWS);
    // The route record first, every read at a fixed address so that they
    // issue together: the count, each work item's expert and (one token)
    // slot, and the combine's ranks and weights (k <= FG here; loaded one
    // rank at a time at the end, each was a memory round trip in every
    // workgroup's tail).  Ranks past k and empty ranks are left out of the
    // sum below; items past the count are not used.  The table's loads are
    // issued first and its LDS stores follow these reads.
    uint64_t tv[kTabPer<3, FG * FGW * 64, 0>];
    table_load<6, 3, FG * FGW * 64, 0>(a.experts, a.n_exp, tv);
    const int nwork = rt.nwork;
    int w_e[FG], w_s[FG];
    bool on[FG];
    float wq[FG];
#pragma unroll
    for (int q = 0; q < FG; q++) {
        w_e[q] = rt.work[q].expert;
        w_s[q] = rt.work[q].slot[0];
        on[q] = (q < a.k) & (rt.idx[q] >= 0);    // '&': the load is not skipped
        wq[q] = rt.w[q];
    }
    asm volatile("" ::"s"(nwork), "s"(w_e[0]), "s"(w_e[1]), "s"(w_e[2]), "s"(w_e[3]), "s"(w_s[0]),
                 "s"(w_s[1]), "s"(w_s[2]), "s"(w_s[3]));   // (as gate/up)
    table_store<3, FG * FGW * 64, 0>(a.n_exp, tv, tab);
    if (nwork == 0) {                            // no expert picked: out = 0, as the combine
        const int row = blockIdx.x * FROWS + threadIdx.x;
        if ((int)threadIdx.x < FROWS && row < a.hidden) a.out[row] = 0.0f;
        return;
    }
    const int g = threadIdx.x / (FGW * 64);
    const int wl = (threadIdx.x >> 6) & (FGW - 1);
    const int lane = threadIdx.x & 63, lig = lane & 31;
    const int gi = g < nwork ? g : 0;            // groups past the experts recompute item 0, store nothing
    const int nst = nwork < FG ? nwork : FG;
    __syncthreads();
    int e_g = w_e[0];
#pragma unroll
    for (int i = 1; i < FG; i++) e_g = gi == i ? w_e[i] : e_g;
    const uint64_t* te = tab + e_g * 3;
    const struct { const uint8_t *dc, *ds; const uint16_t* db; } ex = {
        tab_ptr<const uint8_t*>(te, 0), tab_ptr<const uint8_t*>(te, 1), tab_ptr<const uint16_t*>(te, 2)};
    const MxMat mat[1] = {{ex.dc, ex.ds, a.hidden, a.eid, nb}};
    const int tile0 = blockIdx.x * FROWS;
    const int row0 = tile0 + wl * 2 * FMR + (lane >> 5) * FMR;
    // one input a group, all groups' at once, loaded ahead of the codes
    static_assert(FG * FGW * 64 * XR * 4 >= 4096, "one register chunk holds a 4096-float input");
    float4 xr[FG][XR];
    auto pre = [&]() {
        load_inputs<FG>(xr, nst, a.eid, [&](int i) { return (const float*)(a.h + (size_t)w_s[i] * a.eid); });
    };
    auto stage = [&](int, int) {
        put_inputs<FG>(xs, xr, nst, nb);
        __syncthreads();
    };
    mx_tile<1, NI, FMR>(mat, xs + (size_t)gi * nb * XBP, 1, row0, lig, pre, stage,
                        [&](int, const float (&acc)[1][FMR]) {
#pragma unroll
        for (int r = 0; r < FMR; r++) {
            const float v = qsf::group_sum_last(acc[0][r], 32);
            const int row = row0 + r;
            if (lig == 31 && g < nwork && row < a.hidden)
                part[g * FROWS + (row - tile0)] = ex.db ? v + qsf::f16_bits(ex.db[row]) : v;
        }
    });
    __syncthreads();
    if ((int)threadIdx.x < FROWS) {
        const int row = tile0 + threadIdx.x;
        if (row < a.hidden) {
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < FG; q++)
                if (on[q]) acc += wq[q] * part[q * FROWS + threadIdx.x];
            a.out[row] = acc;
        }
    }
}

// out[t] = sum over the token's ranks of w * d (src/engine.c:1021,
// 1104-1106); slots without an expert are skipped.
// Every rank's index, weight and output is loaded before the sum, without
// branches (slots are clamped into the workspace's MAX_SLOTS rows; ranks
// past k and empty ranks are then left out), so the loads overlap instead of
// each waiting on the rank's expert index.
__global__ void moe_combine_kernel(MoeArgs a) {
    const Route& rt = *a.route;
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.hidden) return;
    bool on[MAX_K];
    float wv[MAX_K], dv[MAX_K];
#pragma unroll
    for (int q = 0; q < MAX_K; q++) {
        const int s = min(t * a.k + q, MAX_SLOTS - 1);
        on[q] = (q < a.k) & (rt.idx[s] >= 0);            // '&': the load is not skipped
        wv[q] = rt.w[s];
        dv[q] = a.d[(size_t)s * a.hidden + i];
    }
    __builtin_amdgcn_sched_barrier(0);                    // every load issued before the sum
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < MAX_K; q++)
        if (on[q]) acc += wv[q] * dv[q];
    a.out[(size_t)t * a.hidden + i] = acc;
}

// Expert kernels with dynamic LDS: the first launch of an instantiation
// allows it what its static LDS leaves of 160 KB (inputs of 8 tokens exceed
// 64 KB).  `timed`
// launches record the library's kernel-timing event pair (diagnostics) when
// it is enabled.
template <auto K>
void launch_lds(dim3 g, dim3 b, size_t lds, hipStream_t s, const MoeArgs& a, bool timed = false) {
    static bool allowed = false;
    if (!allowed) {
        // what the kernel's static LDS leaves of the CU's 160 KB (asking for
        // more fails the call, and its error would be reported at the launch)
        hipFuncAttributes fa = {};
        const size_t st = hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(K)) == hipSuccess
                              ? fa.sharedSizeBytes : (size_t)16384;
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(K),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)(160 * 1024 - st));
        allowed = true;
    }
    hipEvent_t e0, e1;
    if (timed && qk_timing_pair(&e0, &e1))
        hipExtLaunchKernelGGL(K, g, b, (uint32_t)lds, s, e0, e1, 0, a);
    else
        hipLaunchKernelGGL(K, g, b, lds, s, a);
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

// Workspace: routing | h [MAX_TOK*MAX_K][eid] | d [MAX_TOK*MAX_K][hidden].
static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" size_t qk_moe_ws_bytes(int n_exp, int k, int ntok, int hidden, int eid) {
    (void)n_exp; (void)k; (void)ntok;
    return al256(sizeof(Route)) + al256((size_t)MAX_SLOTS * eid * 4) + al256((size_t)MAX_SLOTS * hidden * 4);
}

extern "C" int qk_moe_launch(const qk_mx_expert* d_experts, int n_exp, int k, int norm, int act,
                             int hidden, int eid, int ntok, const float* d_x,
                             const float* d_logits, float* d_out, void* d_ws, int stages,
                             hipStream_t s) {
    if (ntok < 1 || ntok > MAX_TOK || k < 1 || k > MAX_K || n_exp < 1 || n_exp > MAX_EXP ||
        hidden < 1 || eid < 1 || (hidden % 4) || (eid % 4) || hidden > 4096 || eid > 4096)
        return -2;
    MoeArgs a = {};
    a.experts = d_experts;
    a.n_exp = n_exp; a.k = k; a.norm = norm; a.act = act;
    a.hidden = hidden; a.eid = eid; a.ntok = ntok;
    a.x = d_x; a.logits = d_logits; a.out = d_out;
    uint8_t* ws = (uint8_t*)d_ws;
    a.route = (Route*)ws;
    ws += al256(sizeof(Route));
    a.h = (float*)ws;
    ws += al256((size_t)MAX_SLOTS * eid * 4);
    a.d = (float*)ws;
    // work items: distinct experts, at most min(n_exp, ntok*k)
    const int items = ntok * k < n_exp ? ntok * k : n_exp;
    const dim3 block_dn(DN_WAVES * 64), block_gu(GU_WAVES * 64);
    constexpr int rows_gu = GU_WAVES * 2 * GU_MR;
    constexpr int rows_dn = DN_WAVES * 2 * DN_MR;
    const dim3 g_gu((eid + rows_gu - 1) / rows_gu, items), g_dn((hidden + rows_dn - 1) / rows_dn, items);
    // one token with the fused down: gate/up routes in-kernel (no route launch)
    const bool one = ntok == 1 && k <= FG;
    if (!one && (stages & 1)) hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(MAX_TOK * 64), 0, s, a);
    const int tch = ntok < TCH ? ntok : TCH;
    // inputs (one token: then the expert table's gate/up pointers)
    const size_t lds_gu = (size_t)tch * ((hidden + 31) / 32) * XBP * 4 + (one ? (size_t)n_exp * 6 * 8 : 0),
                 lds_dn = (size_t)tch * ((eid + 31) / 32) * XBP * 4;
    const int ni_gu = (hidden + 1023) / 1024, ni_dn = (eid + 1023) / 1024;
#define QK_GU(NI)                                                                        \
    if (one) launch_lds<moe_gate_up_kernel<NI, true>>(g_gu, block_gu, lds_gu, s, a, true); \
    else launch_lds<moe_gate_up_kernel<NI, false>>(g_gu, block_gu, lds_gu, s, a, true);
    if (stages & 2) {
        switch (ni_gu) {
        case 1: QK_GU(1) break;
        case 2: QK_GU(2) break;
        case 3: QK_GU(3) break;
        default: QK_GU(4) break;
        }
    }
#undef QK_GU
    if (!(stages & 4)) return hipGetLastError() == hipSuccess ? 0 : -1;
    if (one) {
        // one token: down and combine in one launch
        const dim3 g_f((hidden + FROWS - 1) / FROWS), b_f(FG * FGW * 64);
        const size_t lds_f = (size_t)FG * ((eid + 31) / 32) * XBP * 4 + (size_t)FG * FROWS * 4 +
                             (size_t)n_exp * 3 * 8;
        switch (ni_dn) {
        case 1: launch_lds<moe_down_fused_kernel<1>>(g_f, b_f, lds_f, s, a); break;
        case 2: launch_lds<moe_down_fused_kernel<2>>(g_f, b_f, lds_f, s, a); break;
        case 3: launch_lds<moe_down_fused_kernel<3>>(g_f, b_f, lds_f, s, a); break;
        default: launch_lds<moe_down_fused_kernel<4>>(g_f, b_f, lds_f, s, a); break;
        }
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    switch (ni_dn) {
    case 1: launch_lds<moe_down_kernel<1>>(g_dn, block_dn, lds_dn, s, a); break;
    case 2: launch_lds<moe_down_kernel<2>>(g_dn, block_dn, lds_dn, s, a); break;
    case 3: launch_lds<moe_down_kernel<3>>(g_dn, block_dn, lds_dn, s, a); break;
    default: launch_lds<moe_down_kernel<4>>(g_dn, block_dn, lds_dn, s, a); break;
    }
    hipLaunchKernelGGL(moe_combine_kernel, dim3((hidden + 255) / 256, ntok), dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
