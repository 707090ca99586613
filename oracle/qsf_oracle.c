/*
 * qsf_oracle.c - CPU restatement of QStream's quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library; libqsf_hip never links it.
 *
 * Build strictly: -O2 -std=c11 -ffp-contract=off -fno-fast-math.  Each
 * multiply and add is then rounded separately, in the reference's order,
 * and the matvec results equal a strict build of the reference bit for bit
 * (checked in tests/test_oracle.py against oracle/_ref).
 *
 * Citations are relative to the QStream source tree.
 */
#include "qsf_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}
static float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 -> binary32 by field arithmetic (src/quant.c:11-39).
 * Subnormal halves are renormalised; Inf/NaN keep their payload bits. */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 31u) return bits_to_f32(sign | 0x7F800000u | (m << 13));
    if (e == 0u) {
        if (m == 0u) return bits_to_f32(sign);
        /* value = m * 2^-24; shift the leading one up to bit 10 */
        int shifts = 0;
        while ((m & 0x400u) == 0u) { m <<= 1; shifts++; }
        m &= 0x3FFu;
        return bits_to_f32(sign | ((uint32_t)(113 - shifts) << 23) | (m << 13));
    }
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_fp16_to_fp32_array(const uint16_t* in, float* out, int n) {
    for (int i = 0; i < n; i++) out[i] = orc_fp16_to_fp32(in[i]);
}

/* Block bytes: 4 bytes of fp16 metadata + packed codes (src/quant.c:69-85).
 * Types 5..8 and the outlier types have no fixed block in the reference. */
size_t orc_block_bytes(int qt, int bs) {
    switch (qt) {
    case ORC_Q2: case ORC_Q2SYM: return 4 + (size_t)(bs * 2 + 7) / 8;
    case ORC_Q3:                 return 4 + (size_t)(bs * 3 + 7) / 8;
    case ORC_Q4: case ORC_Q4SYM: return 4 + (size_t)(bs * 4 + 7) / 8;
    case 7:                      return (size_t)bs * 2;
    default:                     return 0;
    }
}

/* Field value of code i in a block's packed area (after the 4-byte meta).
 * 2-bit: LSB-first crumbs (src/quant.c:104-108); 3-bit: LSB-first
 * bitstream (src/quant.c:123-131); 4-bit: even i low nibble
 * (src/quant.c:145-152). */
static unsigned code_at(int bits, const uint8_t* packed, int i) {
    if (bits == 2) return (packed[i >> 2] >> ((i & 3) * 2)) & 3u;
    if (bits == 4) return (packed[i >> 1] >> ((i & 1) * 4)) & 15u;
    /* 3-bit: bits 3i..3i+2; only touch the second byte when needed */
    int bit = 3 * i, byte = bit >> 3, off = bit & 7;
    unsigned v = packed[byte] >> off;
    if (off > 5) v |= (unsigned)packed[byte + 1] << (8 - off);
    return v & 7u;
}

static int dense_type_of(int qt) {
    if (qt == ORC_Q2 || qt == ORC_Q2SYM || qt == ORC_Q2_OUTLIER) return ORC_Q2;
    if (qt == ORC_Q3) return ORC_Q3;
    if (qt == ORC_Q4SYM) return ORC_Q4SYM;
    return ORC_Q4;
}

static int qt_bits(int qt) {
    if (qt == ORC_Q2 || qt == ORC_Q2SYM || qt == ORC_Q2_OUTLIER) return 2;
    if (qt == ORC_Q3) return 3;
    return 4;
}

void orc_unpack_codes(int qt, const void* block, int count, int8_t* codes) {
    const uint8_t* packed = (const uint8_t*)block + 4;
    int bits = qt_bits(qt);
    for (int i = 0; i < count; i++) {
        unsigned c = code_at(bits, packed, i);
        /* 4-bit sym: two's-complement nibble (src/quant.c:166-174) */
        codes[i] = (qt == ORC_Q4SYM && c >= 8u) ? (int8_t)((int)c - 16) : (int8_t)c;
    }
}

void orc_unpack_codes_many(int qt, const void* blocks, int nblocks, int bs, int8_t* codes) {
    size_t bb = orc_block_bytes(dense_type_of(qt), bs);
    for (int b = 0; b < nblocks; b++)
        orc_unpack_codes(qt, (const uint8_t*)blocks + (size_t)b * bb, bs, codes + (size_t)b * bs);
}

/* src/quant.c:95-177: v = scale*q + zero (asym) or scale*q (4-bit sym,
 * whose bytes 2-3 are reserved). */
void orc_dequant_block(int qt, const void* block, float* out, int count) {
    const uint8_t* p = (const uint8_t*)block;
    float scale = orc_fp16_to_fp32(rd_u16(p));
    int8_t codes[256];
    orc_unpack_codes(qt, block, count, codes);
    if (qt == ORC_Q4SYM) {
        for (int i = 0; i < count; i++) out[i] = scale * (float)codes[i];
        return;
    }
    float zero = orc_fp16_to_fp32(rd_u16(p + 2));
    for (int i = 0; i < count; i++) {
        float prod = scale * (float)codes[i];
        out[i] = prod + zero;
    }
}

/* Block type used by the dense slot the engine dispatches to
 * (src/engine.c:141-152): 0,1 -> 2-bit, 2 -> 3-bit, 4 -> 4-bit sym,
 * everything else -> 4-bit asym. */
static int dense_type(int qt) {
    if (qt == ORC_Q2 || qt == ORC_Q2SYM || qt == ORC_Q2_OUTLIER) return ORC_Q2;
    if (qt == ORC_Q3) return ORC_Q3;
    if (qt == ORC_Q4SYM) return ORC_Q4SYM;
    return ORC_Q4;
}

/* src/kernels_scalar.c:16-109: per row, per block, dequantise then a
 * sequential fp32 dot; out[r] is written, not accumulated. */
static void matvec_dense(int qt, const void* w, const float* x, float* y,
                         int rows, int cols, int bs) {
    size_t bb = orc_block_bytes(qt, bs);
    int nb = (cols + bs - 1) / bs;
    const uint8_t* wp = (const uint8_t*)w;
    float buf[256];
    for (int r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (int b = 0, col = 0; b < nb; b++, col += bs) {
            int count = (col + bs <= cols) ? bs : cols - col;
            orc_dequant_block(qt, wp, buf, count);
            for (int k = 0; k < count; k++) {
                float prod = buf[k] * x[col + k];
                acc = acc + prod;
            }
            wp += bb;
        }
        y[r] = acc;
    }
}

/* src/quant.c:387-495: [u32 n][n x {u32 flat_idx, u16 fp16}][blocks].
 * Base matvec over the blocks, then in table order out[idx/cols] +=
 * fp16(v) * x[idx%cols] when the row is in range; duplicates add twice. */
void orc_matvec_outlier(int qt, const void* payload, const float* x, float* y,
                        int rows, int cols, int bs) {
    const uint8_t* p = (const uint8_t*)payload;
    uint32_t n = rd_u32(p);
    const uint8_t* ent = p + 4;
    const uint8_t* blocks = ent + (size_t)n * 6;
    matvec_dense(dense_type(qt), blocks, x, y, rows, cols, bs);
    if (cols <= 0) return; /* the reference would divide by zero here */
    for (uint32_t i = 0; i < n; i++, ent += 6) {
        uint32_t flat = rd_u32(ent);
        uint32_t r = flat / (uint32_t)cols, c = flat % (uint32_t)cols;
        if ((int)r < rows && (int)c < cols && r < 0x80000000u) {
            float v = orc_fp16_to_fp32(rd_u16(ent + 4));
            float prod = v * x[c];
            y[r] = y[r] + prod;
        }
    }
}

/* OCP MX v1.0 E2M1: sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0.
 * Same table as tools/convert_hf.py:1472-1475. */
float orc_e2m1_to_fp32(uint8_t nib) {
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float v = mag[nib & 7u];
    return (nib & 8u) ? -v : v;
}

/* OCP MX v1.0 E8M0: 2^(e-127); 0xFF is NaN. */
float orc_e8m0_to_fp32(uint8_t e) {
    if (e == 0xFFu) return bits_to_f32(0x7FC00000u);
    return ldexpf(1.0f, (int)e - 127);
}

/* MXFP4 matvec: element 2j is the low nibble of byte j, 2j+1 the high
 * nibble (tools/convert_hf.py:1488-1492); every element of a 32-block is
 * multiplied by the block scale; fp32 sequential dot like the dense path. */
void orc_matvec_mxfp4(const void* w, const float* x, float* y, int rows, int cols) {
    int nb = (cols + 31) / 32;
    const uint8_t* codes = (const uint8_t*)w;
    const uint8_t* scales = codes + (size_t)rows * nb * 16;
    for (int r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = codes + ((size_t)r * nb + b) * 16;
            float s = orc_e8m0_to_fp32(scales[(size_t)r * nb + b]);
            int count = (32 * b + 32 <= cols) ? 32 : cols - 32 * b;
            for (int j = 0; j < count; j++) {
                uint8_t nib = (uint8_t)((blk[j >> 1] >> ((j & 1) * 4)) & 15u);
                float v = orc_e2m1_to_fp32(nib) * s;
                float prod = v * x[32 * b + j];
                acc = acc + prod;
            }
        }
        y[r] = acc;
    }
}

size_t orc_payload_bytes(int qt, const void* payload, int rows, int cols, int bs) {
    if (rows <= 0 || cols <= 0) return qt == ORC_Q2_OUTLIER || qt == ORC_Q4_OUTLIER ? 4 : 0;
    if (qt == ORC_MXFP4) return (size_t)rows * (size_t)((cols + 31) / 32) * 17;
    size_t nb = (size_t)((cols + bs - 1) / bs);
    size_t dense = (size_t)rows * nb * orc_block_bytes(dense_type(qt), bs);
    if (qt == ORC_Q2_OUTLIER || qt == ORC_Q4_OUTLIER)
        return 4 + 6 * (size_t)rd_u32((const uint8_t*)payload) + dense;
    return dense;
}

/* Dispatch like get_matvec_fn (src/engine.c:141-152) plus the MXFP4 type. */
void orc_matvec(int qt, const void* w, const float* x, float* y,
                int rows, int cols, int bs) {
    if (qt == ORC_Q2_OUTLIER || qt == ORC_Q4_OUTLIER) {
        orc_matvec_outlier(qt, w, x, y, rows, cols, bs);
    } else if (qt == ORC_MXFP4) {
        orc_matvec_mxfp4(w, x, y, rows, cols);
    } else {
        matvec_dense(dense_type(qt), w, x, y, rows, cols, bs);
    }
}

/* src/kernels_scalar.c:187-214 */
void orc_softmax(const float* in, float* out, int n) {
    if (n <= 0) return;
    float mx = in[0];
    for (int i = 1; i < n; i++) if (in[i] > mx) mx = in[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { out[i] = expf(in[i] - mx); sum = sum + out[i]; }
    if (sum < 1e-30f) {
        for (int i = 0; i < n; i++) out[i] = 1.0f / (float)n;
        return;
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) out[i] = out[i] * inv;
}

/* Activation by header enum (types.h:59-66), as the MoE path selects it
 * (src/engine.c:1070-1077); bodies from src/kernels_scalar.c:129-147. */
void orc_act(int act, float* x, int n) {
    if (act == 2) {                       /* SiLU */
        for (int i = 0; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
    } else if (act == 0 || act == 1) {    /* GELU, tanh form */
        const float c = 0.7978845608f;
        for (int i = 0; i < n; i++) {
            float v = x[i];
            float cube = 0.044715f * v * v * v;
            float inner = c * (v + cube);
            float half = 0.5f * v;
            x[i] = half * (1.0f + tanhf(inner));
        }
    } else {                              /* ReLU */
        for (int i = 0; i < n; i++) if (x[i] < 0.0f) x[i] = 0.0f;
    }
}

/* src/engine.c:987-1018: strict '>' insertion keeps the lower expert id on
 * ties; slots start at (-1, -1e30). */
void orc_topk(const float* probs, int n_exp, int k, int norm_topk, int* idx, float* w) {
    for (int i = 0; i < k; i++) { idx[i] = -1; w[i] = -1e30f; }
    for (int e = 0; e < n_exp; e++) {
        float p = probs[e];
        for (int i = 0; i < k; i++) {
            if (p > w[i]) {
                for (int j = k - 1; j > i; j--) { w[j] = w[j - 1]; idx[j] = idx[j - 1]; }
                w[i] = p; idx[i] = e;
                break;
            }
        }
    }
    if (norm_topk) {
        float s = 0.0f;
        for (int i = 0; i < k; i++) s = s + w[i];
        if (s > 0.0f) {
            float inv = 1.0f / s;
            for (int i = 0; i < k; i++) w[i] = w[i] * inv;
        }
    }
}

static void add_bias(float* v, const uint16_t* b, int n) {
    if (!b) return;
    for (int i = 0; i < n; i++) v[i] = v[i] + orc_fp16_to_fp32(b[i]);
}

/* src/engine.c:951-1107 for one token. */
void orc_moe_token(const orc_expert* ex, int n_exp, int k, int norm_topk, int act,
                   int hidden, int eid, const float* x, const float* logits, float* out) {
    float* probs = (float*)malloc(sizeof(float) * (size_t)n_exp);
    int* idx = (int*)malloc(sizeof(int) * (size_t)k);
    float* w = (float*)malloc(sizeof(float) * (size_t)k);
    float* g = (float*)malloc(sizeof(float) * (size_t)eid);
    float* u = (float*)malloc(sizeof(float) * (size_t)eid);
    float* d = (float*)malloc(sizeof(float) * (size_t)hidden);
    orc_softmax(logits, probs, n_exp);
    orc_topk(probs, n_exp, k, norm_topk, idx, w);
    for (int i = 0; i < hidden; i++) out[i] = 0.0f;
    for (int a = 0; a < k; a++) {
        int e = idx[a];
        if (e < 0) continue;
        orc_matvec_mxfp4(ex[e].gate, x, g, eid, hidden);
        add_bias(g, ex[e].gate_bias, eid);
        orc_matvec_mxfp4(ex[e].up, x, u, eid, hidden);
        add_bias(u, ex[e].up_bias, eid);
        orc_act(act, g, eid);
        for (int i = 0; i < eid; i++) g[i] = g[i] * u[i];
        orc_matvec_mxfp4(ex[e].down, g, d, hidden, eid);
        add_bias(d, ex[e].down_bias, hidden);
        for (int i = 0; i < hidden; i++) {
            float prod = w[a] * d[i];
            out[i] = out[i] + prod;
        }
    }
    free(probs); free(idx); free(w); free(g); free(u); free(d);
}

/* M token-by-token src/kernels_scalar.c:64-85 matvecs on float(bf16 x)
 * (the engine prefills one token at a time, src/engine.c:1289-1295).
 * The weights are dequantised once (the same values matvec_dense makes per
 * call) and four rows run as independent chains; each row keeps
 * matvec_dense's sequential order, so y is bit-identical to the token loop
 * (tests/test_oracle.py checks that). */
void orc_prefill_4bit(const void* w, const uint16_t* x_bf16, float* y,
                      int m, int n, int k, int bs) {
    if (m <= 0 || n <= 0) return;
    size_t bb = orc_block_bytes(ORC_Q4, bs);
    int nb = k > 0 ? (k + bs - 1) / bs : 0;
    float* xf = (float*)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
    float* wd = (float*)malloc(sizeof(float) * (size_t)n * (size_t)(k > 0 ? k : 1));
    const uint8_t* wp = (const uint8_t*)w;
    for (int r = 0; r < n; r++)
        for (int b = 0, col = 0; b < nb; b++, col += bs) {
            int count = (col + bs <= k) ? bs : k - col;
            orc_dequant_block(ORC_Q4, wp, wd + (size_t)r * k + col, count);
            wp += bb;
        }
    for (int t = 0; t < m; t++) {
        for (int i = 0; i < k; i++)
            xf[i] = bits_to_f32((uint32_t)x_bf16[(size_t)t * k + i] << 16);
        float* yt = y + (size_t)t * n;
        int r = 0;
        for (; r + 4 <= n; r += 4) {
            const float* w0 = wd + (size_t)r * k;
            const float* w1 = w0 + k;
            const float* w2 = w1 + k;
            const float* w3 = w2 + k;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            for (int i = 0; i < k; i++) {
                float p0 = w0[i] * xf[i], p1 = w1[i] * xf[i];
                float p2 = w2[i] * xf[i], p3 = w3[i] * xf[i];
                a0 = a0 + p0; a1 = a1 + p1; a2 = a2 + p2; a3 = a3 + p3;
            }
            yt[r] = a0; yt[r + 1] = a1; yt[r + 2] = a2; yt[r + 3] = a3;
        }
        for (; r < n; r++) {
            const float* w0 = wd + (size_t)r * k;
            float a0 = 0.0f;
            for (int i = 0; i < k; i++) {
                float p0 = w0[i] * xf[i];
                a0 = a0 + p0;
            }
            yt[r] = a0;
        }
    }
    free(wd);
    free(xf);
}

/* ---- decode glue ---------------------------------------------------------- */
void orc_rms_norm(const float* in, float* out, const float* w, int dim, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < dim; i++) {
        float sq = in[i] * in[i];
        ss = ss + sq;
    }
    float rms = sqrtf(ss / (float)dim + eps);
    float inv = 1.0f / rms;
    for (int i = 0; i < dim; i++) {
        float t = in[i] * inv;
        out[i] = t * w[i];
    }
}

void orc_layer_norm(const float* in, float* out, const float* w, const float* b,
                    int dim, float eps) {
    float mean = 0.0f;
    for (int i = 0; i < dim; i++) mean = mean + in[i];
    mean = mean / (float)dim;
    float var = 0.0f;
    for (int i = 0; i < dim; i++) {
        float d = in[i] - mean;
        float sq = d * d;
        var = var + sq;
    }
    var = var / (float)dim;
    float inv_std = 1.0f / sqrtf(var + eps);
    for (int i = 0; i < dim; i++) {
        float t = (in[i] - mean) * inv_std;
        out[i] = t * w[i];
        if (b) out[i] = out[i] + b[i];
    }
}

void orc_vec_add(const float* a, const float* b, float* o, int n) {
    for (int i = 0; i < n; i++) o[i] = a[i] + b[i];
}

void orc_vec_mul(const float* a, const float* b, float* o, int n) {
    for (int i = 0; i < n; i++) o[i] = a[i] * b[i];
}

/* One head's rotation; the angle is reduced in double as the reference
 * does (fmod by 2 pi), then cos/sin in float. */
static void rope_head(float* h, int head_dim, int position, float theta) {
    for (int i = 0; i < head_dim; i += 2) {
        float freq = 1.0f / powf(theta, (float)i / (float)head_dim);
        double angle = (double)position * (double)freq;
        angle = fmod(angle, 2.0 * 3.14159265358979323846);
        float c = cosf((float)angle), s = sinf((float)angle);
        float a0 = h[i], a1 = h[i + 1];
        float p0 = a0 * c, p1 = a1 * s, p2 = a0 * s, p3 = a1 * c;
        h[i] = p0 - p1;
        h[i + 1] = p2 + p3;
    }
}

void orc_rope(float* q, float* k, int head_dim, int position, float theta,
              int n_heads, int n_kv_heads) {
    for (int h = 0; h < n_heads; h++) rope_head(q + (size_t)h * head_dim, head_dim, position, theta);
    for (int h = 0; h < n_kv_heads; h++) rope_head(k + (size_t)h * head_dim, head_dim, position, theta);
}

/* absmax int8 with round half away from zero and a +-127 clamp */
static float kv_quant_row(const float* src, int8_t* dst, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = src[i] < 0 ? -src[i] : src[i];
        if (a > amax) amax = a;
    }
    float scale = amax / 127.0f;
    if (amax > 1e-30f) {
        float inv = 127.0f / amax;
        for (int i = 0; i < n; i++) {
            float v = src[i] * inv;
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            float r = v + (v >= 0 ? 0.5f : -0.5f);
            dst[i] = (int8_t)r;
        }
    } else {
        memset(dst, 0, (size_t)n);
    }
    return scale;
}

void orc_kv_store(int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq,
                  int n_kv, int head_dim, int position, const float* k, const float* v) {
    for (int h = 0; h < n_kv; h++) {
        size_t row = (size_t)h * max_seq + position;
        ks[row] = kv_quant_row(k + (size_t)h * head_dim, kc + row * head_dim, head_dim);
        vs[row] = kv_quant_row(v + (size_t)h * head_dim, vc + row * head_dim, head_dim);
    }
}

void orc_attention(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                   const float* vs, int max_seq, int n_heads, int n_kv, int head_dim,
                   int position, float* out) {
    int seq = position + 1, groups = n_heads / n_kv;
    float* scores = (float*)malloc(sizeof(float) * (size_t)seq);
    float inv_sqrt_d = 1.0f / sqrtf((float)head_dim);
    for (int h = 0; h < n_heads; h++) {
        int kvh = h / groups;
        const float* qh = q + (size_t)h * head_dim;
        for (int p = 0; p < seq; p++) {
            size_t row = (size_t)kvh * max_seq + p;
            const int8_t* kr = kc + row * head_dim;
            float sc = ks[row], dot = 0.0f;
            for (int d = 0; d < head_dim; d++) {
                float kv = (float)kr[d] * sc;
                float prod = qh[d] * kv;
                dot = dot + prod;
            }
            scores[p] = dot * inv_sqrt_d;
        }
        orc_softmax(scores, scores, seq);
        float* oh = out + (size_t)h * head_dim;
        for (int d = 0; d < head_dim; d++) oh[d] = 0.0f;
        for (int p = 0; p < seq; p++) {
            size_t row = (size_t)kvh * max_seq + p;
            const int8_t* vr = vc + row * head_dim;
            float sv = scores[p] * vs[row];
            for (int d = 0; d < head_dim; d++) {
                float prod = sv * (float)vr[d];
                oh[d] = oh[d] + prod;
            }
        }
    }
    free(scores);
}

int orc_residual_check(float* res, const float* x, int n) {
    int bad = -1;
    for (int i = 0; i < n; i++) res[i] = res[i] + x[i];
    for (int i = 0; i < n; i++)
        if (res[i] != res[i] || res[i] > 1e30f || res[i] < -1e30f) { bad = i; break; }
    return bad;
}

void orc_embed_row(int qt, const void* table, int bs, int hd, int token, float* out) {
    if (qt == 7) {   /* QSF_QUANT_FP16: hd halfs per row */
        const uint8_t* r = (const uint8_t*)table + (size_t)token * hd * 2;
        for (int i = 0; i < hd; i++) out[i] = orc_fp16_to_fp32(rd_u16(r + 2 * (size_t)i));
        return;
    }
    int dt = dense_type(qt);
    size_t bb = orc_block_bytes(dt, bs);
    int nb = (hd + bs - 1) / bs;
    const uint8_t* bp = (const uint8_t*)table + (size_t)token * nb * bb;
    for (int b = 0; b < nb; b++, bp += bb) {
        int count = (b + 1 < nb) ? bs : hd - b * bs;
        orc_dequant_block(dt, bp, out + (size_t)b * bs, count);
    }
}

