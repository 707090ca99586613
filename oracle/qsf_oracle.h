/*
 * qsf_oracle.h - CPU restatement of QStream's quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product path (libqsf_hip) never links or calls it.
 *
 * Every function restates one reference function and cites it
 * (paths relative to the QStream source tree).  Loop order and the
 * separate multiply/add roundings of the reference are kept, so a build
 * with -ffp-contract=off reproduces the strict reference bit for bit.
 */
#ifndef QSF_ORACLE_H
#define QSF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quant type ids, include/qsf/types.h:43-56; 11 is the MXFP4 type this
 * build adds in an unused slot. */
enum {
    ORC_Q2 = 0, ORC_Q2SYM = 1, ORC_Q3 = 2, ORC_Q4 = 3, ORC_Q4SYM = 4,
    ORC_Q2_OUTLIER = 9, ORC_Q4_OUTLIER = 10, ORC_MXFP4 = 11
};

/* src/quant.c:11-39 */
float    orc_fp16_to_fp32(uint16_t h);
/* bulk form: writes the fp32 bit patterns (NaN payloads intact) */
void     orc_fp16_to_fp32_array(const uint16_t* in, float* out, int n);
/* src/quant.c:69-85 (0 for types without a fixed block) */
size_t   orc_block_bytes(int qt, int bs);
/* Raw integer codes of one block (2/3/4-bit: unsigned field value;
 * 4-bit sym: the two's-complement value as int8).  src/quant.c:95-177 */
void     orc_unpack_codes(int qt, const void* block, int count, int8_t* codes);
/* orc_unpack_codes over nblocks consecutive blocks (bulk enumeration). */
void     orc_unpack_codes_many(int qt, const void* blocks, int nblocks, int bs, int8_t* codes);
/* Dequantised values of one block, src/quant.c:95-177 */
void     orc_dequant_block(int qt, const void* block, float* out, int count);
/* Dense matvec, src/kernels_scalar.c:16-109 */
void     orc_matvec(int qt, const void* w, const float* x, float* y,
                    int rows, int cols, int bs);
/* Outlier matvec: base pass + additive sparse pass, src/quant.c:387-495 */
void     orc_matvec_outlier(int qt, const void* payload, const float* x,
                            float* y, int rows, int cols, int bs);
/* Size in bytes of a tensor payload (outlier types read n from payload) */
size_t   orc_payload_bytes(int qt, const void* payload, int rows, int cols,
                           int bs);

/* MXFP4 (OCP MX v1.0): E2M1 element, E8M0 block scale.
 * Element order and LUT from tools/convert_hf.py:1456-1495; the scale is
 * 2^(E-127) (E=255 is NaN), not the raw byte the converter multiplies by. */
float    orc_e2m1_to_fp32(uint8_t nibble);
float    orc_e8m0_to_fp32(uint8_t e);
/* Payload layout: codes plane [rows][nblk][16 B], then scales [rows][nblk]
 * with nblk = ceil(cols/32). */
void     orc_matvec_mxfp4(const void* w, const float* x, float* y,
                          int rows, int cols);

/* src/kernels_scalar.c:187-214 */
void     orc_softmax(const float* in, float* out, int n);
/* src/kernels_scalar.c:129-147 */
void     orc_act(int act, float* x, int n);
/* Top-K by strict '>' insertion, src/engine.c:987-1006, and the optional
 * renormalisation, src/engine.c:1009-1018. */
void     orc_topk(const float* probs, int n_exp, int k, int norm_topk,
                  int* idx, float* w);

/* One token through the MoE FFN, src/engine.c:951-1107, experts in MXFP4.
 * gate/up: [eid][hidden]; down: [hidden][eid]; biases fp16 or NULL.
 * logits: router output [n_exp] (the router matvec itself is the caller's). */
typedef struct {
    const void* gate;  const uint16_t* gate_bias;
    const void* up;    const uint16_t* up_bias;
    const void* down;  const uint16_t* down_bias;
} orc_expert;
void     orc_moe_token(const orc_expert* experts, int n_exp, int k,
                       int norm_topk, int act, int hidden, int eid,
                       const float* x, const float* logits, float* out);

/* Batched prefill oracle: M independent 4-bit matvecs on float(bf16(x)).
 * The reference prefills token by token (src/engine.c:1289-1295). */
void     orc_prefill_4bit(const void* w, const uint16_t* x_bf16, float* y,
                          int m, int n, int k, int bs);

/* ---- decode glue around the matvecs (device-resident decode step) ----- */
/* src/kernels_scalar.c:172-185 (bias ignored, as there) */
void     orc_rms_norm(const float* in, float* out, const float* w, int dim, float eps);
/* src/kernels_scalar.c:148-169; b may be NULL */
void     orc_layer_norm(const float* in, float* out, const float* w, const float* b,
                        int dim, float eps);
/* src/kernels_scalar.c:112-118 */
void     orc_vec_add(const float* a, const float* b, float* o, int n);
void     orc_vec_mul(const float* a, const float* b, float* o, int n);
/* apply_rope, src/engine.c:204-235: q [n_heads][head_dim], k [n_kv][head_dim]
 * rotated in place, pair (i, i+1) by position * theta^(-i/head_dim). */
void     orc_rope(float* q, float* k, int head_dim, int position, float theta,
                  int n_heads, int n_kv_heads);
/* kv_cache_store, src/engine.c:240-300, for one layer: caches
 * [n_kv][max_seq][head_dim] int8, scales [n_kv][max_seq]; row `position`. */
void     orc_kv_store(int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq,
                      int n_kv, int head_dim, int position, const float* k, const float* v);
/* The attention loop of src/engine.c:879-923 for one layer over positions
 * 0..position: out [n_heads][head_dim]. */
void     orc_attention(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                       const float* vs, int max_seq, int n_heads, int n_kv, int head_dim,
                       int position, float* out);
/* Residual add and the NaN/Inf check, src/engine.c:1172-1187: res += x;
 * returns the first index with NaN or |res| > 1e30, or -1. */
int      orc_residual_check(float* res, const float* x, int n);
/* Embedding row dequantisation, src/engine.c:709-765: row `token` of a
 * [vocab][ceil(hd/bs) blocks] table of type qt (FP16 = 7: hd halfs). */
void     orc_embed_row(int qt, const void* table, int bs, int hd, int token, float* out);

#ifdef __cplusplus
}
#endif
#endif
