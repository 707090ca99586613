/*
 * qsf_hip.h - C ABI of libqsf_hip, the MI355X (gfx950) backend for
 * QStream's quantized matrix-vector hot path.
 *
 * Plain C: pointers, sizes and ints only.  Reference citations are relative
 * to the QStream source tree (include/, src/, tools/).
 *
 * Two layers:
 *  1. Drop-in table slots with exactly the qsf_matvec_fn signature
 *     (include/qsf/kernels.h:53-58).  They take host pointers like the CPU
 *     kernels, are synchronous on return, and upload a weight payload to HBM
 *     the first time its host pointer is seen (device weight arena).
 *  2. Device-pointer entry points for callers whose activations already live
 *     in HBM (the device-resident engine path and the benchmarks).
 *
 * Status codes are QSFError values (include/qsf/error.h:14-32): 0 = QSF_OK,
 * 4 = QSF_ERR_OUT_OF_MEMORY, 11 = QSF_ERR_INVALID_INPUT, 15 = QSF_ERR_INTERNAL.
 * The void table slots report through qsf_set_error() when the host engine
 * links one (src/error.c:43-53) and through qsf_hip_last_error(); on failure
 * they fill the output with quiet NaN (there is no CPU fallback).
 */
#ifndef QSF_HIP_H
#define QSF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QSF_HIP_QUANT_MXFP4 11   /* quant type added in an unused enum slot */

/* ---- lifecycle ----------------------------------------------------------- */
/* Select the GPU and create the library's stream.  Called implicitly by the
 * first table-slot call (device 0).  Replaces nothing in the reference: the
 * CPU backend needs no device (src/engine.c:435-439 is where it is called). */
int         qsf_hip_init(int device);
/* Free every tensor, workspace and stream. */
void        qsf_hip_shutdown(void);
int         qsf_hip_last_error(void);
const char* qsf_hip_last_error_detail(void);

/* ---- 1. drop-in table slots (qsf_matvec_fn) ------------------------------ */
/* Synchronous: host x in, host y out, weights from the device arena.  The
 * first call with a weight pointer uploads its payload; later calls run from
 * HBM.  A pointer whose geometry, outlier count or sampled payload words
 * differ from what was uploaded is uploaded again and marked volatile (every
 * later call uploads it).  Rewriting a buffer that a slot has seen, without
 * qsf_hip_arena_forget, is only safe once the pointer is volatile: the first
 * rewrite is caught by the sampled words alone, not by a full comparison. */
/* src/kernels_scalar.c:16-37 (2-bit; also QSF_QUANT_2BIT_SYM, src/engine.c:143) */
void qsf_matvec_2bit_hip(const void* weights_q, const float* input, float* output,
                         int rows, int cols, int block_size);
/* src/kernels_scalar.c:40-61 */
void qsf_matvec_3bit_hip(const void* weights_q, const float* input, float* output,
                         int rows, int cols, int block_size);
/* src/kernels_scalar.c:64-85 (also every type the engine maps to the 4-bit slot) */
void qsf_matvec_4bit_hip(const void* weights_q, const float* input, float* output,
                         int rows, int cols, int block_size);
/* src/kernels_scalar.c:88-109; decodes nibbles as two's complement like the
 * scalar reference (src/quant.c:166-174) */
void qsf_matvec_4bit_sym_hip(const void* weights_q, const float* input, float* output,
                             int rows, int cols, int block_size);
/* src/quant.c:387-445 / src/kernels_avx2.c:420-488; weights_q points at the
 * payload's [u32 n] outlier header */
void qsf_matvec_outlier_2bit_hip(const void* weights_q, const float* input, float* output,
                                 int rows, int cols, int block_size);
/* src/quant.c:447-495 / src/kernels_avx2.c:491-549 */
void qsf_matvec_outlier_4bit_hip(const void* weights_q, const float* input, float* output,
                                 int rows, int cols, int block_size);
/* New slot (no reference kernel): MXFP4 E2M1 codes + E8M0 scales per 32
 * elements, element order of tools/convert_hf.py:1456-1495, payload
 * [rows][cols/32][16 B codes] then [rows][cols/32] scales.  block_size is
 * ignored (always 32). */
void qsf_matvec_mxfp4_hip(const void* weights_q, const float* input, float* output,
                          int rows, int cols, int block_size);

/* src/kernels.c:7-65 (qsf_kernels_init).  Writes the six matvec slots at the
 * head of a QSFKernelTable (include/qsf/kernels.h:91-98) -- call it after
 * qsf_kernels_init() so the remaining CPU slots stay as they are.  When
 * mxfp4_slot is non-NULL it receives qsf_matvec_mxfp4_hip (the slot the
 * engine appends to the table for quant type 11). */
void qsf_kernels_init_hip(void* kernel_table, const void* platform, void** mxfp4_slot);

/* No counterpart in the reference: a tuning knob of the slots above.  A
 * slot call learns which weight pointer the engine calls next with the same
 * x (k after q, up after gate: src/engine.c:848-866, 1118-1125); once the
 * same one has followed twice running, the call also runs up to n such
 * successors in its own launch and holds their results until they are
 * called.  A held result is served only when that later call passes every
 * check a call makes and finds x, the tensor and the arena unchanged, and
 * only for groups whose launch gives each matrix the arithmetic it gets
 * alone: every result is bit-identical to the call made by itself.  A held
 * result not called for costs one GEMV and its predecessor the successor.
 * n = 0 turns it off; default 2 (q, k, v); at most 7.  n < 0 only queries.
 * Returns the previous setting. */
int qsf_hip_slot_lookahead(int n);

/* ---- device weight arena (replaces mmap streaming, src/file_access.c:80-88) */
typedef struct qsf_hip_tensor qsf_hip_tensor;   /* opaque */

/* Upload one tensor payload (as find_tensor returns it, src/engine.c:183-202)
 * and register its host pointer; later table-slot calls with that pointer
 * run from HBM.  Returns NULL on error. */
qsf_hip_tensor* qsf_hip_tensor_upload(const void* host_payload, int quant_type,
                                      int rows, int cols, int block_size);
/* Gate and up weights of one FFN (two payloads of the same plain block
 * format and shape, no outlier table) uploaded as one interleaved tensor of
 * 2 * rows rows for qsf_hip_gate_up_act_dev.  Not registered for any host
 * pointer.  No counterpart in the reference: the engine's two matvecs and
 * activation product (src/engine.c:1118-1140) in one launch, for a
 * device-resident engine.  Returns NULL on error. */
qsf_hip_tensor* qsf_hip_tensor_upload_pair(const void* gate_payload, const void* up_payload,
                                           int quant_type, int rows, int cols, int block_size);
/* Tensor registered for this host pointer, or NULL. */
qsf_hip_tensor* qsf_hip_tensor_lookup(const void* host_payload);
void            qsf_hip_tensor_free(qsf_hip_tensor* t);
/* Forget a host pointer and its volatile mark.  Required before a slot call
 * with a buffer the caller has rewritten since a slot last saw it, unless
 * the pointer is already volatile.  Returns QSF_ERR_INVALID_INPUT when the pointer
 * is not registered. */
int             qsf_hip_arena_forget(const void* host_payload);
/* Forget every registered pointer in [base, base + bytes), e.g. all tensors
 * of an LZ4 layer buffer after it is decompressed again (src/engine.c:786-789).
 * Returns the number forgotten, or -QSF_ERR_OUT_OF_MEMORY. */
int             qsf_hip_arena_forget_range(const void* base, size_t bytes);
/* Bytes of HBM held by the arena. */
size_t          qsf_hip_arena_bytes(void);
/* On-disk payload bytes of a registered tensor. */
size_t          qsf_hip_tensor_payload_bytes(const qsf_hip_tensor* t);

/* ---- 2. device-pointer entry points --------------------------------------- */
/* y[rows] = W x[cols] on `stream` (hipStream_t; NULL = the default stream);
 * asynchronous.  d_x, d_y are device pointers.  Calls that use the library
 * workspace (all but the prepared form) must not overlap on different
 * streams. */
int qsf_hip_matvec_dev(const qsf_hip_tensor* t, const float* d_x, float* d_y, void* stream);
/* n (<= 8) tensors with the same type/cols/block size sharing one x in one
 * launch (q/k/v, gate/up). */
int qsf_hip_matvec_group_dev(const qsf_hip_tensor* const* t, int n, const float* d_x,
                             float* const* d_y, void* stream);

/* Split form of the two calls above, for callers that share one x between
 * several launches or fuse the activation preparation upstream: prepare x
 * once (block-fixed-point digits, qsf_hip_xprep_bytes bytes of device
 * memory, 256-B aligned), then run any number of GEMVs on it.  d_x must
 * still be passed: the outlier pass reads it. */
size_t qsf_hip_xprep_bytes(int quant_type, int block_size, int cols);
int qsf_hip_xprep_dev(int quant_type, int block_size, int cols, const float* d_x,
                      void* d_xq, void* stream);
int qsf_hip_matvec_group_prepared_dev(const qsf_hip_tensor* const* t, int n,
                                      const float* d_x, const void* d_xq,
                                      float* const* d_y, void* stream);

/* Kernel timing (diagnostics; no counterpart in the reference).  While
 * enabled, each decode GEMV, batched-prefill and MoE gate/up launch records a
 * HIP event pair at the kernel's own start and end on its stream (up to 4096
 * launches; enabling resets the record).  _read waits for the recorded launches and writes their
 * durations in microseconds; it returns how many it wrote, or a negative
 * status.  Do not enable it while a graph is being captured. */
int qsf_hip_kernel_timing(int enable);
int qsf_hip_kernel_timing_read(float* us, int max);

/* Decode GEMV engine for the tensors uploaded from now on (no counterpart
 * in the reference).  1 (default): 3-bit tensors whose shape the int8
 * matrix-core kernel covers (cols 16..16384) are stored in its fragment
 * order and every decode GEMV over them (one-launch, gate/up, fused
 * residual + norm, table slots, prepared-x) takes that kernel; all other
 * tensors are stored in row-plane order (each row's block bytes regrouped
 * into aligned 16-byte planes) and take the dot-product kernels.  2: the same
 * for the 2- and 4-bit formats too.  0: row-plane order and dot-product
 * kernels for every tensor.  Either way the device copy is not in on-disk
 * order; the library reads it, callers do not.  A tensor keeps the engine it was uploaded
 * with.  For A/B comparisons and tests; both engines meet the same 1e-5
 * bound, their results differ in fp32 rounding.  engine < 0 only queries.
 * Returns the previous setting. */
int qsf_hip_gemv_engine(int engine);

/* ---- QSF model file -> device arena (src/format.c:11-284, engine.c:183-202) */
/* qsf_crc32 of src/format.c:11-34 (ISO 3309 CRC-32). */
uint32_t qsf_hip_crc32(const void* data, size_t len);

typedef struct qsf_hip_model qsf_hip_model;   /* opaque */
/* Header fields (include/qsf/types.h:185-245, zero defaults resolved as
 * src/format.c:37-99 and 137-160 do) and what the load found. */
typedef struct {
    uint32_t num_layers, hidden_dim, num_heads, num_kv_heads, vocab_size, max_seq_len,
             intermediate_dim, head_dim, block_size;
    uint32_t quant_type, activation, norm_type, pos_enc_type, ffn_type, attn_type;
    uint32_t has_bias, weight_tied, num_experts, num_active_experts, expert_intermediate_dim;
    uint32_t moe_norm_topk;
    float    rope_theta, norm_epsilon;
    uint32_t num_tensors;        /* tensor records in all layers */
    uint32_t has_embedding;
    uint32_t crc_mismatches;     /* header, layers, embedding, final section */
    uint32_t size_mismatch;      /* total_file_size differs from the file */
    uint32_t moe_layers;         /* layers given a device MXFP4 expert table */
    size_t   device_bytes;       /* bytes uploaded to HBM */
} qsf_hip_model_info;
/* Load an uncompressed QSF file: validate the header (src/format.c:37-99),
 * check every CRC (a mismatch is counted and warned about, as the
 * reference only warns, src/format.c:129-135, 226-233), walk each layer's
 * tensor records (src/engine.c:183-202) and upload every matrix to HBM and
 * every FP16 vector (norms, biases) as fp32, plus the embedding table and
 * the final norm / output head (src/engine.c:403-420, 664-679).  The file
 * is fully checked before any device work.  NULL on error
 * (qsf_hip_last_error: 1 not found, 2 corrupted, 3 version, 6 invalid
 * model, 15 LZ4-compressed layers, which this build does not read). */
qsf_hip_model* qsf_hip_model_load(const char* path);
/* The same load from a QSF file already in memory (size bytes at data, read
 * only during the call; nothing in the model points into it afterwards).
 * No counterpart in the reference: for engines that hold the file in
 * their own buffers, and for checking the parse under a sanitizer. */
qsf_hip_model* qsf_hip_model_load_mem(const void* data, size_t size);
void qsf_hip_model_free(qsf_hip_model* m);
int qsf_hip_model_get_info(const qsf_hip_model* m, qsf_hip_model_info* out);
/* Matrix (tensor_type of include/qsf/types.h:118-162) of a layer, or NULL. */
const qsf_hip_tensor* qsf_hip_model_tensor(const qsf_hip_model* m, int layer, int tensor_type);
/* FP16 vector tensor of a layer as device fp32 (*n elements), or NULL. */
const float* qsf_hip_model_vector(const qsf_hip_model* m, int layer, int tensor_type, int* n);
/* Embedding table: blockwise (for qsf_hip_embed_row_dev), or FP16. */
const qsf_hip_tensor* qsf_hip_model_embedding(const qsf_hip_model* m);
const uint16_t* qsf_hip_model_embedding_fp16(const qsf_hip_model* m);
/* Output head for the logits matvec: the embedding table when tied. */
const qsf_hip_tensor* qsf_hip_model_output_head(const qsf_hip_model* m);
/* Final norm weight (and bias, NULL when absent) as device fp32. */
const float* qsf_hip_model_final_norm(const qsf_hip_model* m, const float** bias);
/* Device expert table of an MoE layer (ffn_type 3, num_experts > 1) whose
 * gate/up/down experts are all MXFP4, built at load with their FP16 biases
 * (src/engine.c:1024-1107); NULL otherwise.  Owned by the model. */
struct qsf_hip_moe* qsf_hip_model_moe(const qsf_hip_model* m, int layer);

/* ---- MoE FFN with MXFP4 experts (src/engine.c:951-1107) ------------------ */
typedef struct qsf_hip_moe qsf_hip_moe;         /* opaque device expert table */
/* gate/up: [expert_dim][hidden], down: [hidden][expert_dim], all MXFP4
 * tensors from qsf_hip_tensor_upload.  Bias arrays are host fp16 vectors per
 * expert (the MOE_*_BIAS tensors, src/engine.c:1039-1046); the outer array or
 * any entry may be NULL. */
qsf_hip_moe* qsf_hip_moe_create(int n_experts, int hidden, int expert_dim,
                                const qsf_hip_tensor* const* gate,
                                const qsf_hip_tensor* const* up,
                                const qsf_hip_tensor* const* down,
                                const uint16_t* const* gate_bias,
                                const uint16_t* const* up_bias,
                                const uint16_t* const* down_bias);
void qsf_hip_moe_free(qsf_hip_moe* m);
/* For each of ntok tokens (any count: they run in launches of up to 8, in
 * order on `stream`; top_k <= 8): softmax(router logits), top_k by strict
 * '>' insertion, optional renormalisation, then per selected expert
 * gate/up + bias, activation (QSFActivation: 2 SiLU, 0/1 GELU, else ReLU)
 * times up, down + bias, weighted sum in rank order.  d_x [ntok][hidden],
 * d_logits [ntok][n_experts], d_out [ntok][hidden]; asynchronous. */
int qsf_hip_moe_forward_dev(qsf_hip_moe* m, int top_k, int norm_topk, int activation,
                            int ntok, const float* d_x, const float* d_logits,
                            float* d_out, void* stream);
/* Measurement aid (no counterpart in the reference): the stages
 * qsf_hip_moe_forward_dev launches from now on, bit 0 the routing launch
 * (batches of more than one token; one token routes inside its gate/up
 * launch), bit 1 gate/up, bit 2 down and the weighted sum.  Default 7 (the
 * whole FFN).  A stage left out leaves the object's workspace as the last
 * call that ran it wrote it, so forward calls with masks 1, 2, 4 in turn on
 * the same inputs give the output of one call with 7; any other mask leaves
 * d_out unwritten or stale, for timing one stage's launches on their own.
 * Masks other than 7 need ntok <= 8.  mask < 0 only queries; returns the
 * previous mask. */
int qsf_hip_moe_stages(int mask);

/* Batched prefill through the 4-bit format (no reference kernel: the engine
 * runs one qsf_matvec_4bit call per token, src/engine.c:1289-1295):
 * d_y[m][rows] = W . float(d_x[m][cols]) for m tokens.  W is a 4-bit
 * asymmetric tensor (block 64, 128 or 256, no outliers).  Per block,
 * s * (sum q x) + z * (sum x): the integer codes (exact in bf16) meet bf16 x
 * on MFMA with fp32 accumulation, the scale is applied in fp32 every 64
 * codes, and the zero-point term runs on exact bf16 splits of z and of the
 * block sums; nothing is rounded below fp32 (about 1e-6 rel-L2 against the
 * scalar matvec on float(x)).  d_x is bf16 [m][cols] (16-byte aligned,
 * cols >= 32, cols % 8 == 0); asynchronous on `stream`.  Uses the library
 * workspace (x repacked into fragment order with the block-sum splits,
 * about 2*m*cols bytes plus 16 per block and token): calls must not overlap
 * with other workspace users on other streams.  The workspace grows as
 * needed; an outgrown one is kept until qsf_hip_shutdown, so graphs
 * captured with it stay valid. */
int qsf_hip_prefill_4bit_dev(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                             float* d_y, void* stream);

/* Allocation-free form of qsf_hip_prefill_4bit_dev (no counterpart in the
 * reference).  For callers that cannot allocate device memory: code under
 * HIP graph capture and serving loops that forbid hipMalloc.  Same inputs,
 * outputs and results; the packed activations go to a static per-GPU
 * scratch array of QSF_HIP_PREFILL_SCRATCH_BYTES instead of the library
 * workspace, and nothing is allocated or freed.  A call that needs more
 * scratch than that (about 2 * m * (cols + 8 * cols / block_size) bytes,
 * m rounded up to 16 and both column counts to 256; config 4's 512 x 4096
 * at block 64 needs 4.7 MB) fails with QSF_ERR_INVALID_INPUT.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (different streams, or graphs
 * replayed concurrently) race on it. */
#define QSF_HIP_PREFILL_SCRATCH_BYTES (16 << 20)
int qsf_hip_prefill_4bit_dev_noalloc(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                                     float* d_y, void* stream);

/* qsf_hip_prefill_4bit_dev in two halves (no counterpart in the reference):
 * pack x (bf16 [m][cols]) once into a caller buffer of
 * qsf_hip_prefill_pack_bytes(m, cols, bs) bytes (16-byte aligned), then run
 * the GEMM of every 4-bit tensor with those cols and block size that
 * shares this x (q/k/v, gate/up) over it.  Results are those of
 * qsf_hip_prefill_4bit_dev.  Asynchronous on `stream`. */
size_t qsf_hip_prefill_pack_bytes(int m, int cols, int block_size);
int qsf_hip_prefill_pack_dev(const uint16_t* d_x_bf16, int m, int cols, int block_size, void* d_packed,
                             void* stream);
int qsf_hip_prefill_4bit_packed_dev(const qsf_hip_tensor* t, const void* d_packed, int m, float* d_y,
                                    void* stream);

/* Diagnostic (no counterpart in the reference): one launch that streams the
 * device bytes of n <= 8 tensors once (blocks, scales, outlier CSR) and does
 * nothing else, the floor a one-launch GEMV over them is measured against.
 * d_sink: one uint32 of device memory, written only in the unlikely case a
 * workgroup's checksum equals a fixed constant.  Asynchronous. */
int qsf_hip_stream_read_dev(const qsf_hip_tensor* const* t, int n, uint32_t* d_sink, void* stream);
/* The bf16 matrix-core ceiling the prefill is set beside (a diagnostic, no
 * counterpart in the reference): one launch in which every CU runs
 * independent v_mfma_f32_16x16x32_bf16 chains `iters` long with no memory
 * traffic.  d_sink: one uint32 of device memory, written only if the sum of
 * the accumulators has a fixed bit pattern.  Asynchronous; returns the
 * launch's FLOP, or a negative value on error. */
double qsf_hip_mfma_peak_dev(int iters, uint32_t* d_sink, void* stream);

/* ---- device-resident decode glue ------------------------------------------
 * The per-layer work between the projections of one decode step
 * (src/engine.c:709-1187), so an engine that keeps its activations in HBM
 * needs no host round trip.  All take device pointers and are asynchronous
 * on `stream`.  Layouts: q [n_heads][head_dim], k and v [n_kv][head_dim];
 * one layer's KV cache [n_kv][max_seq][head_dim] int8 with per-position
 * scales [n_kv][max_seq] (src/engine.c:240-327). */
/* src/kernels_scalar.c:172-185 (called at src/engine.c:805-815, 940-948, 1190-1196) */
int qsf_hip_rms_norm_dev(const float* d_in, float* d_out, const float* d_w, int dim, float eps,
                         void* stream);
/* src/kernels_scalar.c:148-169; d_b may be NULL */
int qsf_hip_layer_norm_dev(const float* d_in, float* d_out, const float* d_w, const float* d_b,
                           int dim, float eps, void* stream);
/* apply_rope, src/engine.c:204-235.  The frequency table 1/theta^(2j/head_dim)
 * is computed once on the host with the C library's powf, as the reference
 * does (theta <= 0 means 10000, src/engine.c:873). */
typedef struct qsf_hip_rope qsf_hip_rope;
qsf_hip_rope* qsf_hip_rope_create(int head_dim, float theta);
void qsf_hip_rope_free(qsf_hip_rope* r);
int qsf_hip_rope_dev(const qsf_hip_rope* r, float* d_q, float* d_k, int n_heads, int n_kv_heads,
                     int position, void* stream);
/* kv_cache_store, src/engine.c:240-300: row `position` of one layer's cache;
 * int8 codes and scales bit-exact. */
int qsf_hip_kv_store_dev(int8_t* d_kc, int8_t* d_vc, float* d_ks, float* d_vs, int max_seq,
                         int n_kv_heads, int head_dim, int position, const float* d_k,
                         const float* d_v, void* stream);
/* The attention loop of src/engine.c:879-923 over positions 0..position
 * (grouped-query heads: head h reads KV head h / (n_heads / n_kv_heads));
 * d_out [n_heads][head_dim].  head_dim a multiple of 16 up to 256,
 * position < 16384.  Uses a library workspace for per-chunk partial
 * results (grown on first use: run once eagerly before capturing a graph;
 * calls must not overlap on different streams). */
int qsf_hip_attention_dev(const float* d_q, const int8_t* d_kc, const int8_t* d_vc,
                          const float* d_ks, const float* d_vs, int max_seq, int n_heads,
                          int n_kv_heads, int head_dim, int position, float* d_out, void* stream);
/* gate = act(gate) * up, src/engine.c:1128-1140 (QSFActivation: 2 SiLU,
 * 0/1 GELU, else ReLU) */
int qsf_hip_act_mul_dev(float* d_gate, const float* d_up, int n, int activation, void* stream);
/* d_out[i] = act(gate_i . x) * (up_i . x) over a tensor from
 * qsf_hip_tensor_upload_pair, in one GEMV launch: the results equal the
 * gate/up GEMV followed by qsf_hip_act_mul_dev bit for bit.  Replaces
 * src/engine.c:1118-1140 for a device-resident engine. */
int qsf_hip_gate_up_act_dev(const qsf_hip_tensor* pair, const float* d_x, float* d_out, int activation,
                            void* stream);
/* res += x, src/engine.c:937 and 1174; with d_bad, the NaN/Inf check of
 * src/engine.c:1176-1187: *d_bad = first index holding NaN or |v| > 1e30,
 * or -1 (written on every call; nothing to clear beforehand). */
int qsf_hip_residual_dev(float* d_res, const float* d_x, int n, int* d_bad, void* stream);
/* Fused forms of the sequences a layer step runs back to back; each equals
 * its separate calls bit for bit, in one launch instead of two.
 * Residual + NaN check + the next norm: res += x (src/engine.c:937, 1174),
 * the check of 1176-1187 into d_bad (may be NULL), then d_out = norm(res)
 * (RMS, or layer norm with d_b when layer_norm != 0; 940-948, 805-815). */
int qsf_hip_residual_norm_dev(float* d_res, const float* d_x, int n, int* d_bad, const float* d_w,
                              const float* d_b, float eps, int layer_norm, float* d_out, void* stream);
/* Residual + NaN check + RMS norm fused into the matvec that consumes the
 * norm (src/engine.c:1174-1187 and 940-948 ahead of the q/k/v matvecs at
 * 848-866, or 937 and 805-815 ahead of gate/up at 1118-1125): d_res_out =
 * d_res + d_x, *d_bad as in qsf_hip_residual_dev (d_bad may be NULL), and
 * the rows multiply rms_norm(d_res_out) * d_w.  Equal bit for bit to
 * qsf_hip_residual_norm_dev followed by qsf_hip_matvec_group_dev /
 * qsf_hip_gate_up_act_dev, in one launch instead of two.  No counterpart in
 * the reference, which runs these steps one after another.  d_res_out is a
 * second residual buffer (not d_res or d_x: every workgroup reads d_res
 * while one writes d_res_out), and d_y / d_out alias none of the three.
 * Blockwise tensors without outliers, cols <= 8192; otherwise
 * QSF_ERR_INVALID_INPUT and nothing runs. */
int qsf_hip_residual_norm_matvec_group_dev(const qsf_hip_tensor* const* t, int n, const float* d_res,
                                           float* d_res_out, const float* d_x, int* d_bad,
                                           const float* d_w, float eps, float* const* d_y, void* stream);
int qsf_hip_residual_norm_gate_up_act_dev(const qsf_hip_tensor* pair, const float* d_res, float* d_res_out,
                                          const float* d_x, int* d_bad, const float* d_w, float eps,
                                          float* d_out, int activation, void* stream);
/* RoPE of q and k (apply_rope, src/engine.c:204-235) and the int8 KV store
 * of the rotated k and of v at `position` (kv_cache_store, 240-300);
 * head_dim <= 256. */
int qsf_hip_rope_kv_store_dev(const qsf_hip_rope* r, float* d_q, float* d_k, const float* d_v,
                              int n_heads, int n_kv_heads, int position, int8_t* d_kc, int8_t* d_vc,
                              float* d_ks, float* d_vs, int max_seq, void* stream);
/* qsf_hip_rope_kv_store_dev followed by qsf_hip_attention_dev (the
 * sequence src/engine.c:870-923 runs: apply_rope, kv_cache_store, the
 * attention loop), in two launches instead of three for head_dim 64, 128
 * and 256: the cache rows, scales and d_out equal the two calls' bit for
 * bit.  On return d_q and d_k hold either their inputs or the rotated
 * values (rotated only for other head dims, which run the two calls):
 * neither is read after this step.  Same limits and workspace as
 * qsf_hip_attention_dev.  No counterpart in the reference, which runs the
 * three steps one after another. */
int qsf_hip_rope_kv_attention_dev(const qsf_hip_rope* r, float* d_q, float* d_k, const float* d_v,
                                  int n_heads, int n_kv_heads, int position, int8_t* d_kc, int8_t* d_vc,
                                  float* d_ks, float* d_vs, int max_seq, float* d_out, void* stream);
/* Embedding lookup, src/engine.c:709-765: row `token` of a blockwise table
 * uploaded with qsf_hip_tensor_upload (rows = vocab, cols = hidden),
 * dequantised bit-exactly; or of an FP16 table [vocab][hd] in device memory.
 * Blockwise types 0, 2, 3 and 4 only, the ones the engine's lookup reads
 * (its row size, qsf_quant_block_size, is 0 for the outlier and MXFP4 types,
 * and type 1 rows are dequantised as 4-bit): others fail with E_INVALID. */
int qsf_hip_embed_row_dev(const qsf_hip_tensor* table, int token, float* d_out, void* stream);
int qsf_hip_embed_row_fp16_dev(const uint16_t* d_table, int hd, int token, float* d_out,
                               void* stream);

/* Bit-exact unpack of `nblocks` QSF blocks already in device memory (the
 * same device code paths the GEMV uses): codes int8[nblocks*bs] (2/3/4-bit
 * field values; 4-bit sym as two's complement), meta u32[nblocks] (first
 * block dword: fp16 scale | fp16 zero << 16), dequantised fp32[nblocks*bs]
 * (scale*q + zero with separate roundings, src/quant.c:95-177).
 * Any output pointer may be NULL. */
int qsf_hip_unpack_dev(int quant_type, const void* d_blocks, int nblocks, int block_size,
                       int8_t* d_codes, uint32_t* d_meta, float* d_dequant, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* QSF_HIP_H */
