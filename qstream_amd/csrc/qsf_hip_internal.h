/*
 * qsf_hip_internal.h - contract between the C11 host layer (host/qsf_hip.c)
 * and the gfx950 kernels (the csrc .hip files).  Plain C: no C++ types cross it.
 */
#ifndef QSF_HIP_INTERNAL_H
#define QSF_HIP_INTERNAL_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quant type ids (include/qsf/types.h:43-56) plus MXFP4 in unused slot 11. */
enum {
    QK_Q2 = 0, QK_Q2SYM = 1, QK_Q3 = 2, QK_Q4 = 3, QK_Q4SYM = 4,
    QK_Q2_OUTLIER = 9, QK_Q4_OUTLIER = 10, QK_MXFP4 = 11
};

/* Kernel formats of the decode GEMV (what the device unpacks). */
enum { QK_FMT_2 = 0, QK_FMT_3 = 1, QK_FMT_4 = 2, QK_FMT_4SYM = 3 };

/* A weight tensor resident in HBM.  Block bytes are the QSF on-disk blocks,
 * unchanged, relocated to a 256-byte aligned region; an outlier table is
 * re-encoded as per-row CSR (file order kept inside a row, out-of-range
 * entries dropped, duplicates kept). */
typedef struct qsf_hip_tensor {
    int      qt, rows, cols, bs;
    int      fmt;               /* QK_FMT_* or -1 for MXFP4 */
    int      nb;                /* blocks per row */
    int      block_bytes;
    const void* host_key;       /* registry key (host payload pointer) */
    size_t   payload_bytes;     /* on-disk payload size (algorithmic bytes) */
    uint8_t* d_blocks;          /* rows*nb*block_bytes (MXFP4: codes plane) */
    uint8_t* d_scales;          /* MXFP4: E8M0 plane rows*nb, else NULL */
    uint32_t n_outliers;        /* entries in the file table */
    uint32_t n_csr;             /* entries kept (in range) */
    uint32_t* d_row_ptr;        /* rows+1, or NULL */
    uint32_t* d_oent;           /* n_csr packed entries col | fp16 << 16 (cols <= 65536), or NULL */
    uint32_t* d_ocol;           /* else n_csr column indices ... */
    uint16_t* d_oval;           /* ... and n_csr fp16 values */
    void*    d_alloc;           /* base of the single device allocation */
    size_t   alloc_bytes;       /* its parts (blocks, scales, CSR) up to the tail pad */
    int      frag;              /* 1: d_blocks in fragment order (below) */
    int      frag_nq;           /* fragment order: 4-block quads a row, ceil(nb / 4) */
    int      plane;             /* 1: d_blocks in row-plane order (below); with frag
                                 * 0 as well: on-disk order */
    int      registry_owned;    /* uploaded implicitly by a table-slot call */
    const void* succ;           /* table slots: the key called next with the same x ... */
    int      succ_hits;         /* ... this many times since it last differed */
    struct qsf_hip_tensor* prev; /* list of live tensors (freed at shutdown) */
    struct qsf_hip_tensor* next;
} qsf_hip_tensor;

#define QK_MAX_GROUP 8

/* Fragment order: the device layout of a dense tensor the matrix-core GEMV
 * covers (qk_mfma_layout).  The on-disk blocks, unchanged, regrouped into
 * tiles of 16 rows x 4 blocks: tile t = (row / 16) * nq + b / 4 (nq =
 * ceil(nb / 4)) holds 64 blocks, lane L = 16 (b % 4) + row % 16 holding block
 * b of row `row`.  A tile is 64 * bb bytes: bb / 16 planes of 64 x 16 bytes
 * (plane i: bytes [16 i, 16 i + 16) of every lane's block, lane-major), then
 * a plane of 64 x (bb % 16) bytes with the rest.  Blocks past nb and rows
 * past `rows` in a tile are zero.  So a wave reads a tile with 16-byte loads
 * that each cover 1 KB of contiguous memory. */
size_t qk_frag_bytes(int rows, int nb, int block_bytes);
/* byte j of block b of row `row` in fragment order */
size_t qk_frag_offset(size_t row, int b, int j, int nq, int block_bytes);
/* Row-plane order: the device layout of every other dense tensor.  Rows
 * stay where they are on disk (nb * bb bytes each); inside a row:
 *  - blocks of at most 64 codes (read whole, one a lane): bytes
 *    [16 i, 16 i + 16) of block b sit at i * nb * 16 + 16 b (plane i, for
 *    i < bb / 16), and the last bb % 16 bytes of block b at
 *    (bb / 16) * nb * 16 + (bb % 16) b (the tail plane);
 *  - blocks of 128 or 256 codes (read as 64-code parts, one a lane): the
 *    meta dwords first (block b at 4 b), then the parts' code bytes, part
 *    u = b * (bs / 64) + p holding codes [64 p, 64 p + 64) of block b, in
 *    the same planes over parts (16-byte planes of np = nb * bs / 64 parts,
 *    then a tail plane of cwb % 16 bytes a part, cwb = the part's code
 *    bytes: 16, 24 or 32).
 * So a wave's 16-byte loads of consecutive blocks or parts each read one
 * aligned, contiguous run of 1 KB where the on-disk order gives
 * dword-aligned loads that straddle lines and reads each line twice (codes,
 * then meta). */
int qk_plane_layout(int fmt, int bs);
/* byte j of block b of a row of nb blocks of bs codes in row-plane order,
 * from the row's first byte */
size_t qk_plane_offset(int b, int j, int nb, int block_bytes, int bs);

/* 1 when the matrix-core GEMV covers tensors of this format (QK_FMT_*),
 * block size and column count (with an outlier table when `outliers`), so
 * that they are uploaded in fragment order */
int qk_mfma_layout(int fmt, int bs, int cols, int outliers);

/* Per-call prepared activation: block-fixed-point digits of x. */
size_t qk_xprep_bytes(int fmt, int bs, int cols);

/* n floats from host-mapped `src` to device `d_dst` (both 16-B aligned) */
int qk_stage_f32(float* d_dst, const float* src, int n, hipStream_t s);

/* qk_xprep from x in host-mapped memory, also writing fp32 x to d_xcopy
 * (room for ceil(cols/bs)*bs floats): the table slots' one x dispatch */
int qk_xprep_stage(int fmt, int bs, int cols, const float* x, float* d_xcopy, void* d_ws,
                   hipStream_t s);

/* x preparation into ws (qk_xprep_bytes(fmt, bs, cols) bytes, 256-B aligned) */
int qk_xprep(int fmt, int bs, int cols, const float* d_x, void* d_ws, hipStream_t s);
/* GEMV over n tensors sharing x.  mode: QK_RUN_BOTH prepares x inside the
 * GEMV workgroups (one launch); QK_RUN_GEMV reads digits prepared into ws by
 * qk_xprep; QK_RUN_BOTH | QK_RUN_STANDALONE_PREP launches both kernels. */
enum { QK_RUN_XPREP = 1, QK_RUN_GEMV = 2, QK_RUN_BOTH = 3, QK_RUN_STANDALONE_PREP = 4 };
int qk_gemv_group(const qsf_hip_tensor* const* t, int n, const float* d_x,
                  float* const* d_y, void* d_ws, int mode, hipStream_t s);
/* One-launch GEMV over a paired tensor (row 2i gate_i, row 2i+1 up_i, no
 * outliers): y[i] = act(gate_i x) * (up_i x), act a QSFActivation >= 0.
 * -2 when the plan cannot take two-row tiles. */
int qk_gemv_pair_act(const qsf_hip_tensor* t, const float* d_x, float* d_y, int act, hipStream_t s);
/* Residual + RMS norm fused ahead of a one-launch GEMV: res_out = res_in +
 * x (the matvec's x argument is the increment), the NaN check into *bad
 * (may be NULL), then the rows multiply rms_norm(res_out) * w.  Equal bit
 * for bit to qk_residual_norm followed by the plain GEMV.  res_out must
 * differ from res_in and x, and y from all three.  -2 when the plan is not
 * the one-launch whole-row kernel without outliers, or cols > 8192. */
typedef struct {
    const float* res_in;
    float* res_out;
    const float* w;
    int* bad;
    float eps;
} qk_norm_args;
int qk_gemv_group_norm(const qsf_hip_tensor* const* t, int n, const qk_norm_args* nm,
                       const float* d_x, float* const* d_y, hipStream_t s);
int qk_gemv_pair_act_norm(const qsf_hip_tensor* t, const qk_norm_args* nm, const float* d_x,
                          float* d_y, int act, hipStream_t s);
/* One-launch decode GEMV on the int8 matrix cores (gemv_mfma.hip) over n
 * tensors in fragment order sharing fp32 x in HBM: the path qk_gemv_group
 * takes for them in every mode (a prepared x is not used).  A group's
 * matrices must all have outlier tables or none.  act1: paired rows
 * (qk_gemv_pair_act); nm: the fused residual + norm (qk_gemv_group_norm), or
 * NULL.  Returns -2 when the call is not covered.  A row's arithmetic
 * depends on its matrix's shape and its outlier entries only, never on the
 * group or the grid. */
int qk_gemv_mfma(const qsf_hip_tensor* const* t, int n, const float* d_x, float* const* d_y,
                 int act1, const qk_norm_args* nm, hipStream_t s);
/* Engine for tensors uploaded from now on: 1 (default) the matrix-core GEMV
 * and fragment order for the 3-bit formats where qk_mfma_layout covers the
 * shape, 2 the same for every format, 0 the dot-product kernels and on-disk
 * order for all; < 0 only queries.  Returns the previous setting. */
int qk_gemv_mfma_enable(int on);

/* What fixes a row's arithmetic in qk_gemv_group(t, n, ..., mode): the
 * kernel instantiation, row-group width, tile rows and chunk.  A tensor's
 * rows come out bit-identical in two launches whose signatures are equal
 * (0: the group is not supported). */
uint64_t qk_gemv_signature(const qsf_hip_tensor* const* t, int n, int mode);

/* Kernel timing of main-path GEMV and prefill launches (event pair at the
 * kernel's own start and end): on/off (on resets the record), then read
 * durations in us.  qk_timing_pair hands a launcher the next event pair for
 * hipExtLaunchKernel, or returns 0 when timing is off or the record is full. */
int qk_timing(int enable);
int qk_timing_read(float* us, int max);
int qk_timing_pair(hipEvent_t* start, hipEvent_t* stop);

/* Bit-exact unpack checks: codes as int8 [nblocks][bs], meta bits u32 per
 * block (scale | zero << 16); dequantised fp32 [nblocks][bs]. */
int qk_unpack(int qt, const void* d_blocks, int nblocks, int bs,
              int8_t* d_codes, uint32_t* d_meta, float* d_deq, hipStream_t s);

/* MXFP4 GEMV for T tokens: y[t][rows] = W x[t]. */
int qk_mxfp4_gemv(const qsf_hip_tensor* t, const float* d_x, int ntok,
                  float* d_y, hipStream_t s);

/* MoE FFN (src/engine.c:951-1107) for ntok <= 8 tokens, experts in MXFP4.
 * Device-side expert table entry: codes/scales of gate, up ([eid][hidden])
 * and down ([hidden][eid]) plus optional fp16 biases (NULL = none). */
typedef struct {
    const uint8_t* gc; const uint8_t* gs; const uint16_t* gb;
    const uint8_t* uc; const uint8_t* us; const uint16_t* ub;
    const uint8_t* dc; const uint8_t* ds; const uint16_t* db;
} qk_mx_expert;
size_t qk_moe_ws_bytes(int n_exp, int k, int ntok, int hidden, int eid);
/* stages: bit 0 the routing launch (more than one token; one token routes
 * in the gate/up launch), bit 1 gate/up, bit 2 down and combine; a stage
 * left out leaves the workspace as the previous call's stage wrote it. */
int qk_moe_launch(const qk_mx_expert* d_experts, int n_exp, int k, int norm, int act,
                  int hidden, int eid, int ntok, const float* d_x, const float* d_logits,
                  float* d_out, void* d_ws, int stages, hipStream_t s);

/* 4-bit prefill on MFMA: y[m][n] = W[n] . float(x_bf16[m]).  d_ws holds
 * the per-block sums of x and x itself in MFMA fragment order:
 * qk_prefill_ws_bytes(m, cols, bs) bytes, 16-byte aligned. */
size_t qk_prefill_ws_bytes(int m, int cols, int bs);

/* The same prefill with the packed activations in a file-scope device array
 * of QK_PREFILL_SCRATCH_BYTES per GPU instead of a caller workspace: no
 * allocation.  qk_prefill_scratch_init looks up the current device's address
 * of that array (once per device); qk_prefill_4bit_noalloc returns -3 when
 * the call needs more than the array holds. */
#define QK_PREFILL_SCRATCH_BYTES (16 << 20)
#define QK_MAX_DEVICES 64
int qk_prefill_scratch_init(void);
int qk_prefill_4bit_noalloc(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                            float* d_y, hipStream_t s);
/* One streaming read of n device ranges (16-byte aligned), the floor of a
 * launch that reads those bytes once.  A workgroup stores its checksum to
 * *sink only if it equals a fixed 32-bit constant, which keeps every load
 * live and in practice stores nothing. */
int qk_stream_read(const void* const* ptr, const size_t* bytes, int n, uint32_t* sink, hipStream_t s);
/* The bf16 matrix-core ceiling: every CU runs independent
 * v_mfma_f32_16x16x32_bf16 chains `iters` long, with no memory traffic.
 * Returns the launch's FLOP (< 0 on a bad argument or launch failure). */
double qk_mfma_peak(int iters, uint32_t* sink, hipStream_t s);

/* The two halves of qk_prefill_4bit: x bf16 [m][cols] packed into d_ws
 * (qk_prefill_ws_bytes), and the GEMM of a 4-bit tensor with those cols and
 * block size over it. */
int qk_prefill_pack(const uint16_t* d_x_bf16, int m, int cols, int bs, void* d_ws, hipStream_t s);
int qk_prefill_gemm(const qsf_hip_tensor* t, const void* d_ws, int m, float* d_y, hipStream_t s);
int qk_prefill_4bit(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                    float* d_y, void* d_ws, hipStream_t s);

/* Decode glue (decode_glue.hip), all asynchronous on `s`.  Layouts: q
 * [n_heads][head_dim], k/v [n_kv][head_dim]; one layer's KV cache
 * [n_kv][max_seq][head_dim] int8 with scales [n_kv][max_seq].  freq is the
 * head_dim/2 RoPE frequency table.  qk_attention returns -2 for a head_dim
 * above 256 or not a multiple of 16, more than QK_ATT_MAX_SEQ positions
 * or n_heads not a multiple
 * of n_kv; ws holds qk_attention_ws_bytes of per-chunk partial results. */
#define QK_ATT_MAX_SEQ 16384
int qk_norm(const float* in, float* out, const float* w, const float* b, int dim, float eps,
            int layer, hipStream_t s);
int qk_rope(float* q, float* k, const float* freq, int head_dim, int n_heads, int n_kv,
            int position, hipStream_t s);
int qk_kv_store(int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq, int n_kv,
                int head_dim, int position, const float* k, const float* v, hipStream_t s);
size_t qk_attention_ws_bytes(int n_heads, int head_dim, int position);
int qk_attention(const float* q, const int8_t* kc, const int8_t* vc, const float* ks,
                 const float* vs, int max_seq, int n_heads, int n_kv, int head_dim,
                 int position, float* out, void* ws, hipStream_t s);
int qk_act_mul(float* gate, const float* up, int n, int act, hipStream_t s);
int qk_residual(float* res, const float* x, int n, int* bad, hipStream_t s);
int qk_residual_norm(float* res, const float* x, int n, int* bad, const float* w, const float* b,
                     float eps, int layer, float* out, hipStream_t s);
int qk_rope_kv_store(float* q, float* k, const float* v, const float* freq, int head_dim, int n_heads,
                     int n_kv, int position, int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq,
                     hipStream_t s);
/* qk_rope_kv_store then qk_attention, for head_dim 64, 128 or 256 in two
 * launches (RoPE, KV store and the chunk pass in one); other head dims run
 * the two calls.  The cache, scales and out are theirs bit for bit; q and
 * k are rotated in place only on the two-call path. */
int qk_rope_kv_attention(float* q, float* k, const float* v, const float* freq, int head_dim, int n_heads,
                         int n_kv, int position, int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq,
                         float* out, void* ws, hipStream_t s);
int qk_embed_row(const qsf_hip_tensor* t, int token, float* out, hipStream_t s);
int qk_embed_row_fp16(const uint16_t* table, int hd, int token, float* out, hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif
