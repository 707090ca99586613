/*
 * qsf_loader.c - QSF model file -> device weight arena.
 *
 * Replaces, for this path, the mmap streaming of src/file_access.c and the
 * per-token tensor walk of src/engine.c:183-202: one pass over the file at
 * load time validates the header (src/format.c:37-99), checks the header,
 * layer, embedding and final-section CRC-32s (src/format.c:11-34,
 * 129-135, 226-233; a mismatch warns and is counted, as the reference only
 * warns), walks every layer's [24-byte QSFTensorHeader][data] records
 * (include/qsf/types.h:264-273) and uploads each matrix to HBM once.  FP16
 * vectors (norm weights, biases) become device fp32 arrays.  The engine
 * then asks for tensors by (layer, tensor type) instead of scanning bytes.
 *
 * The file is parsed and checked completely before the GPU is touched, so
 * a malformed file is rejected without a device.  LZ4-compressed layers
 * are refused (the reference needs liblz4 for them, src/format.c:239-281,
 * and this build links none).
 */
#define _DEFAULT_SOURCE
#include "qsf_hip.h"
#include "qsf_host.h"

#include <fcntl.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

enum {
    E_OK = 0, E_NOT_FOUND = 1, E_CORRUPTED = 2, E_VERSION = 3, E_OOM = 4, E_INVALID_MODEL = 6,
    E_IO = 8, E_INTERNAL = 15
};

/* ---- CRC-32 (ISO 3309, reflected 0xEDB88320), src/format.c:11-34 ------- */
static uint32_t g_crc_table[256];
static pthread_once_t g_crc_once = PTHREAD_ONCE_INIT;

static void crc_table_init(void) {
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int j = 0; j < 8; j++) c = (c >> 1) ^ ((c & 1u) ? 0xEDB88320u : 0u);
        g_crc_table[i] = c;
    }
}

uint32_t qsf_hip_crc32(const void* data, size_t len) {
    pthread_once(&g_crc_once, crc_table_init);
    const uint8_t* p = (const uint8_t*)data;
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < len; i++) c = g_crc_table[(c ^ p[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

/* ---- little-endian field reads (the structs are packed, LE) ----------- */
static uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t le32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static uint64_t le64(const uint8_t* p) { return (uint64_t)le32(p) | ((uint64_t)le32(p + 4) << 32); }
static float lef(const uint8_t* p) {
    uint32_t u = le32(p);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Payload bytes of a matrix as the engine's matvec reads it: the block
 * type get_matvec_fn dispatches to (src/engine.c:141-152), plus the
 * outlier table of the *_outlier types.  0 when it cannot be sized. */
static size_t block_bytes_of(int qt, int bs) {
    switch (qt) {
    case 0: case 1: case 9: return 4 + (size_t)(2 * bs + 7) / 8;
    case 2: return 4 + (size_t)(3 * bs + 7) / 8;
    default: return 4 + (size_t)(4 * bs + 7) / 8;   /* 3, 4, 10 and every other type */
    }
}

/* a * b * c, or 0 when it does not fit a size_t */
static size_t mul3(size_t a, size_t b, size_t c) {
    size_t ab, abc;
    if (__builtin_mul_overflow(a, b, &ab) || __builtin_mul_overflow(ab, c, &abc)) return 0;
    return abc;
}

/* Bytes the upload of a [rows][cols] matrix of type qt reads from `data`
 * (avail bytes there): MXFP4 records, or the dense blocks behind the
 * outlier table of types 9 and 10.  0 when it cannot be sized. */
static size_t matrix_bytes(int qt, const uint8_t* data, size_t avail, uint32_t rows, uint32_t cols,
                           int bs) {
    if (qt == QSF_HIP_QUANT_MXFP4) return mul3(rows, ((size_t)cols + 31) / 32, 17);
    const size_t dense = mul3(rows, ((size_t)cols + (uint32_t)bs - 1) / (uint32_t)bs, block_bytes_of(qt, bs));
    if (dense == 0 && rows > 0 && cols > 0) return 0;
    if (qt == 9 || qt == 10) {
        if (avail < 4) return 0;
        const size_t table = 4 + 6 * (size_t)le32(data);
        return dense > SIZE_MAX - table ? 0 : table + dense;
    }
    return dense;
}

/* ---- parsed file ------------------------------------------------------- */
typedef struct {
    uint16_t type;
    uint8_t qt;          /* resolved (0xFF -> layer or model default) */
    uint32_t rows, cols;
    const uint8_t* data;
    uint32_t data_size;
    qsf_hip_tensor* t;   /* matrices */
    float* d_vec;        /* FP16 vectors, as fp32 */
    size_t n_vec;
} rec_t;

typedef struct {
    int n;
    rec_t* recs;
    qsf_hip_moe* moe;    /* MXFP4 expert table of an MoE layer, or NULL */
} layer_t;

struct qsf_hip_model {
    qsf_hip_model_info info;
    layer_t* layers;
    qsf_hip_tensor* embedding;        /* blockwise table [vocab][hidden] */
    uint16_t* d_embedding_fp16;       /* or an FP16 table */
    qsf_hip_tensor* output_head;      /* separate head; NULL when tied */
    float* d_final_norm_w;
    float* d_final_norm_b;
};

static void free_model(qsf_hip_model* m) {
    if (!m) return;
    if (m->layers) {
        for (uint32_t l = 0; l < m->info.num_layers; l++) {
            for (int i = 0; i < m->layers[l].n; i++) {
                if (m->layers[l].recs[i].t) qsf_hip_tensor_free(m->layers[l].recs[i].t);
                qsf_host_device_free(m->layers[l].recs[i].d_vec);
            }
            free(m->layers[l].recs);
            qsf_hip_moe_free(m->layers[l].moe);
        }
        free(m->layers);
    }
    if (m->embedding) qsf_hip_tensor_free(m->embedding);
    qsf_host_device_free(m->d_embedding_fp16);
    if (m->output_head) qsf_hip_tensor_free(m->output_head);
    qsf_host_device_free(m->d_final_norm_w);
    qsf_host_device_free(m->d_final_norm_b);
    free(m);
}

void qsf_hip_model_free(qsf_hip_model* m) { free_model(m); }

/* first record of a tensor type in a layer (find_tensor, src/engine.c:183-202) */
static const rec_t* find_rec_in(const layer_t* L, int type) {
    for (int i = 0; i < L->n; i++)
        if (L->recs[i].type == (uint16_t)type) return &L->recs[i];
    return NULL;
}

static int warn_crc(qsf_hip_model* m, const char* what, uint32_t got, uint32_t want) {
    fprintf(stderr, "[qsf_hip] %s CRC mismatch (got 0x%08X, expected 0x%08X)\n", what, got, want);
    m->info.crc_mismatches++;
    return 0;
}

/* src/format.c:37-99 */
static int parse_header(const uint8_t* h, size_t fsize, qsf_hip_model_info* in) {
    if (le32(h) != 0x51534631u) return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: bad magic number");
    if (le32(h + 4) > 1u) return qsf_host_fail(E_VERSION, "qsf_hip_model_load: file version too new");
    if (le32(h + 8) < 256u) return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: header_size too small");
    in->num_layers = le32(h + 16);
    in->hidden_dim = le32(h + 20);
    in->num_heads = le32(h + 24);
    in->num_kv_heads = le32(h + 28);
    in->vocab_size = le32(h + 32);
    in->max_seq_len = le32(h + 36);
    in->intermediate_dim = le32(h + 40);
    in->head_dim = le32(h + 44);
    in->quant_type = h[48];
    in->activation = h[49];
    in->norm_type = h[50];
    in->pos_enc_type = h[51];
    in->rope_theta = lef(h + 52);
    in->norm_epsilon = lef(h + 56);
    in->block_size = le32(h + 60);
    in->has_bias = h[140];
    in->ffn_type = h[141];
    in->attn_type = h[142];
    in->weight_tied = h[143] == 1 || le32(h + 156) == 1;
    in->num_experts = h[173];
    in->num_active_experts = h[174];
    in->moe_norm_topk = h[175];
    in->expert_intermediate_dim = le32(h + 177);
    if (in->num_layers == 0 || in->num_layers > 1000u)
        return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: invalid num_layers %u", in->num_layers);
    if (in->hidden_dim == 0 || in->num_heads == 0 || in->hidden_dim % in->num_heads)
        return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: hidden_dim %u / num_heads %u",
                             in->hidden_dim, in->num_heads);
    if (in->num_kv_heads == 0) in->num_kv_heads = in->num_heads;
    if (in->num_heads % in->num_kv_heads)
        return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: num_heads not divisible by num_kv_heads");
    if (in->vocab_size < 100) return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: vocab_size too small");
    if (in->block_size == 0) in->block_size = 64;
    if (in->block_size < 32 || in->block_size > 256 || (in->block_size & (in->block_size - 1)))
        return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: block_size must be a power of 2, 32-256");
    if (in->head_dim == 0) in->head_dim = in->hidden_dim / in->num_heads;
    uint64_t total = le64(h + 160);
    in->size_mismatch = total != 0 && total != fsize;
    return E_OK;
}

/* Walk one layer's records (src/engine.c:183-202) and size-check them. */
static int parse_layer(const uint8_t* data, size_t size, int num_tensors, uint8_t layer_qt,
                       const qsf_hip_model_info* in, layer_t* out, int li) {
    out->recs = calloc((size_t)(num_tensors ? num_tensors : 1), sizeof(rec_t));
    if (!out->recs) return qsf_host_fail(E_OOM, "qsf_hip_model_load: layer records");
    size_t off = 0;
    for (int i = 0; i < num_tensors; i++) {
        if (off + 24 > size)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: layer %d tensor %d header past the layer end",
                                 li, i);
        const uint8_t* th = data + off;
        rec_t* r = &out->recs[out->n++];
        r->type = le16(th);
        uint8_t qt = th[2];
        if (qt == 0xFF) qt = layer_qt;
        if (qt == 0xFF) qt = (uint8_t)in->quant_type;
        r->qt = qt;
        r->rows = le32(th + 4);
        r->cols = le32(th + 8);
        r->data_size = le32(th + 12);
        uint32_t n_out = le32(th + 16);
        off += 24;
        if (off + r->data_size > size)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: layer %d tensor %d data past the layer end",
                                 li, i);
        r->data = data + off;
        off += r->data_size;
        /* a separate outlier table after the data (never written by the
         * converter, which keeps outliers inside the payload) */
        off += (size_t)n_out * 6;
        if (qt == 7) {
            if (r->data_size < 2) return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: empty FP16 tensor");
            continue;
        }
        size_t need = matrix_bytes(qt, r->data, r->data_size, r->rows, r->cols, (int)in->block_size);
        if (r->rows == 0 || r->cols == 0 || need == 0 || need > r->data_size || r->rows > 0x7FFFFFFFu ||
            r->cols > 0x7FFFFFFFu)
            return qsf_host_fail(E_INVALID_MODEL,
                                 "qsf_hip_model_load: layer %d tensor type %u (%ux%u, quant %u) holds %u "
                                 "bytes, its matvec reads %zu", li, r->type, r->rows, r->cols, qt,
                                 r->data_size, need);
    }
    return E_OK;
}

/* Error code of a failed upload: the recorded one, never 0 (a load that
 * reports success must hold every tensor). */
static int upload_failed(void) {
    const int e = qsf_hip_last_error();
    return e ? e : qsf_host_fail(E_INTERNAL, "qsf_hip_model_load: upload failed");
}

static float* fp16_to_device(const uint8_t* p, size_t n) {
    float* h = malloc(sizeof(float) * (n ? n : 1));
    if (!h) {
        qsf_host_fail(E_OOM, "qsf_hip_model_load: vector");
        return NULL;
    }
    for (size_t i = 0; i < n; i++) h[i] = qsf_host_fp16(le16(p + 2 * i));
    float* d = qsf_host_device_floats(h, n);
    free(h);
    return d;
}

static int load_mapped(qsf_hip_model* m, const uint8_t* f, size_t fsize) {
    qsf_hip_model_info* in = &m->info;
    if (fsize < 256) return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: file too small for a header");
    int rc = parse_header(f, fsize, in);
    if (rc) return rc;
    uint32_t hcrc = qsf_hip_crc32(f, 168);
    if (hcrc != le32(f + 168)) warn_crc(m, "header", hcrc, le32(f + 168));
    const int bs = (int)in->block_size, hd = (int)in->hidden_dim;

    /* layer index, src/format.c:146-180 */
    uint64_t lio = le64(f + 64);
    size_t lis = (size_t)in->num_layers * 48;
    if (lio == 0 || lio > fsize || lis > fsize - lio)
        return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: invalid layer index offset");
    m->layers = calloc(in->num_layers, sizeof(layer_t));
    if (!m->layers) return qsf_host_fail(E_OOM, "qsf_hip_model_load: layers");
    for (uint32_t l = 0; l < in->num_layers; l++) {
        const uint8_t* e = f + lio + 48 * (size_t)l;
        uint64_t off = le64(e);
        uint32_t csize = le32(e + 8);
        uint8_t lqt = e[16], comp = e[17];
        uint16_t nt = le16(e + 18);
        uint32_t crc = le32(e + 20);
        if (comp != 0)
            return qsf_host_fail(E_INTERNAL, "qsf_hip_model_load: layer %u is LZ4-compressed; this build "
                                             "reads uncompressed layers only", l);
        if (off > fsize || csize > fsize - off)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: layer %u data past the end of the file", l);
        if (crc != 0) {
            uint32_t got = qsf_hip_crc32(f + off, csize);
            if (got != crc) {
                char what[32];
                snprintf(what, sizeof what, "layer %u", l);
                warn_crc(m, what, got, crc);
            }
        }
        rc = parse_layer(f + off, csize, nt, lqt, in, &m->layers[l], (int)l);
        if (rc) return rc;
        in->num_tensors += (uint32_t)m->layers[l].n;
    }

    /* embedding section (types.h:276-286; engine.c:709-765) */
    const uint8_t* emb = NULL;
    uint32_t emb_qt = 0;
    size_t emb_row_bytes = 0;
    uint64_t eo = le64(f + 72);
    if (eo) {
        if (eo > fsize || fsize - eo < 32)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: embedding header past the end");
        const uint8_t* eh = f + eo;
        emb_qt = le32(eh);
        uint32_t nvec = le32(eh + 8), dim = le32(eh + 12), nchunks = le32(eh + 24), ecrc = le32(eh + 20);
        if (eh[16] != 0)
            return qsf_host_fail(E_INTERNAL, "qsf_hip_model_load: compressed embedding not supported");
        if (nvec != in->vocab_size || dim != in->hidden_dim)
            return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: embedding %ux%u, model %ux%u", nvec,
                                 dim, in->vocab_size, in->hidden_dim);
        uint64_t dofs = eo + 32 + (nchunks > 1 ? 8ull * nchunks : 0);
        if (dofs > fsize)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: embedding data past the end");
        /* the span the upload reads: FP16 rows at the engine's stride of
         * ceil(dim / bs) blocks of 2 * bs bytes (engine.c:718-721 with
         * quant.c:82), else the table as a matrix of its type (outlier
         * table and MXFP4 records included) */
        if (emb_qt == 7) emb_row_bytes = (((size_t)dim + (uint32_t)bs - 1) / (uint32_t)bs) * (uint32_t)bs * 2;
        size_t esize = emb_qt == 7 ? mul3(nvec, emb_row_bytes, 1)
                                   : matrix_bytes((int)emb_qt, f + dofs, fsize - dofs, nvec, dim, bs);
        if (esize == 0 && nvec > 0 && dim > 0)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: embedding size cannot be computed");
        if (esize > fsize - dofs)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: embedding data past the end");
        emb = f + dofs;
        uint32_t got = qsf_hip_crc32(emb, esize);
        if (ecrc != 0 && got != ecrc) warn_crc(m, "embedding", got, ecrc);
        in->has_embedding = 1;
    }

    /* final section (types.h:300-306; engine.c:403-420, 664-679) */
    const uint8_t* norm = NULL;
    const uint8_t* head = NULL;
    uint32_t norm_size = 0, head_size = 0;
    uint64_t fo = le64(f + 80);
    if (fo) {
        if (fo > fsize || fsize - fo < 16)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: final header past the end");
        const uint8_t* fh = f + fo;
        norm_size = le32(fh + 4);
        head_size = le32(fh + 8);
        uint32_t fcrc = le32(fh + 12);
        if ((size_t)norm_size + head_size > fsize - fo - 16)
            return qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load: final section past the end");
        if (norm_size < (uint32_t)hd * 2)
            return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: final norm shorter than hidden_dim");
        norm = fh + 16;
        uint32_t got = qsf_hip_crc32(norm, (size_t)norm_size + head_size);
        if (fcrc != 0 && got != fcrc) warn_crc(m, "final section", got, fcrc);
        if (!in->weight_tied && head_size > 0) {
            head = norm + norm_size;
            size_t need = matrix_bytes(in->quant_type, head, head_size, in->vocab_size, in->hidden_dim, bs);
            if (need == 0 || need > head_size)
                return qsf_host_fail(E_INVALID_MODEL, "qsf_hip_model_load: output head holds %u bytes, "
                                                      "its matvec reads %zu", head_size, need);
        }
    }

    /* everything checked: upload */
    if (qsf_hip_init(0) != E_OK) return upload_failed();
    for (uint32_t l = 0; l < in->num_layers; l++) {
        for (int i = 0; i < m->layers[l].n; i++) {
            rec_t* r = &m->layers[l].recs[i];
            if (r->qt == 7) {
                r->n_vec = r->data_size / 2;
                r->d_vec = fp16_to_device(r->data, r->n_vec);
                if (!r->d_vec) return upload_failed();
                in->device_bytes += r->n_vec * 4;
            } else {
                r->t = qsf_host_upload_owned(r->data, r->qt, (int)r->rows, (int)r->cols, bs);
                if (!r->t) return upload_failed();
                in->device_bytes += qsf_hip_tensor_payload_bytes(r->t);
            }
        }
    }
    /* MoE layers whose experts are all MXFP4: one device expert table per
     * layer (gate/up/down tensors and their FP16 biases, the
     * QSF_MOE_*(e) records of include/qsf/types.h:145-162) */
    if (in->ffn_type == 3 && in->num_experts > 1) {
        const int ne = (int)in->num_experts;
        const int eid = (int)(in->expert_intermediate_dim ? in->expert_intermediate_dim
                                                          : in->intermediate_dim);
        const qsf_hip_tensor** tt = calloc((size_t)ne * 3, sizeof *tt);
        const uint16_t** bb = calloc((size_t)ne * 3, sizeof *bb);
        if (!tt || !bb) {
            free(tt);
            free(bb);
            return qsf_host_fail(E_OOM, "qsf_hip_model_load: expert tables");
        }
        for (uint32_t l = 0; l < in->num_layers && !rc; l++) {
            int all = 1;
            for (int e = 0; e < ne && all; e++) {
                for (int j = 0; j < 3; j++) {
                    const rec_t* w = find_rec_in(&m->layers[l], 23 + 6 * e + 2 * j);
                    const rec_t* b = find_rec_in(&m->layers[l], 24 + 6 * e + 2 * j);
                    if (!w || w->qt != QSF_HIP_QUANT_MXFP4) {
                        all = 0;
                        break;
                    }
                    const uint32_t blen = j < 2 ? (uint32_t)eid : in->hidden_dim;
                    tt[3 * e + j] = w->t;
                    bb[3 * e + j] = b && b->qt == 7 && b->data_size >= 2 * blen ? (const uint16_t*)b->data
                                                                               : NULL;
                }
            }
            if (!all) continue;
            /* the bias vectors are copied from the mapping at creation */
            const qsf_hip_tensor *g[256], *u[256], *d[256];
            const uint16_t *gb[256], *ub[256], *db[256];
            for (int e = 0; e < ne; e++) {
                g[e] = tt[3 * e]; u[e] = tt[3 * e + 1]; d[e] = tt[3 * e + 2];
                gb[e] = bb[3 * e]; ub[e] = bb[3 * e + 1]; db[e] = bb[3 * e + 2];
            }
            m->layers[l].moe = qsf_hip_moe_create(ne, hd, eid, g, u, d, gb, ub, db);
            if (m->layers[l].moe) {
                in->moe_layers++;
            } else if (qsf_hip_last_error() == 11) {
                /* a shape the expert table does not take (hidden or expert
                 * dim not a multiple of 4): the experts stay ordinary tensors */
                fprintf(stderr, "[qsf_hip] layer %u: no MXFP4 expert table (%s); experts load as tensors\n",
                        l, qsf_hip_last_error_detail());
            } else {
                rc = upload_failed();
            }
        }
        free(tt);
        free(bb);
        if (rc) return rc;
    }
    if (emb) {
        if (emb_qt == 7) {
            /* [vocab][hd] on the device: rows padded to whole blocks in the
             * file are packed (sizes checked above) */
            const size_t nb = (size_t)in->vocab_size * hd * 2;
            if (emb_row_bytes == (size_t)hd * 2) {
                m->d_embedding_fp16 = (uint16_t*)qsf_host_device_bytes(emb, nb);
            } else {
                uint8_t* packed = malloc(nb ? nb : 1);
                if (!packed) return qsf_host_fail(E_OOM, "qsf_hip_model_load: FP16 embedding staging");
                for (size_t r = 0; r < in->vocab_size; r++)
                    memcpy(packed + r * hd * 2, emb + r * emb_row_bytes, (size_t)hd * 2);
                m->d_embedding_fp16 = (uint16_t*)qsf_host_device_bytes(packed, nb);
                free(packed);
            }
            if (!m->d_embedding_fp16) return upload_failed();
            in->device_bytes += nb;
        } else {
            m->embedding = qsf_host_upload_owned(emb, (int)emb_qt, (int)in->vocab_size, hd, bs);
            if (!m->embedding) return upload_failed();
            in->device_bytes += qsf_hip_tensor_payload_bytes(m->embedding);
        }
    }
    if (norm) {
        m->d_final_norm_w = fp16_to_device(norm, (size_t)hd);
        if (!m->d_final_norm_w) return upload_failed();
        if ((in->has_bias & 0x08) && norm_size >= (uint32_t)hd * 4) {
            m->d_final_norm_b = fp16_to_device(norm + 2 * (size_t)hd, (size_t)hd);
            if (!m->d_final_norm_b) return upload_failed();
        }
        if (head) {
            m->output_head = qsf_host_upload_owned(head, in->quant_type, (int)in->vocab_size, hd, bs);
            if (!m->output_head) return upload_failed();
            in->device_bytes += qsf_hip_tensor_payload_bytes(m->output_head);
        }
    }
    return E_OK;
}

qsf_hip_model* qsf_hip_model_load(const char* path) {
    if (!path) {
        qsf_host_fail(E_NOT_FOUND, "qsf_hip_model_load: null path");
        return NULL;
    }
    int fd = open(path, O_RDONLY);
    if (fd < 0) {
        qsf_host_fail(E_NOT_FOUND, "qsf_hip_model_load: cannot open %s", path);
        return NULL;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        qsf_host_fail(E_IO, "qsf_hip_model_load: cannot stat %s", path);
        return NULL;
    }
    size_t fsize = (size_t)st.st_size;
    void* map = mmap(NULL, fsize, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        qsf_host_fail(E_IO, "qsf_hip_model_load: cannot map %s", path);
        return NULL;
    }
    qsf_hip_model* m = calloc(1, sizeof *m);
    int rc = m ? load_mapped(m, (const uint8_t*)map, fsize) : qsf_host_fail(E_OOM, "qsf_hip_model_load");
    munmap(map, fsize);
    if (rc) {
        free_model(m);
        return NULL;
    }
    return m;
}

qsf_hip_model* qsf_hip_model_load_mem(const void* data, size_t size) {
    if (!data || size == 0) {
        qsf_host_fail(E_CORRUPTED, "qsf_hip_model_load_mem: empty buffer");
        return NULL;
    }
    qsf_hip_model* m = calloc(1, sizeof *m);
    int rc = m ? load_mapped(m, (const uint8_t*)data, size) : qsf_host_fail(E_OOM, "qsf_hip_model_load_mem");
    if (rc) {
        free_model(m);
        return NULL;
    }
    return m;
}

int qsf_hip_model_get_info(const qsf_hip_model* m, qsf_hip_model_info* out) {
    if (!m || !out) return qsf_host_fail(11, "qsf_hip_model_get_info: null argument");
    *out = m->info;
    return E_OK;
}

static const rec_t* find_rec(const qsf_hip_model* m, int layer, int type) {
    if (!m || layer < 0 || (uint32_t)layer >= m->info.num_layers) return NULL;
    return find_rec_in(&m->layers[layer], type);
}

qsf_hip_moe* qsf_hip_model_moe(const qsf_hip_model* m, int layer) {
    if (!m || layer < 0 || (uint32_t)layer >= m->info.num_layers) return NULL;
    return m->layers[layer].moe;
}

const qsf_hip_tensor* qsf_hip_model_tensor(const qsf_hip_model* m, int layer, int tensor_type) {
    const rec_t* r = find_rec(m, layer, tensor_type);
    return r ? r->t : NULL;
}

const float* qsf_hip_model_vector(const qsf_hip_model* m, int layer, int tensor_type, int* n) {
    const rec_t* r = find_rec(m, layer, tensor_type);
    if (n) *n = r && r->d_vec ? (int)r->n_vec : 0;
    return r ? r->d_vec : NULL;
}

const qsf_hip_tensor* qsf_hip_model_embedding(const qsf_hip_model* m) {
    return m ? m->embedding : NULL;
}

const uint16_t* qsf_hip_model_embedding_fp16(const qsf_hip_model* m) {
    return m ? m->d_embedding_fp16 : NULL;
}

const qsf_hip_tensor* qsf_hip_model_output_head(const qsf_hip_model* m) {
    if (!m) return NULL;
    return m->info.weight_tied ? m->embedding : m->output_head;
}

const float* qsf_hip_model_final_norm(const qsf_hip_model* m, const float** bias) {
    if (bias) *bias = m ? m->d_final_norm_b : NULL;
    return m ? m->d_final_norm_w : NULL;
}
