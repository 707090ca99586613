/*
 * qsf_hip.c - C11 host layer of libqsf_hip.
 *
 * Fills QStream's matvec table slots (src/kernels.c:7-65) with functions of
 * the qsf_matvec_fn type (include/qsf/kernels.h:53-58) that run on the GPU,
 * and keeps weight payloads resident in HBM (device weight arena) instead of
 * streaming them from the mmap'd file (src/file_access.c:80-88).
 *
 * Behaviour the engine relies on (src/engine.c:141-152, call sites in
 * engine.c) is kept: synchronous on return, output fully overwritten,
 * rows <= 0 a no-op, cols == 0 writes zeros, outlier entries applied
 * additively with out-of-range rows skipped (src/quant.c:423-444).
 */
#define _POSIX_C_SOURCE 200809L   /* clock_gettime */
#include "qsf_hip.h"
#include "qsf_host.h"
#include "../csrc/qsf_hip_internal.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ---- errors --------------------------------------------------------------- */
enum { E_OK = 0, E_OOM = 4, E_INVALID = 11, E_INTERNAL = 15 };

/* The engine's error sink (src/error.c:43-53), used when the host links it. */
extern void qsf_set_error(int err, const char* detail) __attribute__((weak));

static _Thread_local int g_err;
static _Thread_local char g_err_detail[256];

static int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err_detail, sizeof g_err_detail, fmt, ap);
    va_end(ap);
    g_err = code;
    if (qsf_set_error) qsf_set_error(code, g_err_detail);
    return code;
}

int qsf_host_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err_detail, sizeof g_err_detail, fmt, ap);
    va_end(ap);
    g_err = code;
    if (qsf_set_error) qsf_set_error(code, g_err_detail);
    return code;
}

int qsf_hip_last_error(void) { return g_err; }
const char* qsf_hip_last_error_detail(void) { return g_err_detail; }

/* ---- device state ----------------------------------------------------------- */
typedef struct {
    int ready, device;
    hipStream_t stream;
    void* ws;          size_t ws_bytes;       /* prefill workspace */
    void* att_ws;      size_t att_ws_bytes;   /* attention partials */
    float* d_x;        size_t d_x_n;          /* device copy of a table slot's x */
    void* slot_xq;     size_t slot_xq_bytes;  /* a table slot's prepared x */
    int xq_ok, xq_fmt, xq_bs, xq_cols;        /* slot_xq and d_x hold h_x prepared so */
    float* h_x;        size_t h_x_n;          /* host-mapped, coherent: slot x ... */
    float* h_y;        size_t h_y_n;          /* ... and y (the kernel writes it) */
    uint32_t* h_flag;  uint32_t* d_flag;      /* host-mapped completion word (slot_wait) */
    uint32_t flag_seq;
    size_t arena_bytes;
} dev_state;

static dev_state g_dev;
static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;

#define HIPCHK(call, code)                                                        \
    do {                                                                          \
        hipError_t e_ = (call);                                                   \
        if (e_ != hipSuccess)                                                     \
            return fail(code, "%s: %s", #call, hipGetErrorString(e_));           \
    } while (0)

static int init_locked(int device) {
    if (g_dev.ready) return E_OK;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail(E_INTERNAL, "qsf_hip: no GPU visible");
    if (device < 0 || device >= n) return fail(E_INVALID, "qsf_hip: device %d of %d", device, n);
    HIPCHK(hipSetDevice(device), E_INTERNAL);
    HIPCHK(hipStreamCreateWithFlags(&g_dev.stream, hipStreamNonBlocking), E_INTERNAL);
    /* device address of the allocation-free prefill's scratch array; a
     * failure here surfaces as that entry point's error (it retries the
     * lookup on its first call on a device) */
    (void)qk_prefill_scratch_init();
    g_dev.device = device;
    g_dev.ready = 1;
    return E_OK;
}

int qsf_hip_init(int device) {
    pthread_mutex_lock(&g_lock);
    int rc = init_locked(device);
    pthread_mutex_unlock(&g_lock);
    return rc;
}

/* Buffers a grow-only device buffer has outgrown.  A caller may have
 * captured a graph whose kernels hold the old address (the device-pointer
 * entry points run on the caller's stream), so an outgrown buffer is never
 * freed before qsf_hip_shutdown; growth is by 1.5x, so the retired buffers
 * together stay below twice the live one. */
static void** g_retired;
static size_t g_retired_n, g_retired_cap;

static int retire_dev(void* p) {
    if (!p) return E_OK;
    if (g_retired_n == g_retired_cap) {
        size_t cap = g_retired_cap ? 2 * g_retired_cap : 16;
        void** nr = realloc(g_retired, cap * sizeof *nr);
        if (!nr) return fail(E_OOM, "qsf_hip: retired-buffer list");
        g_retired = nr;
        g_retired_cap = cap;
    }
    g_retired[g_retired_n++] = p;
    return E_OK;
}

/* grow-only device buffer */
static int ensure_dev(void** p, size_t* have, size_t need) {
    if (*have >= need) return E_OK;
    size_t sz = need < 4096 ? 4096 : need + need / 2;
    void* np = NULL;
    HIPCHK(hipMalloc(&np, sz), E_OOM);
    if (retire_dev(*p) != E_OK) {
        hipFree(np);
        return E_OOM;
    }
    *p = np;
    *have = sz;
    return E_OK;
}

/* grow-only pinned host buffer, mapped into the device address space and
 * coherent (fine-grained): kernels read and write it directly and the host
 * sees a kernel's stores once the stream has been synchronised.  Only the
 * synchronous table slots use these, so the old buffer is idle when freed. */
static int ensure_host(void** p, size_t* have, size_t need) {
    if (*have >= need) return E_OK;
    if (*p) hipHostFree(*p);
    *p = NULL;
    *have = 0;
    size_t sz = need < 4096 ? 4096 : need + need / 2;
    HIPCHK(hipHostMalloc(p, sz, hipHostMallocMapped | hipHostMallocCoherent), E_OOM);
    *have = sz;
    return E_OK;
}

/* ---- tensor payload geometry (src/quant.c:69-85) ------------------------- */
static int kernel_fmt(int qt) {
    switch (qt) {
    case QK_Q2: case QK_Q2SYM: case QK_Q2_OUTLIER: return QK_FMT_2;
    case QK_Q3: return QK_FMT_3;
    case QK_Q4SYM: return QK_FMT_4SYM;
    case QK_MXFP4: return -1;
    default: return QK_FMT_4;   /* the engine maps every other type to 4-bit */
    }
}

static int fmt_bits(int fmt) { return fmt == QK_FMT_2 ? 2 : fmt == QK_FMT_3 ? 3 : 4; }

static int is_outlier(int qt) { return qt == QK_Q2_OUTLIER || qt == QK_Q4_OUTLIER; }

static uint32_t rd_u32(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

/* ---- registry: host payload pointer -> device tensor --------------------- */
typedef struct {
    const void* key;
    qsf_hip_tensor* t;
    uint64_t fp;       /* fingerprint of sampled payload words */
    int vol;           /* the bytes at key have changed once: upload on every call */
} reg_slot;

static reg_slot* g_reg;
static size_t g_reg_cap, g_reg_n;
static uint64_t g_reg_gen;   /* bumped whenever an entry goes */

/* Table-slot results computed ahead (host_matvec): entry 0 is the call that
 * launched them, entries 1..n-1 the calls it expects next, each with its key,
 * tensor, predecessor key and place in h_y.  Valid while the registry
 * generation is gen and x is unchanged. */
typedef struct {
    const void* key;
    const void* pred;
    const qsf_hip_tensor* t;
    size_t off;
    int rows, used;
} ahead_entry;

static struct {
    int n;
    uint64_t gen;
    const void* last;   /* key of the last completed call on prepared x */
    ahead_entry e[QK_MAX_GROUP];
} g_ahead;

static int g_lookahead = 2;   /* successors a slot call may run with itself */

static size_t hash_ptr(const void* p) {
    uint64_t v = (uint64_t)(uintptr_t)p;
    v ^= v >> 33; v *= 0xff51afd7ed558ccdULL; v ^= v >> 33;
    return (size_t)v;
}

static uint64_t fingerprint(const uint8_t* p, size_t n) {
    uint64_t h = 1469598103934665603ULL ^ n;
    if (n == 0) return h;
    size_t pos[9] = {0, n / 8, n / 4, 3 * n / 8, n / 2, 5 * n / 8, 3 * n / 4, 7 * n / 8, n - 1};
    for (int i = 0; i < 9; i++) {
        size_t a = pos[i] > n - 8 && n >= 8 ? n - 8 : pos[i];
        uint64_t w = 0;
        memcpy(&w, p + a, n >= 8 ? 8 : 1);
        h = (h ^ w) * 1099511628211ULL;
    }
    return h;
}

static reg_slot* reg_find(const void* key) {
    if (!g_reg_cap) return NULL;
    for (size_t i = hash_ptr(key) & (g_reg_cap - 1);; i = (i + 1) & (g_reg_cap - 1)) {
        if (g_reg[i].key == key) return &g_reg[i];
        if (!g_reg[i].key) return NULL;
    }
}

static int reg_put(const void* key, qsf_hip_tensor* t, uint64_t fp, int vol) {
    if ((g_reg_n + 1) * 2 > g_reg_cap) {
        size_t cap = g_reg_cap ? g_reg_cap * 2 : 256;
        reg_slot* nr = calloc(cap, sizeof *nr);
        if (!nr) return fail(E_OOM, "qsf_hip: registry");
        for (size_t i = 0; i < g_reg_cap; i++) {
            if (!g_reg[i].key) continue;
            size_t j = hash_ptr(g_reg[i].key) & (cap - 1);
            while (nr[j].key) j = (j + 1) & (cap - 1);
            nr[j] = g_reg[i];
        }
        free(g_reg);
        g_reg = nr;
        g_reg_cap = cap;
    }
    size_t i = hash_ptr(key) & (g_reg_cap - 1);
    while (g_reg[i].key && g_reg[i].key != key) i = (i + 1) & (g_reg_cap - 1);
    if (!g_reg[i].key) g_reg_n++;
    g_reg[i].key = key;
    g_reg[i].t = t;
    g_reg[i].fp = fp;
    g_reg[i].vol = vol;
    return E_OK;
}

static void reg_del(const void* key) {
    reg_slot* s = reg_find(key);
    if (!s) return;
    g_reg_gen++;
    size_t i = (size_t)(s - g_reg);
    g_reg[i].key = NULL;
    g_reg[i].t = NULL;
    g_reg_n--;
    /* re-insert the rest of the probe run */
    for (size_t j = (i + 1) & (g_reg_cap - 1); g_reg[j].key; j = (j + 1) & (g_reg_cap - 1)) {
        reg_slot tmp = g_reg[j];
        g_reg[j].key = NULL;
        g_reg_n--;
        reg_put(tmp.key, tmp.t, tmp.fp, tmp.vol);
    }
}

/* ---- upload --------------------------------------------------------------- */
/* Ownership: tensors returned by qsf_hip_tensor_upload belong to the caller
 * (freed by qsf_hip_tensor_free); tensors a table-slot call uploads belong to
 * the registry.  Registering a new tensor for a host pointer drops the old
 * entry and frees it only if the registry owned it.  Every live tensor is on
 * g_live so qsf_hip_shutdown can free them all. */
static qsf_hip_tensor* g_live;

static void tensor_destroy(qsf_hip_tensor* t) {
    if (!t) return;
    if (t->prev) t->prev->next = t->next;
    else if (g_live == t) g_live = t->next;
    if (t->next) t->next->prev = t->prev;
    if (t->d_alloc) {
        hipFree(t->d_alloc);
        g_dev.arena_bytes -= t->payload_bytes;
    }
    free(t);
}

static void tensor_link(qsf_hip_tensor* t) {
    t->prev = NULL;
    t->next = g_live;
    if (g_live) g_live->prev = t;
    g_live = t;
}

/* unregister a host pointer; free its tensor if the registry owned it */
static void reg_drop(const void* key) {
    reg_slot* s = reg_find(key);
    if (!s) return;
    qsf_hip_tensor* t = s->t;
    reg_del(key);
    if (t && t->registry_owned) tensor_destroy(t);
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

/* Fragment order (qsf_hip_internal.h): 16-row x 4-block tiles of 64 blocks,
 * each block's bytes spread over 16-byte planes and a tail plane. */
size_t qk_frag_bytes(int rows, int nb, int block_bytes) {
    return (size_t)((rows + 15) / 16) * (size_t)((nb + 3) / 4) * 64 * (size_t)block_bytes;
}

size_t qk_frag_offset(size_t row, int b, int j, int nq, int block_bytes) {
    const size_t tile = (row >> 4) * (size_t)nq + (size_t)(b >> 2);
    const size_t lane = (size_t)((b & 3) * 16) + (row & 15);
    const int k = block_bytes >> 4;
    const size_t base = tile * 64 * (size_t)block_bytes;
    return j < 16 * k ? base + (size_t)(j >> 4) * 1024 + lane * 16 + (size_t)(j & 15)
                      : base + (size_t)k * 1024 + lane * (size_t)(block_bytes & 15) + (size_t)(j - 16 * k);
}

/* The on-disk blocks [rows][nb][bb] into fragment order (dst zeroed). */
static void frag_permute(uint8_t* dst, const uint8_t* src, int rows, int nb, int bb) {
    const int nq = (nb + 3) / 4, k = bb / 16, tb = bb % 16;
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const uint8_t* s = src + ((size_t)r * nb + b) * bb;
            uint8_t* tile = dst + (((size_t)(r >> 4) * nq + (size_t)(b >> 2)) * 64) * bb;
            const size_t lane = (size_t)((b & 3) * 16 + (r & 15));
            for (int i = 0; i < k; i++) memcpy(tile + (size_t)i * 1024 + lane * 16, s + 16 * i, 16);
            if (tb) memcpy(tile + (size_t)k * 1024 + lane * tb, s + 16 * k, (size_t)tb);
        }
}

/* Row-plane order (qsf_hip_internal.h): every dense format the dot-product
 * GEMV reads (blocks of up to 64 codes whole, larger ones as 64-code parts). */
int qk_plane_layout(int fmt, int bs) {
    return fmt >= 0 && (bs == 32 || bs == 64 || bs == 128 || bs == 256);
}

size_t qk_plane_offset(int b, int j, int nb, int block_bytes, int bs) {
    if (bs <= 64) {
        const int k = block_bytes >> 4;
        return j < 16 * k ? (size_t)(j >> 4) * (size_t)nb * 16 + (size_t)b * 16 + (size_t)(j & 15)
                          : (size_t)k * (size_t)nb * 16 + (size_t)b * (size_t)(block_bytes & 15) +
                                (size_t)(j - 16 * k);
    }
    if (j < 4) return (size_t)b * 4 + (size_t)j;
    const int P = bs / 64, cwb = (block_bytes - 4) / P, k = cwb >> 4;
    const size_t np = (size_t)nb * P, u = (size_t)b * P + (size_t)((j - 4) / cwb);
    const int c = (j - 4) % cwb;
    return c < 16 * k ? (size_t)nb * 4 + (size_t)(c >> 4) * np * 16 + u * 16 + (size_t)(c & 15)
                      : (size_t)nb * 4 + (size_t)k * np * 16 + u * (size_t)(cwb & 15) + (size_t)(c - 16 * k);
}

/* The on-disk blocks [rows][nb][bb] into row-plane order (the layout
 * qk_plane_offset addresses). */
static void plane_permute(uint8_t* dst, const uint8_t* src, int rows, int nb, int bb, int bs) {
    const size_t rb = (size_t)nb * bb;
    if (bs <= 64) {
        const int k = bb / 16, tb = bb % 16;
        for (int r = 0; r < rows; r++) {
            const uint8_t* s = src + (size_t)r * rb;
            uint8_t* d = dst + (size_t)r * rb;
            for (int b = 0; b < nb; b++) {
                for (int i = 0; i < k; i++)
                    memcpy(d + (size_t)i * nb * 16 + (size_t)b * 16, s + (size_t)b * bb + 16 * i, 16);
                if (tb) memcpy(d + (size_t)k * nb * 16 + (size_t)b * tb, s + (size_t)b * bb + 16 * k, (size_t)tb);
            }
        }
        return;
    }
    /* part planes: the meta plane, then each 64-code part's code bytes in
     * 16-byte planes and a tail plane (whole runs per part) */
    const int P = bs / 64, cwb = (bb - 4) / P, k = cwb / 16, tb = cwb % 16;
    const size_t np = (size_t)nb * P;
    for (int r = 0; r < rows; r++) {
        const uint8_t* s = src + (size_t)r * rb;
        uint8_t* d = dst + (size_t)r * rb;
        for (int b = 0; b < nb; b++) {
            memcpy(d + (size_t)b * 4, s + (size_t)b * bb, 4);
            for (int p = 0; p < P; p++) {
                const uint8_t* cs = s + (size_t)b * bb + 4 + (size_t)p * cwb;
                const size_t u = (size_t)b * P + (size_t)p;
                for (int i = 0; i < k; i++) memcpy(d + (size_t)nb * 4 + (size_t)i * np * 16 + u * 16, cs + 16 * i, 16);
                if (tb) memcpy(d + (size_t)nb * 4 + (size_t)k * np * 16 + u * (size_t)tb, cs + 16 * k, (size_t)tb);
            }
        }
    }
}

static qsf_hip_tensor* upload_locked(const void* host, int qt, int rows, int cols, int bs) {
    if (init_locked(g_dev.ready ? g_dev.device : 0) != E_OK) return NULL;
    if (!host || rows < 0 || cols < 0) {
        fail(E_INVALID, "qsf_hip_tensor_upload: bad arguments");
        return NULL;
    }
    const int fmt = kernel_fmt(qt);
    if (fmt >= 0 && !(bs == 32 || bs == 64 || bs == 128 || bs == 256)) {
        fail(E_INVALID, "qsf_hip: block size %d not in {32,64,128,256}", bs);
        return NULL;
    }
    qsf_hip_tensor* t = calloc(1, sizeof *t);
    if (!t) { fail(E_OOM, "qsf_hip: tensor"); return NULL; }
    t->qt = qt; t->rows = rows; t->cols = cols; t->bs = fmt >= 0 ? bs : 32; t->fmt = fmt;
    t->host_key = host;
    const uint8_t* p = (const uint8_t*)host;
    size_t blocks_bytes, scales_bytes = 0;
    uint32_t n_out = 0;
    if (fmt < 0) {
        t->nb = (cols + 31) / 32;
        t->block_bytes = 16;
        blocks_bytes = (size_t)rows * t->nb * 16;
        scales_bytes = (size_t)rows * t->nb;
        t->payload_bytes = blocks_bytes + scales_bytes;
    } else {
        t->nb = (cols + bs - 1) / bs;
        t->block_bytes = 4 + (bs * fmt_bits(fmt) + 7) / 8;
        blocks_bytes = (size_t)rows * t->nb * t->block_bytes;
        t->payload_bytes = blocks_bytes;
        if (is_outlier(qt)) {
            n_out = rd_u32(p);
            t->payload_bytes += 4 + 6 * (size_t)n_out;
        }
    }
    t->n_outliers = n_out;
    /* device order of the blocks: fragment order where the matrix-core GEMV
     * is the engine for the format and covers the shape (engine 1 takes it
     * for the 3-bit formats, whose unpack is the costliest on the vector
     * units; 2 for every format), else row-plane order. */
    const int engine = qk_gemv_mfma_enable(-1);
    t->frag = fmt >= 0 && rows > 0 && (engine == 2 || (engine == 1 && fmt == QK_FMT_3)) &&
              qk_mfma_layout(fmt, bs, cols, is_outlier(qt));
    t->frag_nq = (t->nb + 3) / 4;
    t->plane = !t->frag && rows > 0 && qk_plane_layout(fmt, t->bs);
    const size_t dev_blocks_bytes = t->frag ? qk_frag_bytes(rows, t->nb, t->block_bytes) : blocks_bytes;

    /* CSR of the outlier table: stable counting sort by row keeps file order
     * within a row; entries with row >= rows are dropped (src/quant.c:432-434). */
    uint32_t* row_ptr = NULL;
    uint32_t* ocol = NULL;
    uint16_t* oval = NULL;
    uint32_t kept = 0;
    if (is_outlier(qt) && rows > 0 && cols > 0) {
        const uint8_t* ent = p + 4;
        row_ptr = calloc((size_t)rows + 1, sizeof *row_ptr);
        ocol = malloc(sizeof *ocol * (n_out ? n_out : 1));
        oval = malloc(sizeof *oval * (n_out ? n_out : 1));
        if (!row_ptr || !ocol || !oval) {
            free(row_ptr); free(ocol); free(oval); free(t);
            fail(E_OOM, "qsf_hip: outlier CSR");
            return NULL;
        }
        for (uint32_t i = 0; i < n_out; i++) {
            uint32_t flat = rd_u32(ent + 6 * (size_t)i);
            uint32_t r = flat / (uint32_t)cols;
            if (r < (uint32_t)rows) row_ptr[r + 1]++;
        }
        for (int r = 0; r < rows; r++) row_ptr[r + 1] += row_ptr[r];
        kept = row_ptr[rows];
        uint32_t* fill = malloc(sizeof *fill * ((size_t)rows + 1));
        if (!fill) {
            free(row_ptr); free(ocol); free(oval); free(t);
            fail(E_OOM, "qsf_hip: outlier CSR");
            return NULL;
        }
        memcpy(fill, row_ptr, sizeof *fill * ((size_t)rows + 1));
        for (uint32_t i = 0; i < n_out; i++) {
            const uint8_t* e = ent + 6 * (size_t)i;
            uint32_t flat = rd_u32(e);
            uint32_t r = flat / (uint32_t)cols;
            if (r >= (uint32_t)rows) continue;
            uint32_t at = fill[r]++;
            ocol[at] = flat % (uint32_t)cols;
            memcpy(&oval[at], e + 4, 2);
        }
        free(fill);
    }
    t->n_csr = kept;

    /* Entries are packed into one dword (col | fp16 << 16) when every column
     * fits 16 bits: one 4-byte load per entry instead of two loads. */
    const int packed = cols <= 65536;
    if (row_ptr && packed)
        for (uint32_t i = 0; i < kept; i++) ocol[i] |= (uint32_t)oval[i] << 16;

    /* one allocation: [blocks][scales][row_ptr][ocol][oval], 256-B aligned parts */
    size_t off_blocks = 0;
    size_t off_scales = align256(dev_blocks_bytes);
    size_t off_rp = off_scales + align256(scales_bytes);
    size_t rp_bytes = row_ptr ? ((size_t)rows + 1) * 4 : 0;
    size_t off_oc = off_rp + align256(rp_bytes);
    size_t off_ov = off_oc + align256((size_t)kept * 4);
    size_t total = off_ov + (packed ? 0 : align256((size_t)kept * 2));
    if (total == 0) total = 256;
    /* blocks are read with 16-byte vector loads that may reach 12 bytes past
     * the last block: keep a tail pad */
    total += 256;
    t->alloc_bytes = total - 256;    /* the parts, without the tail pad */
    hipError_t he = hipMalloc(&t->d_alloc, total);
    if (he != hipSuccess) {
        free(row_ptr); free(ocol); free(oval); free(t);
        fail(E_OOM, "qsf_hip: hipMalloc(%zu): %s", total, hipGetErrorString(he));
        return NULL;
    }
    uint8_t* base = (uint8_t*)t->d_alloc;
    t->d_blocks = base + off_blocks;
    const uint8_t* host_blocks = is_outlier(qt) ? p + 4 + 6 * (size_t)n_out : p;
    if (t->frag || t->plane) {
        uint8_t* fb = calloc(dev_blocks_bytes ? dev_blocks_bytes : 1, 1);
        if (!fb) {
            hipFree(t->d_alloc);
            free(row_ptr); free(ocol); free(oval); free(t);
            fail(E_OOM, "qsf_hip: %s staging (%zu bytes)", t->frag ? "fragment-order" : "row-plane",
                 dev_blocks_bytes);
            return NULL;
        }
        if (t->frag) frag_permute(fb, host_blocks, rows, t->nb, t->block_bytes);
        else plane_permute(fb, host_blocks, rows, t->nb, t->block_bytes, t->bs);
        he = hipMemcpy(t->d_blocks, fb, dev_blocks_bytes, hipMemcpyHostToDevice);
        free(fb);
    } else {
        he = hipMemcpy(t->d_blocks, host_blocks, blocks_bytes, hipMemcpyHostToDevice);
    }
    if (he == hipSuccess && scales_bytes) {
        t->d_scales = base + off_scales;
        he = hipMemcpy(t->d_scales, p + blocks_bytes, scales_bytes, hipMemcpyHostToDevice);
    }
    if (he == hipSuccess && row_ptr) {
        t->d_row_ptr = (uint32_t*)(base + off_rp);
        he = hipMemcpy(t->d_row_ptr, row_ptr, rp_bytes, hipMemcpyHostToDevice);
        if (packed) {
            t->d_oent = (uint32_t*)(base + off_oc);
            if (he == hipSuccess && kept)
                he = hipMemcpy(t->d_oent, ocol, (size_t)kept * 4, hipMemcpyHostToDevice);
        } else {
            t->d_ocol = (uint32_t*)(base + off_oc);
            t->d_oval = (uint16_t*)(base + off_ov);
            if (he == hipSuccess && kept)
                he = hipMemcpy(t->d_ocol, ocol, (size_t)kept * 4, hipMemcpyHostToDevice);
            if (he == hipSuccess && kept)
                he = hipMemcpy(t->d_oval, oval, (size_t)kept * 2, hipMemcpyHostToDevice);
        }
    }
    free(row_ptr); free(ocol); free(oval);
    if (he != hipSuccess) {
        hipFree(t->d_alloc);
        free(t);
        fail(E_INTERNAL, "qsf_hip: upload: %s", hipGetErrorString(he));
        return NULL;
    }
    g_dev.arena_bytes += t->payload_bytes;
    tensor_link(t);
    return t;
}

qsf_hip_tensor* qsf_hip_tensor_upload(const void* host, int qt, int rows, int cols, int bs) {
    pthread_mutex_lock(&g_lock);
    qsf_hip_tensor* t = upload_locked(host, qt, rows, cols, bs);
    if (t) {
        reg_drop(host);
        if (reg_put(host, t, fingerprint(host, t->payload_bytes), 0) != E_OK) {
            tensor_destroy(t);
            t = NULL;
        }
    }
    pthread_mutex_unlock(&g_lock);
    return t;
}

/* Gate and up weights of one FFN as one tensor of 2 * rows rows, block rows
 * interleaved (row 2i = gate row i, row 2i+1 = up row i), so that one
 * two-row GEMV tile holds both rows of an output.  Not registered: no host
 * pointer stands for it.  Plain block formats only (no outlier table). */
qsf_hip_tensor* qsf_hip_tensor_upload_pair(const void* gate, const void* up, int qt, int rows,
                                           int cols, int bs) {
    if (!gate || !up || rows <= 0 || cols <= 0 || kernel_fmt(qt) < 0 || is_outlier(qt) ||
        !(bs == 32 || bs == 64 || bs == 128 || bs == 256)) {
        fail(E_INVALID, "qsf_hip_tensor_upload_pair: bad arguments (type %d, %dx%d, block %d)", qt,
             rows, cols, bs);
        return NULL;
    }
    const size_t row_bytes = (size_t)((cols + bs - 1) / bs) * (4 + (bs * fmt_bits(kernel_fmt(qt)) + 7) / 8);
    uint8_t* both = malloc(2 * (size_t)rows * row_bytes);
    if (!both) {
        fail(E_OOM, "qsf_hip_tensor_upload_pair: host staging");
        return NULL;
    }
    for (int r = 0; r < rows; r++) {
        memcpy(both + (2 * (size_t)r) * row_bytes, (const uint8_t*)gate + (size_t)r * row_bytes, row_bytes);
        memcpy(both + (2 * (size_t)r + 1) * row_bytes, (const uint8_t*)up + (size_t)r * row_bytes, row_bytes);
    }
    pthread_mutex_lock(&g_lock);
    qsf_hip_tensor* t = upload_locked(both, qt, 2 * rows, cols, bs);
    if (t) t->host_key = NULL;
    pthread_mutex_unlock(&g_lock);
    free(both);
    return t;
}

qsf_hip_tensor* qsf_host_upload_owned(const void* host, int qt, int rows, int cols, int bs) {
    pthread_mutex_lock(&g_lock);
    qsf_hip_tensor* t = upload_locked(host, qt, rows, cols, bs);
    pthread_mutex_unlock(&g_lock);
    return t;
}

void* qsf_host_device_bytes(const void* host, size_t n) {
    pthread_mutex_lock(&g_lock);
    void* d = NULL;
    int rc = init_locked(g_dev.ready ? g_dev.device : 0);
    if (!rc && hipMalloc(&d, n ? n : 1) != hipSuccess) {
        fail(E_OOM, "qsf_hip: device buffer of %zu bytes", n);
        d = NULL;
    }
    if (d && n && hipMemcpy(d, host, n, hipMemcpyHostToDevice) != hipSuccess) {
        hipFree(d);
        d = NULL;
        fail(E_INTERNAL, "qsf_hip: device buffer upload");
    }
    pthread_mutex_unlock(&g_lock);
    return d;
}

float* qsf_host_device_floats(const float* host, size_t n) {
    return (float*)qsf_host_device_bytes(host, sizeof(float) * n);
}

void qsf_host_device_free(void* p) {
    if (p) hipFree(p);
}

float qsf_host_fp16(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
    if (e == 31u) {
        u = sign | 0x7F800000u | (m << 13);
    } else if (e == 0u) {
        if (m == 0u) {
            u = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            u = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

qsf_hip_tensor* qsf_hip_tensor_lookup(const void* host) {
    pthread_mutex_lock(&g_lock);
    reg_slot* s = reg_find(host);
    qsf_hip_tensor* t = s ? s->t : NULL;
    pthread_mutex_unlock(&g_lock);
    return t;
}

void qsf_hip_tensor_free(qsf_hip_tensor* t) {
    if (!t) return;
    pthread_mutex_lock(&g_lock);
    reg_slot* s = reg_find(t->host_key);
    if (s && s->t == t) reg_del(t->host_key);
    tensor_destroy(t);
    pthread_mutex_unlock(&g_lock);
}

int qsf_hip_arena_forget(const void* host) {
    pthread_mutex_lock(&g_lock);
    int found = reg_find(host) != NULL;
    reg_drop(host);
    pthread_mutex_unlock(&g_lock);
    return found ? E_OK : E_INVALID;
}

int qsf_hip_arena_forget_range(const void* base, size_t bytes) {
    const uintptr_t lo = (uintptr_t)base, hi = lo + bytes;
    int n = 0;
    pthread_mutex_lock(&g_lock);
    /* collect first: reg_drop moves entries of a probe run */
    const void** keys = g_reg_n ? malloc(g_reg_n * sizeof *keys) : NULL;
    if (g_reg_n && !keys) {
        pthread_mutex_unlock(&g_lock);
        return -fail(E_OOM, "qsf_hip_arena_forget_range");
    }
    for (size_t i = 0; i < g_reg_cap; i++)
        if (g_reg[i].key && (uintptr_t)g_reg[i].key >= lo && (uintptr_t)g_reg[i].key < hi)
            keys[n++] = g_reg[i].key;
    for (int i = 0; i < n; i++) reg_drop(keys[i]);
    free(keys);
    pthread_mutex_unlock(&g_lock);
    return n;
}

size_t qsf_hip_arena_bytes(void) { return g_dev.arena_bytes; }
size_t qsf_hip_tensor_payload_bytes(const qsf_hip_tensor* t) { return t ? t->payload_bytes : 0; }

void qsf_hip_shutdown(void) {
    pthread_mutex_lock(&g_lock);
    while (g_live) tensor_destroy(g_live);
    free(g_reg);
    g_reg = NULL;
    g_reg_cap = g_reg_n = 0;
    g_reg_gen++;
    memset(&g_ahead, 0, sizeof g_ahead);
    if (g_dev.ready) {
        hipStreamSynchronize(g_dev.stream);
        if (g_dev.ws) hipFree(g_dev.ws);
        if (g_dev.att_ws) hipFree(g_dev.att_ws);
        if (g_dev.d_x) hipFree(g_dev.d_x);
        if (g_dev.slot_xq) hipFree(g_dev.slot_xq);
        if (g_dev.h_x) hipHostFree(g_dev.h_x);
        if (g_dev.h_y) hipHostFree(g_dev.h_y);
        if (g_dev.h_flag) hipHostFree(g_dev.h_flag);
        for (size_t i = 0; i < g_retired_n; i++) hipFree(g_retired[i]);
        hipStreamDestroy(g_dev.stream);
    }
    free(g_retired);
    g_retired = NULL;
    g_retired_n = g_retired_cap = 0;
    memset(&g_dev, 0, sizeof g_dev);
    pthread_mutex_unlock(&g_lock);
}

/* ---- device-pointer entry points ----------------------------------------- */
/* Device-pointer entry points run on the caller's stream; NULL is the HIP
 * default (null) stream, as everywhere in HIP.  Only the synchronous table
 * slots use the library's own stream. */
static hipStream_t pick_stream(void* s) { return (hipStream_t)s; }

static int group_locked(const qsf_hip_tensor* const* t, int n, const float* d_x,
                        float* const* d_y, void* stream) {
    if (n <= 0 || n > QK_MAX_GROUP || !t) return fail(E_INVALID, "qsf_hip: group of %d", n);
    for (int i = 0; i < n; i++) {
        if (!t[i] || !d_y || !d_y[i]) return fail(E_INVALID, "qsf_hip: null tensor/output");
        if (t[i]->fmt < 0) return fail(E_INVALID, "qsf_hip: MXFP4 tensor in the dense path");
        if (t[i]->fmt != t[0]->fmt || t[i]->bs != t[0]->bs || t[i]->cols != t[0]->cols)
            return fail(E_INVALID, "qsf_hip: grouped tensors differ in type/cols/block");
    }
    if (t[0]->cols > 0 && !d_x) return fail(E_INVALID, "qsf_hip: null input");
    /* the one-launch form prepares x inside the GEMV workgroups: no
     * workspace, so nothing is allocated on this path */
    int rc = qk_gemv_group(t, n, d_x, d_y, NULL, QK_RUN_BOTH, pick_stream(stream));
    if (rc) return fail(E_INTERNAL, "qsf_hip: GEMV launch failed (%d)", rc);
    return E_OK;
}

size_t qsf_hip_xprep_bytes(int qt, int bs, int cols) {
    int fmt = kernel_fmt(qt);
    return fmt < 0 || cols <= 0 ? 0 : qk_xprep_bytes(fmt, bs, cols);
}

int qsf_hip_xprep_dev(int qt, int bs, int cols, const float* d_x, void* d_xq, void* stream) {
    int fmt = kernel_fmt(qt);
    if (fmt < 0 || !(bs == 32 || bs == 64 || bs == 128 || bs == 256) || cols < 0 ||
        (cols > 0 && (!d_x || !d_xq)) || ((uintptr_t)d_xq & 255))
        return fail(E_INVALID, "qsf_hip_xprep_dev: bad arguments");
    if (!g_dev.ready) return fail(E_INVALID, "qsf_hip: not initialised");
    if (qk_xprep(fmt, bs, cols, d_x, d_xq, pick_stream(stream)))
        return fail(E_INTERNAL, "qsf_hip_xprep_dev: launch failed");
    return E_OK;
}

int qsf_hip_matvec_group_prepared_dev(const qsf_hip_tensor* const* t, int n, const float* d_x,
                                      const void* d_xq, float* const* d_y, void* stream) {
    if (n <= 0 || n > QK_MAX_GROUP || !t || !d_y)
        return fail(E_INVALID, "qsf_hip: group of %d", n);
    for (int i = 0; i < n; i++) {
        if (!t[i] || !d_y[i] || t[i]->fmt < 0 || t[i]->fmt != t[0]->fmt ||
            t[i]->bs != t[0]->bs || t[i]->cols != t[0]->cols)
            return fail(E_INVALID, "qsf_hip: grouped tensors differ in type/cols/block");
    }
    if (t[0]->cols > 0 && (!d_x || !d_xq || ((uintptr_t)d_xq & 255)))
        return fail(E_INVALID, "qsf_hip: prepared input missing or misaligned");
    if (!g_dev.ready) return fail(E_INVALID, "qsf_hip: not initialised");
    if (qk_gemv_group(t, n, d_x, d_y, (void*)d_xq, QK_RUN_GEMV, pick_stream(stream)))
        return fail(E_INTERNAL, "qsf_hip: GEMV launch failed");
    return E_OK;
}

int qsf_hip_matvec_group_dev(const qsf_hip_tensor* const* t, int n, const float* d_x,
                             float* const* d_y, void* stream) {
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? group_locked(t, n, d_x, d_y, stream)
                         : fail(E_INVALID, "qsf_hip: not initialised");
    pthread_mutex_unlock(&g_lock);
    return rc;
}

static int mxfp4_locked(const qsf_hip_tensor* t, const float* d_x, float* d_y, void* stream) {
    int rc = qk_mxfp4_gemv(t, d_x, 1, d_y, pick_stream(stream));
    return rc ? fail(E_INTERNAL, "qsf_hip: MXFP4 launch failed (%d)", rc) : E_OK;
}

int qsf_hip_matvec_dev(const qsf_hip_tensor* t, const float* d_x, float* d_y, void* stream) {
    if (!t) return fail(E_INVALID, "qsf_hip: null tensor");
    pthread_mutex_lock(&g_lock);
    int rc;
    if (!g_dev.ready) rc = fail(E_INVALID, "qsf_hip: not initialised");
    else if (t->rows <= 0) rc = E_OK;
    else if (t->fmt < 0) rc = mxfp4_locked(t, d_x, d_y, stream);
    else rc = group_locked(&t, 1, d_x, &d_y, stream);
    pthread_mutex_unlock(&g_lock);
    return rc;
}

_Static_assert(QSF_HIP_PREFILL_SCRATCH_BYTES == QK_PREFILL_SCRATCH_BYTES,
               "public and kernel-side scratch sizes differ");

static int prefill_check(const char* who, const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m) {
    if (!t) return fail(E_INVALID, "%s: null tensor", who);
    if (t->fmt != QK_FMT_4 || t->n_outliers || !(t->bs == 64 || t->bs == 128 || t->bs == 256))
        return fail(E_INVALID, "%s: needs a 4-bit asymmetric tensor with "
                               "block 64, 128 or 256 and no outliers", who);
    if (m < 0 || t->cols < 32 || t->cols % 8 != 0 || ((uintptr_t)d_x_bf16 & 15u) != 0 ||
        (m > 0 && !d_x_bf16 && !strstr(who, "packed")))
        return fail(E_INVALID, "%s: m >= 0, cols >= 32, cols %% 8 == 0 "
                               "and a 16-byte aligned x are required", who);
    return E_OK;
}

int qsf_hip_prefill_4bit_dev(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                             float* d_y, void* stream) {
    if (prefill_check("qsf_hip_prefill_4bit_dev", t, d_x_bf16, m)) return g_err;
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? E_OK : fail(E_INVALID, "qsf_hip: not initialised");
    if (rc == E_OK) rc = ensure_dev(&g_dev.ws, &g_dev.ws_bytes, qk_prefill_ws_bytes(m, t->cols, t->bs));
    if (rc == E_OK && qk_prefill_4bit(t, d_x_bf16, m, d_y, g_dev.ws, pick_stream(stream)))
        rc = fail(E_INTERNAL, "qsf_hip_prefill_4bit_dev: launch failed");
    pthread_mutex_unlock(&g_lock);
    return rc;
}

int qsf_hip_prefill_4bit_dev_noalloc(const qsf_hip_tensor* t, const uint16_t* d_x_bf16, int m,
                                     float* d_y, void* stream) {
    if (prefill_check("qsf_hip_prefill_4bit_dev_noalloc", t, d_x_bf16, m)) return g_err;
    const size_t need = qk_prefill_ws_bytes(m, t->cols, t->bs);
    if (need > (size_t)QSF_HIP_PREFILL_SCRATCH_BYTES)
        return fail(E_INVALID, "qsf_hip_prefill_4bit_dev_noalloc: %d tokens x %d columns need "
                               "%zu bytes of scratch, more than its %d (use "
                               "qsf_hip_prefill_4bit_dev, or split the tokens)",
                    m, t->cols, need, QSF_HIP_PREFILL_SCRATCH_BYTES);
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? E_OK : fail(E_INVALID, "qsf_hip: not initialised");
    if (rc == E_OK) {
        int r = qk_prefill_4bit_noalloc(t, d_x_bf16, m, d_y, pick_stream(stream));
        if (r) rc = fail(E_INTERNAL, "qsf_hip_prefill_4bit_dev_noalloc: %s",
                         r == -1 ? "no address for this device's scratch array" : "launch failed");
    }
    pthread_mutex_unlock(&g_lock);
    return rc;
}

size_t qsf_hip_prefill_pack_bytes(int m, int cols, int bs) { return qk_prefill_ws_bytes(m, cols, bs); }

int qsf_hip_prefill_pack_dev(const uint16_t* d_x_bf16, int m, int cols, int bs, void* d_packed,
                             void* stream) {
    if (m < 0 || cols < 32 || cols % 8 != 0 || !(bs == 64 || bs == 128 || bs == 256) ||
        ((uintptr_t)d_x_bf16 & 15u) != 0 || ((uintptr_t)d_packed & 15u) != 0 || (m > 0 && !d_packed))
        return fail(E_INVALID, "qsf_hip_prefill_pack_dev: m >= 0, cols >= 32, cols %% 8 == 0, block "
                               "64/128/256 and 16-byte aligned x and packed buffer are required");
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? E_OK : fail(E_INVALID, "qsf_hip: not initialised");
    if (rc == E_OK && qk_prefill_pack(d_x_bf16, m, cols, bs, d_packed, pick_stream(stream)))
        rc = fail(E_INTERNAL, "qsf_hip_prefill_pack_dev: %d tokens x %d columns: launch failed", m, cols);
    pthread_mutex_unlock(&g_lock);
    return rc;
}

int qsf_hip_prefill_4bit_packed_dev(const qsf_hip_tensor* t, const void* d_packed, int m, float* d_y,
                                    void* stream) {
    if (prefill_check("qsf_hip_prefill_4bit_packed_dev", t, NULL, m)) return g_err;
    if (((uintptr_t)d_packed & 15u) != 0 || (m > 0 && !d_packed))
        return fail(E_INVALID, "qsf_hip_prefill_4bit_packed_dev: a 16-byte aligned packed buffer is required");
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? E_OK : fail(E_INVALID, "qsf_hip: not initialised");
    if (rc == E_OK && qk_prefill_gemm(t, d_packed, m, d_y, pick_stream(stream)))
        rc = fail(E_INTERNAL, "qsf_hip_prefill_4bit_packed_dev: launch failed");
    pthread_mutex_unlock(&g_lock);
    return rc;
}

int qsf_hip_stream_read_dev(const qsf_hip_tensor* const* t, int n, uint32_t* d_sink, void* stream) {
    if (!t || n <= 0 || n > QK_MAX_GROUP || !d_sink)
        return fail(E_INVALID, "qsf_hip_stream_read_dev: 1..%d tensors and a sink are required", QK_MAX_GROUP);
    const void* ptr[QK_MAX_GROUP];
    size_t bytes[QK_MAX_GROUP];
    for (int i = 0; i < n; i++) {
        if (!t[i]) return fail(E_INVALID, "qsf_hip_stream_read_dev: null tensor %d", i);
        ptr[i] = t[i]->d_alloc;
        bytes[i] = t[i]->alloc_bytes;
    }
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? E_OK : fail(E_INVALID, "qsf_hip: not initialised");
    if (rc == E_OK && qk_stream_read(ptr, bytes, n, d_sink, pick_stream(stream)))
        rc = fail(E_INTERNAL, "qsf_hip_stream_read_dev: launch failed");
    pthread_mutex_unlock(&g_lock);
    return rc;
}

double qsf_hip_mfma_peak_dev(int iters, uint32_t* d_sink, void* stream) {
    if (iters <= 0 || !d_sink) {
        fail(E_INVALID, "qsf_hip_mfma_peak_dev: iters > 0 and a sink are required");
        return -1.0;
    }
    pthread_mutex_lock(&g_lock);
    double flop = -1.0;
    if (!g_dev.ready) fail(E_INVALID, "qsf_hip: not initialised");
    else if ((flop = qk_mfma_peak(iters, d_sink, pick_stream(stream))) < 0)
        fail(E_INTERNAL, "qsf_hip_mfma_peak_dev: launch failed");
    pthread_mutex_unlock(&g_lock);
    return flop;
}

int qsf_hip_unpack_dev(int qt, const void* d_blocks, int nblocks, int bs, int8_t* d_codes,
                       uint32_t* d_meta, float* d_deq, void* stream) {
    if (kernel_fmt(qt) < 0 || !(bs == 32 || bs == 64 || bs == 128 || bs == 256))
        return fail(E_INVALID, "qsf_hip_unpack_dev: type %d block %d", qt, bs);
    pthread_mutex_lock(&g_lock);
    int rc = init_locked(0);
    if (!rc && qk_unpack(qt, d_blocks, nblocks, bs, d_codes, d_meta, d_deq, pick_stream(stream)))
        rc = fail(E_INTERNAL, "qsf_hip_unpack_dev: launch failed");
    pthread_mutex_unlock(&g_lock);
    return rc;
}

int qsf_hip_kernel_timing(int enable) {
    pthread_mutex_lock(&g_lock);
    int rc = qk_timing(enable);
    pthread_mutex_unlock(&g_lock);
    return rc ? fail(E_INTERNAL, "qsf_hip_kernel_timing") : E_OK;
}

int qsf_hip_kernel_timing_read(float* us, int max) {
    if (!us || max < 0) return -fail(E_INVALID, "qsf_hip_kernel_timing_read: bad buffer");
    pthread_mutex_lock(&g_lock);
    int n = qk_timing_read(us, max);
    pthread_mutex_unlock(&g_lock);
    return n < 0 ? -fail(E_INTERNAL, "qsf_hip_kernel_timing_read: event query failed") : n;
}

/* ---- device-resident decode glue (src/engine.c:709-1187) ------------------ */
static int glue_rc(const char* who, int r) {
    if (r == 0) return E_OK;
    return fail(r == -2 ? E_INVALID : E_INTERNAL, "%s: %s", who,
                r == -2 ? "unsupported shape" : "launch failed");
}

int qsf_hip_rms_norm_dev(const float* d_in, float* d_out, const float* d_w, int dim, float eps,
                         void* stream) {
    if (dim < 0 || (dim > 0 && (!d_in || !d_out || !d_w)))
        return fail(E_INVALID, "qsf_hip_rms_norm_dev: bad arguments");
    return glue_rc("qsf_hip_rms_norm_dev", qk_norm(d_in, d_out, d_w, NULL, dim, eps, 0, pick_stream(stream)));
}

int qsf_hip_layer_norm_dev(const float* d_in, float* d_out, const float* d_w, const float* d_b,
                           int dim, float eps, void* stream) {
    if (dim < 0 || (dim > 0 && (!d_in || !d_out || !d_w)))
        return fail(E_INVALID, "qsf_hip_layer_norm_dev: bad arguments");
    return glue_rc("qsf_hip_layer_norm_dev", qk_norm(d_in, d_out, d_w, d_b, dim, eps, 1, pick_stream(stream)));
}

struct qsf_hip_rope {
    int head_dim;
    float* d_freq;     /* head_dim/2 frequencies */
};

qsf_hip_rope* qsf_hip_rope_create(int head_dim, float theta) {
    if (head_dim <= 0 || head_dim % 2) {
        fail(E_INVALID, "qsf_hip_rope_create: head_dim %d must be even and positive", head_dim);
        return NULL;
    }
    if (theta <= 0) theta = 10000.0f;          /* src/engine.c:873 */
    int n = head_dim / 2;
    float* f = malloc(sizeof(float) * (size_t)n);
    qsf_hip_rope* r = calloc(1, sizeof *r);
    if (!f || !r) {
        free(f); free(r);
        fail(E_OOM, "qsf_hip_rope_create");
        return NULL;
    }
    /* the reference's frequency, by the host C library (src/engine.c:210) */
    for (int j = 0; j < n; j++) f[j] = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
    r->head_dim = head_dim;
    if (hipMalloc((void**)&r->d_freq, sizeof(float) * (size_t)n) != hipSuccess ||
        hipMemcpy(r->d_freq, f, sizeof(float) * (size_t)n, hipMemcpyHostToDevice) != hipSuccess) {
        if (r->d_freq) hipFree(r->d_freq);
        free(f); free(r);
        fail(E_OOM, "qsf_hip_rope_create: device table");
        return NULL;
    }
    free(f);
    return r;
}

void qsf_hip_rope_free(qsf_hip_rope* r) {
    if (!r) return;
    hipFree(r->d_freq);
    free(r);
}

int qsf_hip_rope_dev(const qsf_hip_rope* r, float* d_q, float* d_k, int n_heads, int n_kv_heads,
                     int position, void* stream) {
    if (!r || n_heads < 0 || n_kv_heads < 0 || position < 0 ||
        (n_heads > 0 && !d_q) || (n_kv_heads > 0 && !d_k))
        return fail(E_INVALID, "qsf_hip_rope_dev: bad arguments");
    return glue_rc("qsf_hip_rope_dev", qk_rope(d_q, d_k, r->d_freq, r->head_dim, n_heads, n_kv_heads,
                                               position, pick_stream(stream)));
}

int qsf_hip_kv_store_dev(int8_t* d_kc, int8_t* d_vc, float* d_ks, float* d_vs, int max_seq,
                         int n_kv_heads, int head_dim, int position, const float* d_k,
                         const float* d_v, void* stream) {
    if (!d_kc || !d_vc || !d_ks || !d_vs || !d_k || !d_v || n_kv_heads < 0 || head_dim <= 0 ||
        position < 0 || position >= max_seq)
        return fail(E_INVALID, "qsf_hip_kv_store_dev: bad arguments (position %d of %d)",
                    position, max_seq);
    return glue_rc("qsf_hip_kv_store_dev", qk_kv_store(d_kc, d_vc, d_ks, d_vs, max_seq, n_kv_heads,
                                                       head_dim, position, d_k, d_v,
                                                       pick_stream(stream)));
}

int qsf_hip_attention_dev(const float* d_q, const int8_t* d_kc, const int8_t* d_vc,
                          const float* d_ks, const float* d_vs, int max_seq, int n_heads,
                          int n_kv_heads, int head_dim, int position, float* d_out,
                          void* stream) {
    if (!d_q || !d_kc || !d_vc || !d_ks || !d_vs || !d_out || n_heads <= 0 || n_kv_heads <= 0 ||
        head_dim <= 0 || position < 0 || position >= max_seq)
        return fail(E_INVALID, "qsf_hip_attention_dev: bad arguments");
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? E_OK : fail(E_INVALID, "qsf_hip: not initialised");
    if (rc == E_OK)
        rc = ensure_dev(&g_dev.att_ws, &g_dev.att_ws_bytes,
                        qk_attention_ws_bytes(n_heads, head_dim, position));
    if (rc == E_OK)
        rc = glue_rc("qsf_hip_attention_dev",
                     qk_attention(d_q, d_kc, d_vc, d_ks, d_vs, max_seq, n_heads, n_kv_heads, head_dim,
                                  position, d_out, g_dev.att_ws, pick_stream(stream)));
    pthread_mutex_unlock(&g_lock);
    return rc;
}

int qsf_hip_act_mul_dev(float* d_gate, const float* d_up, int n, int activation, void* stream) {
    if (n < 0 || (n > 0 && (!d_gate || !d_up)))
        return fail(E_INVALID, "qsf_hip_act_mul_dev: bad arguments");
    return glue_rc("qsf_hip_act_mul_dev", qk_act_mul(d_gate, d_up, n, activation, pick_stream(stream)));
}

int qsf_hip_gate_up_act_dev(const qsf_hip_tensor* pair, const float* d_x, float* d_out, int activation,
                            void* stream) {
    if (!pair || !d_x || !d_out || pair->rows % 2 || activation < 0)
        return fail(E_INVALID, "qsf_hip_gate_up_act_dev: bad arguments");
    const int rc = qk_gemv_pair_act(pair, d_x, d_out, activation, pick_stream(stream));
    if (rc == -2) return fail(E_INVALID, "qsf_hip_gate_up_act_dev: no two-row plan for this tensor");
    return rc ? fail(E_INTERNAL, "qsf_hip_gate_up_act_dev: launch failed") : E_OK;
}

static int norm_rc(const char* fn, int rc) {
    if (rc == -2)
        return fail(E_INVALID, "%s: no fused plan (outliers, cols > 8192, no rows, or aliased buffers)", fn);
    return rc ? fail(E_INTERNAL, "%s: launch failed", fn) : E_OK;
}

int qsf_hip_residual_norm_matvec_group_dev(const qsf_hip_tensor* const* t, int n, const float* d_res,
                                           float* d_res_out, const float* d_x, int* d_bad,
                                           const float* d_w, float eps, float* const* d_y, void* stream) {
    static const char fn[] = "qsf_hip_residual_norm_matvec_group_dev";
    if (!t || n <= 0 || n > QK_MAX_GROUP || !d_res || !d_res_out || !d_x || !d_w || !d_y)
        return fail(E_INVALID, "%s: bad arguments", fn);
    for (int i = 0; i < n; i++)
        if (!t[i] || t[i]->fmt < 0 || !d_y[i]) return fail(E_INVALID, "%s: blockwise QSF tensors only", fn);
    const qk_norm_args nm = {d_res, d_res_out, d_w, d_bad, eps};
    return norm_rc(fn, qk_gemv_group_norm(t, n, &nm, d_x, d_y, pick_stream(stream)));
}

int qsf_hip_residual_norm_gate_up_act_dev(const qsf_hip_tensor* pair, const float* d_res, float* d_res_out,
                                          const float* d_x, int* d_bad, const float* d_w, float eps,
                                          float* d_out, int activation, void* stream) {
    static const char fn[] = "qsf_hip_residual_norm_gate_up_act_dev";
    if (!pair || pair->fmt < 0 || pair->rows % 2 || activation < 0 || !d_res || !d_res_out || !d_x || !d_w ||
        !d_out)
        return fail(E_INVALID, "%s: bad arguments", fn);
    const qk_norm_args nm = {d_res, d_res_out, d_w, d_bad, eps};
    return norm_rc(fn, qk_gemv_pair_act_norm(pair, &nm, d_x, d_out, activation, pick_stream(stream)));
}

int qsf_hip_residual_dev(float* d_res, const float* d_x, int n, int* d_bad, void* stream) {
    if (n < 0 || (n > 0 && (!d_res || !d_x)))
        return fail(E_INVALID, "qsf_hip_residual_dev: bad arguments");
    return glue_rc("qsf_hip_residual_dev", qk_residual(d_res, d_x, n, d_bad, pick_stream(stream)));
}

int qsf_hip_residual_norm_dev(float* d_res, const float* d_x, int n, int* d_bad, const float* d_w,
                              const float* d_b, float eps, int layer_norm, float* d_out, void* stream) {
    if (n < 0 || (n > 0 && (!d_res || !d_x || !d_w || !d_out)))
        return fail(E_INVALID, "qsf_hip_residual_norm_dev: bad arguments");
    return glue_rc("qsf_hip_residual_norm_dev",
                   qk_residual_norm(d_res, d_x, n, d_bad, d_w, layer_norm ? d_b : NULL, eps, layer_norm != 0,
                                    d_out, pick_stream(stream)));
}

int qsf_hip_rope_kv_store_dev(const qsf_hip_rope* r, float* d_q, float* d_k, const float* d_v,
                              int n_heads, int n_kv_heads, int position, int8_t* d_kc, int8_t* d_vc,
                              float* d_ks, float* d_vs, int max_seq, void* stream) {
    if (!r || n_heads < 0 || n_kv_heads <= 0 || (n_heads > 0 && !d_q) || !d_k || !d_v || !d_kc ||
        !d_vc || !d_ks || !d_vs || position < 0 || position >= max_seq || r->head_dim > 256)
        return fail(E_INVALID, "qsf_hip_rope_kv_store_dev: bad arguments (position %d of %d)", position,
                    max_seq);
    return glue_rc("qsf_hip_rope_kv_store_dev",
                   qk_rope_kv_store(d_q, d_k, d_v, r->d_freq, r->head_dim, n_heads, n_kv_heads, position,
                                    d_kc, d_vc, d_ks, d_vs, max_seq, pick_stream(stream)));
}

int qsf_hip_rope_kv_attention_dev(const qsf_hip_rope* r, float* d_q, float* d_k, const float* d_v,
                                  int n_heads, int n_kv_heads, int position, int8_t* d_kc, int8_t* d_vc,
                                  float* d_ks, float* d_vs, int max_seq, float* d_out, void* stream) {
    static const char fn[] = "qsf_hip_rope_kv_attention_dev";
    if (!r || n_heads <= 0 || n_kv_heads <= 0 || !d_q || !d_k || !d_v || !d_kc || !d_vc || !d_ks || !d_vs ||
        !d_out || position < 0 || position >= max_seq)
        return fail(E_INVALID, "%s: bad arguments (position %d of %d)", fn, position, max_seq);
    pthread_mutex_lock(&g_lock);
    int rc = g_dev.ready ? E_OK : fail(E_INVALID, "qsf_hip: not initialised");
    if (rc == E_OK)
        rc = ensure_dev(&g_dev.att_ws, &g_dev.att_ws_bytes,
                        qk_attention_ws_bytes(n_heads, r->head_dim, position));
    if (rc == E_OK)
        rc = glue_rc(fn, qk_rope_kv_attention(d_q, d_k, d_v, r->d_freq, r->head_dim, n_heads, n_kv_heads,
                                              position, d_kc, d_vc, d_ks, d_vs, max_seq, d_out, g_dev.att_ws,
                                              pick_stream(stream)));
    pthread_mutex_unlock(&g_lock);
    return rc;
}

int qsf_hip_embed_row_dev(const qsf_hip_tensor* t, int token, float* d_out, void* stream) {
    if (!t || !d_out || token < 0 || token >= t->rows)
        return fail(E_INVALID, "qsf_hip_embed_row_dev: bad arguments (token %d)", token);
    /* the engine's lookup reads rows of qsf_quant_block_size(type) blocks
     * and dequantises types 0, 2, 3 and 4 (src/engine.c:718-753,
     * src/quant.c:68-85); for every other blockwise type its row size is 0
     * or its dequantiser reads 4-bit blocks over 2-bit ones */
    if (t->qt != QK_Q2 && t->qt != QK_Q3 && t->qt != QK_Q4 && t->qt != QK_Q4SYM)
        return fail(E_INVALID, "qsf_hip_embed_row_dev: quant type %d has no embedding lookup in the "
                               "engine (types 0, 2, 3, 4; FP16 tables take qsf_hip_embed_row_fp16_dev)", t->qt);
    return glue_rc("qsf_hip_embed_row_dev", qk_embed_row(t, token, d_out, pick_stream(stream)));
}

int qsf_hip_embed_row_fp16_dev(const uint16_t* d_table, int hd, int token, float* d_out,
                               void* stream) {
    if (!d_table || !d_out || hd < 0 || token < 0)
        return fail(E_INVALID, "qsf_hip_embed_row_fp16_dev: bad arguments");
    return glue_rc("qsf_hip_embed_row_fp16_dev",
                   qk_embed_row_fp16(d_table, hd, token, d_out, pick_stream(stream)));
}

/* ---- MoE ------------------------------------------------------------------- */
struct qsf_hip_moe {
    int n_exp, hidden, eid;
    qk_mx_expert* d_table;   /* device expert table */
    void* d_alloc;           /* table + biases */
    void* d_ws;
    size_t ws_bytes;
};

qsf_hip_moe* qsf_hip_moe_create(int n_exp, int hidden, int eid,
                                const qsf_hip_tensor* const* gate, const qsf_hip_tensor* const* up,
                                const qsf_hip_tensor* const* down, const uint16_t* const* gb,
                                const uint16_t* const* ub, const uint16_t* const* db) {
    if (n_exp < 1 || n_exp > 256 || hidden < 4 || eid < 4 || (hidden % 4) || (eid % 4) ||
        !gate || !up || !down) {
        fail(E_INVALID, "qsf_hip_moe_create: bad arguments");
        return NULL;
    }
    for (int e = 0; e < n_exp; e++) {
        const qsf_hip_tensor* t[3] = {gate[e], up[e], down[e]};
        for (int i = 0; i < 3; i++) {
            int r = i < 2 ? eid : hidden, c = i < 2 ? hidden : eid;
            if (!t[i] || t[i]->fmt >= 0 || t[i]->rows != r || t[i]->cols != c) {
                fail(E_INVALID, "qsf_hip_moe_create: expert %d tensor %d is not MXFP4 [%d][%d]",
                     e, i, r, c);
                return NULL;
            }
        }
    }
    pthread_mutex_lock(&g_lock);
    qsf_hip_moe* m = calloc(1, sizeof *m);
    qk_mx_expert* host = calloc((size_t)n_exp, sizeof *host);
    size_t table = align256(sizeof(qk_mx_expert) * (size_t)n_exp);
    size_t hb = align256((size_t)hidden * 2), eb = align256((size_t)eid * 2);
    size_t total = table + (size_t)n_exp * (2 * eb + hb);
    if (!m || !host || hipMalloc(&m->d_alloc, total) != hipSuccess) {
        free(m); free(host);
        fail(E_OOM, "qsf_hip_moe_create: allocation");
        pthread_mutex_unlock(&g_lock);
        return NULL;
    }
    uint8_t* base = (uint8_t*)m->d_alloc;
    m->d_table = (qk_mx_expert*)base;
    uint8_t* bias = base + table;
    int rc = 0;
    for (int e = 0; e < n_exp && !rc; e++, bias += 2 * eb + hb) {
        host[e].gc = gate[e]->d_blocks; host[e].gs = gate[e]->d_scales;
        host[e].uc = up[e]->d_blocks;   host[e].us = up[e]->d_scales;
        host[e].dc = down[e]->d_blocks; host[e].ds = down[e]->d_scales;
        const uint16_t* src[3] = {gb ? gb[e] : NULL, ub ? ub[e] : NULL, db ? db[e] : NULL};
        uint8_t* dst[3] = {bias, bias + eb, bias + 2 * eb};
        size_t n[3] = {(size_t)eid * 2, (size_t)eid * 2, (size_t)hidden * 2};
        const uint16_t** slot[3] = {&host[e].gb, &host[e].ub, &host[e].db};
        for (int i = 0; i < 3; i++) {
            *slot[i] = NULL;
            if (!src[i]) continue;
            if (hipMemcpy(dst[i], src[i], n[i], hipMemcpyHostToDevice) != hipSuccess) rc = 1;
            *slot[i] = (const uint16_t*)dst[i];
        }
    }
    if (!rc && hipMemcpy(m->d_table, host, sizeof(qk_mx_expert) * (size_t)n_exp,
                         hipMemcpyHostToDevice) != hipSuccess)
        rc = 1;
    free(host);
    m->n_exp = n_exp; m->hidden = hidden; m->eid = eid;
    m->ws_bytes = qk_moe_ws_bytes(n_exp, 8, 8, hidden, eid);
    if (!rc && hipMalloc(&m->d_ws, m->ws_bytes) != hipSuccess) rc = 1;

    if (rc) {
        if (m->d_ws) hipFree(m->d_ws);
        hipFree(m->d_alloc);
        free(m);
        fail(E_INTERNAL, "qsf_hip_moe_create: upload failed");
        m = NULL;
    }
    pthread_mutex_unlock(&g_lock);
    return m;
}

void qsf_hip_moe_free(qsf_hip_moe* m) {
    if (!m) return;
    hipFree(m->d_ws);
    hipFree(m->d_alloc);
    free(m);
}

/* Tokens go through in chunks of at most 8 (the kernels' batch), one after
 * another on `stream`, which orders their use of the object's workspace;
 * each token's result does not depend on the others in its chunk. */
static int g_moe_stages = 7;

int qsf_hip_moe_stages(int mask) {
    pthread_mutex_lock(&g_lock);
    const int prev = g_moe_stages;
    if (mask >= 0) g_moe_stages = mask & 7;
    pthread_mutex_unlock(&g_lock);
    return prev;
}

int qsf_hip_moe_forward_dev(qsf_hip_moe* m, int k, int norm, int act, int ntok,
                            const float* d_x, const float* d_logits, float* d_out, void* stream) {
    if (!m || ntok < 1 || k < 1 || k > 8 || !d_x || !d_logits || !d_out)
        return fail(E_INVALID, "qsf_hip_moe_forward_dev: bad arguments (ntok %d, k %d)", ntok, k);
    const int stages = qsf_hip_moe_stages(-1);
    if (stages != 7 && ntok > 8)
        return fail(E_INVALID, "qsf_hip_moe_forward_dev: stages 0x%x need ntok <= 8 (one launch group)", stages);
    for (int t0 = 0; t0 < ntok; t0 += 8) {
        const int nt = ntok - t0 < 8 ? ntok - t0 : 8;
        if (qk_moe_launch(m->d_table, m->n_exp, k, norm, act, m->hidden, m->eid, nt,
                          d_x + (size_t)t0 * m->hidden, d_logits + (size_t)t0 * m->n_exp,
                          d_out + (size_t)t0 * m->hidden, m->d_ws, stages, pick_stream(stream)))
            return fail(E_INTERNAL, "qsf_hip_moe_forward_dev: launch failed (tokens %d..%d)", t0,
                        t0 + nt - 1);
    }
    return E_OK;
}

/* ---- drop-in table slots ---------------------------------------------------- */
static void nan_fill(float* out, int rows) {
    for (int i = 0; i < rows; i++) out[i] = NAN;
}

/* ---- slot look-ahead ----------------------------------------------------------
 * An engine calls the slots in a fixed order each token, and the matrices
 * that share an x follow one another: q, k and v, then gate and up
 * (src/engine.c:848-866, 1118-1125).  Each tensor learns the key called
 * right after it with a bit-identical x; once the same successor has
 * followed twice running, a call on the tensor launches its successors'
 * GEMVs in the same launch (at most g_lookahead of them, same format, block
 * size and length, not volatile) and holds their results in host-mapped
 * memory.  The successor's own call then passes every check a call makes
 * (geometry, fingerprint, the pointer not volatile), and is served the held
 * result only if its tensor, the registry generation and x are all still
 * those the launch used; otherwise it runs as usual.  A group is launched
 * only when each member's rows get the arithmetic they get alone
 * (qk_gemv_signature), so a result never depends on what ran beside it.
 * A held result not asked for costs its predecessor the successor. */
static void ahead_learn(const void* w, int same_x) {
    if (!same_x || !g_ahead.last || g_ahead.last == w) return;
    reg_slot* ps = reg_find(g_ahead.last);
    qsf_hip_tensor* pt = ps ? ps->t : NULL;
    if (!pt) return;
    if (pt->succ == w) {
        if (pt->succ_hits < (1 << 20)) pt->succ_hits++;
    } else {
        pt->succ = w;
        pt->succ_hits = 1;
    }
}

static int ahead_serve(const void* w, const qsf_hip_tensor* t, int rows, float* out) {
    if (g_ahead.gen != g_reg_gen) return 0;
    for (int i = 1; i < g_ahead.n; i++) {
        ahead_entry* e = &g_ahead.e[i];
        if (e->key != w || e->used) continue;
        if (e->t != t || e->rows != rows) return 0;
        memcpy(out, g_dev.h_y + e->off, sizeof(float) * (size_t)rows);
        e->used = 1;
        g_ahead.last = w;
        return 1;
    }
    return 0;
}

static void ahead_drop(void) {
    for (int i = 1; i < g_ahead.n; i++) {
        const ahead_entry* e = &g_ahead.e[i];
        if (e->used) continue;
        reg_slot* ps = reg_find(e->pred);
        if (ps && ps->t && ps->t->succ == e->key) ps->t->succ_hits = 0;
    }
    g_ahead.n = 0;
}

/* the group a call on t launches: t, then its learnt successors */
static int ahead_plan(const qsf_hip_tensor* t, const void* w, const qsf_hip_tensor** grp,
                      const void** keys) {
    int n = 1;
    grp[0] = t;
    keys[0] = w;
    for (const qsf_hip_tensor* cur = t;
         n - 1 < g_lookahead && n < QK_MAX_GROUP && cur->succ && cur->succ_hits >= 2;) {
        const void* k = cur->succ;
        reg_slot* s = reg_find(k);
        if (!s || s->vol || !s->t) break;
        const qsf_hip_tensor* st = s->t;
        if (st->fmt != t->fmt || st->bs != t->bs || st->cols != t->cols) break;
        int dup = 0;
        for (int i = 0; i < n; i++) dup |= keys[i] == k;
        if (dup) break;
        grp[n] = st;
        keys[n++] = k;
        cur = st;
    }
    for (; n > 1; n--) {
        const uint64_t g = qk_gemv_signature(grp, n, QK_RUN_GEMV);
        int ok = g != 0;
        for (int i = 0; i < n && ok; i++) ok = qk_gemv_signature(&grp[i], 1, QK_RUN_GEMV) == g;
        if (ok) break;
    }
    return n;
}

int qsf_hip_gemv_engine(int engine) {
    return qk_gemv_mfma_enable(engine);
}

int qsf_hip_slot_lookahead(int n) {
    pthread_mutex_lock(&g_lock);
    const int old = g_lookahead;
    if (n >= 0) g_lookahead = n < QK_MAX_GROUP - 1 ? n : QK_MAX_GROUP - 1;
    pthread_mutex_unlock(&g_lock);
    return old;
}

/* Wait for the slot stream's work.  The stream writes a fresh sequence
 * number into host-mapped memory once everything queued before it has
 * completed (hipStreamWriteValue32) and the caller spins on that word: about
 * 2.5 us sooner than hipStreamSynchronize returns.  When the word cannot be
 * set up or queued, or has not arrived after 2 ms (a long queue ahead, or
 * a failed kernel), hipStreamSynchronize decides and reports any error. */
static int slot_wait(hipStream_t s) {
    if (!g_dev.h_flag) {
        if (hipHostMalloc((void**)&g_dev.h_flag, 256, hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess)
            g_dev.h_flag = NULL;
        else if (hipHostGetDevicePointer((void**)&g_dev.d_flag, g_dev.h_flag, 0) != hipSuccess) {
            hipHostFree(g_dev.h_flag);
            g_dev.h_flag = NULL;
        } else {
            __atomic_store_n(g_dev.h_flag, g_dev.flag_seq, __ATOMIC_RELEASE);
        }
    }
    if (g_dev.h_flag) {
        const uint32_t seq = ++g_dev.flag_seq;
        if (hipStreamWriteValue32(s, g_dev.d_flag, seq, 0) == hipSuccess) {
            struct timespec t0, t1;
            clock_gettime(CLOCK_MONOTONIC, &t0);
            for (uint32_t i = 1;; i++) {
                if (__atomic_load_n(g_dev.h_flag, __ATOMIC_ACQUIRE) == seq) return E_OK;
                if (!(i & 1023)) {
                    clock_gettime(CLOCK_MONOTONIC, &t1);
                    if ((t1.tv_sec - t0.tv_sec) * 1000000000L + (t1.tv_nsec - t0.tv_nsec) > 2000000L)
                        break;
                }
            }
        }
    }
    const hipError_t e = hipStreamSynchronize(s);
    return e == hipSuccess ? E_OK : fail(E_INTERNAL, "qsf_hip: %s", hipGetErrorString(e));
}

/* Synchronous host-pointer matvec.  The payload is looked up in the arena
 * (uploaded on first sight).  x is written to host-mapped memory and one
 * dispatch prepares it (block fixed point digits) straight from there,
 * leaving an fp32 copy in HBM; the GEMV runs on the prepared x and writes y
 * into host-mapped memory; one wait for the stream (slot_wait) ends the call.  When x
 * is bit-identical to the previous slot call's (gate and up, or q, k and v,
 * of one token share it) and of the same format, block size and length, the
 * prepared x is still in HBM and the call is one dispatch; with a learnt
 * successor it may also have been computed already (look-ahead, above).
 *
 * Stale weights: a pointer's entry is checked against the call's geometry,
 * the outlier count and a fingerprint of nine sampled payload words.  Any
 * mismatch uploads the payload again and marks the pointer volatile: from
 * then on it is uploaded on every call (an engine that decompresses each
 * layer into one reused buffer, src/engine.c:786-789, pays one upload per
 * call and is never served another layer's weights).  A caller that rewrites
 * a buffer whose first change could leave the sampled words equal must call
 * qsf_hip_arena_forget on it first. */
static void host_matvec(int qt, const void* w, const float* in, float* out,
                        int rows, int cols, int bs) {
    if (rows <= 0) return;
    pthread_mutex_lock(&g_lock);
    int rc = init_locked(g_dev.ready ? g_dev.device : 0);
    qsf_hip_tensor* t = NULL;
    if (!rc) {
        reg_slot* s = reg_find(w);
        t = s ? s->t : NULL;
        int vol = s ? s->vol : 0;
        if (t && (vol || t->qt != qt || t->rows != rows || t->cols != cols ||
                  (t->fmt >= 0 && t->bs != bs) ||
                  (is_outlier(qt) && rd_u32((const uint8_t*)w) != t->n_outliers) ||
                  s->fp != fingerprint(w, t->payload_bytes))) {
            vol = 1;
            reg_drop(w);
            t = NULL;
        }
        if (!t) {
            t = upload_locked(w, qt, rows, cols, bs);
            if (t) t->registry_owned = 1;
            if (!t || reg_put(w, t, vol ? 0 : fingerprint(w, t->payload_bytes), vol) != E_OK) {
                if (t) tensor_destroy(t);
                t = NULL;
                rc = g_err ? g_err : E_INTERNAL;
            }
        }
    }
    const int fmt = t ? t->fmt : -1, tbs = t ? t->bs : 32;
    const size_t xn = sizeof(float) * (size_t)(cols > 0 ? cols : 1), yn = sizeof(float) * (size_t)rows;
    /* the prepared x in HBM is this call's x */
    const int same = !rc && cols > 0 && g_dev.xq_ok && fmt >= 0 && g_dev.xq_fmt == fmt &&
                     g_dev.xq_bs == tbs && g_dev.xq_cols == cols && memcmp(g_dev.h_x, in, xn) == 0;
    if (!rc) {
        ahead_learn(w, same);
        if (same && ahead_serve(w, t, rows, out)) {
            pthread_mutex_unlock(&g_lock);
            return;
        }
    }
    ahead_drop();
    const qsf_hip_tensor* grp[QK_MAX_GROUP] = {t};
    const void* keys[QK_MAX_GROUP] = {w};
    size_t off[QK_MAX_GROUP] = {0};
    const int ng = !rc && fmt >= 0 && cols > 0 ? ahead_plan(t, w, grp, keys) : 1;
    size_t ytot = (size_t)rows;
    for (int i = 1; i < ng; i++) {
        off[i] = (ytot + 63) & ~(size_t)63;
        ytot = off[i] + (size_t)grp[i]->rows;
    }
    /* the prepared form writes x up to the last block's end */
    const size_t xpad = sizeof(float) * ((size_t)(cols > 0 ? cols : 1) + 256);
    if (!rc) {
        void* old_x = g_dev.d_x;
        rc = ensure_dev((void**)&g_dev.d_x, &g_dev.d_x_n, xpad);
        if (g_dev.d_x != old_x) g_dev.xq_ok = 0;
    }
    if (!rc && fmt >= 0 && cols > 0) {
        void* old_q = g_dev.slot_xq;
        rc = ensure_dev(&g_dev.slot_xq, &g_dev.slot_xq_bytes, qk_xprep_bytes(fmt, tbs, cols));
        if (g_dev.slot_xq != old_q) g_dev.xq_ok = 0;
    }
    if (!rc) {
        void* old_h = g_dev.h_x;
        rc = ensure_host((void**)&g_dev.h_x, &g_dev.h_x_n, xn);
        if (g_dev.h_x != old_h) g_dev.xq_ok = 0;
    }
    if (!rc) rc = ensure_host((void**)&g_dev.h_y, &g_dev.h_y_n, sizeof(float) * ytot);
    float *hx_dev = NULL, *hy_dev = NULL;
    if (!rc && (hipHostGetDevicePointer((void**)&hx_dev, g_dev.h_x, 0) != hipSuccess ||
                hipHostGetDevicePointer((void**)&hy_dev, g_dev.h_y, 0) != hipSuccess))
        rc = fail(E_INTERNAL, "qsf_hip: host-mapped staging");
    hipStream_t s = g_dev.stream;
    if (!rc && cols > 0) {
        /* buffers may have moved since `same` was taken */
        const int keep = same && g_dev.xq_ok;
        g_dev.xq_ok = 0;
        if (!keep) {
            memcpy(g_dev.h_x, in, xn);
            if (fmt < 0 ? qk_stage_f32(g_dev.d_x, hx_dev, cols, s)
                        : qk_xprep_stage(fmt, tbs, cols, hx_dev, g_dev.d_x, g_dev.slot_xq, s))
                rc = fail(E_INTERNAL, "qsf_hip: x staging");
        }
    }
    if (!rc) {
        float* ys[QK_MAX_GROUP];
        for (int i = 0; i < ng; i++) ys[i] = hy_dev + off[i];
        if (fmt < 0) rc = mxfp4_locked(t, g_dev.d_x, hy_dev, s);
        else if (qk_gemv_group(grp, ng, g_dev.d_x, ys, g_dev.slot_xq,
                               cols > 0 ? QK_RUN_GEMV : QK_RUN_BOTH, s))
            rc = fail(E_INTERNAL, "qsf_hip: GEMV launch failed");
    }
    if (!rc) rc = slot_wait(s);
    if (!rc) {
        memcpy(out, g_dev.h_y, yn);
        /* valid for the next call only after this one completed */
        g_dev.xq_ok = fmt >= 0 && cols > 0;
        g_dev.xq_fmt = fmt;
        g_dev.xq_bs = tbs;
        g_dev.xq_cols = cols;
        g_ahead.last = g_dev.xq_ok ? w : NULL;
        g_ahead.gen = g_reg_gen;
        g_ahead.n = ng > 1 ? ng : 0;
        for (int i = 1; i < ng; i++)
            g_ahead.e[i] = (ahead_entry){keys[i], keys[i - 1], grp[i], off[i], grp[i]->rows, 0};
    } else {
        g_ahead.last = NULL;
        nan_fill(out, rows);
    }
    pthread_mutex_unlock(&g_lock);
}

void qsf_matvec_2bit_hip(const void* w, const float* in, float* out, int rows, int cols, int bs) {
    host_matvec(QK_Q2, w, in, out, rows, cols, bs);
}
void qsf_matvec_3bit_hip(const void* w, const float* in, float* out, int rows, int cols, int bs) {
    host_matvec(QK_Q3, w, in, out, rows, cols, bs);
}
void qsf_matvec_4bit_hip(const void* w, const float* in, float* out, int rows, int cols, int bs) {
    host_matvec(QK_Q4, w, in, out, rows, cols, bs);
}
void qsf_matvec_4bit_sym_hip(const void* w, const float* in, float* out, int rows, int cols, int bs) {
    host_matvec(QK_Q4SYM, w, in, out, rows, cols, bs);
}
void qsf_matvec_outlier_2bit_hip(const void* w, const float* in, float* out, int rows, int cols, int bs) {
    host_matvec(QK_Q2_OUTLIER, w, in, out, rows, cols, bs);
}
void qsf_matvec_outlier_4bit_hip(const void* w, const float* in, float* out, int rows, int cols, int bs) {
    host_matvec(QK_Q4_OUTLIER, w, in, out, rows, cols, bs);
}
void qsf_matvec_mxfp4_hip(const void* w, const float* in, float* out, int rows, int cols, int bs) {
    (void)bs;
    host_matvec(QK_MXFP4, w, in, out, rows, cols, 32);
}

/* The six matvec slots lead QSFKernelTable in this order
 * (include/qsf/kernels.h:91-98). */
typedef void (*matvec_fn)(const void*, const float*, float*, int, int, int);

void qsf_kernels_init_hip(void* kernel_table, const void* platform, void** mxfp4_slot) {
    (void)platform;
    matvec_fn* slot = (matvec_fn*)kernel_table;
    if (slot) {
        slot[0] = qsf_matvec_2bit_hip;
        slot[1] = qsf_matvec_3bit_hip;
        slot[2] = qsf_matvec_4bit_hip;
        slot[3] = qsf_matvec_4bit_sym_hip;
        slot[4] = qsf_matvec_outlier_2bit_hip;
        slot[5] = qsf_matvec_outlier_4bit_hip;
    }
    if (mxfp4_slot) *mxfp4_slot = (void*)qsf_matvec_mxfp4_hip;
}
