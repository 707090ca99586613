/* host_double.c - the device half of libqsf_hip replaced by host reads, for
 * the sanitizer build of the loader (tests/asan/Makefile).  Test
 * infrastructure only.
 *
 * Every entry point the loader (qstream_amd/host/qsf_loader.c) calls after
 * its checks is here, and each one reads every host byte the real upload
 * reads (qstream_amd/host/qsf_hip.c: upload_locked, qsf_host_device_bytes,
 * qsf_hip_moe_create), sized from the QSF format itself: MXFP4 records of
 * 17 bytes per 32 columns, the outlier table's count and 6-byte entries
 * before the blocks of types 9 and 10, and blocks of 4 + ceil(bits * bs / 8)
 * bytes (src/quant.c:69-85).  Under AddressSanitizer a read past what the
 * loader validated then stops the run.
 */
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qsf_hip.h"
#include "qsf_host.h"

struct qsf_hip_tensor {
    size_t payload_bytes;
};
struct qsf_hip_moe {
    int n;
};

static int g_err;
static char g_detail[256];
static volatile uint32_t g_sink;

static void touch(const void* p, size_t n) {
    const uint8_t* b = (const uint8_t*)p;
    uint32_t s = 0;
    for (size_t i = 0; i < n; i++) s += b[i];
    g_sink += s;
}

int qsf_host_fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_detail, sizeof g_detail, fmt, ap);
    va_end(ap);
    g_err = code;
    return code;
}
int qsf_hip_last_error(void) { return g_err; }
const char* qsf_hip_last_error_detail(void) { return g_detail; }
int qsf_hip_init(int device) {
    (void)device;
    return 0;
}

float qsf_host_fp16(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    float f;
    if (e == 0) {
        f = (float)m * (1.0f / 16777216.0f);   /* m * 2^-24 */
        return s ? -f : f;
    }
    const uint32_t bits = s | (e == 31 ? 0x7F800000u | (m << 13) : ((e + 112) << 23) | (m << 13));
    memcpy(&f, &bits, 4);
    return f;
}

qsf_hip_tensor* qsf_host_upload_owned(const void* host, int qt, int rows, int cols, int bs) {
    if (!host || rows < 0 || cols < 0) return NULL;
    const uint8_t* p = (const uint8_t*)host;
    size_t n;
    if (qt == 11) {
        n = (size_t)rows * (((size_t)cols + 31) / 32) * 17;
    } else {
        if (bs != 32 && bs != 64 && bs != 128 && bs != 256) return NULL;
        const int bits = (qt == 0 || qt == 1 || qt == 9) ? 2 : qt == 2 ? 3 : 4;
        n = (size_t)rows * (((size_t)cols + bs - 1) / bs) * (4 + ((size_t)bs * bits + 7) / 8);
        if (qt == 9 || qt == 10) {
            uint32_t n_out;
            memcpy(&n_out, p, 4);
            n += 4 + 6 * (size_t)n_out;
        }
    }
    touch(p, n);
    qsf_hip_tensor* t = malloc(sizeof *t);
    if (t) t->payload_bytes = n;
    return t;
}

void* qsf_host_device_bytes(const void* host, size_t n) {
    touch(host, n);
    return malloc(n ? n : 1);
}
float* qsf_host_device_floats(const float* host, size_t n) {
    touch(host, n * sizeof(float));
    return malloc(n ? n * sizeof(float) : 1);
}
void qsf_host_device_free(void* p) { free(p); }
void qsf_hip_tensor_free(qsf_hip_tensor* t) { free(t); }
size_t qsf_hip_tensor_payload_bytes(const qsf_hip_tensor* t) { return t ? t->payload_bytes : 0; }

qsf_hip_moe* qsf_hip_moe_create(int n_experts, int hidden, int expert_dim, const qsf_hip_tensor* const* gate,
                                const qsf_hip_tensor* const* up, const qsf_hip_tensor* const* down,
                                const uint16_t* const* gate_bias, const uint16_t* const* up_bias,
                                const uint16_t* const* down_bias) {
    (void)gate; (void)up; (void)down;
    for (int e = 0; e < n_experts; e++) {
        if (gate_bias && gate_bias[e]) touch(gate_bias[e], (size_t)expert_dim * 2);
        if (up_bias && up_bias[e]) touch(up_bias[e], (size_t)expert_dim * 2);
        if (down_bias && down_bias[e]) touch(down_bias[e], (size_t)hidden * 2);
    }
    qsf_hip_moe* m = malloc(sizeof *m);
    if (m) m->n = n_experts;
    return m;
}
void qsf_hip_moe_free(qsf_hip_moe* m) { free(m); }
