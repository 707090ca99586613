/* dropin_table.c - the engine's own way into libqsf_hip, as a test program.
 *
 * Test infrastructure.  Compiled against QStream's include/qsf headers and
 * linked with its kernels.c, kernels_scalar.c, kernels_avx2.c and quant.c
 * (oracle/Makefile), it does what src/engine.c:439 and the integration
 * patch do: qsf_kernels_init (src/kernels.c:7-65) fills a real
 * QSFKernelTable (include/qsf/kernels.h:91-126) with the CPU kernels, then
 * qsf_kernels_init_hip, loaded from the path given on the command line,
 * takes over the six matvec slots.  It checks that exactly those six
 * members changed, that the other twelve are the CPU kernels still, and
 * (unless --slots-only) calls every matvec slot through its struct member,
 * as engine.c's get_matvec_fn callers do, against the slots captured before
 * the takeover and the reference's scalar kernels: relative L2 <= 1e-5.
 *
 * usage: dropin_table <path to libqsf_hip.so> [--slots-only]
 * exit 0 and a final "OK" line on success.
 */
#include "qsf/kernels.h"
#include "qsf/quant.h"

#include <dlfcn.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef void (*init_hip_fn)(void* kernel_table, const void* platform, void** mxfp4_slot);

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 7;
    g_rng ^= g_rng << 17;
    return (uint32_t)(g_rng >> 16);
}
static float gauss(void) {   /* sum of 4 uniforms, unit variance */
    float s = 0.f;
    for (int i = 0; i < 4; i++) s += (float)(rnd() & 0xFFFF) / 65536.0f - 0.5f;
    return s * 1.7320508f;
}
static uint16_t f16(float v) {   /* to nearest even; below fp16's normal range -> 0 */
    uint32_t u;
    memcpy(&u, &v, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, m = u & 0x7FFFFFu;
    const int32_t e = (int32_t)((u >> 23) & 0xFF) - 127 + 15;
    if (e <= 0) return (uint16_t)sign;
    uint32_t h = ((uint32_t)e << 10) | (m >> 13);
    const uint32_t rest = m & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* a payload of `qt` (0 2-bit, 2 3-bit, 3 4-bit, 4 4-bit sym, 9/10 outlier) */
static uint8_t* payload(int qt, int rows, int cols, int bs, size_t* bytes) {
    const int base = qt == 9 ? QSF_QUANT_2BIT_ASYM : qt == 10 ? QSF_QUANT_4BIT_ASYM : qt;
    const size_t bb = qsf_quant_block_size((QSFQuantType)base, bs), nb = (size_t)(cols + bs - 1) / bs;
    const uint32_t n_out = (qt == 9 || qt == 10) ? (uint32_t)(rows * cols / 200 + 1) : 0;
    const size_t head = (qt == 9 || qt == 10) ? 4 + 6 * (size_t)n_out : 0;
    *bytes = head + (size_t)rows * nb * bb;
    uint8_t* p = malloc(*bytes);
    if (!p) return NULL;
    if (head) {
        memcpy(p, &n_out, 4);
        for (uint32_t i = 0; i < n_out; i++) {
            uint32_t idx = rnd() % (uint32_t)(rows * cols);
            uint16_t v = f16(gauss() * 0.5f);
            memcpy(p + 4 + 6 * i, &idx, 4);
            memcpy(p + 8 + 6 * i, &v, 2);
        }
    }
    for (size_t b = 0; b < (size_t)rows * nb; b++) {
        uint8_t* blk = p + head + b * bb;
        uint16_t s = f16(0.002f + 0.004f * (float)(rnd() & 0xFF) / 256.0f), z = f16(gauss() * 0.02f);
        memcpy(blk, &s, 2);
        memcpy(blk + 2, &z, 2);
        for (size_t j = 4; j < bb; j++) blk[j] = (uint8_t)rnd();
    }
    return p;
}

static double rel_l2(const float* a, const float* b, int n) {
    double num = 0, den = 0;
    for (int i = 0; i < n; i++) {
        num += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
        den += (double)b[i] * b[i];
    }
    return den > 0 ? sqrt(num / den) : sqrt(num);
}

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s <libqsf_hip.so> [--slots-only]\n", argv[0]);
        return 2;
    }
    const int slots_only = argc > 2 && strcmp(argv[2], "--slots-only") == 0;
    void* lib = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (!lib) {
        fprintf(stderr, "dlopen: %s\n", dlerror());
        return 2;
    }
    init_hip_fn init_hip = (init_hip_fn)dlsym(lib, "qsf_kernels_init_hip");
    const char* names[6] = {"qsf_matvec_2bit_hip", "qsf_matvec_3bit_hip", "qsf_matvec_4bit_hip",
                            "qsf_matvec_4bit_sym_hip", "qsf_matvec_outlier_2bit_hip",
                            "qsf_matvec_outlier_4bit_hip"};
    if (!init_hip) {
        fprintf(stderr, "qsf_kernels_init_hip missing\n");
        return 2;
    }

    /* the engine's start-up: CPU table, then the GPU takeover */
    QSFPlatformInfo platform;
    memset(&platform, 0, sizeof platform);
    __builtin_cpu_init();
    platform.has_avx2 = __builtin_cpu_supports("avx2");
    platform.has_fma = __builtin_cpu_supports("fma");
    platform.has_f16c = 1;
    platform.is_little_endian = 1;
    QSFKernelTable kt, cpu;
    memset(&kt, 0, sizeof kt);
    qsf_kernels_init(&kt, &platform);
    cpu = kt;
    void* mx = NULL;
    init_hip(&kt, &platform, &mx);

    int fails = 0;
    const qsf_matvec_fn got[6] = {kt.matvec_2bit, kt.matvec_3bit, kt.matvec_4bit, kt.matvec_4bit_sym,
                                  kt.matvec_outlier_2bit, kt.matvec_outlier_4bit};
    for (int i = 0; i < 6; i++)
        if ((void*)got[i] != dlsym(lib, names[i])) {
            fprintf(stderr, "slot %d is not %s\n", i, names[i]);
            fails++;
        }
    if (!mx || mx != dlsym(lib, "qsf_matvec_mxfp4_hip")) {
        fprintf(stderr, "mxfp4 slot not returned\n");
        fails++;
    }
    /* every member after the six matvec slots is the CPU kernel still */
    if (memcmp((const char*)&kt + offsetof(QSFKernelTable, vec_add),
               (const char*)&cpu + offsetof(QSFKernelTable, vec_add),
               sizeof kt - offsetof(QSFKernelTable, vec_add)) != 0) {
        fprintf(stderr, "a non-matvec slot changed\n");
        fails++;
    }
    printf("slots: %s (cpu isa %s)\n", fails ? "FAIL" : "ok", platform.has_avx2 ? "avx2" : "scalar");
    if (fails || slots_only) {
        if (!fails) printf("OK\n");
        return fails ? 1 : 0;
    }

    /* every slot through its struct member, against the captured CPU slot
     * and the reference's scalar kernel */
    static const int shapes[][3] = {{64, 64, 64}, {300, 4096, 64}, {37, 1000, 128}, {11008 / 8, 4096, 128},
                                    {5, 33, 32}, {130, 1000, 256}};
    const int qts[6] = {0, 2, 3, 4, 9, 10};
    int cases = 0;
    for (int s = 0; s < (int)(sizeof shapes / sizeof shapes[0]); s++)
        for (int q = 0; q < 6; q++) {
            const int rows = shapes[s][0], cols = shapes[s][1], bs = shapes[s][2], qt = qts[q];
            size_t bytes = 0;
            uint8_t* w = payload(qt, rows, cols, bs, &bytes);
            float* x = malloc(sizeof(float) * cols);
            float *yg = malloc(sizeof(float) * rows), *yc = malloc(sizeof(float) * rows),
                  *ys = malloc(sizeof(float) * rows);
            if (!w || !x || !yg || !yc || !ys) return 2;
            for (int i = 0; i < cols; i++) x[i] = gauss();
            qsf_matvec_fn slot_g, slot_c;
            switch (qt) {
            case 0: slot_g = kt.matvec_2bit; slot_c = cpu.matvec_2bit; break;
            case 2: slot_g = kt.matvec_3bit; slot_c = cpu.matvec_3bit; break;
            case 3: slot_g = kt.matvec_4bit; slot_c = cpu.matvec_4bit; break;
            case 4: slot_g = kt.matvec_4bit_sym; slot_c = cpu.matvec_4bit_sym; break;
            case 9: slot_g = kt.matvec_outlier_2bit; slot_c = cpu.matvec_outlier_2bit; break;
            default: slot_g = kt.matvec_outlier_4bit; slot_c = cpu.matvec_outlier_4bit; break;
            }
            for (int i = 0; i < rows; i++) yg[i] = NAN;
            slot_g(w, x, yg, rows, cols, bs);
            /* without AVX2 the CPU table's outlier slots are quant.c's
             * seven-argument matvecs (src/kernels.c:13-14), not callable
             * through the six-argument slot: compare with scalar only */
            const int cpu_ok = (qt != 9 && qt != 10) || (platform.has_avx2 && platform.has_fma);
            if (cpu_ok) slot_c(w, x, yc, rows, cols, bs);
            /* 4-bit symmetric: the scalar kernel reads codes >= 8 as q - 16
             * (src/quant.c:158-177), the AVX2 slot as q - 8
             * (src/kernels_avx2.c:300-302); this library follows the scalar kernel,
             * so its AVX2 slot is reported, not held to the bar */
            const int cpu_cmp = cpu_ok && !(qt == 4 && platform.has_avx2 && platform.has_fma);
            switch (qt) {
            case 0: qsf_matvec_2bit_scalar(w, x, ys, rows, cols, bs); break;
            case 2: qsf_matvec_3bit_scalar(w, x, ys, rows, cols, bs); break;
            case 3: qsf_matvec_4bit_scalar(w, x, ys, rows, cols, bs); break;
            case 4: qsf_matvec_4bit_sym_scalar(w, x, ys, rows, cols, bs); break;
            case 9: qsf_matvec_outlier_2bit(w, bytes, x, ys, rows, cols, bs); break;
            default: qsf_matvec_outlier_4bit(w, bytes, x, ys, rows, cols, bs); break;
            }
            const double e_s = rel_l2(yg, ys, rows), e_c = cpu_ok ? rel_l2(yg, yc, rows) : e_s;
            const int ok = e_s <= 1e-5 && (!cpu_cmp || e_c <= 1e-5);
            printf("qt %2d %5dx%-5d bs %3d  rel-L2 vs scalar %.2e  vs cpu slot %.2e%s  %s\n", qt, rows, cols, bs,
                   e_s, e_c, cpu_cmp ? "" : " (not held)", ok ? "ok" : "FAIL");
            fails += !ok;
            cases++;
            free(w); free(x); free(yg); free(yc); free(ys);
        }
    printf("%d cases, %d failed\n", cases, fails);
    if (!fails) printf("OK\n");
    return fails ? 1 : 0;
}
