/* mutate_loader.c - seeded byte-mutation sweep of the QSF loader's parse
 * path (test infrastructure; tests/asan/Makefile builds it with
 * AddressSanitizer and UndefinedBehaviorSanitizer).
 *
 * usage: mutate_loader <seed file.qsf> <iterations> <seed> [offsets file]
 *
 * Each iteration copies the file into a heap buffer of exactly its (possibly
 * truncated) length, applies a few mutations -- random bytes, 32/64-bit
 * fields set to boundary values, truncation -- and loads it with
 * qsf_hip_model_load_mem.  A sanitizer report stops the run with a non-zero
 * status (-fno-sanitize-recover); otherwise it prints how many mutants were
 * loaded and how many rejected, and exits 0.  The optional offsets file
 * lists the file's structure fields (one byte offset a line: header fields,
 * layer-index entries, tensor record headers, section headers, outlier
 * counts); half of the mutations land on one of them.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qsf_hip.h"

static uint64_t g_s;
static uint64_t next(void) {   /* splitmix64 */
    uint64_t z = (g_s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

int main(int argc, char** argv) {
    if (argc < 4) {
        fprintf(stderr, "usage: %s <file.qsf> <iterations> <seed>\n", argv[0]);
        return 2;
    }
    FILE* f = fopen(argv[1], "rb");
    if (!f) return 2;
    fseek(f, 0, SEEK_END);
    const size_t size = (size_t)ftell(f);
    fseek(f, 0, SEEK_SET);
    uint8_t* orig = malloc(size);
    if (!orig || fread(orig, 1, size, f) != size) return 2;
    fclose(f);
    const long iters = atol(argv[2]);
    g_s = strtoull(argv[3], NULL, 0);
    size_t hot[4096];
    int n_hot = 0;
    if (argc > 4) {
        FILE* o = fopen(argv[4], "r");
        if (!o) return 2;
        unsigned long long v;
        while (n_hot < 4096 && fscanf(o, "%llu", &v) == 1)
            if (v < size) hot[n_hot++] = (size_t)v;
        fclose(o);
    }
    /* the unmutated file loads */
    qsf_hip_model* m0 = qsf_hip_model_load_mem(orig, size);
    if (!m0) {
        fprintf(stderr, "seed file rejected: %s\n", qsf_hip_last_error_detail());
        return 3;
    }
    qsf_hip_model_free(m0);
    static const uint64_t vals[] = {0, 1, 2, 3, 7, 31, 32, 33, 63, 64, 255, 256, 4096, 65535, 65536,
                                    0x7FFFFFFFull, 0x80000000ull, 0xFFFFFFFFull, 0xFFFFFFFFFFFFFFFFull};
    long loaded = 0, rejected = 0;
    for (long it = 0; it < iters; it++) {
        size_t len = size;
        if (next() % 8 == 0) len = (size_t)(next() % size) + 1;   /* truncate */
        uint8_t* b = malloc(len);
        if (!b) return 2;
        memcpy(b, orig, len);
        const int nm = 1 + (int)(next() % 4);
        for (int k = 0; k < nm; k++) {
            const uint64_t r = next();
            /* header, index and section headers first: the first 512 bytes
             * and the end of the file are where the structure is */
            size_t at = (r & 1) ? (size_t)(next() % (len < 512 ? len : 512)) : (size_t)(next() % len);
            const int from_hot = n_hot && (r & 0x30) != 0;
            if (from_hot) {
                at = hot[next() % (uint64_t)n_hot];
                if (at >= len) at = len - 1;
            }
            switch ((r >> 1) % 3) {
            case 0: b[at] = (uint8_t)next(); break;
            case 1:
                if (!from_hot) at &= ~(size_t)3;
                if (at + 4 <= len) { uint32_t v = (uint32_t)vals[next() % 18]; memcpy(b + at, &v, 4); }
                break;
            default:
                if (!from_hot) at &= ~(size_t)7;
                if (at + 8 <= len) { uint64_t v = vals[next() % 19]; memcpy(b + at, &v, 8); }
                break;
            }
        }
        qsf_hip_model* m = qsf_hip_model_load_mem(b, len);
        if (m) {
            loaded++;
            qsf_hip_model_free(m);
        } else {
            rejected++;
        }
        free(b);
    }
    printf("%s: %ld mutants, %ld loaded, %ld rejected\n", argv[1], iters, loaded, rejected);
    free(orig);
    return 0;
}
