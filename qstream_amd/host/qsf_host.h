/*
 * qsf_host.h - functions the host-layer files share (not part of the
 * public C ABI).
 */
#ifndef QSF_HOST_H
#define QSF_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "qsf_hip.h"

/* Record an error (thread-local detail, qsf_set_error when linked);
 * returns `code`. */
int qsf_host_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

/* Upload a payload into the device arena without registering its host
 * pointer (the caller owns the tensor; qsf_hip_tensor_free releases it).
 * For payloads read from a mapping that is unmapped afterwards. */
qsf_hip_tensor* qsf_host_upload_owned(const void* host, int qt, int rows, int cols, int bs);

/* Device copy of n floats / n bytes (hipMalloc + copy); NULL on failure. */
float* qsf_host_device_floats(const float* host, size_t n);
void* qsf_host_device_bytes(const void* host, size_t n);
void qsf_host_device_free(void* p);

/* IEEE binary16 -> binary32 (src/quant.c:11-39). */
float qsf_host_fp16(uint16_t h);

#endif
