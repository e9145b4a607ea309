/*
 * CLTXHip's C side: device memory, copies and streams for the Swift package, over the HIP
 * runtime's C API. The attention itself is libltx_attn.so (ltx_attn.h).
 */
#include "CLTXHip.h"

#include <hip/hip_runtime_api.h>

int32_t cltx_set_device(int32_t ordinal) { return (int32_t)hipSetDevice(ordinal); }

int32_t cltx_alloc(size_t bytes, void **out) {
    if (!out || bytes == 0) return (int32_t)hipErrorInvalidValue;
    *out = NULL;
    return (int32_t)hipMalloc(out, bytes);
}

int32_t cltx_free(void *ptr) { return ptr ? (int32_t)hipFree(ptr) : 0; }

int32_t cltx_stream_create(void **out) {
    if (!out) return (int32_t)hipErrorInvalidValue;
    return (int32_t)hipStreamCreate((hipStream_t *)out);
}

int32_t cltx_stream_destroy(void *stream) {
    return stream ? (int32_t)hipStreamDestroy((hipStream_t)stream) : 0;
}

int32_t cltx_stream_synchronize(void *stream) {
    return (int32_t)hipStreamSynchronize((hipStream_t)stream);
}

int32_t cltx_host_alloc(size_t bytes, void **out) {
    if (!out || bytes == 0) return (int32_t)hipErrorInvalidValue;
    *out = NULL;
    return (int32_t)hipHostMalloc(out, bytes, hipHostMallocDefault);
}

int32_t cltx_host_free(void *ptr) { return ptr ? (int32_t)hipHostFree(ptr) : 0; }

int32_t cltx_upload(void *dst_device, const void *src_host, size_t bytes, void *stream) {
    if (bytes == 0) return 0;
    return (int32_t)hipMemcpyAsync(dst_device, src_host, bytes, hipMemcpyHostToDevice,
                                   (hipStream_t)stream);
}

int32_t cltx_download(void *dst_host, const void *src_device, size_t bytes, void *stream) {
    if (bytes == 0) return 0;
    return (int32_t)hipMemcpyAsync(dst_host, src_device, bytes, hipMemcpyDeviceToHost,
                                   (hipStream_t)stream);
}

int32_t cltx_mem_info(size_t *free_bytes, size_t *total_bytes) {
    if (!free_bytes || !total_bytes) return (int32_t)hipErrorInvalidValue;
    return (int32_t)hipMemGetInfo(free_bytes, total_bytes);
}

const char *cltx_error_string(int32_t code) { return hipGetErrorString((hipError_t)code); }
