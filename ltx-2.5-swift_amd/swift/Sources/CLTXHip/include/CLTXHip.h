/*
 * CLTXHip -- the thin C target between the Swift package and libltx_attn.so.
 *
 * Swift imports this module and sees two things:
 *   - the attention library's C ABI (ltx_attn.h: ltx_attn_fwd, ltx_linear,
 *     ltx_gemma_attn_fwd, the RoPE table builders, ltx_device_query), unchanged;
 *   - cltx_*: device memory, page-locked host memory, host<->device copies, one stream and a
 *     free-memory query, as plain C over the HIP runtime, so no HIP header has to be
 *     imported into Swift.
 * Every function returns 0 on success or the hipError_t code; cltx_error_string() names it.
 */
#ifndef CLTX_HIP_H
#define CLTX_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <ltx_attn.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Make `ordinal` the calling thread's current device (the explicit selection). */
int32_t cltx_set_device(int32_t ordinal);

/* Device memory: `bytes` (> 0) of device memory, 256-byte aligned, into *out. */
int32_t cltx_alloc(size_t bytes, void **out);
int32_t cltx_free(void *ptr);

/* A stream of the current device (default priority), and a wait for everything on it. */
int32_t cltx_stream_create(void **out);
int32_t cltx_stream_destroy(void *stream);
int32_t cltx_stream_synchronize(void *stream);

/* Page-locked host memory (`bytes` > 0) into *out: copies from and to it run asynchronously,
 * without a staging copy by the runtime. */
int32_t cltx_host_alloc(size_t bytes, void **out);
int32_t cltx_host_free(void *ptr);

/* Copies between host memory and device memory, ordered on `stream`, asynchronous: the host
 * side must stay valid and unchanged until cltx_stream_synchronize(stream) returns (use
 * cltx_host_alloc memory; pageable memory is staged by the runtime, slower). */
int32_t cltx_upload(void *dst_device, const void *src_host, size_t bytes, void *stream);
int32_t cltx_download(void *dst_host, const void *src_device, size_t bytes, void *stream);

/* Free and total device memory of the current device, measured now (hipMemGetInfo). */
int32_t cltx_mem_info(size_t *free_bytes, size_t *total_bytes);

const char *cltx_error_string(int32_t code);

#ifdef __cplusplus
}
#endif

#endif /* CLTX_HIP_H */
