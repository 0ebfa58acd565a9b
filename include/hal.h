/*
 * hal.h -- device contract of the paged KV-cache path (C ABI).
 *
 * The reference names this contract (README.md:197-203,269-276: dev_alloc /
 * dev_free / dev_upload / dev_download / dev_sync / dev_max_alloc) but ships no
 * such file; its nearest realisations are syclb::Device
 * (code/device/sycl/device.h:140-148) and DeviceArena + NOVA_CU
 * (include/nova/memory/arena.h:276-470).  This header defines it, with the
 * reference's abort-on-failure convention (include/nova/config.h:42-63): no
 * function returns an error code; a failing HIP call prints the call, the
 * error string and device free/total memory, then aborts.
 *
 * Implemented by conflux-nova_amd/code/device/hip/hal_hip.hip over HIP.  The
 * stream type is opaque: hipStream_t appears only inside code/device/hip.
 * A NULL stream means the device's default (null) stream.
 */
#ifndef NOVA_HAL_H
#define NOVA_HAL_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* nova_stream_t;
typedef void* nova_event_t;
typedef void* nova_graph_t;

/* ---- the six functions named by the reference (README.md:203) ---- */
/* bytes == 0 returns NULL.  Failure aborts after printing free/total
 * (arena.h:276-288).  Memory is NOT cleared. */
void*    dev_alloc(uint64_t bytes);
void     dev_free(void* p);
/* synchronous host->device / device->host copies (device.h:144-145) */
void     dev_upload(void* dst, const void* src, uint64_t bytes);
void     dev_download(void* dst, const void* src, uint64_t bytes);
/* waits for all work on the device (device.h:147) */
void     dev_sync(void);
/* largest single allocation the build will attempt: free device memory minus a
 * fixed reserve (cf. profile::kMaxAllocBytes, device.h:38) */
uint64_t dev_max_alloc(void);

/* ---- extensions the paged path needs that the six do not cover ----
 * Engine::cow_guard issues device->device page copies (src/model.cpp:180-187)
 * and SessionManager::create clears pages with cudaMemsetAsync
 * (code/session.h:107-118); both run on a per-session stream (session.h:94). */
void     dev_copy_d2d(void* dst, const void* src, uint64_t bytes, nova_stream_t s);
void     dev_upload_async(void* dst, const void* src, uint64_t bytes, nova_stream_t s);
void     dev_download_async(void* dst, const void* src, uint64_t bytes, nova_stream_t s);
/* zero-fill with a kernel (never a memset node, so it is safe under graph capture) */
void     dev_zero(void* dst, uint64_t bytes, nova_stream_t s);
nova_stream_t dev_stream_create(void);          /* default priority, non-blocking */
void     dev_stream_destroy(nova_stream_t s);
void     dev_stream_sync(nova_stream_t s);
/* events, for timing on the stream the kernels run on */
nova_event_t dev_event_create(void);
void     dev_event_destroy(nova_event_t e);
void     dev_event_record(nova_event_t e, nova_stream_t s);
float    dev_event_elapsed_ms(nova_event_t start, nova_event_t stop);  /* syncs on stop */
/* stream capture into a replayable graph (launch-bound layer loops) */
void     dev_graph_begin(nova_stream_t s);
nova_graph_t dev_graph_end(nova_stream_t s);
void     dev_graph_launch(nova_graph_t g, nova_stream_t s);
void     dev_graph_destroy(nova_graph_t g);
/* device facts */
int      dev_cu_count(void);
int      dev_count(void);                        /* 0 when no GPU is visible */
const char* dev_arch_name(void);                 /* e.g. "gfx950" */

#ifdef __cplusplus
}
#endif
#endif
