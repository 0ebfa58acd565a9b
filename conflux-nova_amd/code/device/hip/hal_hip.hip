// hal_hip.hip -- the device contract (include/hal.h) over HIP for gfx950.
//
// dev_alloc/dev_free/dev_upload/dev_download/dev_sync/dev_max_alloc are the six
// functions the reference names for code/device/hal.h (README.md:203); their
// behaviour follows syclb::Device (code/device/sycl/device.h:140-148) and the
// NOVA_CU abort convention (include/nova/memory/arena.h:276-289).  The rest are
// the copy / zero / stream / event / graph extensions the paged path needs.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "hal.h"
#include "../../kernel/hip/check.h"

namespace {

hipStream_t S(nova_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Zero-fill kernel: 16 B per lane on the aligned body, byte tail handled by the
// first lanes.  Used instead of hipMemsetAsync so the clear is an ordinary
// kernel node if a caller captures it into a graph.
__global__ void zero_kernel(uint8_t* __restrict__ p, uint64_t n16, uint64_t tail_off, uint32_t tail) {
    const uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint4* q = reinterpret_cast<uint4*>(p);
    for (uint64_t k = i; k < n16; k += stride) q[k] = make_uint4(0u, 0u, 0u, 0u);
    if (i < tail) p[tail_off + i] = 0;
}

}  // namespace

extern "C" {

void* dev_alloc(uint64_t bytes) {
    if (bytes == 0) return nullptr;
    void* p = nullptr;
    NOVA_HIP(hipMalloc(&p, bytes));
    return p;
}

void dev_free(void* p) {
    if (p) NOVA_HIP(hipFree(p));
}

void dev_upload(void* dst, const void* src, uint64_t bytes) {
    if (bytes) NOVA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
}

void dev_download(void* dst, const void* src, uint64_t bytes) {
    if (bytes) NOVA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
}

void dev_sync(void) { NOVA_HIP(hipDeviceSynchronize()); }

uint64_t dev_max_alloc(void) {
    size_t f = 0, t = 0;
    NOVA_HIP(hipMemGetInfo(&f, &t));
    const uint64_t reserve = 2ull << 30;   // keep 2 GiB for workspaces and the runtime
    return f > reserve ? (uint64_t)f - reserve : 0;
}

void dev_copy_d2d(void* dst, const void* src, uint64_t bytes, nova_stream_t s) {
    if (bytes) NOVA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(s)));
}

void dev_upload_async(void* dst, const void* src, uint64_t bytes, nova_stream_t s) {
    if (bytes) NOVA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, S(s)));
}

void dev_download_async(void* dst, const void* src, uint64_t bytes, nova_stream_t s) {
    if (bytes) NOVA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, S(s)));
}

void dev_zero(void* dst, uint64_t bytes, nova_stream_t s) {
    if (!bytes) return;
    const uintptr_t a = reinterpret_cast<uintptr_t>(dst);
    NOVA_REQUIRE(a % 16 == 0);
    const uint64_t n16 = bytes / 16;
    const uint32_t tail = (uint32_t)(bytes - n16 * 16);
    uint64_t blocks = (n16 + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, S(s),
                       static_cast<uint8_t*>(dst), n16, n16 * 16, tail);
    NOVA_LAUNCHED();
}

nova_stream_t dev_stream_create(void) {
    hipStream_t s = nullptr;
    NOVA_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    return s;
}
void dev_stream_destroy(nova_stream_t s) { if (s) NOVA_HIP(hipStreamDestroy(S(s))); }
void dev_stream_sync(nova_stream_t s) { NOVA_HIP(hipStreamSynchronize(S(s))); }

nova_event_t dev_event_create(void) {
    hipEvent_t e = nullptr;
    NOVA_HIP(hipEventCreate(&e));
    return e;
}
void dev_event_destroy(nova_event_t e) { if (e) NOVA_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(e))); }
void dev_event_record(nova_event_t e, nova_stream_t s) {
    NOVA_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(e), S(s)));
}
float dev_event_elapsed_ms(nova_event_t a, nova_event_t b) {
    NOVA_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(b)));
    float ms = 0.f;
    NOVA_HIP(hipEventElapsedTime(&ms, reinterpret_cast<hipEvent_t>(a), reinterpret_cast<hipEvent_t>(b)));
    return ms;
}

void dev_graph_begin(nova_stream_t s) {
    NOVA_REQUIRE(s != nullptr);   // the legacy null stream cannot be captured
    NOVA_HIP(hipStreamBeginCapture(S(s), hipStreamCaptureModeThreadLocal));
}
nova_graph_t dev_graph_end(nova_stream_t s) {
    hipGraph_t g = nullptr;
    NOVA_HIP(hipStreamEndCapture(S(s), &g));
    hipGraphExec_t ex = nullptr;
    NOVA_HIP(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
    NOVA_HIP(hipGraphDestroy(g));
    return ex;
}
void dev_graph_launch(nova_graph_t g, nova_stream_t s) {
    NOVA_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(g), S(s)));
}
void dev_graph_destroy(nova_graph_t g) {
    if (g) NOVA_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(g)));
}

int dev_cu_count(void) {
    int dev = 0, n = 0;
    NOVA_HIP(hipGetDevice(&dev));
    NOVA_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    return n;
}

int dev_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

const char* dev_arch_name(void) {
    static char name[64] = {0};
    static std::once_flag once;
    std::call_once(once, [] {
        hipDeviceProp_t p;
        int dev = 0;
        NOVA_HIP(hipGetDevice(&dev));
        NOVA_HIP(hipGetDeviceProperties(&p, dev));
        std::strncpy(name, p.gcnArchName, sizeof(name) - 1);
    });
    return name;
}

}  // extern "C"
