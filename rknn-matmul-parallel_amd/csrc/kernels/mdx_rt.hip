// mdx_rt.hip — HIP runtime wrappers behind the plain-C device ABI
// (mdx_device.h).  Errors are mapped to MatmulDecoderError codes and the
// last HIP message is kept for diagnostics.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "mdx_device.h"

namespace {

thread_local char g_last_error[256] = "";

int fail(hipError_t e, const char* what) {
    std::snprintf(g_last_error, sizeof g_last_error, "%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? -2 : -4;
}

#define MDX_CHECK(expr, what)                     \
    do {                                          \
        hipError_t e_ = (expr);                   \
        if (e_ != hipSuccess) return fail(e_, what); \
    } while (0)

__global__ void k_fill_u32(uint32_t* dst, uint32_t value, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = value;
}

}  // namespace

// Uncached device memory (MTYPE UC: no L2 allocation) for the one-launch
// step's exchange words.  Every exchange is a store that has to reach memory
// and polls that have to miss every cache; in uncached memory neither goes
// through the XCD's L2 (measured: fp16 layers at KV 512 465.3 -> 443.8
// us/token, int4 at KV 4000 540.7 -> 513.2).  Uncached memory that a kernel
// has read is never returned to the device before the process ends (later
// allocations at the same addresses have held wrong values), so released
// buffers go back to this pool, one list per device, and are handed out
// again to later contexts.  The caller clears a buffer it acquires (on its
// own stream: nothing here synchronises the device, which could meet another
// thread's graph capture).
namespace {
struct UcBuf {
    int dev;
    size_t bytes;
    void* p;
    bool used;
};
std::mutex g_uc_mu;
std::vector<UcBuf>* g_uc = nullptr;   // never destroyed: outlives every context
}  // namespace

extern "C" {

int mdxrt_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

const char* mdxrt_last_error(void) { return g_last_error; }

int mdxrt_malloc(void** p, size_t bytes) {
    *p = nullptr;
    MDX_CHECK(hipMalloc(p, bytes ? bytes : 256), "hipMalloc");
    return 0;
}

int mdxrt_free(void* p) {
    if (p) MDX_CHECK(hipFree(p), "hipFree");
    return 0;
}

int mdxrt_uc_acquire(void** p, size_t bytes) {
    *p = nullptr;
    int dev = 0;
    MDX_CHECK(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_uc_mu);
    if (!g_uc) g_uc = new std::vector<UcBuf>();
    for (UcBuf& u : *g_uc) {
        if (!u.used && u.dev == dev && u.bytes == bytes) {
            u.used = true;
            *p = u.p;
            break;
        }
    }
    if (!*p) {
        void* q = nullptr;
        MDX_CHECK(hipExtMallocWithFlags(&q, bytes, hipDeviceMallocUncached), "hipExtMallocWithFlags(uncached)");
        g_uc->push_back(UcBuf{dev, bytes, q, true});
        *p = q;
    }
    return 0;
}

int mdxrt_uc_release(void* p) {
    if (!p) return 0;
    std::lock_guard<std::mutex> lk(g_uc_mu);
    if (g_uc)
        for (UcBuf& u : *g_uc)
            if (u.p == p) {
                u.used = false;
                return 0;
            }
    std::snprintf(g_last_error, sizeof g_last_error, "mdxrt_uc_release: unknown buffer");
    return -1;
}

int mdxrt_host_alloc(void** p, size_t bytes) {
    *p = nullptr;
    MDX_CHECK(hipHostMalloc(p, bytes ? bytes : 64, hipHostMallocDefault), "hipHostMalloc");
    return 0;
}

int mdxrt_host_free(void* p) {
    if (p) MDX_CHECK(hipHostFree(p), "hipHostFree");
    return 0;
}

int mdxrt_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes) MDX_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return 0;
}

int mdxrt_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes) MDX_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return 0;
}

int mdxrt_h2d_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes)
        MDX_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream),
                  "hipMemcpyAsync H2D");
    return 0;
}

int mdxrt_d2h_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes)
        MDX_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream),
                  "hipMemcpyAsync D2H");
    return 0;
}

int mdxrt_d2d_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes)
        MDX_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream),
                  "hipMemcpyAsync D2D");
    return 0;
}

int mdxrt_stream_create(void** stream) {
    hipStream_t s = nullptr;
    MDX_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = (void*)s;
    return 0;
}

int mdxrt_stream_destroy(void* stream) {
    if (stream) MDX_CHECK(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
    return 0;
}

int mdxrt_stream_sync(void* stream) {
    MDX_CHECK(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return 0;
}

int mdxrt_device_sync(void) {
    MDX_CHECK(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return 0;
}

int mdxrt_graph_begin(void* stream) {
    MDX_CHECK(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal),
              "hipStreamBeginCapture");
    return 0;
}

// A captured graph and its executable instance.  The graph is kept alive as
// long as the instance: the runtime (and tools that trace graph launches) may
// refer to the graph's nodes when the instance is launched.
struct mdx_graph {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

int mdxrt_graph_end(void* stream, void** handle) {
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    *handle = nullptr;
    MDX_CHECK(hipStreamEndCapture((hipStream_t)stream, &g), "hipStreamEndCapture");
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(e, "hipGraphInstantiate");
    }
    mdx_graph* h = new mdx_graph{g, ge};
    *handle = (void*)h;
    return 0;
}

int mdxrt_graph_launch(void* handle, void* stream) {
    MDX_CHECK(hipGraphLaunch(static_cast<mdx_graph*>(handle)->exec, (hipStream_t)stream),
              "hipGraphLaunch");
    return 0;
}

int mdxrt_graph_destroy(void* handle) {
    if (!handle) return 0;
    mdx_graph* h = static_cast<mdx_graph*>(handle);
    hipError_t e1 = hipGraphExecDestroy(h->exec);
    hipError_t e2 = hipGraphDestroy(h->graph);
    delete h;
    if (e1 != hipSuccess) return fail(e1, "hipGraphExecDestroy");
    if (e2 != hipSuccess) return fail(e2, "hipGraphDestroy");
    return 0;
}

int mdxrt_event_create(void** ev) {
    hipEvent_t e = nullptr;
    MDX_CHECK(hipEventCreate(&e), "hipEventCreate");
    *ev = (void*)e;
    return 0;
}

int mdxrt_event_destroy(void* ev) {
    if (ev) MDX_CHECK(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
    return 0;
}

int mdxrt_event_record(void* ev, void* stream) {
    MDX_CHECK(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream), "hipEventRecord");
    return 0;
}

int mdxrt_event_elapsed_ms(void* start, void* stop, float* ms) {
    MDX_CHECK(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize");
    MDX_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), "hipEventElapsedTime");
    return 0;
}

int mdxrt_fill_u32(void* dst, uint32_t value, size_t n, void* stream) {
    if (!n) return 0;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_fill_u32<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
        (uint32_t*)dst, value, n);
    MDX_CHECK(hipGetLastError(), "k_fill_u32");
    return 0;
}

}  // extern "C"
