// Runtime half of the boundary: status strings, device selection, memory,
// copies, the backend stream, events and workspaces
// (core/device.h:26-46, core/device.cpp:183-333, cuda/cuda_utils.cu).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "gh_common.h"

namespace gh {

static thread_local std::string g_err;
static hipStream_t g_stream = nullptr;
static int g_cus = 0;

void set_error(int code, const std::string& msg) {
    (void)code;
    g_err = msg;
}

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_error(code, buf);
    return code;
}

hipStream_t stream() { return g_stream; }

int num_cus() {
    if (g_cus == 0) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&g_cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (g_cus <= 0) g_cus = 256;
    }
    return g_cus;
}

struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
static std::vector<Workspace> g_ws(64);

static uint64_t g_ws_gen = 0;  // bumped whenever a slot gets a new buffer
uint64_t workspace_generation() { return g_ws_gen; }

void* workspace(int slot, size_t bytes) {
    if (slot < 0 || slot >= (int)g_ws.size()) return nullptr;
    Workspace& w = g_ws[(size_t)slot];
    if (w.bytes < bytes) {
        ++g_ws_gen;
        // grow-only; the old buffer may still be read by queued work
        if (w.ptr) {
            (void)hipStreamSynchronize(g_stream);
            (void)hipFree(w.ptr);
        }
        size_t nb = bytes < 256 ? 256 : bytes;
        nb = (nb + 255) & ~(size_t)255;
        if (hipMalloc(&w.ptr, nb) != hipSuccess) {
            w.ptr = nullptr;
            w.bytes = 0;
            return nullptr;
        }
        w.bytes = nb;
    }
    return w.ptr;
}

void free_workspaces() {
    (void)hipStreamSynchronize(g_stream);
    ++g_ws_gen;
    for (Workspace& w : g_ws) {
        if (w.ptr) (void)hipFree(w.ptr);
        w = Workspace{};
    }
}

}  // namespace gh

using namespace gh;

extern "C" {

const char* gh_last_error(void) { return g_err.c_str(); }

int gh_init(int device) {
    int n = 0;
    GH_HIP(hipGetDeviceCount(&n));
    GH_REQUIRE(device >= 0 && device < n, "gh_init: device %d out of range (%d devices)", device, n);
    GH_HIP(hipSetDevice(device));
    hipDeviceProp_t p;
    GH_HIP(hipGetDeviceProperties(&p, device));
    GH_REQUIRE(strstr(p.gcnArchName, "gfx950") != nullptr,
               "gh_init: this backend is built for gfx950 (MI355X), device is %s", p.gcnArchName);
    g_cus = p.multiProcessorCount;
    return GH_OK;
}

int gh_device_info(gh_device_info_t* out) {
    GH_REQUIRE(out != nullptr, "gh_device_info: null output");
    int dev = 0;
    GH_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    GH_HIP(hipGetDeviceProperties(&p, dev));
    memset(out, 0, sizeof *out);
    snprintf(out->name, sizeof out->name, "%s (%s)", p.name, p.gcnArchName);
    out->arch_major = p.major;
    out->arch_minor = p.minor;
    out->compute_units = p.multiProcessorCount;
    GH_HIP(hipMemGetInfo(&out->free_mem, &out->total_mem));
    return GH_OK;
}

int gh_device_alloc(void** out, size_t bytes) {
    GH_REQUIRE(out != nullptr, "gh_device_alloc: null output");
    *out = nullptr;
    if (bytes == 0) return GH_OK;
    // core/device.cpp:256-264: refuse before allocating when it cannot fit
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) == hipSuccess && bytes > free_b)
        return fail(GH_ENOMEM, "gh_device_alloc: %zu bytes requested, %zu free", bytes, free_b);
    hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) return fail(GH_ENOMEM, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    return GH_OK;
}

int gh_device_free(void* p) {
    if (p) GH_HIP(hipFree(p));
    return GH_OK;
}

int gh_device_memset_zero(void* p, size_t bytes) {
    if (!bytes) return GH_OK;
    GH_REQUIRE(p != nullptr, "gh_device_memset_zero: null pointer");
    GH_HIP(hipMemsetAsync(p, 0, bytes, g_stream));
    GH_HIP(hipStreamSynchronize(g_stream));
    return GH_OK;
}

int gh_device_copy(void* dst, int dst_dev, const void* src, int src_dev, size_t bytes) {
    if (!bytes) return GH_OK;
    GH_REQUIRE(dst && src, "gh_device_copy: null pointer");
    GH_REQUIRE((dst_dev == GH_DEV_CPU || dst_dev == GH_DEV_GPU) && (src_dev == GH_DEV_CPU || src_dev == GH_DEV_GPU),
               "gh_device_copy: bad device id");
    if (dst_dev == GH_DEV_CPU && src_dev == GH_DEV_CPU) {
        memcpy(dst, src, bytes);
        return GH_OK;
    }
    hipMemcpyKind k = dst_dev == GH_DEV_GPU ? (src_dev == GH_DEV_GPU ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice)
                                            : hipMemcpyDeviceToHost;
    GH_HIP(hipMemcpyAsync(dst, src, bytes, k, g_stream));
    GH_HIP(hipStreamSynchronize(g_stream));
    return GH_OK;
}

int gh_set_stream(void* s) {
    g_stream = (hipStream_t)s;
    return GH_OK;
}
void* gh_get_stream(void) { return (void*)g_stream; }

int gh_synchronize(void) {
    GH_HIP(hipStreamSynchronize(g_stream));
    return GH_OK;
}

int gh_event_create(void** ev) {
    GH_REQUIRE(ev != nullptr, "gh_event_create: null output");
    hipEvent_t e;
    GH_HIP(hipEventCreate(&e));
    *ev = (void*)e;
    return GH_OK;
}
int gh_event_record(void* ev) {
    GH_HIP(hipEventRecord((hipEvent_t)ev, g_stream));
    return GH_OK;
}
int gh_event_elapsed_ms(void* a, void* b, float* ms) {
    GH_HIP(hipEventSynchronize((hipEvent_t)b));
    GH_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return GH_OK;
}
int gh_event_destroy(void* ev) {
    if (ev) GH_HIP(hipEventDestroy((hipEvent_t)ev));
    return GH_OK;
}

int gh_free_workspace(void) {
    free_workspaces();
    return GH_OK;
}

}  // extern "C"
