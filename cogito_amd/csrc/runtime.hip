// runtime.hip -- device context, error reporting, device memory, staging
// scratch and the registry of device-resident INT4 weights.
//
// One device, one HIP stream (default priority) per process.  Errors never
// abort: they are recorded in a thread-local string (cgx_last_error), the
// same contract as the reference's last-error string
// (src/cuda/cg_cuda.c:29,344-353).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "cgx_internal.h"

namespace {

struct Runtime {
    bool initialized = false;
    int device = 0;
    hipStream_t stream = nullptr;
    char name[256] = {0};
    hipEvent_t events[8] = {};
    void* scratch[CGX_NUM_SLOTS] = {};
    size_t scratch_bytes[CGX_NUM_SLOTS] = {};
    unsigned int* counters = nullptr;
    size_t counter_count = 0;
};

Runtime g_rt;
thread_local char g_err[1024] = {0};

struct QuantEntry {
    const cg_tensor_quant* q;
    cgx_qinfo info;
};
std::vector<QuantEntry> g_quants;

}  // namespace

extern "C" void cgx_set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" const char* cgx_last_error(void) { return g_err; }
extern "C" void cgx_clear_error(void) { g_err[0] = 0; }

#define CGX_TRY(call)                                                      \
    do {                                                                   \
        hipError_t e_ = (call);                                            \
        if (e_ != hipSuccess) {                                            \
            cgx_set_error("%s failed: %s", #call, hipGetErrorString(e_));  \
            return -1;                                                     \
        }                                                                  \
    } while (0)

extern "C" int cgx_init(int device) {
    if (g_rt.initialized) {
        if (device != g_rt.device) {
            cgx_set_error("cgx_init: already bound to device %d", g_rt.device);
            return -1;
        }
        return 0;
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        cgx_set_error("cgx_init: no HIP device is visible");
        return -1;
    }
    if (device < 0 || device >= count) {
        cgx_set_error("cgx_init: device %d out of range (%d visible)", device,
                      count);
        return -1;
    }
    CGX_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    CGX_TRY(hipGetDeviceProperties(&prop, device));
    snprintf(g_rt.name, sizeof(g_rt.name), "%s (%s, %d CUs)", prop.name,
             prop.gcnArchName, prop.multiProcessorCount);
    CGX_TRY(hipStreamCreateWithFlags(&g_rt.stream, hipStreamNonBlocking));
    for (int i = 0; i < 8; i++) CGX_TRY(hipEventCreate(&g_rt.events[i]));
    g_rt.device = device;
    g_rt.initialized = true;
    // the allocation-free verify's workspace address on this device
    if (cgk_verify_static_init(device)) return -1;
    return 0;
}

extern "C" int cgx_device_id(void) { return g_rt.initialized ? g_rt.device : -1; }

extern "C" int cgx_ensure_init(void) {
    return g_rt.initialized ? 0 : cgx_init(0);
}

extern "C" int cgx_device_count(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return count;
}

extern "C" void* cgx_stream(void) {
    if (cgx_ensure_init()) return nullptr;
    return (void*)g_rt.stream;
}

extern "C" const char* cgx_device_name(void) {
    if (cgx_ensure_init()) return "";
    return g_rt.name;
}

extern "C" int cgx_synchronize(void) {
    if (cgx_ensure_init()) return -1;
    CGX_TRY(hipStreamSynchronize(g_rt.stream));
    CGX_TRY(hipGetLastError());
    return 0;
}

extern "C" void* cgx_malloc(size_t bytes) {
    if (cgx_ensure_init()) return nullptr;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        cgx_set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
        return nullptr;
    }
    return p;
}

extern "C" int cgx_free(void* p) {
    if (!p) return 0;
    if (cgx_ensure_init()) return -1;
    CGX_TRY(hipStreamSynchronize(g_rt.stream));
    CGX_TRY(hipFree(p));
    return 0;
}

extern "C" int cgx_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (cgx_ensure_init()) return -1;
    if (!bytes) return 0;
    CGX_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_rt.stream));
    CGX_TRY(hipStreamSynchronize(g_rt.stream));
    return 0;
}

extern "C" int cgx_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (cgx_ensure_init()) return -1;
    if (!bytes) return 0;
    CGX_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_rt.stream));
    CGX_TRY(hipStreamSynchronize(g_rt.stream));
    return 0;
}

extern "C" int cgx_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (cgx_ensure_init()) return -1;
    if (!bytes) return 0;
    CGX_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_rt.stream));
    return 0;
}

// True while the library stream is being captured into a graph.  Calls that
// would record a memset node or allocate, free or synchronise then refuse:
// memset nodes have given wrong results on replays after the first, and an
// allocation or a synchronisation ends the capture with an error.
static bool capturing(const char* who) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g_rt.stream, &st) != hipSuccess || st == hipStreamCaptureStatusNone)
        return false;
    cgx_set_error("%s: the library stream is being captured into a graph (cgx_graph_begin); "
                  "only calls that allocate, clear and synchronise nothing may be captured",
                  who);
    return true;
}

extern "C" int cgx_memset(void* dst, int value, size_t bytes) {
    if (cgx_ensure_init()) return -1;
    if (!bytes) return 0;
    if (capturing("cgx_memset")) return -1;
    CGX_TRY(hipMemsetAsync(dst, value, bytes, g_rt.stream));
    return 0;
}

extern "C" int cgx_is_device_ptr(const void* p) {
    if (!p || cgx_ensure_init()) return 0;
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // unregistered host memory
        return 0;
    }
    return attr.type == hipMemoryTypeDevice ? 1 : 0;
}

extern "C" int cgx_event_record(int slot) {
    if (cgx_ensure_init()) return -1;
    if (slot < 0 || slot >= 8) {
        cgx_set_error("cgx_event_record: slot %d out of range", slot);
        return -1;
    }
    CGX_TRY(hipEventRecord(g_rt.events[slot], g_rt.stream));
    return 0;
}

// Plain streaming read of a buffer: 256-thread blocks, two 16-byte words per
// thread (the shape of the fastest plain read measured on gfx950), each wave
// XOR-folding its two 1 KiB runs into one word of `out`.  A floor for any
// kernel that has to read the same bytes.
typedef unsigned int cgx_u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_stream_read(const cgx_u32x4* __restrict__ p, size_t n16,
                                                     unsigned int* __restrict__ out) {
    const size_t base = (size_t)blockIdx.x * 512 + threadIdx.x;
    unsigned int x = 0;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const size_t j = base + (size_t)i * 256;
        if (j < n16) {
            const cgx_u32x4 v = __builtin_nontemporal_load(p + j);
            x ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if ((threadIdx.x & 63) == 0) out[(size_t)blockIdx.x * 4 + (threadIdx.x >> 6)] = x;
}

extern "C" int cgx_stream_read(const void* buf, size_t bytes, unsigned int* out) {
    if (cgx_ensure_init()) return -1;
    if (!buf || !out || bytes == 0 || (bytes & 15) || ((uintptr_t)buf & 15)) {
        cgx_set_error("cgx_stream_read: a 16-byte aligned buffer of a multiple of 16 bytes "
                      "is required");
        return -1;
    }
    const size_t n16 = bytes / 16, blocks = (n16 + 511) / 512;
    if (blocks > 0x7fffffffu) {
        cgx_set_error("cgx_stream_read: buffer too large");
        return -1;
    }
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)blocks), dim3(256), 0, g_rt.stream,
                       (const cgx_u32x4*)buf, n16, out);
    CGX_TRY(hipGetLastError());
    return 0;
}

extern "C" float cgx_event_elapsed_ms(int a, int b) {
    if (cgx_ensure_init() || a < 0 || a >= 8 || b < 0 || b >= 8) return -1.0f;
    if (hipEventSynchronize(g_rt.events[b]) != hipSuccess) return -1.0f;
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, g_rt.events[a], g_rt.events[b]) != hipSuccess)
        return -1.0f;
    return ms;
}

// ------------------------------------------------------------ graphs
// Capture of the library stream into a HIP graph (thread-local mode: other
// threads' HIP calls are not affected) and its replays on the same stream.
extern "C" int cgx_graph_begin(void) {
    if (cgx_ensure_init()) return -1;
    CGX_TRY(hipStreamBeginCapture(g_rt.stream, hipStreamCaptureModeThreadLocal));
    return 0;
}

extern "C" void* cgx_graph_end(void) {
    if (cgx_ensure_init()) return nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(g_rt.stream, &g);
    if (e != hipSuccess || !g) {
        cgx_set_error("graph capture failed: %s", hipGetErrorString(e));
        (void)hipGetLastError();
        return nullptr;
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        cgx_set_error("graph instantiation failed: %s", hipGetErrorString(e));
        return nullptr;
    }
    return (void*)x;
}

extern "C" int cgx_graph_launch(void* graph) {
    if (cgx_ensure_init()) return -1;
    if (!graph) {
        cgx_set_error("cgx_graph_launch: no graph");
        return -1;
    }
    CGX_TRY(hipGraphLaunch((hipGraphExec_t)graph, g_rt.stream));
    return 0;
}

extern "C" int cgx_graph_free(void* graph) {
    if (!graph) return 0;
    CGX_TRY(hipGraphExecDestroy((hipGraphExec_t)graph));
    return 0;
}

extern "C" void* cgx_scratch(int slot, size_t bytes) {
    if (cgx_ensure_init()) return nullptr;
    if (slot < 0 || slot >= CGX_NUM_SLOTS) {
        cgx_set_error("cgx_scratch: bad slot %d", slot);
        return nullptr;
    }
    if (bytes > g_rt.scratch_bytes[slot]) {
        if (capturing("cgx_scratch (growth)")) return nullptr;
        size_t want = bytes < 4096 ? 4096 : bytes + bytes / 4;
        if (g_rt.scratch[slot]) {
            if (hipStreamSynchronize(g_rt.stream) != hipSuccess ||
                hipFree(g_rt.scratch[slot]) != hipSuccess) {
                cgx_set_error("cgx_scratch: releasing slot %d failed", slot);
                return nullptr;
            }
        }
        g_rt.scratch[slot] = nullptr;
        g_rt.scratch_bytes[slot] = 0;
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) {
            cgx_set_error("cgx_scratch: hipMalloc(%zu) failed: %s", want,
                          hipGetErrorString(e));
            return nullptr;
        }
        g_rt.scratch[slot] = p;
        g_rt.scratch_bytes[slot] = want;
    }
    return g_rt.scratch[slot];
}

extern "C" unsigned int* cgx_counters(size_t count) {
    if (cgx_ensure_init()) return nullptr;
    if (count > g_rt.counter_count) {
        if (capturing("cgx_counters (growth)")) return nullptr;
        size_t want = count < 4096 ? 4096 : count;
        if (g_rt.counters) {
            if (hipStreamSynchronize(g_rt.stream) != hipSuccess ||
                hipFree(g_rt.counters) != hipSuccess) {
                cgx_set_error("cgx_counters: release failed");
                return nullptr;
            }
        }
        g_rt.counters = nullptr;
        g_rt.counter_count = 0;
        void* p = nullptr;
        if (hipMalloc(&p, want * sizeof(unsigned int)) != hipSuccess ||
            hipMemset(p, 0, want * sizeof(unsigned int)) != hipSuccess ||
            hipDeviceSynchronize() != hipSuccess) {
            cgx_set_error("cgx_counters: allocation of %zu counters failed", want);
            return nullptr;
        }
        g_rt.counters = (unsigned int*)p;
        g_rt.counter_count = want;
    }
    return g_rt.counters;
}

extern "C" const void* cgx_dev_in(const void* p, size_t bytes, int slot) {
    if (!p) {
        cgx_set_error("null input pointer");
        return nullptr;
    }
    if (cgx_is_device_ptr(p)) return p;
    void* d = cgx_scratch(slot, bytes);
    if (!d) return nullptr;
    if (bytes &&
        hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, g_rt.stream) != hipSuccess) {
        cgx_set_error("staging copy of %zu bytes failed", bytes);
        return nullptr;
    }
    return d;
}

extern "C" int cgx_quant_lookup(const cg_tensor_quant* q, cgx_qinfo* info) {
    for (const QuantEntry& e : g_quants) {
        if (e.q == q) {
            if (info) *info = e.info;
            return 1;
        }
    }
    return 0;
}

extern "C" void cgx_quant_register(const cg_tensor_quant* q, const cgx_qinfo* info) {
    cgx_quant_unregister(q);
    g_quants.push_back(QuantEntry{q, *info});
}

extern "C" void cgx_quant_unregister(const cg_tensor_quant* q) {
    for (size_t i = 0; i < g_quants.size(); i++) {
        if (g_quants[i].q == q) {
            g_quants.erase(g_quants.begin() + (long)i);
            return;
        }
    }
}
