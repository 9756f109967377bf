// runtime_abi.cpp — af_rt_* device plumbing and status strings (see af_runtime.h).
#include <hip/hip_runtime.h>

#include <cstring>

#include "af_common.h"
#include "af_runtime.h"

extern "C" int af_version(void) { return (0 << 16) | (1 << 8) | 0; }

extern "C" const char* af_status_string(int status) {
    switch (status) {
        case AF_OK: return "ok";
        case AF_ERR_POOL_EXHAUSTED: return "block pool exhausted";
        case AF_ERR_INVALID_ARG: return "invalid argument";
        case AF_ERR_UNSUPPORTED: return "unsupported shape or dtype";
        case AF_ERR_OUT_OF_RANGE: return "position or length out of range";
        case AF_ERR_BAD_BLOCK: return "bad block id";
        case AF_ERR_WORKSPACE: return "workspace missing or too small";
        case AF_ERR_BAD_SEQUENCE: return "unknown sequence id";
        case AF_ERR_NOT_BUILT: return "device code not built";
        case AF_ERR_BAD_FILE: return "bad or truncated weight file";
        case AF_ERR_TIMEOUT: return "decode attention: a split never published its partial";
        default: break;
    }
    if (status > 0) return hipGetErrorString(hipError_t(status));
    return "unknown status";
}

extern "C" int af_rt_device_count(int* count) {
    if (!count) return AF_ERR_INVALID_ARG;
    *count = 0;
    return int(hipGetDeviceCount(count));
}

extern "C" int af_rt_set_device(int device) { return int(hipSetDevice(device)); }

extern "C" int af_rt_device_info(char* name, int name_len, int* compute_units, char* arch,
                                 int arch_len) {
    int dev = 0;
    AF_TRY_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    AF_TRY_HIP(hipGetDeviceProperties(&p, dev));
    if (name && name_len > 0) {
        std::strncpy(name, p.name, size_t(name_len) - 1);
        name[name_len - 1] = 0;
    }
    if (arch && arch_len > 0) {
        std::strncpy(arch, p.gcnArchName, size_t(arch_len) - 1);
        arch[arch_len - 1] = 0;
    }
    if (compute_units) *compute_units = p.multiProcessorCount;
    return AF_OK;
}

extern "C" int af_rt_device_sync(void) { return int(hipDeviceSynchronize()); }
extern "C" int af_rt_last_error(void) { return int(hipGetLastError()); }

extern "C" int af_rt_malloc(void** ptr, size_t bytes) {
    if (!ptr) return AF_ERR_INVALID_ARG;
    *ptr = nullptr;
    return int(hipMalloc(ptr, bytes));
}
extern "C" int af_rt_free(void* ptr) { return int(hipFree(ptr)); }
extern "C" int af_rt_host_malloc(void** ptr, size_t bytes) {
    if (!ptr) return AF_ERR_INVALID_ARG;
    *ptr = nullptr;
    return int(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
}
extern "C" int af_rt_host_free(void* ptr) { return int(hipHostFree(ptr)); }
extern "C" int af_rt_mem_info(size_t* free_bytes, size_t* total_bytes) {
    if (!free_bytes || !total_bytes) return AF_ERR_INVALID_ARG;
    return int(hipMemGetInfo(free_bytes, total_bytes));
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, af_stream_t stream) {
    if ((!dst || !src) && bytes) return AF_ERR_INVALID_ARG;
    if (!bytes) return AF_OK;
    return int(hipMemcpyAsync(dst, src, bytes, kind, static_cast<hipStream_t>(stream)));
}
extern "C" int af_rt_memcpy_h2d(void* dst, const void* src, size_t bytes, af_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyHostToDevice, stream);
}
extern "C" int af_rt_memcpy_d2h(void* dst, const void* src, size_t bytes, af_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream);
}
extern "C" int af_rt_memcpy_d2d(void* dst, const void* src, size_t bytes, af_stream_t stream) {
    return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream);
}

extern "C" int af_rt_stream_create(af_stream_t* stream) {
    if (!stream) return AF_ERR_INVALID_ARG;
    hipStream_t s = nullptr;
    AF_TRY_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));  // default priority
    *stream = s;
    return AF_OK;
}
extern "C" int af_rt_stream_destroy(af_stream_t stream) {
    return int(hipStreamDestroy(static_cast<hipStream_t>(stream)));
}
extern "C" int af_rt_stream_sync(af_stream_t stream) {
    return int(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
}

extern "C" int af_rt_event_create(void** event) {
    if (!event) return AF_ERR_INVALID_ARG;
    hipEvent_t e = nullptr;
    AF_TRY_HIP(hipEventCreate(&e));
    *event = e;
    return AF_OK;
}
extern "C" int af_rt_event_destroy(void* event) {
    return int(hipEventDestroy(static_cast<hipEvent_t>(event)));
}
extern "C" int af_rt_event_record(void* event, af_stream_t stream) {
    return int(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
}
extern "C" int af_rt_event_sync(void* event) {
    return int(hipEventSynchronize(static_cast<hipEvent_t>(event)));
}
extern "C" int af_rt_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (!ms) return AF_ERR_INVALID_ARG;
    return int(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
}

extern "C" int af_rt_capture_begin(af_stream_t stream) {
    if (!stream) return AF_ERR_INVALID_ARG;  // the legacy default stream cannot be captured
    return int(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeGlobal));
}
extern "C" int af_rt_capture_end(af_stream_t stream, void** graph_exec) {
    if (!stream || !graph_exec) return AF_ERR_INVALID_ARG;
    hipGraph_t g = nullptr;
    AF_TRY_HIP(hipStreamEndCapture(static_cast<hipStream_t>(stream), &g));
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return int(e);
    *graph_exec = ge;
    return AF_OK;
}
extern "C" int af_rt_graph_launch(void* graph_exec, af_stream_t stream) {
    return int(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), static_cast<hipStream_t>(stream)));
}
extern "C" int af_rt_graph_destroy(void* graph_exec) {
    return int(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)));
}
