// The HIP runtime calls a host executor needs (allocation, streams, graphs, copies), so
// that it loads libqwen3_5_hip.so alone. Semantics of the reference's runtime.cu:7-74:
// non-blocking streams, synchronous upload/download, queued device copies, graph capture
// in thread-local mode with the sticky error cleared after a failed capture.
#include <hip/hip_runtime.h>

#include "qwen3_5_ops.h"

extern "C" {

uint32_t cs1_abi_version(void) { return CS1_ABI_VERSION; }

const char* cs1_error_string(int code) {
    if (code >= 1000) return "hipBLASLt error (status = code - 1000)";
    return hipGetErrorString(static_cast<hipError_t>(code));
}

int cs1_set_device(int device) { return hipSetDevice(device); }

int cs1_malloc(void** ptr, size_t bytes) { return hipMalloc(ptr, bytes); }

int cs1_free(void* ptr) { return hipFree(ptr); }

int cs1_stream_create(void** stream) {
    return hipStreamCreateWithFlags(reinterpret_cast<hipStream_t*>(stream), hipStreamNonBlocking);
}

int cs1_stream_destroy(void* stream) { return hipStreamDestroy(static_cast<hipStream_t>(stream)); }

int cs1_stream_sync(void* stream) { return hipStreamSynchronize(static_cast<hipStream_t>(stream)); }

int cs1_upload(void* dst, const void* src, size_t bytes, void* stream) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
    return e != hipSuccess ? e : hipStreamSynchronize(st);
}

int cs1_download(void* dst, const void* src, size_t bytes, void* stream) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st);
    return e != hipSuccess ? e : hipStreamSynchronize(st);
}

int cs1_copy_dd(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return hipSuccess;
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream));
}

int cs1_copy2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
               void* stream) {
    if (width == 0 || height == 0) return hipSuccess;
    return hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDeviceToDevice,
                            static_cast<hipStream_t>(stream));
}

int cs1_graph_begin(void* stream) {
    const hipError_t e = hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) (void)hipGetLastError();
    return e;
}

int cs1_graph_end(void* stream, void** exec) {
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &graph);
    if (e == hipSuccess) e = hipGraphInstantiate(reinterpret_cast<hipGraphExec_t*>(exec), graph, nullptr, nullptr, 0);
    if (graph) (void)hipGraphDestroy(graph);
    if (e != hipSuccess) (void)hipGetLastError();
    return e;
}

int cs1_graph_launch(void* exec, void* stream) {
    const hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) (void)hipGetLastError();
    return e;
}

int cs1_graph_destroy(void* exec) { return hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)); }

}  // extern "C"
