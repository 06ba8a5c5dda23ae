// Device, stream, copy and graph entry points of the ABI (reference interface ops.h:22-52,
// bound by cuda.rs:50-133), so that a host executor needs no HIP headers or link of its own.
//
// Error policy of this file:
//  * every failed runtime call is "settled": its code is returned and the runtime's sticky
//    last-error slot is cleared, so one failure never resurfaces as the result of an unrelated
//    later call (an executor falls back to eager mode after a failed capture and keeps going);
//  * empty copies and launches succeed without touching the runtime;
//  * graph capture is thread-local, and a host wait on a capturing stream is refused with
//    hipErrorStreamCaptureUnsupported and marks that capture as spoilt, so ending it reports
//    hipErrorStreamCaptureInvalidated and yields no graph whatever the closure returned. This
//    makes the recovery rules the executor relies on (a capture that failed must end cleanly
//    and the stream must be capturable again; a retained graph keeps replaying) hold by this
//    library's own bookkeeping rather than by how a runtime version reports the event.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "qwen3_5_ops.h"

namespace {

int settle(hipError_t e) {
    if (e != hipSuccess) (void)hipGetLastError();
    return e;
}

// Streams of this thread whose open capture was spoilt by a host wait.
thread_local std::vector<hipStream_t> spoilt;

bool take_spoilt(hipStream_t s) {
    auto it = std::find(spoilt.begin(), spoilt.end(), s);
    if (it == spoilt.end()) return false;
    spoilt.erase(it);
    return true;
}

bool capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

const char* blaslt_string(int status) {
    switch (status) {
        case 1: return "hipBLASLt: handle not initialized";
        case 2: return "hipBLASLt: resource allocation failed";
        case 3: return "hipBLASLt: invalid value";
        case 4: return "hipBLASLt: mapping error";
        case 5: return "hipBLASLt: execution failed";
        case 6: return "hipBLASLt: internal error";
        case 7: return "hipBLASLt: not supported";
        case 8: return "hipBLASLt: architecture mismatch";
        default: return "hipBLASLt: error";
    }
}

}  // namespace

extern "C" {

uint32_t cs1_abi_version(void) { return CS1_ABI_VERSION; }

// Codes of 1000 and above are 1000 + a hipBLASLt status (the ABI's convention for library
// errors); the rest are hipError_t.
const char* cs1_error_string(int code) {
    return code >= 1000 ? blaslt_string(code - 1000) : hipGetErrorString(static_cast<hipError_t>(code));
}

int cs1_set_device(int device) { return settle(hipSetDevice(device)); }

int cs1_malloc(void** ptr, size_t bytes) {
    if (!ptr) return hipErrorInvalidValue;
    return settle(hipMalloc(ptr, bytes));
}

int cs1_free(void* ptr) { return ptr ? settle(hipFree(ptr)) : hipSuccess; }

// Non-blocking (no implicit ordering with the null stream), default priority.
int cs1_stream_create(void** stream) {
    if (!stream) return hipErrorInvalidValue;
    return settle(hipStreamCreateWithFlags(reinterpret_cast<hipStream_t*>(stream), hipStreamNonBlocking));
}

int cs1_stream_destroy(void* stream) { return settle(hipStreamDestroy(static_cast<hipStream_t>(stream))); }

// A host wait on a capturing stream: refused, and the capture is marked spoilt.
int refuse_host_wait(hipStream_t s) {
    if (std::find(spoilt.begin(), spoilt.end(), s) == spoilt.end()) spoilt.push_back(s);
    return hipErrorStreamCaptureUnsupported;
}

int cs1_stream_sync(void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (capturing(s)) return refuse_host_wait(s);
    return settle(hipStreamSynchronize(s));
}

// Host <-> device copies are synchronous: they return once the bytes have arrived, in
// stream order (the executor reuses its host buffers right after the call). Both are host
// waits, so under capture they are refused like cs1_stream_sync (a recorded copy would read or
// write a host buffer the caller has already reused by the time the graph replays).
int cs1_upload(void* dst, const void* src, size_t bytes, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (capturing(s)) return refuse_host_wait(s);
    if (bytes == 0) return hipSuccess;
    return settle(hipMemcpyWithStream(dst, src, bytes, hipMemcpyHostToDevice, s));
}

int cs1_download(void* dst, const void* src, size_t bytes, void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (capturing(s)) return refuse_host_wait(s);
    if (bytes == 0) return hipSuccess;
    return settle(hipMemcpyWithStream(dst, src, bytes, hipMemcpyDeviceToHost, s));
}

// Device copies are queued (and captured like kernels).
int cs1_copy_dd(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return hipSuccess;
    return settle(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
}

int cs1_copy2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
               void* stream) {
    if (width == 0 || height == 0) return hipSuccess;
    return settle(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, height, hipMemcpyDeviceToDevice,
                                   static_cast<hipStream_t>(stream)));
}

int cs1_graph_begin(void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    (void)take_spoilt(s);  // a stale mark from a capture that never ended
    return settle(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
}

// Ends the capture on stream and instantiates it; *exec is null unless this returns 0.
int cs1_graph_end(void* stream, void** exec) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (exec) *exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(s, &graph);
    if (take_spoilt(s) && e == hipSuccess) e = hipErrorStreamCaptureInvalidated;
    if (e == hipSuccess && !exec) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipGraphInstantiateWithFlags(reinterpret_cast<hipGraphExec_t*>(exec), graph, 0);
    if (graph) (void)hipGraphDestroy(graph);
    if (e != hipSuccess && exec) *exec = nullptr;
    return settle(e);
}

int cs1_graph_launch(void* exec, void* stream) {
    if (!exec) return hipErrorInvalidValue;
    return settle(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(stream)));
}

int cs1_graph_destroy(void* exec) {
    return exec ? settle(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec))) : hipSuccess;
}

}  // extern "C"
