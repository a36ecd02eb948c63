// Host side of block streaming: exact-size pinned host buffers, asynchronous host -> device copies on a side
// stream, and events as fences between the copy stream and the compute stream (the role of PinnedHost,
// core/tiers/pinned.py:74-149, and of the copy / event calls of _StreamState, streaming/state.py:47-55,133-161,
// 239-256, in the reference).
//
// Pinned memory is allocated page-locked (hipHostMalloc) rather than registered after the fact; streams are
// created non-blocking at the default priority.
#include "wf_common.h"

#define WF_HIP(call, what)                                   \
    do {                                                     \
        hipError_t _e = (call);                              \
        if (_e != hipSuccess) return ::wf::hip_fail(_e, what); \
    } while (0)

extern "C" int wf_host_alloc(size_t nbytes, void** ptr) {
    if (!ptr) { wf::set_error("wf_host_alloc: null out-pointer"); return WF_EINVAL; }
    *ptr = nullptr;
    if (nbytes == 0) return WF_OK;
    WF_HIP(hipHostMalloc(ptr, nbytes, hipHostMallocDefault), "hipHostMalloc");
    return WF_OK;
}

extern "C" int wf_host_free(void* ptr) {
    if (!ptr) return WF_OK;
    WF_HIP(hipHostFree(ptr), "hipHostFree");
    return WF_OK;
}

extern "C" int wf_h2d_async(void* dst, const void* src, size_t nbytes, void* stream) {
    if (nbytes == 0) return WF_OK;
    if (!dst || !src) { wf::set_error("wf_h2d_async: null pointer"); return WF_EINVAL; }
    WF_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)),
           "hipMemcpyAsync");
    return WF_OK;
}

extern "C" int wf_stream_create(void** stream) {
    if (!stream) { wf::set_error("wf_stream_create: null out-pointer"); return WF_EINVAL; }
    hipStream_t s = nullptr;
    WF_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    *stream = s;
    return WF_OK;
}

extern "C" int wf_stream_destroy(void* stream) {
    if (!stream) return WF_OK;
    WF_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
    return WF_OK;
}

extern "C" int wf_stream_synchronize(void* stream) {
    WF_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
    return WF_OK;
}

extern "C" int wf_event_create(void** event, int timing) {
    if (!event) { wf::set_error("wf_event_create: null out-pointer"); return WF_EINVAL; }
    hipEvent_t e = nullptr;
    WF_HIP(hipEventCreateWithFlags(&e, timing ? hipEventDefault : hipEventDisableTiming), "hipEventCreateWithFlags");
    *event = e;
    return WF_OK;
}

extern "C" int wf_event_destroy(void* event) {
    if (!event) return WF_OK;
    WF_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
    return WF_OK;
}

extern "C" int wf_event_record(void* event, void* stream) {
    WF_HIP(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)), "hipEventRecord");
    return WF_OK;
}

extern "C" int wf_stream_wait_event(void* stream, void* event) {
    WF_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0),
           "hipStreamWaitEvent");
    return WF_OK;
}

// 0: the event's work has completed; 1: not yet; < 0: error
extern "C" int wf_event_query(void* event) {
    hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
    if (e == hipSuccess) return 0;
    if (e == hipErrorNotReady) return 1;
    return wf::hip_fail(e, "hipEventQuery");
}

extern "C" int wf_event_synchronize(void* event) {
    WF_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
    return WF_OK;
}

extern "C" int wf_event_elapsed_ms(void* start, void* end, float* ms) {
    if (!ms) { wf::set_error("wf_event_elapsed_ms: null out-pointer"); return WF_EINVAL; }
    WF_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
           "hipEventElapsedTime");
    return WF_OK;
}
