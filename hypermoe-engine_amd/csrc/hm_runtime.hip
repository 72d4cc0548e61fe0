// hm_runtime.hip -- device runtime half of the C ABI (ComputeBackend surface,
// src/backend/Backend.hpp:36-71): allocation, copies, streams, events.
// Streams are created with default priority and the non-blocking flag
// (the reference's CudaRuntime.cpp:114 uses cudaStreamNonBlocking).
#include "hm_device.h"

#include <string.h>

static thread_local int tl_last_hip_error = 0;
static thread_local hm_stage_timer tl_stage_timer = {nullptr, nullptr};

hm_stage_timer& hm_timer() { return tl_stage_timer; }

void hm_record_hip_error(hipError_t e) { tl_last_hip_error = static_cast<int>(e); }

extern "C" {

int hm_abi_version(void) { return HM_ABI_VERSION; }

const char* hm_status_string(int status) {
    switch (status) {
    case HM_OK: return "ok";
    case HM_ERR_INVALID: return "invalid argument";
    case HM_ERR_OVERFLOW: return "size overflow";
    case HM_ERR_RUNTIME: return "HIP runtime failure";
    case HM_ERR_UNSUPPORTED: return "unsupported configuration";
    default: return "unknown status";
    }
}

int hm_last_hip_error(void) { return tl_last_hip_error; }

int hm_device_count(int* count_out) {
    HM_REQUIRE(count_out);
    HM_HIP(hipGetDeviceCount(count_out));
    return HM_OK;
}

int hm_set_device(int ordinal) {
    HM_HIP(hipSetDevice(ordinal));
    return HM_OK;
}

int hm_device_alloc(void** ptr_out, size_t bytes) {
    HM_REQUIRE(ptr_out);
    *ptr_out = nullptr;
    if (bytes == 0) return HM_OK;
    HM_HIP(hipMalloc(ptr_out, bytes));
    return HM_OK;
}

int hm_device_free(void* ptr) {
    if (ptr) HM_HIP(hipFree(ptr));
    return HM_OK;
}

int hm_host_alloc(void** ptr_out, size_t bytes) {
    HM_REQUIRE(ptr_out);
    *ptr_out = nullptr;
    if (bytes == 0) return HM_OK;
    HM_HIP(hipHostMalloc(ptr_out, bytes, hipHostMallocDefault));
    return HM_OK;
}

int hm_host_free(void* ptr) {
    if (ptr) HM_HIP(hipHostFree(ptr));
    return HM_OK;
}

int hm_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return HM_OK;
    HM_REQUIRE(dst && src);
    HM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, hm_stream(stream)));
    return HM_OK;
}

int hm_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return HM_OK;
    HM_REQUIRE(dst && src);
    HM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, hm_stream(stream)));
    return HM_OK;
}

int hm_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return HM_OK;
    HM_REQUIRE(dst && src);
    HM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, hm_stream(stream)));
    return HM_OK;
}

int hm_stream_create(void** stream_out) {
    HM_REQUIRE(stream_out);
    hipStream_t s = nullptr;
    HM_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream_out = s;
    return HM_OK;
}

int hm_stream_destroy(void* stream) {
    if (stream) HM_HIP(hipStreamDestroy(hm_stream(stream)));
    return HM_OK;
}

int hm_stream_synchronize(void* stream) {
    HM_HIP(hipStreamSynchronize(hm_stream(stream)));
    return HM_OK;
}

int hm_event_create(void** event_out) {
    HM_REQUIRE(event_out);
    hipEvent_t e = nullptr;
    HM_HIP(hipEventCreate(&e));
    *event_out = e;
    return HM_OK;
}

int hm_event_destroy(void* event) {
    if (event) HM_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
    return HM_OK;
}

int hm_event_record(void* event, void* stream) {
    HM_REQUIRE(event);
    HM_HIP(hipEventRecord(static_cast<hipEvent_t>(event), hm_stream(stream)));
    return HM_OK;
}

int hm_event_synchronize(void* event) {
    HM_REQUIRE(event);
    HM_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)));
    return HM_OK;
}

int hm_stream_wait_event(void* stream, void* event) {
    HM_REQUIRE(event);
    HM_HIP(hipStreamWaitEvent(hm_stream(stream), static_cast<hipEvent_t>(event), 0));
    return HM_OK;
}

int hm_event_elapsed_ms(float* ms_out, void* start, void* stop) {
    HM_REQUIRE(ms_out && start && stop);
    HM_HIP(hipEventElapsedTime(ms_out, static_cast<hipEvent_t>(start),
                               static_cast<hipEvent_t>(stop)));
    return HM_OK;
}

int hm_mem_info(size_t* free_out, size_t* total_out) {
    HM_REQUIRE(free_out && total_out);
    HM_HIP(hipMemGetInfo(free_out, total_out));
    return HM_OK;
}

}  // extern "C"
