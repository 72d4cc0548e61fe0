// hip_backend.cpp -- HipBackend: the ComputeBackend surface
// (src/backend/Backend.hpp:36-71) for one MI355X over the hm_* C ABI.
#include "hm_backend.hpp"
#include "hm_moe.h"

#include <algorithm>
#include <stdexcept>
#include <string>
#include <utility>

namespace hm::backend {

void throwOnStatus(int status, std::string_view operation) {
    if (status == HM_OK) return;
    std::string msg(operation);
    msg += ": ";
    msg += hm_status_string(status);
    const int hip = hm_last_hip_error();
    if (hip != 0) msg += " (hipError " + std::to_string(hip) + ")";
    switch (status) {
    case HM_ERR_INVALID: throw std::invalid_argument(msg);
    case HM_ERR_OVERFLOW: throw std::overflow_error(msg);
    default: throw std::runtime_error(msg);
    }
}

// ---- DeviceBuffer (src/backend/Backend.cpp:1-80 semantics) ----------------

DeviceBuffer::DeviceBuffer(std::shared_ptr<ComputeBackend> backend, std::size_t sizeBytes)
    : backend_(std::move(backend)), size_(sizeBytes) {
    if (!backend_) throw std::invalid_argument("device buffer requires a backend");
    data_ = backend_->allocate(sizeBytes);
}

DeviceBuffer::DeviceBuffer(std::shared_ptr<ComputeBackend> backend, void* data,
                           std::size_t sizeBytes, std::function<void(void*)> releaser)
    : backend_(std::move(backend)), data_(data), size_(sizeBytes), releaser_(std::move(releaser)) {}

DeviceBuffer::~DeviceBuffer() { reset(); }

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : backend_(std::move(other.backend_)),
      data_(std::exchange(other.data_, nullptr)),
      size_(std::exchange(other.size_, 0)),
      releaser_(std::move(other.releaser_)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
        reset();
        backend_ = std::move(other.backend_);
        data_ = std::exchange(other.data_, nullptr);
        size_ = std::exchange(other.size_, 0);
        releaser_ = std::move(other.releaser_);
    }
    return *this;
}

void DeviceBuffer::reset() noexcept {
    if (data_ != nullptr) {
        if (releaser_) releaser_(data_);
        else if (backend_) backend_->free(data_);
    }
    data_ = nullptr;
    size_ = 0;
    backend_.reset();
    releaser_ = {};
}

// ---- HipBackend -------------------------------------------------------------

HipBackend::HipBackend(int ordinal) : ordinal_(ordinal) {
    if (ordinal < 0) throw std::invalid_argument("HIP device ordinal must be non-negative");
    int count = 0;
    if (hm_device_count(&count) != HM_OK || ordinal >= count) {
        available_ = false;  // no device: every device call throws
        return;
    }
    throwOnStatus(hm_set_device(ordinal_), "HIP set device");
    void* stream = nullptr;
    throwOnStatus(hm_stream_create(&stream), "HIP compute stream");
    compute_ = stream;
    available_ = true;
}

HipBackend::~HipBackend() {
    if (!available_) return;
    makeCurrent();
    (void)hm_stream_synchronize(compute_);
    std::scoped_lock lock(mutex_);
    for (const auto& [p, n] : allocations_) {
        (void)n;
        (void)hm_device_free(p);
    }
    for (const auto& [p, n] : pinned_) {
        (void)n;
        (void)hm_host_free(p);
    }
    (void)hm_stream_destroy(compute_);
}

void HipBackend::requireAvailable(std::string_view operation) const {
    if (!available_) {
        throw std::runtime_error(std::string(operation) + ": no HIP device is available");
    }
}

void HipBackend::makeCurrent() const { (void)hm_set_device(ordinal_); }

void* HipBackend::allocate(std::size_t sizeBytes) {
    if (sizeBytes == 0) throw std::invalid_argument("HIP allocation size must be nonzero");
    requireAvailable("HIP allocate");
    makeCurrent();
    void* p = nullptr;
    throwOnStatus(hm_device_alloc(&p, sizeBytes), "HIP allocate");
    std::scoped_lock lock(mutex_);
    allocations_.emplace(p, sizeBytes);
    stats_.allocatedBytes += sizeBytes;
    stats_.peakAllocatedBytes = std::max(stats_.peakAllocatedBytes, stats_.allocatedBytes);
    return p;
}

void HipBackend::free(void* pointer) noexcept {
    if (pointer == nullptr) return;
    {
        std::scoped_lock lock(mutex_);
        const auto it = allocations_.find(pointer);
        if (it == allocations_.end()) return;
        stats_.allocatedBytes -= it->second;
        allocations_.erase(it);
    }
    makeCurrent();
    (void)hm_device_free(pointer);
}

void HipBackend::recordTransfer(std::size_t bytes, bool toDevice,
                                std::chrono::nanoseconds elapsed) {
    std::scoped_lock lock(mutex_);
    if (toDevice) stats_.hostToDeviceBytes += bytes;
    else stats_.deviceToHostBytes += bytes;
    stats_.transferTime += elapsed;
}

void HipBackend::copyToDevice(void* destination, const void* source, std::size_t sizeBytes,
                              StreamHandle stream) {
    if (sizeBytes == 0) return;
    if (destination == nullptr || source == nullptr) {
        throw std::invalid_argument("HIP copy received a null pointer");
    }
    requireAvailable("HIP copy to device");
    makeCurrent();
    const auto start = std::chrono::steady_clock::now();
    throwOnStatus(hm_memcpy_h2d(destination, source, sizeBytes, stream), "HIP copy to device");
    if (stream == nullptr) throwOnStatus(hm_stream_synchronize(nullptr), "HIP copy to device");
    recordTransfer(sizeBytes, true, std::chrono::steady_clock::now() - start);
}

void HipBackend::copyFromDevice(void* destination, const void* source, std::size_t sizeBytes,
                                StreamHandle stream) {
    if (sizeBytes == 0) return;
    if (destination == nullptr || source == nullptr) {
        throw std::invalid_argument("HIP copy received a null pointer");
    }
    requireAvailable("HIP copy from device");
    makeCurrent();
    const auto start = std::chrono::steady_clock::now();
    throwOnStatus(hm_memcpy_d2h(destination, source, sizeBytes, stream), "HIP copy from device");
    if (stream == nullptr) throwOnStatus(hm_stream_synchronize(nullptr), "HIP copy from device");
    recordTransfer(sizeBytes, false, std::chrono::steady_clock::now() - start);
}

void HipBackend::copyOnDevice(void* destination, const void* source, std::size_t sizeBytes,
                              StreamHandle stream) {
    if (sizeBytes == 0) return;
    if (destination == nullptr || source == nullptr) {
        throw std::invalid_argument("HIP copy received a null pointer");
    }
    requireAvailable("HIP device copy");
    makeCurrent();
    throwOnStatus(hm_memcpy_d2d(destination, source, sizeBytes, stream), "HIP device copy");
    if (stream == nullptr) throwOnStatus(hm_stream_synchronize(nullptr), "HIP device copy");
}

void HipBackend::synchronize(StreamHandle stream) {
    requireAvailable("HIP synchronize");
    makeCurrent();
    const auto start = std::chrono::steady_clock::now();
    if (stream == nullptr) {
        // the whole engine: the compute stream and the null stream
        throwOnStatus(hm_stream_synchronize(compute_), "HIP synchronize");
        throwOnStatus(hm_stream_synchronize(nullptr), "HIP synchronize");
    } else {
        throwOnStatus(hm_stream_synchronize(stream), "HIP synchronize");
    }
    std::scoped_lock lock(mutex_);
    ++stats_.synchronizationCount;
    stats_.synchronizationTime += std::chrono::steady_clock::now() - start;
}

MemoryInfo HipBackend::getMemoryInfo() const {
    MemoryInfo info;
    {
        std::scoped_lock lock(mutex_);
        info.allocatedBytes = stats_.allocatedBytes;
    }
    if (!available_) return info;
    makeCurrent();
    std::size_t freeBytes = 0, totalBytes = 0;
    throwOnStatus(hm_mem_info(&freeBytes, &totalBytes), "HIP memory info");
    info.freeBytes = freeBytes;
    info.totalBytes = totalBytes;
    return info;
}

BackendStats HipBackend::stats() const {
    std::scoped_lock lock(mutex_);
    return stats_;
}

StreamHandle HipBackend::createStream() {
    requireAvailable("HIP create stream");
    makeCurrent();
    void* s = nullptr;
    throwOnStatus(hm_stream_create(&s), "HIP create stream");
    return s;
}

void HipBackend::destroyStream(StreamHandle stream) noexcept {
    if (stream != nullptr && stream != compute_) (void)hm_stream_destroy(stream);
}

EventHandle HipBackend::createEvent() {
    requireAvailable("HIP create event");
    makeCurrent();
    void* e = nullptr;
    throwOnStatus(hm_event_create(&e), "HIP create event");
    return e;
}

void HipBackend::recordEvent(EventHandle event, StreamHandle stream) {
    if (event == nullptr) throw std::invalid_argument("HIP record event: null event");
    throwOnStatus(hm_event_record(event, stream), "HIP record event");
}

void HipBackend::waitEvent(EventHandle event) {
    if (event == nullptr) throw std::invalid_argument("HIP wait event: null event");
    throwOnStatus(hm_event_synchronize(event), "HIP wait event");
}

void HipBackend::destroyEvent(EventHandle event) noexcept {
    if (event != nullptr) (void)hm_event_destroy(event);
}

void* HipBackend::allocatePinned(std::size_t sizeBytes) {
    if (sizeBytes == 0) throw std::invalid_argument("pinned allocation size must be nonzero");
    requireAvailable("HIP pinned allocate");
    makeCurrent();
    void* p = nullptr;
    throwOnStatus(hm_host_alloc(&p, sizeBytes), "HIP pinned allocate");
    std::scoped_lock lock(mutex_);
    pinned_.emplace(p, sizeBytes);
    return p;
}

void HipBackend::freePinned(void* pointer) noexcept {
    if (pointer == nullptr) return;
    {
        std::scoped_lock lock(mutex_);
        if (pinned_.erase(pointer) == 0) return;
    }
    (void)hm_host_free(pointer);
}

}  // namespace hm::backend
