// hm_backend.hpp -- C++20 device backend over the HIP C ABI (hm_moe.h).
//
// The ComputeBackend surface of the reference (src/backend/Backend.hpp:36-71,
// modelled on CpuBackend, src/backend/CpuBackend.cpp:21-116), implemented
// for one MI355X by HipBackend.  The interface is kept member for member so
// code written against the reference's backend compiles against this one;
// the implementation is this engine's own and reaches HIP only through the
// hm_* C functions.
//
// Errors follow the reference's categories: std::invalid_argument for bad
// arguments, std::overflow_error for size arithmetic, std::runtime_error for
// device failures (the HIP error code is in the message).
#pragma once

#include <chrono>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <string_view>
#include <unordered_map>

namespace hm::backend {

using StreamHandle = void*;  // hipStream_t
using EventHandle = void*;   // hipEvent_t

enum class BackendKind {
    Cpu,
    Hip,
};

struct MemoryInfo {
    std::uint64_t totalBytes{};
    std::uint64_t freeBytes{};
    std::uint64_t allocatedBytes{};
};

struct BackendStats {
    std::uint64_t allocatedBytes{};
    std::uint64_t peakAllocatedBytes{};
    std::uint64_t hostToDeviceBytes{};
    std::uint64_t deviceToHostBytes{};
    std::uint64_t synchronizationCount{};
    std::chrono::nanoseconds transferTime{};
    std::chrono::nanoseconds synchronizationTime{};
};

class ComputeBackend {
public:
    virtual ~ComputeBackend() = default;

    [[nodiscard]] virtual BackendKind kind() const noexcept = 0;
    [[nodiscard]] virtual std::string_view name() const noexcept = 0;
    [[nodiscard]] virtual int deviceOrdinal() const noexcept = 0;
    [[nodiscard]] virtual bool isAvailable() const noexcept = 0;

    [[nodiscard]] virtual void* allocate(std::size_t sizeBytes) = 0;
    virtual void free(void* pointer) noexcept = 0;

    virtual void copyToDevice(void* destination, const void* source, std::size_t sizeBytes,
                              StreamHandle stream = nullptr) = 0;
    virtual void copyFromDevice(void* destination, const void* source, std::size_t sizeBytes,
                                StreamHandle stream = nullptr) = 0;
    virtual void synchronize(StreamHandle stream = nullptr) = 0;

    [[nodiscard]] virtual MemoryInfo getMemoryInfo() const = 0;
    [[nodiscard]] virtual BackendStats stats() const = 0;

    [[nodiscard]] virtual StreamHandle createStream() = 0;
    virtual void destroyStream(StreamHandle stream) noexcept = 0;
    [[nodiscard]] virtual EventHandle createEvent() = 0;
    virtual void recordEvent(EventHandle event, StreamHandle stream) = 0;
    virtual void waitEvent(EventHandle event) = 0;
    virtual void destroyEvent(EventHandle event) noexcept = 0;

    [[nodiscard]] virtual void* allocatePinned(std::size_t sizeBytes) = 0;
    virtual void freePinned(void* pointer) noexcept = 0;
    [[nodiscard]] virtual bool supportsPinnedMemory() const noexcept = 0;
};

// Owning handle of one allocation (src/backend/Backend.hpp:73-100): freed
// through its backend, or through a custom releaser.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(std::shared_ptr<ComputeBackend> backend, std::size_t sizeBytes);
    DeviceBuffer(std::shared_ptr<ComputeBackend> backend, void* data, std::size_t sizeBytes,
                 std::function<void(void*)> releaser);
    ~DeviceBuffer();

    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;

    void reset() noexcept;
    [[nodiscard]] void* data() noexcept { return data_; }
    [[nodiscard]] const void* data() const noexcept { return data_; }
    [[nodiscard]] std::size_t size() const noexcept { return size_; }
    [[nodiscard]] explicit operator bool() const noexcept { return data_ != nullptr; }
    [[nodiscard]] const std::shared_ptr<ComputeBackend>& backend() const noexcept {
        return backend_;
    }

private:
    std::shared_ptr<ComputeBackend> backend_;
    void* data_{};
    std::size_t size_{};
    std::function<void(void*)> releaser_;
};

// Throws the reference's exception category for a non-zero hm_status.
void throwOnStatus(int status, std::string_view operation);

// One MI355X.  Owns a compute stream (default priority) on which the tensor
// backend and the MoE block launch; copies with a null stream are
// synchronous.  isAvailable() is false on a machine without a HIP device,
// and every device call then throws std::runtime_error.  Thread-safe.
class HipBackend final : public ComputeBackend {
public:
    explicit HipBackend(int ordinal = 0);
    ~HipBackend() override;
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;

    [[nodiscard]] BackendKind kind() const noexcept override { return BackendKind::Hip; }
    [[nodiscard]] std::string_view name() const noexcept override { return "HIP (gfx950)"; }
    [[nodiscard]] int deviceOrdinal() const noexcept override { return ordinal_; }
    [[nodiscard]] bool isAvailable() const noexcept override { return available_; }

    [[nodiscard]] void* allocate(std::size_t sizeBytes) override;
    void free(void* pointer) noexcept override;
    void copyToDevice(void* destination, const void* source, std::size_t sizeBytes,
                      StreamHandle stream = nullptr) override;
    void copyFromDevice(void* destination, const void* source, std::size_t sizeBytes,
                        StreamHandle stream = nullptr) override;
    void synchronize(StreamHandle stream = nullptr) override;

    [[nodiscard]] MemoryInfo getMemoryInfo() const override;
    [[nodiscard]] BackendStats stats() const override;

    [[nodiscard]] StreamHandle createStream() override;
    void destroyStream(StreamHandle stream) noexcept override;
    [[nodiscard]] EventHandle createEvent() override;
    void recordEvent(EventHandle event, StreamHandle stream) override;
    void waitEvent(EventHandle event) override;
    void destroyEvent(EventHandle event) noexcept override;

    [[nodiscard]] void* allocatePinned(std::size_t sizeBytes) override;
    void freePinned(void* pointer) noexcept override;
    [[nodiscard]] bool supportsPinnedMemory() const noexcept override { return available_; }

    // Device-to-device copy on `stream` (asynchronous unless stream is null).
    void copyOnDevice(void* destination, const void* source, std::size_t sizeBytes,
                      StreamHandle stream = nullptr);
    // The stream every launch of this engine goes to.
    [[nodiscard]] StreamHandle computeStream() const noexcept { return compute_; }

private:
    void requireAvailable(std::string_view operation) const;
    void makeCurrent() const;
    void recordTransfer(std::size_t bytes, bool toDevice, std::chrono::nanoseconds elapsed);

    int ordinal_{};
    bool available_{};
    StreamHandle compute_{};
    mutable std::mutex mutex_;
    std::unordered_map<void*, std::size_t> allocations_;
    std::unordered_map<void*, std::size_t> pinned_;
    BackendStats stats_;
};

}  // namespace hm::backend
