// HipMoEAdapter.hpp -- the reference-side glue of the MI355X MoE block.
//
// Compiled inside the reference tree (src/backend/hip/HipMoEAdapter.cpp
// with HYPERMOE_HAS_HIP), against the reference's headers and this build's
// include/ directory; links libhm_host.so.  It gives the reference:
//   - HipComputeBackend, a hypermoe::backend::ComputeBackend
//     (src/backend/Backend.hpp:36-71) that forwards every call to
//     hm::backend::HipBackend;
//   - toHm: a reference TensorView as an hm TensorView of the same storage
//     (the caller's tensor keeps owning it);
//   - toReference: an hm tensor, or a whole hm::BatchLayerExecutionResult,
//     as the reference's (src/core/runtime/MoERuntime.hpp:33-39), member by
//     member; tensors keep their hm owner through the shared_ptr<void>.
// The reference's DeviceType and BackendKind have CPU/Cuda only; the
// integration adds HIP = 2 to both (and to tensor::isValid), which device
// tensors need.  Host (CPU) tensors convert with the headers unchanged.
#pragma once

#include "backend/Backend.hpp"
#include "runtime/MoERuntime.hpp"
#include "tensor/Tensor.hpp"
#include "tensor/TensorView.hpp"

#include "hm_backend.hpp"
#include "hm_moe_block.hpp"
#include "hm_tensor.hpp"

#include <memory>

namespace hypermoe::backend::hip {

// the enumerator values the integration adds
inline constexpr auto kHipBackendKind = static_cast<BackendKind>(2);
inline constexpr auto kHipDeviceType = static_cast<tensor::DeviceType>(2);

class HipComputeBackend final : public ComputeBackend {
public:
    explicit HipComputeBackend(std::shared_ptr<hm::backend::HipBackend> hip);

    [[nodiscard]] BackendKind kind() const noexcept override { return kHipBackendKind; }
    [[nodiscard]] std::string_view name() const noexcept override { return hip_->name(); }
    [[nodiscard]] int deviceOrdinal() const noexcept override { return hip_->deviceOrdinal(); }
    [[nodiscard]] bool isAvailable() const noexcept override { return hip_->isAvailable(); }

    [[nodiscard]] void* allocate(std::size_t sizeBytes) override { return hip_->allocate(sizeBytes); }
    void free(void* pointer) noexcept override { hip_->free(pointer); }
    void copyToDevice(void* destination, const void* source, std::size_t sizeBytes,
                      StreamHandle stream = nullptr) override {
        hip_->copyToDevice(destination, source, sizeBytes, stream);
    }
    void copyFromDevice(void* destination, const void* source, std::size_t sizeBytes,
                        StreamHandle stream = nullptr) override {
        hip_->copyFromDevice(destination, source, sizeBytes, stream);
    }
    void synchronize(StreamHandle stream = nullptr) override { hip_->synchronize(stream); }

    [[nodiscard]] MemoryInfo getMemoryInfo() const override;
    [[nodiscard]] BackendStats stats() const override;

    [[nodiscard]] StreamHandle createStream() override { return hip_->createStream(); }
    void destroyStream(StreamHandle stream) noexcept override { hip_->destroyStream(stream); }
    [[nodiscard]] EventHandle createEvent() override { return hip_->createEvent(); }
    void recordEvent(EventHandle event, StreamHandle stream) override { hip_->recordEvent(event, stream); }
    void waitEvent(EventHandle event) override { hip_->waitEvent(event); }
    void destroyEvent(EventHandle event) noexcept override { hip_->destroyEvent(event); }

    [[nodiscard]] void* allocatePinned(std::size_t sizeBytes) override { return hip_->allocatePinned(sizeBytes); }
    void freePinned(void* pointer) noexcept override { hip_->freePinned(pointer); }
    [[nodiscard]] bool supportsPinnedMemory() const noexcept override { return hip_->supportsPinnedMemory(); }

    [[nodiscard]] const std::shared_ptr<hm::backend::HipBackend>& hip() const noexcept { return hip_; }

private:
    std::shared_ptr<hm::backend::HipBackend> hip_;
};

}  // namespace hypermoe::backend::hip

namespace hypermoe::integration {

[[nodiscard]] hm::tensor::TensorView toHm(tensor::TensorView view);
[[nodiscard]] tensor::Tensor toReference(const hm::tensor::Tensor& t);
[[nodiscard]] runtime::BatchLayerExecutionResult toReference(hm::BatchLayerExecutionResult r);

}  // namespace hypermoe::integration
