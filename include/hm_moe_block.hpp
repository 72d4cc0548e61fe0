// hm_moe_block.hpp -- the device-resident MoE block behind the reference's
// block entry.
//
// HipMoEBlock::executeBatch keeps the signature and result shape of
// MoERuntime::executeBatch (src/core/runtime/MoERuntime.hpp:57-60) and
// BatchLayerExecutionResult (MoERuntime.hpp:33-39); the routing types follow
// src/router/RouterDecision.hpp:10-43 and src/router/RouterConfig.hpp:22-29,
// ExpertBatch src/experts/ExpertBatch.hpp:10-18, ExecutionMetadata
// src/runtime/InferenceContext.hpp:13-25.  One call is one launch sequence
// on the backend's compute stream (hm_moe_block_forward: route -> permute ->
// grouped SwiGLU experts -> combine); the routing metadata comes back through
// pinned memory once the stream reaches it (launchBatch returns before that,
// executeBatch waits for it).  All experts of a layer stay
// resident in HBM (DeviceExpertLayer), so the reference's scheduler, leases
// and residency tiers have no counterpart here.
#pragma once

#include "hm_backend.hpp"
#include "hm_tensor.hpp"

#include <array>
#include <chrono>
#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <span>
#include <string>
#include <vector>

struct hm_layer;

namespace hm {

using LayerId = std::uint32_t;
using ExpertId = std::uint32_t;

namespace router {

enum class RoutingNormalization {
    None,
    Softmax,
};

struct RouterConfig {
    std::size_t expertCount{};
    std::size_t topK{1};
    RoutingNormalization normalization{RoutingNormalization::Softmax};
    bool renormalizeSelected{};

    // RouterConfig::validate: 0 < topK <= expertCount.
    void validate() const;
};

struct RouterDecision {
    LayerId layerId{};
    std::vector<ExpertId> selectedExpertIds;
    std::vector<float> routingScores;

    [[nodiscard]] bool valid() const noexcept {
        return !selectedExpertIds.empty() && selectedExpertIds.size() == routingScores.size();
    }
};

struct ExpertTokenGroup {
    ExpertId expertId{};
    std::vector<std::size_t> tokenIndices;
    std::vector<float> routingScores;
};

struct BatchRouterDecision {
    LayerId layerId{};
    std::vector<RouterDecision> tokens;
    std::vector<ExpertTokenGroup> expertGroups;

    [[nodiscard]] bool valid() const noexcept;
};

}  // namespace router

struct ExpertBatch {
    LayerId layerId{};
    ExpertId expertId{};
    std::vector<std::size_t> tokenIndices;
    std::vector<float> routingWeights;

    // ExpertBatch::validate (src/experts/ExpertBatch.cpp:9-22).
    void validate(std::size_t tokenCount) const;
    [[nodiscard]] std::size_t size() const noexcept { return tokenIndices.size(); }
};

namespace runtime {

struct ExecutionMetadata {
    std::size_t expertAssignments{};
    std::size_t uniqueExperts{};
    std::size_t expertCacheHits{};    // every selected expert is resident: = uniqueExperts
    std::size_t expertCacheMisses{};  // always 0
    std::uint64_t expertPayloadBytes{};
    std::uint64_t expertTransferBytes{};  // always 0: nothing moves per call
    std::string tensorBackend;
    // Device time between the stage events of the launch sequence.
    std::chrono::nanoseconds routingTime{};           // router
    std::chrono::nanoseconds schedulingTime{};        // permute + activation digits
    std::chrono::nanoseconds expertExecutionTime{};   // gate/up + down GEMMs
    std::chrono::nanoseconds expertCombinationTime{}; // weighted combine
};

struct BatchLayerExecutionResult {
    router::BatchRouterDecision routing;
    std::vector<ExpertBatch> expertBatches;
    // One [n_e x H] FP32 device tensor per expert batch, in batch order
    // (views into one grouped buffer), or empty when the block was built
    // with keepExpertOutputs = false.
    std::vector<tensor::Tensor> expertOutputs;
    tensor::Tensor output;  // [T x H] FP32 on the device
    ExecutionMetadata execution;
};

}  // namespace runtime

using runtime::BatchLayerExecutionResult;
using runtime::ExecutionMetadata;

// Per-projection affine INT8 parameters of one expert.
struct ExpertQuantization {
    tensor::quantization::QuantizationParameters gate, up, down;
};

// One layer's experts resident in HBM in the kernels' layout.  Built from the
// reference's packed payload: per expert gate [H x I] | up [H x I] |
// down [I x H], row-major (ExpertPacker.cpp:228-230), INT8 with one
// {scale, zero point} per projection, or FP32.
class DeviceExpertLayer {
public:
    static std::shared_ptr<DeviceExpertLayer> fromPayload(
        std::shared_ptr<backend::HipBackend> backend, std::span<const std::byte> payload,
        std::size_t experts, std::size_t hidden, std::size_t intermediate, tensor::DType dtype,
        std::span<const ExpertQuantization> quantization = {});
    ~DeviceExpertLayer();

    [[nodiscard]] std::size_t experts() const noexcept { return experts_; }
    [[nodiscard]] std::size_t hidden() const noexcept { return hidden_; }
    [[nodiscard]] std::size_t intermediate() const noexcept { return intermediate_; }
    [[nodiscard]] tensor::DType dtype() const noexcept { return dtype_; }
    [[nodiscard]] std::uint64_t expertBytes() const noexcept;
    [[nodiscard]] const hm_layer& descriptor() const noexcept { return *desc_; }

private:
    DeviceExpertLayer() = default;
    std::shared_ptr<backend::HipBackend> backend_;
    std::size_t experts_{}, hidden_{}, intermediate_{};
    tensor::DType dtype_{tensor::DType::INT8};
    std::unique_ptr<backend::DeviceBuffer> packed_, scale_, zeroPoint_;
    std::unique_ptr<hm_layer> desc_;
};

struct BlockOptions {
    // Digit planes of the INT8 path's activations (gate/up input, down
    // input).  2 keeps the FP32 result within 1e-4 of the W8A32 reference;
    // 3 within 1e-5.
    int limbsX{2};
    int limbsZ{3};
    // Run the INT8 expert GEMMs on the scalar kernels (same integers and
    // float operations as the MFMA kernels; for pinning them).
    bool genericKernels{false};
    // Return per-expert outputs (BatchLayerExecutionResult::expertOutputs).
    bool keepExpertOutputs{true};
};

class HipMoEBlock;

// The result of HipMoEBlock::launchBatch while its work is queued: the
// combined output is a device tensor that work on the backend's compute
// stream may use at once; get() waits for the call's routing metadata
// (copied to pinned host memory behind the kernels) and builds the
// reference-shaped result.  The block must outlive its pending results.
// Movable, not copyable; dropping one without get() is allowed.
class PendingBatchResult {
public:
    PendingBatchResult(PendingBatchResult&& other) noexcept;
    PendingBatchResult& operator=(PendingBatchResult&&) = delete;
    PendingBatchResult(const PendingBatchResult&) = delete;
    ~PendingBatchResult();

    // [T x H] FP32 on the device (ordered after the call on the compute stream).
    [[nodiscard]] const tensor::Tensor& output() const noexcept { return output_; }
    // Waits for the call and returns the result executeBatch returns (the
    // output tensor moves into it); the routing checks and exceptions are
    // executeBatch's.  Once only.
    [[nodiscard]] BatchLayerExecutionResult get();

private:
    friend class HipMoEBlock;
    PendingBatchResult() = default;
    HipMoEBlock* block_{};
    void* slot_{};  // the block's staging slot of this call
    LayerId layerId_{};
    std::size_t tokens_{}, hidden_{}, topK_{}, experts_{};
    std::uint64_t expertBytes_{};
    tensor::Tensor output_;
    std::shared_ptr<backend::DeviceBuffer> expertOut_;
};

class HipMoEBlock {
public:
    HipMoEBlock(std::shared_ptr<backend::HipBackend> backend, router::RouterConfig config,
                BlockOptions options = {});
    ~HipMoEBlock();
    HipMoEBlock(const HipMoEBlock&) = delete;
    HipMoEBlock& operator=(const HipMoEBlock&) = delete;

    void addLayer(LayerId layerId, std::shared_ptr<const DeviceExpertLayer> layer);

    // MoERuntime::executeBatch: hiddenStates [T x H] and routerWeights
    // [H x E], FP32 tensors on this backend's device.  Serialised per block
    // (the reference's executionMutex_).  Equal to launchBatch(...).get().
    [[nodiscard]] BatchLayerExecutionResult executeBatch(LayerId layerId,
                                                         tensor::TensorView hiddenStates,
                                                         tensor::TensorView routerWeights);
    // The same with the residual of TransformerBlock::execute
    // (TransformerBlock.cpp:88-104): output = residual + MoE(hiddenStates).
    [[nodiscard]] BatchLayerExecutionResult executeBatch(LayerId layerId,
                                                         tensor::TensorView hiddenStates,
                                                         tensor::TensorView routerWeights,
                                                         tensor::TensorView residual);

    // The same call without waiting for it: the kernels and the routing
    // metadata's copies to pinned memory are queued on the compute stream
    // and nothing here synchronises with the device.  The reference's block
    // entry blocks on its routing read-back (CudaTensorBackend.cpp:636-640);
    // a caller that needs the routing only later (or never) keeps the
    // stream full instead.  Output buffers of calls whose results were
    // released are reused by later calls of the same shape.
    [[nodiscard]] PendingBatchResult launchBatch(LayerId layerId, tensor::TensorView hiddenStates,
                                                 tensor::TensorView routerWeights,
                                                 tensor::TensorView residual = {});

    [[nodiscard]] const router::RouterConfig& config() const noexcept { return config_; }

private:
    friend class PendingBatchResult;
    struct Staging;
    Staging* acquireSlot(std::size_t pairs, std::size_t experts);
    void releaseSlot(Staging* slot) noexcept;
    std::shared_ptr<backend::DeviceBuffer> outputBuffer(
        std::vector<std::shared_ptr<backend::DeviceBuffer>>& pool, std::size_t bytes);
    BatchLayerExecutionResult materialize(PendingBatchResult& pending);

    std::shared_ptr<backend::HipBackend> backend_;
    router::RouterConfig config_;
    BlockOptions options_;
    std::map<LayerId, std::shared_ptr<const DeviceExpertLayer>> layers_;
    std::mutex executionMutex_;
    std::unique_ptr<backend::DeviceBuffer> workspace_;
    // staging slots (device routing arrays, pinned copies, events), one per
    // call in flight, and the released output buffers kept for reuse
    std::mutex poolMutex_;
    std::vector<std::unique_ptr<Staging>> slots_;
    std::vector<std::shared_ptr<backend::DeviceBuffer>> outPool_, expertOutPool_;
};

}  // namespace hm
