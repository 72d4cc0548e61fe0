// HipMoEAdapter.cpp -- see HipMoEAdapter.hpp.
#include "HipMoEAdapter.hpp"

#include <utility>

namespace hypermoe::backend::hip {

HipComputeBackend::HipComputeBackend(std::shared_ptr<hm::backend::HipBackend> hip)
    : hip_(std::move(hip)) {}

MemoryInfo HipComputeBackend::getMemoryInfo() const {
    const auto m = hip_->getMemoryInfo();
    return {m.totalBytes, m.freeBytes, m.allocatedBytes};
}

BackendStats HipComputeBackend::stats() const {
    const auto s = hip_->stats();
    return {s.allocatedBytes, s.peakAllocatedBytes, s.hostToDeviceBytes, s.deviceToHostBytes,
            s.synchronizationCount, s.transferTime, s.synchronizationTime};
}

}  // namespace hypermoe::backend::hip

namespace hypermoe::integration {

namespace {

hm::tensor::Device toHm(tensor::Device d) {
    return d.type == tensor::DeviceType::CPU ? hm::tensor::Device::cpu()
                                             : hm::tensor::Device::hip(d.ordinal);
}

tensor::Device toReference(hm::tensor::Device d) {
    if (d.type == hm::tensor::DeviceType::CPU) return tensor::Device::cpu();
    return {backend::hip::kHipDeviceType, d.ordinal};
}

}  // namespace

hm::tensor::TensorView toHm(tensor::TensorView view) {
    // DType numbering is the same on both sides (FP32 0, FP16 1, BF16 2,
    // INT8 3).  A read-only reference view (of a const tensor) becomes a
    // read-only hm view; the caller's tensor keeps owning the storage.
    auto t = hm::tensor::Tensor::fromStorage(
        hm::tensor::Shape(view.shape().dimensions()), static_cast<hm::tensor::DType>(view.dtype()),
        toHm(view.device()), const_cast<void*>(view.data()), view.storageBytes(), view.lockOwner());
    if (view.mutableData() != nullptr) return hm::tensor::TensorView(t);
    return hm::tensor::TensorView(static_cast<const hm::tensor::Tensor&>(t));
}

tensor::Tensor toReference(const hm::tensor::Tensor& t) {
    if (!t.valid()) return {};
    return tensor::Tensor::fromStorage(tensor::Shape(t.shape().dimensions()),
                                       static_cast<tensor::DType>(t.dtype()),
                                       toReference(t.device()), const_cast<void*>(t.data()),
                                       t.storageBytes(), t.owner());
}

runtime::BatchLayerExecutionResult toReference(hm::BatchLayerExecutionResult r) {
    runtime::BatchLayerExecutionResult out;
    out.routing.layerId = r.routing.layerId;
    out.routing.tokens.reserve(r.routing.tokens.size());
    for (auto& d : r.routing.tokens)
        out.routing.tokens.push_back({d.layerId, std::move(d.selectedExpertIds), std::move(d.routingScores)});
    out.routing.expertGroups.reserve(r.routing.expertGroups.size());
    for (auto& g : r.routing.expertGroups)
        out.routing.expertGroups.push_back({g.expertId, std::move(g.tokenIndices), std::move(g.routingScores)});
    out.expertBatches.reserve(r.expertBatches.size());
    for (auto& b : r.expertBatches)
        out.expertBatches.push_back({b.layerId, b.expertId, std::move(b.tokenIndices), std::move(b.routingWeights)});
    out.expertOutputs.reserve(r.expertOutputs.size());
    for (const auto& t : r.expertOutputs) out.expertOutputs.push_back(toReference(t));
    out.output = toReference(r.output);
    const auto& e = r.execution;
    out.execution = {e.expertAssignments, e.uniqueExperts, e.expertCacheHits, e.expertCacheMisses,
                     e.expertPayloadBytes, e.expertTransferBytes, std::move(r.execution.tensorBackend),
                     e.routingTime, e.schedulingTime, e.expertExecutionTime, e.expertCombinationTime};
    return out;
}

}  // namespace hypermoe::integration
