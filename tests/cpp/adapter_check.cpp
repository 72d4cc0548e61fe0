// Drop-in check of the reference-side adapter (hypermoe-engine_amd/integration):
// compiled against the reference's own headers and sources (Tensor, Shape,
// TensorView) where the reference tree is mounted, linked with libhm_host.so.
// An hm::BatchLayerExecutionResult built on the host goes through toReference
// into the reference's hypermoe::runtime::BatchLayerExecutionResult
// (src/core/runtime/MoERuntime.hpp:33-39) and every member is compared; a
// reference TensorView goes through toHm; HipComputeBackend is used through
// the reference's ComputeBackend interface (src/backend/Backend.hpp:36-71).
#include "HipMoEAdapter.hpp"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <vector>

#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            std::fprintf(stderr, "adapter check failed: %s (line %d)\n", #c, __LINE__); \
            std::exit(1);                                                     \
        }                                                                     \
    } while (0)

namespace {

hm::tensor::Tensor host_tensor(std::size_t rows, std::size_t cols, float base) {
    auto store = std::make_shared<std::vector<float>>(rows * cols);
    for (std::size_t i = 0; i < store->size(); ++i) (*store)[i] = base + (float)i;
    return hm::tensor::Tensor::fromStorage(hm::tensor::Shape({rows, cols}), hm::tensor::DType::FP32,
                                           hm::tensor::Device::cpu(), store->data(),
                                           store->size() * sizeof(float), store);
}

void same_tensor(const hypermoe::tensor::Tensor& r, const hm::tensor::Tensor& h) {
    CHECK(r.valid());
    CHECK(r.shape().dimensions() == h.shape().dimensions());
    CHECK(static_cast<unsigned>(r.dtype()) == static_cast<unsigned>(h.dtype()));
    CHECK(r.device().type == hypermoe::tensor::DeviceType::CPU);
    CHECK(r.data() == h.data());
    CHECK(r.storageBytes() == h.storageBytes());
}

}  // namespace

int main() {
    // ---- an hm result as the block returns it (host tensors here)
    hm::BatchLayerExecutionResult h;
    h.routing.layerId = 7;
    h.routing.tokens = {{7, {3, 1}, {0.6f, 0.4f}}, {7, {1, 5}, {0.7f, 0.3f}}};
    h.routing.expertGroups = {{1, {0, 1}, {0.4f, 0.7f}}, {3, {0}, {0.6f}}, {5, {1}, {0.3f}}};
    h.expertBatches = {{7, 1, {0, 1}, {0.4f, 0.7f}}, {7, 3, {0}, {0.6f}}, {7, 5, {1}, {0.3f}}};
    for (std::size_t b = 0; b < 3; ++b)
        h.expertOutputs.push_back(host_tensor(h.expertBatches[b].size(), 4, 10.0f * (float)b));
    h.output = host_tensor(2, 4, 100.0f);
    h.execution.expertAssignments = 4;
    h.execution.uniqueExperts = 3;
    h.execution.expertCacheHits = 3;
    h.execution.expertPayloadBytes = 12345;
    h.execution.tensorBackend = "hip";
    h.execution.routingTime = std::chrono::nanoseconds(11);
    h.execution.schedulingTime = std::chrono::nanoseconds(12);
    h.execution.expertExecutionTime = std::chrono::nanoseconds(13);
    h.execution.expertCombinationTime = std::chrono::nanoseconds(14);
    const hm::BatchLayerExecutionResult keep = h;  // the move source's copy

    const hypermoe::runtime::BatchLayerExecutionResult r = hypermoe::integration::toReference(std::move(h));
    CHECK(r.routing.layerId == 7);
    CHECK(r.routing.valid());
    CHECK(r.routing.tokens.size() == keep.routing.tokens.size());
    for (std::size_t i = 0; i < r.routing.tokens.size(); ++i) {
        CHECK(r.routing.tokens[i].layerId == keep.routing.tokens[i].layerId);
        CHECK(r.routing.tokens[i].selectedExpertIds == keep.routing.tokens[i].selectedExpertIds);
        CHECK(r.routing.tokens[i].routingScores == keep.routing.tokens[i].routingScores);
    }
    CHECK(r.routing.expertGroups.size() == keep.routing.expertGroups.size());
    for (std::size_t i = 0; i < r.routing.expertGroups.size(); ++i) {
        CHECK(r.routing.expertGroups[i].expertId == keep.routing.expertGroups[i].expertId);
        CHECK(r.routing.expertGroups[i].tokenIndices == keep.routing.expertGroups[i].tokenIndices);
        CHECK(r.routing.expertGroups[i].routingScores == keep.routing.expertGroups[i].routingScores);
    }
    CHECK(r.expertBatches.size() == keep.expertBatches.size());
    for (std::size_t i = 0; i < r.expertBatches.size(); ++i) {
        CHECK(r.expertBatches[i].layerId == keep.expertBatches[i].layerId);
        CHECK(r.expertBatches[i].expertId == keep.expertBatches[i].expertId);
        CHECK(r.expertBatches[i].tokenIndices == keep.expertBatches[i].tokenIndices);
        CHECK(r.expertBatches[i].routingWeights == keep.expertBatches[i].routingWeights);
        r.expertBatches[i].validate(2);  // the reference's own consistency check
    }
    CHECK(r.expertOutputs.size() == keep.expertOutputs.size());
    for (std::size_t i = 0; i < r.expertOutputs.size(); ++i) same_tensor(r.expertOutputs[i], keep.expertOutputs[i]);
    same_tensor(r.output, keep.output);
    CHECK(static_cast<const float*>(r.output.data())[5] == 105.0f);
    CHECK(r.execution.expertAssignments == 4 && r.execution.uniqueExperts == 3);
    CHECK(r.execution.expertCacheHits == 3 && r.execution.expertCacheMisses == 0);
    CHECK(r.execution.expertPayloadBytes == 12345 && r.execution.expertTransferBytes == 0);
    CHECK(r.execution.tensorBackend == "hip");
    CHECK(r.execution.routingTime.count() == 11 && r.execution.schedulingTime.count() == 12);
    CHECK(r.execution.expertExecutionTime.count() == 13 && r.execution.expertCombinationTime.count() == 14);

    // ---- a reference view into an hm view of the same storage
    auto store = std::make_shared<std::vector<float>>(6, 2.5f);
    const auto rt = hypermoe::tensor::Tensor::fromStorage(
        hypermoe::tensor::Shape({2, 3}), hypermoe::tensor::DType::FP32, hypermoe::tensor::Device::cpu(),
        store->data(), store->size() * sizeof(float), store);
    const hm::tensor::TensorView hv = hypermoe::integration::toHm(hypermoe::tensor::TensorView(rt));
    CHECK(hv.shape().dimensions() == std::vector<std::size_t>({2, 3}));
    CHECK(hv.dtype() == hm::tensor::DType::FP32);
    CHECK(hv.device() == hm::tensor::Device::cpu());
    CHECK(hv.data() == store->data());
    CHECK(hv.lockOwner() == rt.view().lockOwner());

#ifdef HM_ADAPTER_HIP_ENUMS
    // ---- device tensors (the reference built with the HIP enumerators of
    // integration/reference_enums.py): a result whose tensors live on HIP
    // device 1 converts into reference tensors the reference's own
    // Tensor::fromStorage accepts (src/tensor/Tensor.cpp:14-26), with the
    // device, storage and shape kept.  The device pointer is never
    // dereferenced on the host.
    {
        void* devp = reinterpret_cast<void*>(std::uintptr_t{1} << 40);
        std::shared_ptr<void> dev_owner(devp, [](void*) {});
        auto dev_tensor = [&](std::size_t rows, std::size_t cols, std::size_t off) {
            return hm::tensor::Tensor::fromStorage(
                hm::tensor::Shape({rows, cols}), hm::tensor::DType::FP32, hm::tensor::Device::hip(1),
                static_cast<char*>(devp) + off, rows * cols * sizeof(float), dev_owner);
        };
        hm::BatchLayerExecutionResult d = keep;
        d.expertOutputs.clear();
        for (std::size_t b = 0; b < 3; ++b)
            d.expertOutputs.push_back(dev_tensor(d.expertBatches[b].size(), 4, 4096 * (b + 1)));
        d.output = dev_tensor(2, 4, 0);
        const hm::BatchLayerExecutionResult dkeep = d;
        const hypermoe::runtime::BatchLayerExecutionResult rd = hypermoe::integration::toReference(std::move(d));
        auto same_dev = [&](const hypermoe::tensor::Tensor& t, const hm::tensor::Tensor& ht) {
            CHECK(t.valid());
            CHECK(t.device().type == hypermoe::tensor::DeviceType::HIP);
            CHECK(t.device().type == hypermoe::backend::hip::kHipDeviceType);
            CHECK(t.device().ordinal == 1);
            CHECK(hypermoe::tensor::toString(t.device().type) == "HIP");
            CHECK(t.data() == ht.data());
            CHECK(t.storageBytes() == ht.storageBytes());
            CHECK(t.shape().dimensions() == ht.shape().dimensions());
        };
        CHECK(rd.expertOutputs.size() == 3);
        for (std::size_t i = 0; i < 3; ++i) same_dev(rd.expertOutputs[i], dkeep.expertOutputs[i]);
        same_dev(rd.output, dkeep.output);
        CHECK(rd.routing.valid() && rd.routing.expertGroups.size() == 3);
        // and a reference HIP view back into an hm view of the same storage
        const hm::tensor::TensorView dv = hypermoe::integration::toHm(hypermoe::tensor::TensorView(rd.output));
        CHECK(dv.device() == hm::tensor::Device::hip(1));
        CHECK(dv.data() == rd.output.data());
        CHECK(hypermoe::backend::hip::kHipBackendKind == hypermoe::backend::BackendKind::Hip);
        std::printf("adapter device tensors ok\n");
    }
#endif

    // ---- the backend through the reference's interface
    auto hip = std::make_shared<hm::backend::HipBackend>(0);
    std::unique_ptr<hypermoe::backend::ComputeBackend> b =
        std::make_unique<hypermoe::backend::hip::HipComputeBackend>(hip);
    CHECK(b->kind() == hypermoe::backend::hip::kHipBackendKind);
    CHECK(b->name() == hip->name());
    CHECK(b->deviceOrdinal() == 0);
    CHECK(b->isAvailable() == hip->isAvailable());
    CHECK(b->supportsPinnedMemory() == hip->supportsPinnedMemory());
    std::printf("adapter ok (HIP backend %s)\n", b->isAvailable() ? "available" : "not available here");
    return 0;
}
