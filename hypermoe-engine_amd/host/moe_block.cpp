// moe_block.cpp -- HipMoEBlock::executeBatch and the device-resident expert
// layer (see hm_moe_block.hpp).
#include "hm_moe_block.hpp"
#include "hm_moe.h"

#include <cmath>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <utility>

namespace hm {

using backend::DeviceBuffer;
using backend::throwOnStatus;
using tensor::DType;
using tensor::DeviceType;
using tensor::Tensor;
using tensor::TensorView;

namespace router {

void RouterConfig::validate() const {
    if (expertCount == 0) throw std::invalid_argument("router requires experts");
    if (expertCount > std::numeric_limits<std::uint32_t>::max()) {
        throw std::invalid_argument("router expert count exceeds runtime IDs");
    }
    if (topK == 0 || topK > expertCount) {
        throw std::invalid_argument("router top-k must be within expert count");
    }
    if (normalization != RoutingNormalization::None &&
        normalization != RoutingNormalization::Softmax) {
        throw std::invalid_argument("router normalization is unsupported");
    }
}

bool BatchRouterDecision::valid() const noexcept {
    if (tokens.empty()) return false;
    for (const auto& t : tokens) {
        if (!t.valid() || t.layerId != layerId) return false;
    }
    for (const auto& g : expertGroups) {
        if (g.tokenIndices.empty() || g.tokenIndices.size() != g.routingScores.size()) {
            return false;
        }
    }
    return true;
}

}  // namespace router

void ExpertBatch::validate(std::size_t tokenCount) const {
    if (tokenCount == 0 || tokenIndices.empty() || tokenIndices.size() != routingWeights.size()) {
        throw std::invalid_argument("expert batch metadata is incomplete");
    }
    std::unordered_set<std::size_t> seen;
    for (std::size_t i = 0; i < tokenIndices.size(); ++i) {
        if (tokenIndices[i] >= tokenCount || !std::isfinite(routingWeights[i]) ||
            !seen.insert(tokenIndices[i]).second) {
            throw std::invalid_argument("expert batch contains an invalid token assignment");
        }
    }
}

// ---- DeviceExpertLayer ----------------------------------------------------------

DeviceExpertLayer::~DeviceExpertLayer() = default;

std::uint64_t DeviceExpertLayer::expertBytes() const noexcept {
    return 3ull * hidden_ * intermediate_ * tensor::sizeOf(dtype_);
}

std::shared_ptr<DeviceExpertLayer> DeviceExpertLayer::fromPayload(
    std::shared_ptr<backend::HipBackend> backend, std::span<const std::byte> payload,
    std::size_t experts, std::size_t hidden, std::size_t intermediate, DType dtype,
    std::span<const ExpertQuantization> quantization) {
    if (!backend) throw std::invalid_argument("expert layer requires a HIP backend");
    if (experts == 0 || hidden == 0 || intermediate == 0) {
        throw std::invalid_argument("expert layer dimensions must be nonzero");
    }
    if (dtype != DType::INT8 && dtype != DType::FP32) {
        throw std::invalid_argument("expert layer dtype must be INT8 or FP32");
    }
    const auto bytes = hm_packed_layer_bytes((int64_t)experts, (int64_t)hidden,
                                             (int64_t)intermediate, (int32_t)dtype);
    if (bytes == 0) throw std::overflow_error("expert layer byte size overflow");
    if (payload.size() != bytes) {
        throw std::invalid_argument("expert payload size does not match [E x 3 x H x I]");
    }
    if (dtype == DType::INT8 && quantization.size() != experts) {
        throw std::invalid_argument("INT8 expert layer needs one parameter set per expert");
    }
    std::vector<float> scale;
    std::vector<std::int32_t> zp;
    if (dtype == DType::INT8) {
        for (const auto& q : quantization) {
            for (const auto* p : {&q.gate, &q.up, &q.down}) {
                tensor::quantization::validateInt8Parameters(*p);
                scale.push_back(p->scale);
                zp.push_back(p->zeroPoint);
            }
        }
    }

    auto layer = std::shared_ptr<DeviceExpertLayer>(new DeviceExpertLayer());
    layer->backend_ = backend;
    layer->experts_ = experts;
    layer->hidden_ = hidden;
    layer->intermediate_ = intermediate;
    layer->dtype_ = dtype;
    layer->packed_ = std::make_unique<DeviceBuffer>(backend, bytes);
    auto stream = backend->computeStream();
    {
        // upload the reference layout once, re-lay it out on the device
        DeviceBuffer staging(backend, bytes);
        backend->copyToDevice(staging.data(), payload.data(), bytes, nullptr);
        throwOnStatus(hm_pack_layer(staging.data(), (int64_t)experts, (int64_t)hidden,
                                    (int64_t)intermediate, (int32_t)dtype,
                                    layer->packed_->data(), stream),
                      "pack expert layer");
        backend->synchronize(stream);
    }
    if (dtype == DType::INT8) {
        layer->scale_ = std::make_unique<DeviceBuffer>(backend, scale.size() * sizeof(float));
        layer->zeroPoint_ = std::make_unique<DeviceBuffer>(backend, zp.size() * sizeof(int32_t));
        backend->copyToDevice(layer->scale_->data(), scale.data(), scale.size() * sizeof(float));
        backend->copyToDevice(layer->zeroPoint_->data(), zp.data(), zp.size() * sizeof(int32_t));
    }
    layer->desc_ = std::make_unique<hm_layer>();
    *layer->desc_ = hm_layer{(int64_t)experts,
                             (int64_t)hidden,
                             (int64_t)intermediate,
                             (int32_t)dtype,
                             layer->packed_->data(),
                             layer->scale_ ? static_cast<const float*>(layer->scale_->data())
                                           : nullptr,
                             layer->zeroPoint_
                                 ? static_cast<const int32_t*>(layer->zeroPoint_->data())
                                 : nullptr};
    return layer;
}

// ---- HipMoEBlock -------------------------------------------------------------

// Pinned host copies of the routing metadata and the device buffers they
// come from, sized for the largest batch seen.
// One call in flight: the routing arrays the kernels write on the device,
// their pinned host copy, the call's stage events and its completion event.
// A slot is owned by one pending result at a time; `inFlight` marks copies
// that nobody has waited for yet (a result dropped without get()), so the
// next owner waits before it reuses the pinned memory.
struct HipMoEBlock::Staging {
    std::shared_ptr<backend::HipBackend> backend;
    std::size_t pairs{}, experts{};
    std::unique_ptr<DeviceBuffer> device;
    void* host{};
    // byte offsets inside both buffers; `zero` is a host word that stays 0
    // (the source of the status reset, never written after allocation)
    std::size_t ids{}, scores{}, counts{}, offsets{}, ptok{}, pw{}, status{}, zero{}, total{};
    std::array<backend::EventHandle, HM_BLOCK_EVENTS> events{};
    backend::EventHandle done{};
    bool busy{};
    bool inFlight{};

    ~Staging() {
        for (auto e : events) backend->destroyEvent(e);
        backend->destroyEvent(done);
        if (host) backend->freePinned(host);
    }
    void ensure(std::size_t p, std::size_t e) {
        if (done == nullptr) {
            for (auto& ev : events) ev = backend->createEvent();
            done = backend->createEvent();
        }
        if (p <= pairs && e <= experts && device) return;
        pairs = std::max(p, pairs);
        experts = std::max(e, experts);
        std::size_t at = 0;
        auto take = [&](std::size_t n) {
            const auto o = at;
            at += (n + 255) & ~std::size_t{255};
            return o;
        };
        ids = take(pairs * 4);
        scores = take(pairs * 4);
        counts = take(experts * 4);
        offsets = take((experts + 1) * 4);
        ptok = take(pairs * 4);
        pw = take(pairs * 4);
        status = take(4);
        zero = take(4);
        total = at;
        if (host) {
            backend->freePinned(host);
            host = nullptr;
        }
        device = std::make_unique<DeviceBuffer>(backend, total);
        host = backend->allocatePinned(total);
        *hostAt<int32_t>(zero) = 0;
    }
    template <class T>
    T* dev(std::size_t off) const {
        return reinterpret_cast<T*>(static_cast<char*>(device->data()) + off);
    }
    template <class T>
    T* hostAt(std::size_t off) const {
        return reinterpret_cast<T*>(static_cast<char*>(host) + off);
    }
};

HipMoEBlock::HipMoEBlock(std::shared_ptr<backend::HipBackend> backend,
                         router::RouterConfig config, BlockOptions options)
    : backend_(std::move(backend)), config_(config), options_(options) {
    if (!backend_) throw std::invalid_argument("MoE block requires a HIP backend");
    config_.validate();
    if (options_.limbsX < 1 || options_.limbsX > 3 || options_.limbsZ < 1 || options_.limbsZ > 3) {
        throw std::invalid_argument("activation digit planes must be 1, 2 or 3");
    }
}

HipMoEBlock::~HipMoEBlock() {
    try {
        if (backend_->isAvailable()) backend_->synchronize(backend_->computeStream());
    } catch (...) {
    }
}

void HipMoEBlock::addLayer(LayerId layerId, std::shared_ptr<const DeviceExpertLayer> layer) {
    if (!layer) throw std::invalid_argument("MoE block layer is null");
    if (layer->experts() != config_.expertCount) {
        throw std::invalid_argument("expert layer does not match the router's expert count");
    }
    std::scoped_lock lock(executionMutex_);
    layers_[layerId] = std::move(layer);
}

BatchLayerExecutionResult HipMoEBlock::executeBatch(LayerId layerId, TensorView hiddenStates,
                                                    TensorView routerWeights) {
    return launchBatch(layerId, hiddenStates, routerWeights).get();
}

BatchLayerExecutionResult HipMoEBlock::executeBatch(LayerId layerId, TensorView hiddenStates,
                                                    TensorView routerWeights,
                                                    TensorView residual) {
    if (!residual) throw std::invalid_argument("MoE block residual is empty");
    return launchBatch(layerId, hiddenStates, routerWeights, residual).get();
}

HipMoEBlock::Staging* HipMoEBlock::acquireSlot(std::size_t pairs, std::size_t experts) {
    Staging* slot = nullptr;
    {
        std::scoped_lock lock(poolMutex_);
        for (auto& s : slots_) {
            if (!s->busy) {
                slot = s.get();
                break;
            }
        }
        if (slot == nullptr) {
            slots_.push_back(std::make_unique<Staging>());
            slot = slots_.back().get();
            slot->backend = backend_;
        }
        slot->busy = true;
    }
    try {
        // copies of a result dropped without get() may still be landing
        if (slot->inFlight) {
            backend_->waitEvent(slot->done);
            slot->inFlight = false;
        }
        slot->ensure(pairs, experts);
    } catch (...) {
        releaseSlot(slot);
        throw;
    }
    return slot;
}

void HipMoEBlock::releaseSlot(Staging* slot) noexcept {
    std::scoped_lock lock(poolMutex_);
    slot->busy = false;
}

// A released output buffer of this size (only the pool still owns it; the
// call's kernels are ordered after every earlier use on the compute stream),
// else a new one, kept for reuse while the pool has room.
std::shared_ptr<DeviceBuffer> HipMoEBlock::outputBuffer(
    std::vector<std::shared_ptr<DeviceBuffer>>& pool, std::size_t bytes) {
    constexpr std::size_t kKeep = 4;
    std::scoped_lock lock(poolMutex_);
    for (auto& b : pool) {
        if (b.use_count() == 1 && b->size() == bytes) return b;
    }
    auto b = std::make_shared<DeviceBuffer>(backend_, bytes);
    if (pool.size() < kKeep) {
        pool.push_back(b);
    } else {
        for (auto& old : pool) {
            if (old.use_count() == 1) {
                old = b;
                break;
            }
        }
    }
    return b;
}

PendingBatchResult::PendingBatchResult(PendingBatchResult&& o) noexcept
    : block_(o.block_), slot_(o.slot_), layerId_(o.layerId_), tokens_(o.tokens_),
      hidden_(o.hidden_), topK_(o.topK_), experts_(o.experts_), expertBytes_(o.expertBytes_),
      output_(std::move(o.output_)), expertOut_(std::move(o.expertOut_)) {
    o.block_ = nullptr;
    o.slot_ = nullptr;
}

PendingBatchResult::~PendingBatchResult() {
    if (block_ && slot_) block_->releaseSlot(static_cast<HipMoEBlock::Staging*>(slot_));
}

BatchLayerExecutionResult PendingBatchResult::get() {
    if (!block_ || !slot_) throw std::logic_error("MoE block result was already taken");
    // the slot goes back to the block whether or not the result builds
    struct Release {
        PendingBatchResult* p;
        ~Release() {
            p->block_->releaseSlot(static_cast<HipMoEBlock::Staging*>(p->slot_));
            p->block_ = nullptr;
            p->slot_ = nullptr;
        }
    } release{this};
    return block_->materialize(*this);
}

PendingBatchResult HipMoEBlock::launchBatch(LayerId layerId, TensorView hidden,
                                            TensorView routerWeights, TensorView residual) {
    std::scoped_lock executionLock(executionMutex_);
    const auto dev = tensor::Device::hip(backend_->deviceOrdinal());
    if (!hidden || hidden.shape().rank() != 2 || hidden.dtype() != DType::FP32 ||
        hidden.device() != dev) {
        throw std::invalid_argument(
            "MoE runtime requires rank-2 FP32 hidden states on its tensor backend");
    }
    const auto it = layers_.find(layerId);
    if (it == layers_.end()) throw std::out_of_range("MoE block has no experts for this layer");
    const auto& layer = *it->second;
    const std::size_t T = hidden.shape()[0], H = hidden.shape()[1];
    const std::size_t E = config_.expertCount, k = config_.topK;
    if (H != layer.hidden()) {
        throw std::invalid_argument("hidden width does not match the expert layer");
    }
    if (!routerWeights || routerWeights.shape().rank() != 2 ||
        routerWeights.dtype() != DType::FP32 || routerWeights.device() != dev ||
        routerWeights.shape()[0] != H || routerWeights.shape()[1] != E) {
        throw std::invalid_argument("router weights must be [hidden x experts] FP32");
    }
    if (residual && (residual.shape() != hidden.shape() || residual.dtype() != DType::FP32 ||
                     residual.device() != dev)) {
        throw std::invalid_argument("MoE block residual must match the hidden states");
    }
    if (T > (std::size_t)std::numeric_limits<int32_t>::max() / k) {
        throw std::overflow_error("router assignment count overflow");
    }
    const auto hOwner = hidden.lockOwner(), wOwner = routerWeights.lockOwner();
    const auto rOwner = residual ? residual.lockOwner() : std::shared_ptr<void>();
    if (!hOwner || !wOwner || (residual && !rOwner)) {
        throw std::invalid_argument("MoE block received expired tensor storage");
    }

    const auto stream = backend_->computeStream();
    const std::uint32_t routeFlags =
        (config_.normalization == router::RoutingNormalization::Softmax ? HM_ROUTE_SOFTMAX : 0u) |
        (config_.renormalizeSelected ? HM_ROUTE_RENORM : 0u);
    const std::uint32_t execFlags = options_.genericKernels ? HM_EXEC_GENERIC : 0u;
    const std::size_t wsBytes =
        hm_moe_block_workspace_bytes(&layer.descriptor(), (int64_t)T, (int32_t)k,
                                     options_.limbsX, options_.limbsZ, execFlags);
    if (wsBytes == 0) throw std::invalid_argument("MoE block configuration is invalid");
    if (!workspace_ || workspace_->size() < wsBytes) {
        // queued calls may still use the smaller workspace
        if (workspace_) backend_->synchronize(stream);
        workspace_ = std::make_unique<DeviceBuffer>(backend_, wsBytes);
    }
    const std::size_t P = T * k;

    PendingBatchResult pending;
    pending.block_ = this;
    Staging* slot = acquireSlot(P, E);
    pending.slot_ = slot;
    pending.layerId_ = layerId;
    pending.tokens_ = T;
    pending.hidden_ = H;
    pending.topK_ = k;
    pending.experts_ = E;
    pending.expertBytes_ = layer.expertBytes();
    // callee-allocated outputs (MoERuntime.cpp:134), reused once released
    auto out = outputBuffer(outPool_, T * H * sizeof(float));
    if (options_.keepExpertOutputs) pending.expertOut_ = outputBuffer(expertOutPool_, P * H * sizeof(float));

    auto& st = *slot;
    hm_block_io io{};
    io.out = static_cast<float*>(out->data());
    io.ids = st.dev<uint32_t>(st.ids);
    io.scores = st.dev<float>(st.scores);
    io.counts = st.dev<int32_t>(st.counts);
    io.offsets = st.dev<int32_t>(st.offsets);
    io.perm_tokens = st.dev<int32_t>(st.ptok);
    io.perm_weights = st.dev<float>(st.pw);
    io.expert_out = pending.expertOut_ ? static_cast<float*>(pending.expertOut_->data()) : nullptr;
    io.status = st.dev<int32_t>(st.status);
    io.residual = residual ? static_cast<const float*>(residual.data()) : nullptr;
    io.events = st.events.data();
    try {
        backend_->copyToDevice(io.status, st.hostAt<int32_t>(st.zero), 4, stream);
        throwOnStatus(hm_moe_block_forward(&layer.descriptor(),
                                           static_cast<const float*>(hidden.data()),
                                           static_cast<const float*>(routerWeights.data()),
                                           (int64_t)T, (int32_t)k, routeFlags | execFlags,
                                           options_.limbsX, options_.limbsZ, &io,
                                           workspace_->data(), workspace_->size(), stream),
                      "MoE block forward");
        // routing metadata to pinned memory behind the kernels, then the
        // call's completion event; nothing here waits for the device
        backend_->copyFromDevice(st.hostAt<void>(st.ids), io.ids, P * 4, stream);
        backend_->copyFromDevice(st.hostAt<void>(st.scores), io.scores, P * 4, stream);
        backend_->copyFromDevice(st.hostAt<void>(st.counts), io.counts, E * 4, stream);
        backend_->copyFromDevice(st.hostAt<void>(st.offsets), io.offsets, (E + 1) * 4, stream);
        backend_->copyFromDevice(st.hostAt<void>(st.ptok), io.perm_tokens, P * 4, stream);
        backend_->copyFromDevice(st.hostAt<void>(st.pw), io.perm_weights, P * 4, stream);
        backend_->copyFromDevice(st.hostAt<void>(st.status), io.status, 4, stream);
        backend_->recordEvent(st.done, stream);
        st.inFlight = true;
    } catch (...) {
        // the launched work may still read the inputs: drain before unwinding
        try {
            backend_->synchronize(stream);
        } catch (...) {
        }
        throw;  // `pending` releases the slot
    }
    pending.output_ = Tensor::fromDeviceBuffer(tensor::Shape{T, H}, DType::FP32, dev, std::move(out));
    return pending;
}

BatchLayerExecutionResult HipMoEBlock::materialize(PendingBatchResult& pending) {
    auto& st = *static_cast<Staging*>(pending.slot_);
    backend_->waitEvent(st.done);
    st.inFlight = false;
    const std::size_t T = pending.tokens_, H = pending.hidden_, k = pending.topK_;
    const std::size_t E = pending.experts_, P = T * k;
    const LayerId layerId = pending.layerId_;
    const auto dev = tensor::Device::hip(backend_->deviceOrdinal());

    const auto status = *st.hostAt<int32_t>(st.status);
    if (status & HM_STATUS_NONFINITE_SCORE) {
        throw std::runtime_error("router produced a non-finite score");
    }
    if (status & HM_STATUS_SOFTMAX_FAILED) {
        throw std::runtime_error("router softmax normalization failed");
    }
    if (status & HM_STATUS_RENORM_FAILED) {
        throw std::runtime_error("selected router scores cannot be renormalized");
    }

    BatchLayerExecutionResult result;
    auto& routing = result.routing;
    routing.layerId = layerId;
    routing.tokens.resize(T);
    const auto* ids = st.hostAt<const uint32_t>(st.ids);
    const auto* scores = st.hostAt<const float>(st.scores);
    for (std::size_t t = 0; t < T; ++t) {
        auto& d = routing.tokens[t];
        d.layerId = layerId;
        d.selectedExpertIds.assign(ids + t * k, ids + (t + 1) * k);
        d.routingScores.assign(scores + t * k, scores + (t + 1) * k);
    }
    const auto* counts = st.hostAt<const int32_t>(st.counts);
    const auto* offsets = st.hostAt<const int32_t>(st.offsets);
    const auto* ptok = st.hostAt<const int32_t>(st.ptok);
    const auto* pw = st.hostAt<const float>(st.pw);
    const auto& expertOut = pending.expertOut_;
    auto& meta = result.execution;
    meta.tensorBackend = "HIP tensor backend";
    for (std::size_t e = 0; e < E; ++e) {
        const auto n = (std::size_t)counts[e];
        if (n == 0) continue;
        const auto lo = (std::size_t)offsets[e];
        router::ExpertTokenGroup g;
        g.expertId = (ExpertId)e;
        g.tokenIndices.assign(ptok + lo, ptok + lo + n);
        g.routingScores.assign(pw + lo, pw + lo + n);
        ExpertBatch batch{layerId, (ExpertId)e, g.tokenIndices, g.routingScores};
        batch.validate(T);
        meta.expertAssignments += n;
        routing.expertGroups.push_back(std::move(g));
        if (expertOut) {
            auto* base = static_cast<char*>(expertOut->data()) + lo * H * sizeof(float);
            result.expertOutputs.push_back(Tensor::fromStorage(
                tensor::Shape{n, H}, DType::FP32, dev, base, n * H * sizeof(float), expertOut));
        }
        result.expertBatches.push_back(std::move(batch));
    }
    if (result.expertBatches.empty()) throw std::runtime_error("router produced no expert batches");
    if (meta.expertAssignments != P) {
        throw std::runtime_error("router expert groups omit token assignments");
    }
    if (!routing.valid()) throw std::runtime_error("router returned an invalid batch decision");
    meta.uniqueExperts = result.expertBatches.size();
    meta.expertCacheHits = meta.uniqueExperts;
    meta.expertPayloadBytes = meta.uniqueExperts * pending.expertBytes_;
    auto span = [&](int a, int b) {
        float ms = 0.0F;
        throwOnStatus(hm_event_elapsed_ms(&ms, st.events[a], st.events[b]), "block stage timing");
        return std::chrono::nanoseconds((long long)std::llround(ms * 1e6));
    };
    meta.routingTime = span(0, 1);
    meta.schedulingTime = span(1, 3);
    meta.expertExecutionTime = span(3, 5);
    meta.expertCombinationTime = span(5, 6);
    result.output = std::move(pending.output_);
    return result;
}

}  // namespace hm
