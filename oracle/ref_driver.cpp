// ref_driver.cpp -- extern "C" entry points over the compiled reference.
//
// TEST INFRASTRUCTURE ONLY.  This file is this build's own code; it is
// compiled (oracle/Makefile, target `ref`) together with the reference's CPU
// sources, which are read in place from /root/reference and never copied.
// The resulting oracle/_ref/libhm_ref.so is used in this container to write
// the golden vectors under tests/golden/ and to pin the C restatement in
// hm_oracle.c.  Every function returns 0 on success, -1 on
// std::invalid_argument, -2 on std::overflow_error, -3 on any other
// exception.
#include "core/runtime/MoERuntime.hpp"
#include "experts/ExpertExecutor.hpp"
#include "hypermoe/experts/cache_policy.hpp"
#include "hypermoe/experts/expert_manager.hpp"
#include "memory/TransferManager.hpp"
#include "models/ModelManifest.hpp"
#include "storage/ExpertIndex.hpp"
#include "models/ExpertWeightMap.hpp"
#include "backend/CpuBackend.hpp"
#include "backend/cuda/Int8GemmPlan.hpp"
#include "router/CpuRouterBackend.hpp"
#include "router/Router.hpp"
#include "scheduler/Scheduler.hpp"
#include "storage/DiskLoader.hpp"
#include "storage/ExpertStore.hpp"
#include "tensor/activation/Activation.hpp"
#include "tensor/backend/CpuTensorBackend.hpp"
#include "tensor/quantization/Quantization.hpp"
#include "transformer/norm/RMSNorm.hpp"
#include "validation/CorrectnessOracle.hpp"

#include <unistd.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <memory>
#include <span>
#include <stdexcept>
#include <vector>

namespace {

using namespace hypermoe;

template <class F>
int guarded(F&& body) {
    try {
        body();
        return 0;
    } catch (const std::invalid_argument&) {
        return -1;
    } catch (const std::overflow_error&) {
        return -2;
    } catch (...) {
        return -3;
    }
}

tensor::Tensor hostTensor(tensor::CpuTensorBackend& cpu, tensor::Shape shape,
                          tensor::DType dtype, const void* data) {
    auto t = cpu.allocateTensor(shape, dtype);
    std::memcpy(t.data(), data, t.view().bytes());
    return t;
}

router::RouterConfig routerConfig(std::int64_t experts, std::int32_t topK,
                                  std::int32_t softmax, std::int32_t renorm) {
    return {static_cast<std::size_t>(experts), static_cast<std::size_t>(topK),
            softmax ? router::RoutingNormalization::Softmax
                    : router::RoutingNormalization::None,
            renorm != 0};
}

} // namespace

extern "C" {

int hmref_rmsnorm(const float* x, const float* gamma, float* y,
                  std::int64_t rows, std::int64_t width, float eps) {
    return guarded([&] {
        auto cpu = std::make_shared<tensor::CpuTensorBackend>();
        auto in = hostTensor(*cpu, {std::size_t(rows), std::size_t(width)},
                             tensor::DType::FP32, x);
        auto g = hostTensor(*cpu, {std::size_t(width)}, tensor::DType::FP32, gamma);
        transformer::norm::RMSNorm norm(cpu, std::size_t(width), eps);
        auto out = norm.execute(in, g);
        std::memcpy(y, out.data(), out.view().bytes());
    });
}

// Router::routeBatch on CpuRouterBackend.  ids/scores [T x k] rank order;
// counts[E] per expert; perm_tokens/perm_weights [T*k] in group order.
int hmref_route_batch(const float* h, const float* w, std::int64_t tokens,
                      std::int64_t hidden, std::int64_t experts,
                      std::int32_t topK, std::int32_t softmax,
                      std::int32_t renorm, std::uint32_t* ids, float* scores,
                      std::int32_t* counts, std::int32_t* permTokens,
                      float* permWeights) {
    return guarded([&] {
        tensor::CpuTensorBackend cpu;
        auto hs = hostTensor(cpu, {std::size_t(tokens), std::size_t(hidden)},
                             tensor::DType::FP32, h);
        auto ws = hostTensor(cpu, {std::size_t(hidden), std::size_t(experts)},
                             tensor::DType::FP32, w);
        router::Router r(routerConfig(experts, topK, softmax, renorm),
                         std::make_shared<router::CpuRouterBackend>());
        const auto batch = r.routeBatch(0, hs, ws);
        for (std::size_t t = 0; t < batch.tokens.size(); ++t) {
            for (std::size_t j = 0; j < std::size_t(topK); ++j) {
                ids[t * topK + j] = batch.tokens[t].selectedExpertIds[j];
                scores[t * topK + j] = batch.tokens[t].routingScores[j];
            }
        }
        std::memset(counts, 0, sizeof(std::int32_t) * std::size_t(experts));
        std::size_t pos = 0;
        for (const auto& group : batch.expertGroups) {
            counts[group.expertId] = std::int32_t(group.tokenIndices.size());
            for (std::size_t i = 0; i < group.tokenIndices.size(); ++i, ++pos) {
                permTokens[pos] = std::int32_t(group.tokenIndices[i]);
                permWeights[pos] = group.routingScores[i];
            }
        }
    });
}

int hmref_matmul_f32(const float* x, const float* wt, float* y,
                     std::int64_t rows, std::int64_t inner, std::int64_t cols) {
    return guarded([&] {
        tensor::CpuTensorBackend cpu;
        auto a = hostTensor(cpu, {std::size_t(rows), std::size_t(inner)}, tensor::DType::FP32, x);
        auto b = hostTensor(cpu, {std::size_t(inner), std::size_t(cols)}, tensor::DType::FP32, wt);
        auto c = cpu.allocateTensor({std::size_t(rows), std::size_t(cols)}, tensor::DType::FP32);
        cpu.matmul(a, b, c);
        std::memcpy(y, c.data(), c.view().bytes());
    });
}

int hmref_matmul_w8a32(const float* x, const std::int8_t* q, float scale,
                       std::int32_t zp, float* y, std::int64_t rows,
                       std::int64_t inner, std::int64_t cols) {
    return guarded([&] {
        tensor::CpuTensorBackend cpu;
        auto a = hostTensor(cpu, {std::size_t(rows), std::size_t(inner)}, tensor::DType::FP32, x);
        auto b = hostTensor(cpu, {std::size_t(inner), std::size_t(cols)}, tensor::DType::INT8, q);
        auto c = cpu.allocateTensor({std::size_t(rows), std::size_t(cols)}, tensor::DType::FP32);
        cpu.matmulInt8Weights(a, b, {scale, zp}, c);
        std::memcpy(y, c.data(), c.view().bytes());
    });
}

int hmref_silu(const float* x, float* y, std::int64_t n) {
    return guarded([&] {
        for (std::int64_t i = 0; i < n; ++i) y[i] = tensor::activation::silu(x[i]);
    });
}

int hmref_quantize_int8(const float* w, std::int64_t n, std::int8_t* q,
                        float* scale, std::int32_t* zp, float* maxError) {
    return guarded([&] {
        const auto r = tensor::quantization::quantizeInt8(
            std::span<const float>(w, std::size_t(n)));
        std::memcpy(q, r.bytes.data(), r.bytes.size());
        *scale = r.parameters.scale;
        *zp = r.parameters.zeroPoint;
        *maxError = r.maximumAbsoluteError;
    });
}

// planInt8Gemm (backend/cuda/Int8GemmPlan.cpp:29-53); mode 0 auto,
// 1 reference, 2 cooperative.  out = {implementation, partitions, blocks,
// scratchElements}.
int hmref_plan_int8_gemm(std::int64_t rows, std::int64_t inner,
                         std::int64_t cols, std::int32_t mode,
                         std::int64_t* out) {
    return guarded([&] {
        const auto m = static_cast<backend::cuda::Int8GemmMode>(mode);
        const auto p = backend::cuda::planInt8Gemm(std::size_t(rows), std::size_t(inner),
                                                   std::size_t(cols), m);
        out[0] = static_cast<std::int64_t>(p.implementation);
        out[1] = std::int64_t(p.partitions);
        out[2] = std::int64_t(p.blocks);
        out[3] = std::int64_t(p.scratchElements);
    });
}

// MoERuntime::executeBatch on the CPU backend over an ExpertStore written to a
// temporary directory, wired like tests/support/ExpertPipelineFixture.hpp.
// payload: per expert gate[HxI] | up[HxI] | down[IxH] (int8 or float);
// scale/zp [E x 3] for INT8.  out [T x H]; ids/scores [T x k];
// groupCounts [E]; expertOut [T*k x H] in group order (optional).
int hmref_moe_block(const void* payload, std::int32_t isInt8,
                    const float* scale, const std::int32_t* zp,
                    std::int64_t experts, std::int64_t hidden,
                    std::int64_t intermediate, const float* h,
                    const float* routerW, std::int64_t tokens,
                    std::int32_t topK, std::int32_t softmax,
                    std::int32_t renorm, float* out, std::uint32_t* ids,
                    float* scores, std::int32_t* groupCounts,
                    float* expertOut) {
    static std::atomic_uint64_t sequence{};
    std::filesystem::path path;
    const int rc = guarded([&] {
        do {
            path = std::filesystem::temp_directory_path() /
                   ("hmref-moe-" + std::to_string(::getpid()) + "-" +
                    std::to_string(sequence.fetch_add(1)));
        } while (!std::filesystem::create_directory(path));
        const std::size_t H = std::size_t(hidden), I = std::size_t(intermediate);
        const std::size_t elem = isInt8 ? 1 : sizeof(float);
        const std::size_t projBytes = H * I * elem;
        const std::size_t expertBytes = 3 * projBytes;
        const auto qtype = isInt8 ? QuantizationType::Int8 : QuantizationType::Fp32;
        std::vector<storage::ExpertBlob> blobs;
        for (std::size_t e = 0; e < std::size_t(experts); ++e) {
            const auto* src = static_cast<const std::byte*>(payload) + e * expertBytes;
            blobs.push_back({0, std::uint32_t(e), static_cast<std::uint32_t>(qtype),
                             std::vector<std::byte>(src, src + expertBytes)});
        }
        storage::ExpertStore::create(path, blobs, "{}");
        auto store = std::make_shared<storage::ExpertStore>(path);
        auto loader = std::make_shared<storage::DiskLoader>(store);
        auto compute = std::make_shared<backend::CpuBackend>();
        auto transfers = std::make_shared<TransferManager>(loader, compute, 2);
        const std::size_t budget = expertBytes * std::size_t(experts) + (1U << 20);
        MemoryManager memory(budget, budget);
        ExpertManager manager(memory, std::make_unique<LruCachePolicy>(), transfers);
        auto scheduler = std::make_shared<scheduler::Scheduler>(
            transfers, nullptr, 2, MemoryTier::Ram, budget);
        models::ExpertWeightMap mappings;
        for (std::size_t e = 0; e < std::size_t(experts); ++e) {
            const auto record = store->index().find(0, std::uint32_t(e)).value();
            manager.registerExpert({std::uint32_t(e), 0, expertBytes, qtype, MemoryTier::Nvme});
            scheduler->registerExpert(0, std::uint32_t(e));
            const models::ExpertWeightType types[3] = {models::ExpertWeightType::GATE,
                                                       models::ExpertWeightType::UP,
                                                       models::ExpertWeightType::DOWN};
            for (std::size_t p = 0; p < 3; ++p) {
                const tensor::Shape shape = p < 2 ? tensor::Shape{H, I} : tensor::Shape{I, H};
                std::optional<tensor::quantization::QuantizationParameters> params;
                std::optional<tensor::quantization::QuantizedDType> qd;
                if (isInt8) {
                    params = tensor::quantization::QuantizationParameters{
                        scale[e * 3 + p], zp[e * 3 + p]};
                    qd = tensor::quantization::QuantizedDType::INT8;
                }
                mappings.add(0, std::uint32_t(e), types[p],
                             {"expert", shape,
                              isInt8 ? tensor::DType::INT8 : tensor::DType::FP32, qd,
                              record.offset + p * projBytes, projBytes, 0,
                              std::uint32_t(e), params});
            }
        }
        auto tensors = std::make_shared<tensor::CpuTensorBackend>();
        auto routerPtr = std::make_shared<router::Router>(
            routerConfig(experts, topK, softmax, renorm),
            std::make_shared<router::CpuRouterBackend>());
        auto executor = std::make_shared<ExpertMlpExecutor>(tensors);
        {
            runtime::MoERuntime rt(routerPtr, scheduler, manager, std::move(mappings),
                                   tensors, executor, nullptr, nullptr, true);
            auto hs = hostTensor(*tensors, {std::size_t(tokens), H}, tensor::DType::FP32, h);
            auto rw = hostTensor(*tensors, {H, std::size_t(experts)}, tensor::DType::FP32, routerW);
            const auto result = rt.executeBatch(0, hs, rw);
            std::memcpy(out, result.output.data(), result.output.view().bytes());
            for (std::size_t t = 0; t < std::size_t(tokens); ++t) {
                for (std::size_t j = 0; j < std::size_t(topK); ++j) {
                    ids[t * topK + j] = result.routing.tokens[t].selectedExpertIds[j];
                    scores[t * topK + j] = result.routing.tokens[t].routingScores[j];
                }
            }
            std::memset(groupCounts, 0, sizeof(std::int32_t) * std::size_t(experts));
            std::size_t row = 0;
            for (std::size_t g = 0; g < result.expertBatches.size(); ++g) {
                const auto& b = result.expertBatches[g];
                groupCounts[b.expertId] = std::int32_t(b.tokenIndices.size());
                if (expertOut) {
                    std::memcpy(expertOut + row * H, result.expertOutputs[g].data(),
                                result.expertOutputs[g].view().bytes());
                }
                row += b.tokenIndices.size();
            }
        }
        scheduler->shutdown();
    });
    std::error_code ignored;
    if (!path.empty()) std::filesystem::remove_all(path, ignored);
    return rc;
}

// ---- packed artefact (experts.index / manifest.json) -----------------------

// storage::ExpertStore::crc32 (ExpertStore.cpp:183-192).
std::uint32_t hmref_crc32(const void* data, std::size_t bytes) {
    return storage::ExpertStore::crc32(
        std::span<const std::byte>(static_cast<const std::byte*>(data), bytes));
}

// storage::ExpertIndex(records, projections).save(path).  records: 6 u64
// per record (layer, expert, offset, size, quantization, checksum);
// projections: 16 u64 per record (layer, expert, type, dtype, rank,
// reserved, offset, size, shape[4], checksum, trailing, 0, 0).
int hmref_index_save(const char* path, const std::uint64_t* records, std::size_t nrec,
                     const std::uint64_t* projections, std::size_t nproj) {
    return guarded([&] {
        std::vector<storage::ExpertRecord> rs;
        for (std::size_t i = 0; i < nrec; ++i) {
            const auto* r = records + 6 * i;
            rs.push_back({std::uint32_t(r[0]), std::uint32_t(r[1]), r[2], r[3],
                          std::uint32_t(r[4]), std::uint32_t(r[5])});
        }
        std::vector<storage::ProjectionRecord> ps;
        for (std::size_t i = 0; i < nproj; ++i) {
            const auto* p = projections + 16 * i;
            storage::ProjectionRecord o;
            o.layer_id = std::uint32_t(p[0]);
            o.expert_id = std::uint32_t(p[1]);
            o.projection_type = static_cast<storage::ProjectionType>(p[2]);
            o.dtype = std::uint32_t(p[3]);
            o.rank = std::uint32_t(p[4]);
            o.reserved = std::uint32_t(p[5]);
            o.offset = p[6];
            o.size = p[7];
            for (int d = 0; d < 4; ++d) o.shape[d] = p[8 + d];
            o.checksum = std::uint32_t(p[12]);
            o.trailing_reserved = std::uint32_t(p[13]);
            ps.push_back(o);
        }
        storage::ExpertIndex(std::move(rs), std::move(ps)).save(path);
    });
}

// storage::ExpertIndex::load(path): counts, and the records in the layout
// of hmref_index_save (up to the capacities).  -3 on StorageError.
int hmref_index_load(const char* path, std::uint64_t* records, std::size_t rcap,
                     std::uint64_t* projections, std::size_t pcap, std::size_t* nrec,
                     std::size_t* nproj) {
    return guarded([&] {
        const auto index = storage::ExpertIndex::load(path);
        *nrec = index.records().size();
        *nproj = index.projections().size();
        for (std::size_t i = 0; i < std::min(rcap, *nrec); ++i) {
            const auto& r = index.records()[i];
            const std::uint64_t v[6] = {r.layer_id, r.expert_id, r.offset, r.size,
                                        r.quantization_type, r.checksum};
            std::memcpy(records + 6 * i, v, sizeof v);
        }
        for (std::size_t i = 0; i < std::min(pcap, *nproj); ++i) {
            const auto& p = index.projections()[i];
            const std::uint64_t v[16] = {p.layer_id, p.expert_id,
                                         static_cast<std::uint64_t>(p.projection_type), p.dtype,
                                         p.rank, p.reserved, p.offset, p.size, p.shape[0],
                                         p.shape[1], p.shape[2], p.shape[3], p.checksum,
                                         p.trailing_reserved, 0, 0};
            std::memcpy(projections + 16 * i, v, sizeof v);
        }
    });
}

// models::ModelManifest::load(path) (with its validate()), then toJson()
// into out (NUL-terminated, truncated to cap).
int hmref_manifest_load(const char* path, char* out, std::size_t cap) {
    return guarded([&] {
        const auto json = models::ModelManifest::load(path).toJson();
        if (out && cap) {
            const auto n = std::min(cap - 1, json.size());
            std::memcpy(out, json.data(), n);
            out[n] = '\0';
        }
    });
}

} // extern "C"
