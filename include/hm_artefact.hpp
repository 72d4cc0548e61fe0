// hm_artefact.hpp -- the reference's packed model artefact, read into a
// device-resident expert table.
//
// A packed model directory (README.md:154-169) holds
//   experts.bin    4 KiB-aligned expert payloads (gate | up | down, each
//                  [K x N] row-major INPUT_OUTPUT, INT8 or FP32) and the
//                  routers' [H x E] FP32 matrices,
//   experts.index  little-endian records: v1 = expert records, v2 adds one
//                  projection record (role, dtype, shape, CRC32) per
//                  gate/up/down (src/storage/ExpertIndex.hpp:15-55,
//                  ExpertIndex.cpp:59-206),
//   manifest.json  hypermoe.model-manifest.v3 (src/models/ModelManifest.hpp:
//                  37-63,117-121; ModelManifest.cpp:483-599 writes it): model
//                  config, router config, the tensors (with the per-projection
//                  INT8 {scale, zero_point}) and the expert mappings.
// ExpertIndex keeps the reference's format and validation rules; the
// manifest reader takes the fields the MoE block needs (config, router,
// tensors, experts) with the reference's checks on them and ignores the
// attention-side bindings.  PackedModel maps experts.bin, checks every
// expert's and projection's CRC32 (ExpertStore.cpp:183-192: reflected
// 0xEDB88320) and hands a layer to DeviceExpertLayer, which lays it out for
// the kernels on the device.  This replaces the reference's scheduler,
// leases and residency tiers for the all-resident case.
#pragma once

#include "hm_moe_block.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <memory>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace hm {
namespace storage {

// ExpertIndex.hpp:15-24
struct ExpertRecord {
    std::uint32_t layer_id{};
    std::uint32_t expert_id{};
    std::uint64_t offset{};
    std::uint64_t size{};
    std::uint32_t quantization_type{};
    std::uint32_t checksum{};

    friend bool operator==(const ExpertRecord&, const ExpertRecord&) = default;
};

enum class ProjectionType : std::uint32_t { Gate = 0, Up = 1, Down = 2 };

// ExpertIndex.hpp:28-41
struct ProjectionRecord {
    std::uint32_t layer_id{};
    std::uint32_t expert_id{};
    ProjectionType projection_type{ProjectionType::Gate};
    std::uint32_t dtype{};
    std::uint32_t rank{};
    std::uint32_t reserved{};
    std::uint64_t offset{};
    std::uint64_t size{};
    std::array<std::uint64_t, 4> shape{};
    std::uint32_t checksum{};
    std::uint32_t trailing_reserved{};

    friend bool operator==(const ProjectionRecord&, const ProjectionRecord&) = default;
};

class StorageError : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

// CRC-32 (IEEE 802.3, reflected polynomial 0xEDB88320, initial value and
// final xor 0xFFFFFFFF), the checksum of experts.index.
[[nodiscard]] std::uint32_t crc32(std::span<const std::byte> bytes) noexcept;

class ExpertIndex {
public:
    static constexpr std::uint32_t formatVersion = 2;
    static constexpr std::uint32_t legacyFormatVersion = 1;
    static constexpr std::size_t serializedRecordSize = 32;
    static constexpr std::size_t serializedProjectionRecordSize = 80;

    ExpertIndex() = default;
    explicit ExpertIndex(std::vector<ExpertRecord> records,
                         std::vector<ProjectionRecord> projections = {});

    [[nodiscard]] static ExpertIndex load(const std::filesystem::path& path);
    void save(const std::filesystem::path& path) const;

    [[nodiscard]] std::optional<ExpertRecord> find(std::uint32_t layerId,
                                                   std::uint32_t expertId) const noexcept;
    [[nodiscard]] std::optional<ProjectionRecord> findProjection(
        std::uint32_t layerId, std::uint32_t expertId, ProjectionType type) const noexcept;
    [[nodiscard]] std::span<const ExpertRecord> records() const noexcept { return records_; }
    [[nodiscard]] std::span<const ProjectionRecord> projections() const noexcept {
        return projections_;
    }
    [[nodiscard]] std::size_t size() const noexcept { return records_.size(); }

private:
    void validateAndIndex();

    std::vector<ExpertRecord> records_;
    std::vector<ProjectionRecord> projections_;
    std::unordered_map<std::uint64_t, std::size_t> lookup_;
    std::unordered_map<std::uint64_t, std::array<std::size_t, 3>> projectionLookup_;
};

}  // namespace storage

namespace models {

enum class TensorLayout : std::uint32_t { InputOutput = 0, OutputInput = 1 };

// ModelManifest.hpp:37-63
struct ManifestTensor {
    std::string name;
    std::string sourceFile;
    std::uint64_t offset{};
    std::uint64_t size{};
    tensor::DType dtype{tensor::DType::FP32};
    std::vector<std::uint64_t> shape;
    std::optional<tensor::quantization::QuantizationParameters> quantization;
};

struct ProjectionLocation {
    std::string tensorName;
    std::uint64_t offset{};
    std::uint64_t size{};
    std::vector<std::uint64_t> shape;
    TensorLayout layout{TensorLayout::OutputInput};
};

struct ManifestExpertMapping {
    std::uint32_t layerId{};
    std::uint32_t expertId{};
    ProjectionLocation gate, up, down;
};

struct ManifestRouterTensor {
    std::uint32_t layerId{};
    std::string tensorName;
};

struct ManifestRouter {
    router::RouterConfig config;
    std::vector<ManifestRouterTensor> tensors;
    TensorLayout layout{TensorLayout::OutputInput};
};

// The block-side view of ModelManifest (schema v3, or legacy v2).
class PackedManifest {
public:
    static constexpr const char* schemaVersion = "hypermoe.model-manifest.v3";
    static constexpr const char* legacySchemaVersion = "hypermoe.model-manifest.v2";

    std::string schema;
    std::string modelName;
    std::size_t layerCount{};
    std::size_t expertCount{};
    std::size_t hiddenSize{};
    std::size_t intermediateSize{};
    ManifestRouter router;
    std::vector<ManifestTensor> tensors;
    std::vector<ManifestExpertMapping> experts;

    [[nodiscard]] static PackedManifest load(const std::filesystem::path& path);
    [[nodiscard]] static PackedManifest parse(const std::string& json);
    [[nodiscard]] const ManifestTensor* findTensor(const std::string& name) const noexcept;
    [[nodiscard]] const ManifestExpertMapping* findExpert(std::uint32_t layerId,
                                                          std::uint32_t expertId) const noexcept;
    // The reference's manifest checks on what the block reads.
    void validate() const;
};

}  // namespace models

// One layer of a packed model in host memory, in DeviceExpertLayer's input
// form: experts back to back, each gate [H x I] | up [H x I] | down [I x H]
// row-major INPUT_OUTPUT.
struct PackedLayer {
    std::vector<std::byte> payload;
    std::vector<ExpertQuantization> quantization;  // INT8 only
    tensor::DType dtype{tensor::DType::INT8};
    std::size_t experts{}, hidden{}, intermediate{};
};

class PackedModel {
public:
    // Opens a packed model directory: index, manifest, and a read-only
    // mapping of experts.bin.  With verifyChecksums, every payload the
    // loader reads is checked against its CRC32 first.
    explicit PackedModel(const std::filesystem::path& directory, bool verifyChecksums = true);
    ~PackedModel();
    PackedModel(const PackedModel&) = delete;
    PackedModel& operator=(const PackedModel&) = delete;

    [[nodiscard]] const models::PackedManifest& manifest() const noexcept { return manifest_; }
    [[nodiscard]] const storage::ExpertIndex& index() const noexcept { return index_; }
    [[nodiscard]] router::RouterConfig routerConfig() const { return manifest_.router.config; }

    // Every expert of the layer, ascending id (StorageError if one is
    // missing, malformed or corrupt).
    [[nodiscard]] PackedLayer readLayer(LayerId layerId) const;
    // The layer's router matrix [H x E] FP32 (INPUT_OUTPUT).
    [[nodiscard]] std::vector<float> readRouter(LayerId layerId) const;
    // readLayer, uploaded and laid out on the backend's device.
    [[nodiscard]] std::shared_ptr<DeviceExpertLayer> loadLayer(
        std::shared_ptr<backend::HipBackend> backend, LayerId layerId) const;

private:
    [[nodiscard]] std::span<const std::byte> bytes(std::uint64_t offset, std::uint64_t size) const;

    std::filesystem::path directory_;
    bool verify_{true};
    storage::ExpertIndex index_;
    models::PackedManifest manifest_;
    const std::byte* map_{nullptr};
    std::size_t mapSize_{};
};

}  // namespace hm
