// artefact.cpp -- the packed model artefact (experts.bin / experts.index /
// manifest.json) read into device-resident expert tables.  The formats and
// validation rules follow the reference's writers and readers
// (src/storage/ExpertIndex.cpp:59-206, src/storage/ExpertStore.cpp:183-192,
// src/models/ModelManifest.cpp:191-345,483-742,
// tools/model_convert/ExpertPacker.cpp:150-280); the code is this build's.
#include "hm_artefact.h"
#include "hm_artefact.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <fstream>
#include <limits>
#include <map>
#include <set>
#include <sstream>
#include <utility>

namespace hm {
namespace storage {
namespace {

constexpr char kMagic[8] = {'H', 'M', 'O', 'E', 'I', 'D', 'X', '\0'};
constexpr std::uint32_t kEndianMarker = 0x01020304u;
constexpr std::size_t kHeaderSize = 32;

struct Crc32Table {
    std::uint32_t t[256];
    Crc32Table() {
        for (std::uint32_t i = 0; i < 256; ++i) {
            std::uint32_t c = i;
            for (int b = 0; b < 8; ++b) c = (c & 1u) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
            t[i] = c;
        }
    }
};

// Little-endian cursor over a byte image of the index file.
class Reader {
public:
    explicit Reader(const std::vector<unsigned char>& b) : b_(b) {}
    template <typename T>
    T get() {
        if (pos_ + sizeof(T) > b_.size()) throw StorageError("truncated expert index");
        T v = 0;
        for (std::size_t i = 0; i < sizeof(T); ++i) v |= static_cast<T>(b_[pos_ + i]) << (8 * i);
        pos_ += sizeof(T);
        return v;
    }
    std::size_t pos() const { return pos_; }

private:
    const std::vector<unsigned char>& b_;
    std::size_t pos_{0};
};

template <typename T>
void put(std::string& out, T v) {
    for (std::size_t i = 0; i < sizeof(T); ++i) out.push_back(static_cast<char>((v >> (8 * i)) & 0xffu));
}

std::uint64_t key(std::uint32_t layer, std::uint32_t expert) {
    return (static_cast<std::uint64_t>(layer) << 32) | expert;
}

bool validQuantizationType(std::uint32_t q) { return q <= 7; }  // Fp32 .. Fp8 (expert.hpp:14-23)
bool validDType(std::uint32_t d) { return d <= 3; }             // FP32 .. INT8

}  // namespace

std::uint32_t crc32(std::span<const std::byte> bytes) noexcept {
    static const Crc32Table table;
    std::uint32_t c = 0xffffffffu;
    for (const std::byte b : bytes) c = table.t[(c ^ std::to_integer<std::uint32_t>(b)) & 0xffu] ^ (c >> 8);
    return ~c;
}

ExpertIndex::ExpertIndex(std::vector<ExpertRecord> records, std::vector<ProjectionRecord> projections)
    : records_(std::move(records)), projections_(std::move(projections)) {
    validateAndIndex();
}

ExpertIndex ExpertIndex::load(const std::filesystem::path& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw StorageError("cannot open expert index: " + path.string());
    std::vector<unsigned char> b((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    if (b.size() < sizeof(kMagic) || std::memcmp(b.data(), kMagic, sizeof(kMagic)) != 0)
        throw StorageError("invalid expert index magic: " + path.string());
    Reader r(b);
    for (std::size_t i = 0; i < sizeof(kMagic); ++i) (void)r.get<std::uint8_t>();
    const auto version = r.get<std::uint32_t>();
    const auto endian = r.get<std::uint32_t>();
    const auto recordSize = r.get<std::uint32_t>();
    const auto extensionSize = r.get<std::uint32_t>();
    const auto count = r.get<std::uint64_t>();
    if (version != legacyFormatVersion && version != formatVersion)
        throw StorageError("unsupported expert index version");
    if (endian != kEndianMarker) throw StorageError("invalid expert index endian marker");
    if (recordSize != serializedRecordSize ||
        (version == legacyFormatVersion && extensionSize != 0) ||
        (version == formatVersion && extensionSize != serializedProjectionRecordSize))
        throw StorageError("unsupported expert index record size");
    const std::uint64_t fileSize = b.size();
    if (count > (std::numeric_limits<std::uint64_t>::max() - kHeaderSize) / serializedRecordSize)
        throw StorageError("expert index size does not match its record count");
    const std::uint64_t baseSize = kHeaderSize + count * serializedRecordSize;
    if (fileSize < baseSize || (version == legacyFormatVersion && fileSize != baseSize))
        throw StorageError("expert index size does not match its record count");
    std::vector<ExpertRecord> records;
    records.reserve(count);
    for (std::uint64_t i = 0; i < count; ++i) {
        ExpertRecord rec;
        rec.layer_id = r.get<std::uint32_t>();
        rec.expert_id = r.get<std::uint32_t>();
        rec.offset = r.get<std::uint64_t>();
        rec.size = r.get<std::uint64_t>();
        rec.quantization_type = r.get<std::uint32_t>();
        rec.checksum = r.get<std::uint32_t>();
        records.push_back(rec);
    }
    std::vector<ProjectionRecord> projections;
    if (version == formatVersion) {
        const auto pcount = r.get<std::uint64_t>();
        const std::uint64_t pbase = baseSize + 8;
        if (pcount > (std::numeric_limits<std::uint64_t>::max() - pbase) /
                         serializedProjectionRecordSize ||
            fileSize != pbase + pcount * serializedProjectionRecordSize)
            throw StorageError("expert projection index size is invalid");
        projections.reserve(pcount);
        for (std::uint64_t i = 0; i < pcount; ++i) {
            ProjectionRecord p;
            p.layer_id = r.get<std::uint32_t>();
            p.expert_id = r.get<std::uint32_t>();
            p.projection_type = static_cast<ProjectionType>(r.get<std::uint32_t>());
            p.dtype = r.get<std::uint32_t>();
            p.rank = r.get<std::uint32_t>();
            p.reserved = r.get<std::uint32_t>();
            p.offset = r.get<std::uint64_t>();
            p.size = r.get<std::uint64_t>();
            for (auto& d : p.shape) d = r.get<std::uint64_t>();
            p.checksum = r.get<std::uint32_t>();
            p.trailing_reserved = r.get<std::uint32_t>();
            projections.push_back(p);
        }
    }
    if (r.pos() != b.size()) throw StorageError("expert index contains trailing data");
    return ExpertIndex(std::move(records), std::move(projections));
}

void ExpertIndex::save(const std::filesystem::path& path) const {
    std::string out(kMagic, sizeof(kMagic));
    put<std::uint32_t>(out, projections_.empty() ? legacyFormatVersion : formatVersion);
    put<std::uint32_t>(out, kEndianMarker);
    put<std::uint32_t>(out, static_cast<std::uint32_t>(serializedRecordSize));
    put<std::uint32_t>(out, projections_.empty()
                                ? 0u
                                : static_cast<std::uint32_t>(serializedProjectionRecordSize));
    put<std::uint64_t>(out, records_.size());
    for (const auto& rec : records_) {
        put(out, rec.layer_id);
        put(out, rec.expert_id);
        put(out, rec.offset);
        put(out, rec.size);
        put(out, rec.quantization_type);
        put(out, rec.checksum);
    }
    if (!projections_.empty()) {
        put<std::uint64_t>(out, projections_.size());
        for (const auto& p : projections_) {
            put(out, p.layer_id);
            put(out, p.expert_id);
            put(out, static_cast<std::uint32_t>(p.projection_type));
            put(out, p.dtype);
            put(out, p.rank);
            put(out, p.reserved);
            put(out, p.offset);
            put(out, p.size);
            for (const auto d : p.shape) put(out, d);
            put(out, p.checksum);
            put(out, p.trailing_reserved);
        }
    }
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw StorageError("cannot create expert index: " + path.string());
    f.write(out.data(), static_cast<std::streamsize>(out.size()));
    if (!f) throw StorageError("failed writing expert index: " + path.string());
}

std::optional<ExpertRecord> ExpertIndex::find(std::uint32_t layerId,
                                              std::uint32_t expertId) const noexcept {
    const auto it = lookup_.find(key(layerId, expertId));
    if (it == lookup_.end()) return std::nullopt;
    return records_[it->second];
}

std::optional<ProjectionRecord> ExpertIndex::findProjection(std::uint32_t layerId,
                                                            std::uint32_t expertId,
                                                            ProjectionType type) const noexcept {
    const auto it = projectionLookup_.find(key(layerId, expertId));
    const auto t = static_cast<std::size_t>(type);
    if (it == projectionLookup_.end() || t >= 3 ||
        it->second[t] == std::numeric_limits<std::size_t>::max())
        return std::nullopt;
    return projections_[it->second[t]];
}

// ExpertIndex.cpp:234-306: sizes, codes, ranges, duplicates and the
// projection records' consistency with their expert payloads.
void ExpertIndex::validateAndIndex() {
    lookup_.clear();
    projectionLookup_.clear();
    for (std::size_t i = 0; i < records_.size(); ++i) {
        const auto& rec = records_[i];
        if (rec.size == 0 || !validQuantizationType(rec.quantization_type))
            throw StorageError("expert index contains an invalid size or quantization code");
        if (rec.offset > std::numeric_limits<std::uint64_t>::max() - rec.size)
            throw StorageError("expert index record range overflows");
        if (!lookup_.emplace(key(rec.layer_id, rec.expert_id), i).second)
            throw StorageError("expert index contains a duplicate layer/expert key");
    }
    constexpr std::size_t none = std::numeric_limits<std::size_t>::max();
    for (std::size_t i = 0; i < projections_.size(); ++i) {
        const auto& p = projections_[i];
        const auto type = static_cast<std::uint32_t>(p.projection_type);
        if (p.size == 0 || p.rank == 0 || p.rank > 4 || !validDType(p.dtype) || p.reserved != 0 ||
            p.trailing_reserved != 0 || type > 2)
            throw StorageError("expert index contains an invalid projection record");
        const auto expert = find(p.layer_id, p.expert_id);
        if (!expert || p.offset < expert->offset ||
            p.offset > std::numeric_limits<std::uint64_t>::max() - p.size ||
            p.offset + p.size > expert->offset + expert->size)
            throw StorageError("projection record escapes its expert payload");
        auto& slot = projectionLookup_.try_emplace(key(p.layer_id, p.expert_id),
                                                   std::array<std::size_t, 3>{none, none, none})
                         .first->second[type];
        if (slot != none) throw StorageError("expert index contains a duplicate projection record");
        slot = i;
        std::uint64_t elements = 1;
        for (std::uint32_t d = 0; d < p.rank; ++d) {
            if (p.shape[d] == 0) throw StorageError("projection record contains a zero dimension");
            if (elements > std::numeric_limits<std::uint64_t>::max() / p.shape[d])
                throw StorageError("projection shape size overflows");
            elements *= p.shape[d];
        }
        for (std::uint32_t d = p.rank; d < 4; ++d)
            if (p.shape[d] != 0)
                throw StorageError("projection has dimensions beyond its declared rank");
        const std::uint64_t width = tensor::sizeOf(static_cast<tensor::DType>(p.dtype));
        if (elements > std::numeric_limits<std::uint64_t>::max() / width || elements * width != p.size)
            throw StorageError("projection shape and dtype do not match its size");
    }
}

}  // namespace storage

// ---------------------------------------------------------------------------
// A small JSON reader (objects, arrays, strings with escapes, numbers,
// literals) for the manifest.
// ---------------------------------------------------------------------------
namespace {

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind{Null};
    bool b{};
    std::string text;  // number literal or string value
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> fields;

    const Json* find(const std::string& k) const {
        for (const auto& f : fields)
            if (f.first == k) return &f.second;
        return nullptr;
    }
    const Json& require(const std::string& k) const {
        if (kind != Object) throw std::invalid_argument("manifest value is not an object");
        const Json* v = find(k);
        if (!v) throw std::invalid_argument("manifest is missing field: " + k);
        return *v;
    }
    const std::string& str() const {
        if (kind != String) throw std::invalid_argument("manifest value is not a string");
        return text;
    }
    bool boolean() const {
        if (kind != Bool) throw std::invalid_argument("manifest value is not a boolean");
        return b;
    }
    const std::vector<Json>& array() const {
        if (kind != Array) throw std::invalid_argument("manifest value is not an array");
        return items;
    }
    std::uint64_t u64() const {
        if (kind != Number || text.empty() || text[0] == '-' ||
            text.find_first_of(".eE") != std::string::npos)
            throw std::invalid_argument("manifest value is not an unsigned integer");
        errno = 0;
        char* end = nullptr;
        const unsigned long long v = std::strtoull(text.c_str(), &end, 10);
        if (errno != 0 || *end != '\0') throw std::invalid_argument("manifest integer is out of range");
        return v;
    }
    std::int64_t i64() const {
        if (kind != Number || text.find_first_of(".eE") != std::string::npos)
            throw std::invalid_argument("manifest value is not an integer");
        errno = 0;
        char* end = nullptr;
        const long long v = std::strtoll(text.c_str(), &end, 10);
        if (errno != 0 || *end != '\0') throw std::invalid_argument("manifest integer is out of range");
        return v;
    }
    double number() const {
        if (kind != Number) throw std::invalid_argument("manifest value is not a number");
        return std::strtod(text.c_str(), nullptr);
    }
};

class JsonParser {
public:
    explicit JsonParser(const std::string& s) : s_(s) {}
    Json parse() {
        Json v = value();
        ws();
        if (i_ != s_.size()) fail("trailing characters");
        return v;
    }

private:
    [[noreturn]] void fail(const char* what) {
        throw std::invalid_argument(std::string("manifest JSON: ") + what + " at offset " +
                                    std::to_string(i_));
    }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
    }
    bool eat(char c) {
        ws();
        if (i_ < s_.size() && s_[i_] == c) {
            ++i_;
            return true;
        }
        return false;
    }
    Json value() {
        if (++depth_ > 64) fail("nesting too deep");
        ws();
        if (i_ >= s_.size()) fail("unexpected end");
        Json v;
        const char c = s_[i_];
        if (c == '{') {
            ++i_;
            v.kind = Json::Object;
            if (!eat('}')) {
                do {
                    ws();
                    std::string k = string();
                    if (!eat(':')) fail("expected ':'");
                    v.fields.emplace_back(std::move(k), value());
                } while (eat(','));
                if (!eat('}')) fail("expected '}'");
            }
        } else if (c == '[') {
            ++i_;
            v.kind = Json::Array;
            if (!eat(']')) {
                do v.items.push_back(value());
                while (eat(','));
                if (!eat(']')) fail("expected ']'");
            }
        } else if (c == '"') {
            v.kind = Json::String;
            v.text = string();
        } else if (s_.compare(i_, 4, "true") == 0) {
            i_ += 4;
            v.kind = Json::Bool;
            v.b = true;
        } else if (s_.compare(i_, 5, "false") == 0) {
            i_ += 5;
            v.kind = Json::Bool;
        } else if (s_.compare(i_, 4, "null") == 0) {
            i_ += 4;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            const std::size_t st = i_;
            if (s_[i_] == '-') ++i_;
            while (i_ < s_.size() && (std::isdigit(static_cast<unsigned char>(s_[i_])) || s_[i_] == '.' ||
                                      s_[i_] == 'e' || s_[i_] == 'E' || s_[i_] == '+' || s_[i_] == '-'))
                ++i_;
            v.kind = Json::Number;
            v.text = s_.substr(st, i_ - st);
        } else {
            fail("unexpected character");
        }
        --depth_;
        return v;
    }
    std::string string() {
        if (i_ >= s_.size() || s_[i_] != '"') fail("expected a string");
        ++i_;
        std::string out;
        while (true) {
            if (i_ >= s_.size()) fail("unterminated string");
            const char c = s_[i_++];
            if (c == '"') break;
            if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (i_ >= s_.size()) fail("bad escape");
            const char e = s_[i_++];
            switch (e) {
            case '"': case '\\': case '/': out.push_back(e); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                if (i_ + 4 > s_.size()) fail("bad \\u escape");
                const unsigned cp = static_cast<unsigned>(std::stoul(s_.substr(i_, 4), nullptr, 16));
                i_ += 4;
                if (cp < 0x80) {
                    out.push_back(static_cast<char>(cp));
                } else if (cp < 0x800) {
                    out.push_back(static_cast<char>(0xc0 | (cp >> 6)));
                    out.push_back(static_cast<char>(0x80 | (cp & 0x3f)));
                } else {
                    out.push_back(static_cast<char>(0xe0 | (cp >> 12)));
                    out.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3f)));
                    out.push_back(static_cast<char>(0x80 | (cp & 0x3f)));
                }
                break;
            }
            default: fail("bad escape");
            }
        }
        return out;
    }

    const std::string& s_;
    std::size_t i_{0};
    int depth_{0};
};

std::size_t asSize(const Json& v, const char* what) {
    const auto x = v.u64();
    if (x == 0 || x > std::numeric_limits<std::size_t>::max())
        throw std::invalid_argument(std::string("manifest ") + what + " must be positive");
    return static_cast<std::size_t>(x);
}

std::uint32_t asId(const Json& v) {
    const auto x = v.u64();
    if (x > std::numeric_limits<std::uint32_t>::max()) throw std::invalid_argument("manifest id is out of range");
    return static_cast<std::uint32_t>(x);
}

tensor::DType parseDType(const std::string& s) {
    if (s == "FP32") return tensor::DType::FP32;
    if (s == "FP16") return tensor::DType::FP16;
    if (s == "BF16") return tensor::DType::BF16;
    if (s == "INT8") return tensor::DType::INT8;
    throw std::invalid_argument("unsupported manifest dtype: " + s);
}

models::TensorLayout parseLayout(const std::string& s) {
    if (s == "INPUT_OUTPUT") return models::TensorLayout::InputOutput;
    if (s == "OUTPUT_INPUT") return models::TensorLayout::OutputInput;
    throw std::invalid_argument("unsupported manifest tensor layout: " + s);
}

std::vector<std::uint64_t> parseShape(const Json& v) {
    std::vector<std::uint64_t> out;
    for (const auto& d : v.array()) out.push_back(d.u64());
    return out;
}

models::ProjectionLocation parseProjection(const Json& v) {
    models::ProjectionLocation p;
    p.tensorName = v.require("tensor").str();
    p.offset = v.require("offset").u64();
    p.size = v.require("size").u64();
    p.shape = parseShape(v.require("shape"));
    p.layout = parseLayout(v.require("layout").str());
    return p;
}

std::uint64_t requiredBytes(const std::vector<std::uint64_t>& shape, tensor::DType dtype) {
    std::uint64_t n = 1;
    for (const auto d : shape) {
        if (d != 0 && n > std::numeric_limits<std::uint64_t>::max() / d)
            throw std::overflow_error("manifest tensor size overflow");
        n *= d;
    }
    const std::uint64_t w = tensor::sizeOf(dtype);
    if (n > std::numeric_limits<std::uint64_t>::max() / w) throw std::overflow_error("manifest tensor size overflow");
    return n * w;
}

}  // namespace

namespace models {

PackedManifest PackedManifest::parse(const std::string& json) {
    const Json root = JsonParser(json).parse();
    PackedManifest m;
    m.schema = root.require("schema").str();
    m.modelName = root.require("model_name").str();
    m.layerCount = asSize(root.require("layer_count"), "layer_count");
    m.expertCount = asSize(root.require("expert_count"), "expert_count");
    m.hiddenSize = asSize(root.require("hidden_size"), "hidden_size");
    m.intermediateSize = asSize(root.require("intermediate_size"), "intermediate_size");
    const Json& rv = root.require("router");
    m.router.config.expertCount = asSize(rv.require("expert_count"), "router expert_count");
    m.router.config.topK = asSize(rv.require("top_k"), "router top_k");
    const auto& norm = rv.require("normalization").str();
    if (norm == "SOFTMAX") m.router.config.normalization = router::RoutingNormalization::Softmax;
    else if (norm == "NONE") m.router.config.normalization = router::RoutingNormalization::None;
    else throw std::invalid_argument("unsupported router normalization");
    m.router.config.renormalizeSelected = rv.require("renormalize_selected").boolean();
    m.router.layout = parseLayout(rv.require("layout").str());
    for (const auto& t : rv.require("tensors").array())
        m.router.tensors.push_back({asId(t.require("layer_id")), t.require("tensor").str()});
    for (const auto& t : root.require("tensors").array()) {
        ManifestTensor mt;
        mt.name = t.require("name").str();
        mt.sourceFile = t.require("source_file").str();
        mt.offset = t.require("offset").u64();
        mt.size = t.require("size").u64();
        mt.dtype = parseDType(t.require("dtype").str());
        mt.shape = parseShape(t.require("shape"));
        if (const Json* q = t.find("quantization")) {
            if (q->require("scheme").str() != "PER_TENSOR_AFFINE_INT8")
                throw std::invalid_argument("unsupported manifest quantization scheme");
            const auto zp = q->require("zero_point").i64();
            if (zp < std::numeric_limits<std::int32_t>::min() || zp > std::numeric_limits<std::int32_t>::max())
                throw std::invalid_argument("manifest zero_point is out of range");
            tensor::quantization::QuantizationParameters p{
                static_cast<float>(q->require("scale").number()), static_cast<std::int32_t>(zp)};
            tensor::quantization::validateInt8Parameters(p);
            mt.quantization = p;
        }
        m.tensors.push_back(std::move(mt));
    }
    for (const auto& e : root.require("experts").array()) {
        ManifestExpertMapping x;
        x.layerId = asId(e.require("layer_id"));
        x.expertId = asId(e.require("expert_id"));
        x.gate = parseProjection(e.require("gate"));
        x.up = parseProjection(e.require("up"));
        x.down = parseProjection(e.require("down"));
        m.experts.push_back(std::move(x));
    }
    m.validate();
    return m;
}

PackedManifest PackedManifest::load(const std::filesystem::path& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw storage::StorageError("cannot open manifest: " + path.string());
    std::stringstream ss;
    ss << in.rdbuf();
    return parse(ss.str());
}

const ManifestTensor* PackedManifest::findTensor(const std::string& name) const noexcept {
    for (const auto& t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

const ManifestExpertMapping* PackedManifest::findExpert(std::uint32_t layerId,
                                                        std::uint32_t expertId) const noexcept {
    for (const auto& e : experts)
        if (e.layerId == layerId && e.expertId == expertId) return &e;
    return nullptr;
}

// ModelManifest.cpp:191-345 on the fields read here.
void PackedManifest::validate() const {
    if (schema != schemaVersion && schema != legacySchemaVersion)
        throw std::invalid_argument("unsupported manifest schema");
    if (layerCount == 0 || expertCount == 0 || hiddenSize == 0 || intermediateSize == 0)
        throw std::invalid_argument("manifest model dimensions must be nonzero");
    router.config.validate();
    if (router.config.expertCount != expertCount)
        throw std::invalid_argument("manifest router expert count disagrees with model");
    if (tensors.empty() || experts.empty() || router.tensors.empty())
        throw std::invalid_argument("manifest must contain router and expert tensors");
    std::map<std::string, const ManifestTensor*> byName;
    for (const auto& t : tensors) {
        if (t.name.empty() || t.size == 0)
            throw std::invalid_argument("manifest tensor identity or size is invalid");
        if (t.sourceFile.empty() || t.sourceFile[0] == '/')
            throw std::invalid_argument("manifest tensor source path must be relative");
        if (t.offset > std::numeric_limits<std::uint64_t>::max() - t.size)
            throw std::overflow_error("manifest tensor byte range overflows");
        if (requiredBytes(t.shape, t.dtype) != t.size)
            throw std::invalid_argument("manifest tensor shape does not match byte size");
        if (t.dtype == tensor::DType::INT8 && !t.quantization)
            throw std::invalid_argument("INT8 manifest tensor is missing quantization metadata");
        if (t.dtype != tensor::DType::INT8 && t.quantization)
            throw std::invalid_argument("non-INT8 manifest tensor has quantization metadata");
        if (!byName.emplace(t.name, &t).second) throw std::invalid_argument("duplicate manifest tensor name");
    }
    std::set<std::uint32_t> routerLayers;
    for (const auto& rt : router.tensors) {
        if (rt.layerId >= layerCount || !routerLayers.insert(rt.layerId).second)
            throw std::invalid_argument("manifest router layer is invalid or duplicated");
        const auto it = byName.find(rt.tensorName);
        if (it == byName.end()) throw std::invalid_argument("manifest router references an unknown tensor");
        const std::vector<std::uint64_t> expected =
            router.layout == TensorLayout::OutputInput
                ? std::vector<std::uint64_t>{expertCount, hiddenSize}
                : std::vector<std::uint64_t>{hiddenSize, expertCount};
        if (it->second->shape != expected)
            throw std::invalid_argument("manifest router tensor shape is incompatible");
    }
    std::set<std::pair<std::uint32_t, std::uint32_t>> ids;
    std::map<std::uint32_t, std::size_t> perLayer;
    auto checkProjection = [&](const ProjectionLocation& p, bool down) {
        const auto it = byName.find(p.tensorName);
        if (it == byName.end()) throw std::invalid_argument("expert projection references an unknown tensor");
        const auto& src = *it->second;
        if (p.size == 0 || p.offset < src.offset ||
            p.offset > std::numeric_limits<std::uint64_t>::max() - p.size ||
            p.offset + p.size > src.offset + src.size)
            throw std::invalid_argument("expert projection range escapes source tensor");
        if (requiredBytes(p.shape, src.dtype) != p.size)
            throw std::invalid_argument("expert projection shape does not match its bytes");
        const bool io = p.layout == TensorLayout::InputOutput;
        const std::vector<std::uint64_t> expected =
            (io != down) ? std::vector<std::uint64_t>{hiddenSize, intermediateSize}
                         : std::vector<std::uint64_t>{intermediateSize, hiddenSize};
        if (p.shape != expected)
            throw std::invalid_argument("expert projection shape and layout are incompatible");
    };
    for (const auto& e : experts) {
        if (e.layerId >= layerCount || e.expertId >= expertCount)
            throw std::invalid_argument("manifest expert identity is outside model bounds");
        if (!ids.emplace(e.layerId, e.expertId).second)
            throw std::invalid_argument("duplicate manifest expert mapping");
        ++perLayer[e.layerId];
        const auto g = byName.find(e.gate.tensorName), u = byName.find(e.up.tensorName),
                   d = byName.find(e.down.tensorName);
        if (g == byName.end() || u == byName.end() || d == byName.end() ||
            g->second->dtype != u->second->dtype || g->second->dtype != d->second->dtype)
            throw std::invalid_argument("expert projections must use one storage dtype");
        checkProjection(e.gate, false);
        checkProjection(e.up, false);
        checkProjection(e.down, true);
    }
    for (const auto& [layer, count] : perLayer) {
        if (count != expertCount)
            throw std::invalid_argument("manifest MoE layer does not contain the declared expert count");
        if (!routerLayers.count(layer)) throw std::invalid_argument("manifest MoE layer has no router tensor");
    }
    for (const auto layer : routerLayers)
        if (!perLayer.count(layer)) throw std::invalid_argument("manifest router layer has no expert mappings");
}

}  // namespace models

// ---------------------------------------------------------------------------
// PackedModel
// ---------------------------------------------------------------------------
namespace {

// Exact widenings of 16-bit payloads to FP32 (FP16/BF16 artefacts are
// served by the FP32 expert path).
float bf16ToFloat(std::uint16_t h) {
    const std::uint32_t u = static_cast<std::uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

float fp16ToFloat(std::uint16_t h) {
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    std::uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, u;
    if (exp == 0x1f) {
        u = sign | 0x7f800000u | (man << 13);  // inf / nan
    } else if (exp != 0) {
        u = sign | ((exp + 112) << 23) | (man << 13);
    } else if (man == 0) {
        u = sign;
    } else {  // subnormal: normalise
        int e = -1;
        do {
            ++e;
            man <<= 1;
        } while ((man & 0x400u) == 0);
        u = sign | (static_cast<std::uint32_t>(112 - e) << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

void appendWidened(std::vector<std::byte>& out, std::span<const std::byte> in, tensor::DType dtype) {
    const std::size_t n = in.size() / 2;
    const std::size_t base = out.size();
    out.resize(base + n * sizeof(float));
    for (std::size_t i = 0; i < n; ++i) {
        std::uint16_t h;
        std::memcpy(&h, in.data() + 2 * i, 2);
        const float f = dtype == tensor::DType::BF16 ? bf16ToFloat(h) : fp16ToFloat(h);
        std::memcpy(out.data() + base + i * sizeof(float), &f, sizeof f);
    }
}

}  // namespace

PackedModel::PackedModel(const std::filesystem::path& directory, bool verifyChecksums)
    : directory_(directory), verify_(verifyChecksums) {
    index_ = storage::ExpertIndex::load(directory / "experts.index");
    manifest_ = models::PackedManifest::load(directory / "manifest.json");
    const auto data = directory / "experts.bin";
    const int fd = ::open(data.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw storage::StorageError("cannot open expert payloads: " + data.string());
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        throw storage::StorageError("cannot stat expert payloads: " + data.string());
    }
    mapSize_ = static_cast<std::size_t>(st.st_size);
    if (mapSize_ > 0) {
        void* p = ::mmap(nullptr, mapSize_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            ::close(fd);
            throw storage::StorageError("cannot map expert payloads: " + data.string());
        }
        map_ = static_cast<const std::byte*>(p);
    }
    ::close(fd);
}

PackedModel::~PackedModel() {
    if (map_) ::munmap(const_cast<std::byte*>(map_), mapSize_);
}

std::span<const std::byte> PackedModel::bytes(std::uint64_t offset, std::uint64_t size) const {
    if (offset > mapSize_ || size > mapSize_ - offset)
        throw storage::StorageError("expert payload range is outside experts.bin");
    return {map_ + offset, static_cast<std::size_t>(size)};
}

PackedLayer PackedModel::readLayer(LayerId layerId) const {
    const auto& m = manifest_;
    const std::size_t E = m.expertCount, H = m.hiddenSize, I = m.intermediateSize;
    PackedLayer out;
    out.experts = E;
    out.hidden = H;
    out.intermediate = I;
    for (std::uint32_t e = 0; e < E; ++e) {
        const auto* map = m.findExpert(layerId, e);
        const auto rec = index_.find(layerId, e);
        if (!map || !rec) throw storage::StorageError("packed model is missing an expert of the layer");
        const auto* gt = m.findTensor(map->gate.tensorName);
        const auto dtype = gt->dtype;  // as stored
        const bool widen = dtype == tensor::DType::FP16 || dtype == tensor::DType::BF16;
        const auto table = widen ? tensor::DType::FP32 : dtype;
        if (e == 0) {
            out.dtype = table;
            out.payload.reserve(E * 3 * H * I * tensor::sizeOf(table));
        } else if (table != out.dtype) {
            throw storage::StorageError("experts of one layer use different dtypes");
        }
        const auto expert = bytes(rec->offset, rec->size);
        if (verify_ && storage::crc32(expert) != rec->checksum)
            throw storage::StorageError("expert payload checksum mismatch");
        ExpertQuantization q{};
        const models::ProjectionLocation* locs[3] = {&map->gate, &map->up, &map->down};
        tensor::quantization::QuantizationParameters* qs[3] = {&q.gate, &q.up, &q.down};
        for (int p = 0; p < 3; ++p) {
            const auto& loc = *locs[p];
            if (loc.layout != models::TensorLayout::InputOutput)
                throw storage::StorageError("packed expert projections must be INPUT_OUTPUT");
            const auto* t = m.findTensor(loc.tensorName);
            if (t->sourceFile != "experts.bin")
                throw storage::StorageError("packed expert projection is not in experts.bin");
            if (loc.offset < rec->offset || loc.offset + loc.size > rec->offset + rec->size)
                throw storage::StorageError("projection escapes its expert payload");
            const auto proj = bytes(loc.offset, loc.size);
            if (const auto pr = index_.findProjection(layerId, e, static_cast<storage::ProjectionType>(p))) {
                if (pr->offset != loc.offset || pr->size != loc.size ||
                    pr->dtype != static_cast<std::uint32_t>(dtype))
                    throw storage::StorageError("projection record disagrees with the manifest");
                if (verify_ && storage::crc32(proj) != pr->checksum)
                    throw storage::StorageError("projection payload checksum mismatch");
            }
            if (dtype == tensor::DType::INT8) *qs[p] = *t->quantization;
            if (widen) appendWidened(out.payload, proj, dtype);
            else out.payload.insert(out.payload.end(), proj.begin(), proj.end());
        }
        if (dtype == tensor::DType::INT8) out.quantization.push_back(q);
    }
    return out;
}

std::vector<float> PackedModel::readRouter(LayerId layerId) const {
    const auto& m = manifest_;
    for (const auto& rt : m.router.tensors) {
        if (rt.layerId != layerId) continue;
        const auto* t = m.findTensor(rt.tensorName);
        if (t->dtype != tensor::DType::FP32 || t->sourceFile != "experts.bin")
            throw storage::StorageError("packed router must be FP32 in experts.bin");
        if (m.router.layout != models::TensorLayout::InputOutput)
            throw storage::StorageError("packed router must be INPUT_OUTPUT [H x E]");
        const auto b = bytes(t->offset, t->size);
        std::vector<float> w(b.size() / sizeof(float));
        std::memcpy(w.data(), b.data(), w.size() * sizeof(float));
        return w;
    }
    throw storage::StorageError("packed model has no router for the layer");
}

std::shared_ptr<DeviceExpertLayer> PackedModel::loadLayer(std::shared_ptr<backend::HipBackend> backend,
                                                          LayerId layerId) const {
    const auto layer = readLayer(layerId);
    return DeviceExpertLayer::fromPayload(std::move(backend), layer.payload, layer.experts,
                                          layer.hidden, layer.intermediate, layer.dtype,
                                          layer.quantization);
}

}  // namespace hm

// ---------------------------------------------------------------------------
// C ABI (include/hm_artefact.h)
// ---------------------------------------------------------------------------
namespace {
thread_local std::string tl_error;

template <typename F>
int guarded(F&& f) {
    try {
        f();
        tl_error.clear();
        return HM_OK;
    } catch (const hm::storage::StorageError& e) {
        tl_error = e.what();
        return HM_ERR_STORAGE;
    } catch (const std::overflow_error& e) {
        tl_error = e.what();
        return HM_ERR_OVERFLOW;
    } catch (const std::invalid_argument& e) {
        tl_error = e.what();
        return HM_ERR_INVALID;
    } catch (const std::exception& e) {
        tl_error = e.what();
        return HM_ERR_RUNTIME;
    }
}
}  // namespace

struct hm_packed_model {
    std::unique_ptr<hm::PackedModel> model;
};

extern "C" {

const char* hm_artefact_last_error(void) { return tl_error.c_str(); }

uint32_t hm_crc32(const void* data, size_t bytes) {
    return hm::storage::crc32({static_cast<const std::byte*>(data), bytes});
}

int hm_index_read(const char* path, hm_index_record* records, size_t record_capacity,
                  hm_projection_record* projections, size_t projection_capacity,
                  size_t* record_count, size_t* projection_count) {
    if (!path || !record_count || !projection_count) return HM_ERR_INVALID;
    return guarded([&] {
        const auto index = hm::storage::ExpertIndex::load(path);
        *record_count = index.records().size();
        *projection_count = index.projections().size();
        if (records)
            for (std::size_t i = 0; i < std::min(record_capacity, index.records().size()); ++i) {
                const auto& r = index.records()[i];
                records[i] = {r.layer_id, r.expert_id, r.offset, r.size, r.quantization_type, r.checksum};
            }
        if (projections)
            for (std::size_t i = 0; i < std::min(projection_capacity, index.projections().size()); ++i) {
                const auto& p = index.projections()[i];
                auto& o = projections[i];
                o = {p.layer_id, p.expert_id, static_cast<uint32_t>(p.projection_type), p.dtype, p.rank,
                     p.reserved, p.offset, p.size, {p.shape[0], p.shape[1], p.shape[2], p.shape[3]},
                     p.checksum, p.trailing_reserved};
            }
    });
}

int hm_index_write(const char* path, const hm_index_record* records, size_t record_count,
                   const hm_projection_record* projections, size_t projection_count) {
    if (!path || (record_count && !records) || (projection_count && !projections)) return HM_ERR_INVALID;
    return guarded([&] {
        std::vector<hm::storage::ExpertRecord> rs;
        for (std::size_t i = 0; i < record_count; ++i) {
            const auto& r = records[i];
            rs.push_back({r.layer_id, r.expert_id, r.offset, r.size, r.quantization_type, r.checksum});
        }
        std::vector<hm::storage::ProjectionRecord> ps;
        for (std::size_t i = 0; i < projection_count; ++i) {
            const auto& p = projections[i];
            hm::storage::ProjectionRecord o;
            o.layer_id = p.layer_id;
            o.expert_id = p.expert_id;
            o.projection_type = static_cast<hm::storage::ProjectionType>(p.projection_type);
            o.dtype = p.dtype;
            o.rank = p.rank;
            o.reserved = p.reserved;
            o.offset = p.offset;
            o.size = p.size;
            for (int d = 0; d < 4; ++d) o.shape[d] = p.shape[d];
            o.checksum = p.checksum;
            o.trailing_reserved = p.trailing_reserved;
            ps.push_back(o);
        }
        hm::storage::ExpertIndex(std::move(rs), std::move(ps)).save(path);
    });
}

int hm_packed_open(const char* directory, int verify_checksums, hm_packed_model** out) {
    if (!directory || !out) return HM_ERR_INVALID;
    *out = nullptr;
    return guarded([&] {
        auto m = std::make_unique<hm_packed_model>();
        m->model = std::make_unique<hm::PackedModel>(directory, verify_checksums != 0);
        *out = m.release();
    });
}

void hm_packed_close(hm_packed_model* model) { delete model; }

int hm_packed_info(const hm_packed_model* model, hm_packed_model_info* info) {
    if (!model || !info) return HM_ERR_INVALID;
    return guarded([&] {
        const auto& m = model->model->manifest();
        info->layers = static_cast<uint32_t>(m.layerCount);
        info->experts = static_cast<uint32_t>(m.expertCount);
        info->hidden = m.hiddenSize;
        info->intermediate = m.intermediateSize;
        info->top_k = static_cast<uint32_t>(m.router.config.topK);
        info->route_flags =
            (m.router.config.normalization == hm::router::RoutingNormalization::Softmax ? 1u : 0u) |
            (m.router.config.renormalizeSelected ? 2u : 0u);
        const auto* e0 = m.experts.empty() ? nullptr : m.findTensor(m.experts.front().gate.tensorName);
        info->dtype = e0 && e0->dtype == hm::tensor::DType::INT8 ? 3u : 0u;
    });
}

int hm_packed_read_layer(const hm_packed_model* model, uint32_t layer, void* payload,
                         size_t payload_bytes, float* scale, int32_t* zero_point) {
    if (!model || !payload) return HM_ERR_INVALID;
    return guarded([&] {
        const auto l = model->model->readLayer(layer);
        if (payload_bytes != l.payload.size())
            throw std::invalid_argument("payload buffer size does not match the layer");
        std::memcpy(payload, l.payload.data(), l.payload.size());
        if (l.dtype == hm::tensor::DType::INT8) {
            if (!scale || !zero_point) throw std::invalid_argument("INT8 layer needs scale and zero point buffers");
            for (std::size_t e = 0; e < l.quantization.size(); ++e) {
                const auto& q = l.quantization[e];
                const hm::tensor::quantization::QuantizationParameters* ps[3] = {&q.gate, &q.up, &q.down};
                for (int p = 0; p < 3; ++p) {
                    scale[3 * e + p] = ps[p]->scale;
                    zero_point[3 * e + p] = ps[p]->zeroPoint;
                }
            }
        }
    });
}

int hm_packed_read_router(const hm_packed_model* model, uint32_t layer, float* w, size_t count) {
    if (!model || !w) return HM_ERR_INVALID;
    return guarded([&] {
        const auto r = model->model->readRouter(layer);
        if (count != r.size()) throw std::invalid_argument("router buffer size does not match [H x E]");
        std::memcpy(w, r.data(), r.size() * sizeof(float));
    });
}

}  // extern "C"
