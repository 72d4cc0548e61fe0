// test_host.cpp -- tests of the C++20 host layer (HipBackend,
// HipTensorBackend, HipMoEBlock), in the reference's expect() style
// (tests/phase*_tests.cpp).  Checks come from the CPU oracle
// (oracle/hm_oracle.h), the closed forms of the reference's tests and the
// invariants of the result types.
//
//   test_host cpu   argument checks and host logic; needs no GPU
//   test_host gpu   device behaviour on cuda:0 (HIP)
#include "hm_backend.hpp"
#include "hm_moe.h"
#include "hm_moe_block.hpp"
#include "hm_tensor.hpp"

#include "hm_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

extern "C" {
void hm_synth_normal(uint64_t seed, uint64_t tag, int64_t n, float mean, float std, float* out);
int hm_synth_layer(uint64_t seed, uint64_t layer, int64_t experts, int64_t hidden, int64_t inter,
                   float std, int int8, void* payload, float* scale, int32_t* zp, int threads);
}

using namespace hm;
using tensor::DType;
using tensor::Shape;
using tensor::Tensor;
using tensor::TensorView;

namespace {

int g_checks = 0, g_failures = 0;

void expect(bool cond, const std::string& what) {
    ++g_checks;
    if (!cond) {
        ++g_failures;
        std::fprintf(stderr, "FAIL: %s\n", what.c_str());
    }
}

template <class E>
void expectThrows(const std::function<void()>& f, const std::string& what) {
    ++g_checks;
    try {
        f();
    } catch (const E&) {
        return;
    } catch (const std::exception& e) {
        ++g_failures;
        std::fprintf(stderr, "FAIL: %s: wrong exception: %s\n", what.c_str(), e.what());
        return;
    }
    ++g_failures;
    std::fprintf(stderr, "FAIL: %s: no exception\n", what.c_str());
}

uint32_t bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

bool bitexact(const float* a, const float* b, std::size_t n, std::size_t* first = nullptr) {
    for (std::size_t i = 0; i < n; ++i) {
        if (bits(a[i]) != bits(b[i])) {
            if (first) *first = i;
            return false;
        }
    }
    return true;
}

// ---------------------------------------------------------------- CPU tests

void cpuTests() {
    // Shape and sizes
    expectThrows<std::invalid_argument>([] { Shape s{2, 0}; }, "zero dimension rejected");
    expectThrows<std::overflow_error>(
        [] { Shape s{std::size_t{1} << 40, std::size_t{1} << 40}; }, "element count overflow");
    expect(Shape({3, 4}).elementCount() == 12, "element count");
    expectThrows<std::overflow_error>(
        [] { (void)tensor::tensorBytes(Shape{std::size_t{1} << 62}, DType::FP32); },
        "byte size overflow");

    // TensorView never extends the storage lifetime (TensorView.hpp:10-11)
    TensorView v;
    {
        auto t = tensor::allocateHostTensor(Shape{2, 3}, DType::FP32);
        v = t.view();
        expect(v.valid() && v.writable() && v.bytes() == 24, "view of a live tensor");
    }
    expect(!v.valid() && v.lockOwner() == nullptr, "view expires with its tensor");
    {
        const auto t = tensor::allocateHostTensor(Shape{4}, DType::INT8);
        expect(!TensorView(t).writable(), "view of a const tensor is read-only");
        expectThrows<std::invalid_argument>([&] { (void)t.reshape(Shape{3}); },
                                            "reshape keeps the element count");
    }

    // Quantization parameters (Quantization.cpp:24-43)
    using tensor::quantization::QuantizationParameters;
    using tensor::quantization::validateInt8Parameters;
    expectThrows<std::invalid_argument>([] { validateInt8Parameters({0.0F, 0}); }, "scale 0");
    expectThrows<std::invalid_argument>([] { validateInt8Parameters({NAN, 0}); }, "scale NaN");
    expectThrows<std::invalid_argument>([] { validateInt8Parameters({1.0F, 128}); }, "zp 128");
    expectThrows<std::invalid_argument>([] { validateInt8Parameters({1.0F, -129}); }, "zp -129");
    validateInt8Parameters({0.5F, -128});

    // RouterConfig::validate (RouterConfig.cpp:9-22)
    router::RouterConfig rc{8, 0, router::RoutingNormalization::Softmax, true};
    expectThrows<std::invalid_argument>([&] { rc.validate(); }, "top-k 0");
    rc.topK = 9;
    expectThrows<std::invalid_argument>([&] { rc.validate(); }, "top-k > experts");
    rc.topK = 8;
    rc.validate();

    // ExpertBatch::validate (ExpertBatch.cpp:9-22)
    ExpertBatch b{0, 1, {0, 2}, {0.5F, 0.25F}};
    b.validate(3);
    expect(b.size() == 2, "batch size");
    expectThrows<std::invalid_argument>([&] { b.validate(2); }, "token index out of range");
    ExpertBatch dup{0, 1, {1, 1}, {0.5F, 0.5F}};
    expectThrows<std::invalid_argument>([&] { dup.validate(3); }, "duplicate token");
    ExpertBatch nan{0, 1, {1}, {NAN}};
    expectThrows<std::invalid_argument>([&] { nan.validate(3); }, "non-finite weight");
    ExpertBatch ragged{0, 1, {1, 2}, {0.5F}};
    expectThrows<std::invalid_argument>([&] { ragged.validate(3); }, "ragged metadata");

    // Status mapping (hm_moe.h conventions)
    expectThrows<std::invalid_argument>([] { backend::throwOnStatus(HM_ERR_INVALID, "x"); },
                                        "HM_ERR_INVALID -> invalid_argument");
    expectThrows<std::overflow_error>([] { backend::throwOnStatus(HM_ERR_OVERFLOW, "x"); },
                                      "HM_ERR_OVERFLOW -> overflow_error");
    expectThrows<std::runtime_error>([] { backend::throwOnStatus(HM_ERR_RUNTIME, "x"); },
                                     "HM_ERR_RUNTIME -> runtime_error");
    backend::throwOnStatus(HM_OK, "ok");

    // A backend without a device (this process has none) refuses device work
    auto hip = std::make_shared<backend::HipBackend>(0);
    expect(hip->kind() == backend::BackendKind::Hip && hip->deviceOrdinal() == 0, "backend id");
    if (!hip->isAvailable()) {
        expectThrows<std::runtime_error>([&] { (void)hip->allocate(64); },
                                         "allocate without a device");
        expectThrows<std::runtime_error>([&] { hip->synchronize(); }, "sync without a device");
        expect(!hip->supportsPinnedMemory(), "no pinned memory without a device");
    }
    expectThrows<std::invalid_argument>([&] { (void)hip->allocate(0); }, "zero-byte allocation");
    expectThrows<std::invalid_argument>([] { backend::HipBackend bad(-1); }, "negative ordinal");

    tensor::HipTensorBackend tb(hip);
    auto h1 = tensor::allocateHostTensor(Shape{2, 2}, DType::FP32);
    auto h2 = tensor::allocateHostTensor(Shape{2, 2}, DType::FP32);
    auto h3 = tensor::allocateHostTensor(Shape{2, 2}, DType::FP32);
    expectThrows<std::invalid_argument>([&] { tb.add(h1.view(), h2.view(), h3.view()); },
                                        "HIP add rejects host tensors");
    expectThrows<std::invalid_argument>(
        [&] { tb.matmulInt8Weights(h1.view(), h2.view(), {0.0F, 0}, h3.view()); },
        "INT8 matmul validates its parameters first");

    expectThrows<std::invalid_argument>(
        [&] {
            HipMoEBlock blk(hip, router::RouterConfig{8, 9, router::RoutingNormalization::Softmax,
                                                       true});
        },
        "block validates its router config");
    expectThrows<std::invalid_argument>(
        [&] {
            BlockOptions o;
            o.limbsX = 4;
            HipMoEBlock blk(hip, router::RouterConfig{8, 2, router::RoutingNormalization::Softmax,
                                                       true},
                            o);
        },
        "block validates its digit planes");
}

// ---------------------------------------------------------------- GPU tests

void backendTests(const std::shared_ptr<backend::HipBackend>& hip) {
    const std::size_t n = 1 << 20;
    std::vector<float> src(n), dst(n, -1.0F);
    for (std::size_t i = 0; i < n; ++i) src[i] = (float)i * 0.5F;
    void* d = hip->allocate(n * 4);
    const auto before = hip->stats();
    hip->copyToDevice(d, src.data(), n * 4);
    hip->copyFromDevice(dst.data(), d, n * 4);
    expect(std::memcmp(src.data(), dst.data(), n * 4) == 0, "device round trip");
    const auto after = hip->stats();
    expect(after.hostToDeviceBytes - before.hostToDeviceBytes == n * 4 &&
               after.deviceToHostBytes - before.deviceToHostBytes == n * 4,
           "transfer statistics");
    expect(after.allocatedBytes >= n * 4 && after.peakAllocatedBytes >= after.allocatedBytes,
           "allocation statistics");
    hip->free(d);
    expect(hip->stats().allocatedBytes + n * 4 == after.allocatedBytes, "free updates stats");
    const auto mi = hip->getMemoryInfo();
    expect(mi.totalBytes > (std::uint64_t{100} << 30) && mi.freeBytes <= mi.totalBytes,
           "memory info of an MI355X");

    void* p = hip->allocatePinned(4096);
    expect(p != nullptr && hip->supportsPinnedMemory(), "pinned allocation");
    auto s = hip->createStream();
    auto e0 = hip->createEvent(), e1 = hip->createEvent();
    void* d2 = hip->allocate(4096);
    hip->recordEvent(e0, s);
    hip->copyToDevice(d2, p, 4096, s);
    hip->recordEvent(e1, s);
    hip->waitEvent(e1);
    float ms = -1.0F;
    expect(hm_event_elapsed_ms(&ms, e0, e1) == HM_OK && ms >= 0.0F, "event timing");
    hip->destroyEvent(e0);
    hip->destroyEvent(e1);
    hip->destroyStream(s);
    hip->free(d2);
    hip->freePinned(p);
}

void tensorBackendTests(const std::shared_ptr<backend::HipBackend>& hip) {
    tensor::HipTensorBackend tb(hip);
    expect(tb.available() && tb.device() == tensor::Device::hip(0), "tensor backend device");

    // copyTensor in every direction
    auto host = tensor::allocateHostTensor(Shape{3, 5}, DType::FP32);
    auto* hv = static_cast<float*>(host.data());
    for (int i = 0; i < 15; ++i) hv[i] = (float)i - 7.25F;
    auto dev = tb.allocateTensor(Shape{3, 5}, DType::FP32);
    auto dev2 = tb.allocateTensor(Shape{3, 5}, DType::FP32);
    auto back = tensor::allocateHostTensor(Shape{3, 5}, DType::FP32);
    tb.copyTensor(host.view(), dev.view());
    tb.copyTensor(dev.view(), dev2.view());
    tb.copyTensor(dev2.view(), back.view());
    expect(std::memcmp(host.data(), back.data(), 60) == 0, "copyTensor H2D/D2D/D2H");
    auto wrong = tb.allocateTensor(Shape{5, 3}, DType::FP32);
    expectThrows<std::invalid_argument>([&] { tb.copyTensor(dev.view(), wrong.view()); },
                                        "copy shape mismatch");

    // matmulInt8Weights vs the reference arithmetic at the reference's INT8
    // GEMM test inputs (tests/phase23_tests.cpp:189-240): x = ((i%29)-14)/29,
    // q = ((i*13)%255)-127, scale 0.003, zp -3; tolerance 1e-5 + 1e-5|ref|.
    const std::size_t shapes[][3] = {{1, 8, 8},    {1, 257, 65},  {2, 513, 33},  {1, 1031, 31},
                                     {1, 2048, 768}, {1, 768, 2048}, {3, 129, 7}, {1, 4097, 67}};
    for (const auto& sh : shapes) {
        const std::size_t M = sh[0], K = sh[1], N = sh[2];
        auto x = tensor::allocateHostTensor(Shape{M, K}, DType::FP32);
        auto q = tensor::allocateHostTensor(Shape{K, N}, DType::INT8);
        auto* xp = static_cast<float*>(x.data());
        auto* qp = static_cast<int8_t*>(q.data());
        for (std::size_t i = 0; i < M * K; ++i) xp[i] = (float)((int)(i % 29) - 14) / 29.0F;
        for (std::size_t i = 0; i < K * N; ++i) qp[i] = (int8_t)((int)((i * 13) % 255) - 127);
        auto dx = tb.allocateTensor(x.shape(), DType::FP32);
        auto dq = tb.allocateTensor(q.shape(), DType::INT8);
        auto dy = tb.allocateTensor(Shape{M, N}, DType::FP32);
        tb.copyTensor(x.view(), dx.view());
        tb.copyTensor(q.view(), dq.view());
        tb.matmulInt8Weights(dx.view(), dq.view(), {0.003F, -3}, dy.view());
        auto y = tensor::allocateHostTensor(Shape{M, N}, DType::FP32);
        tb.copyTensor(dy.view(), y.view());
        std::vector<float> ref(M * N);
        hmo_matmul_w8a32(xp, qp, 0.003F, -3, ref.data(), (int64_t)M, (int64_t)K, (int64_t)N);
        const auto* yp = static_cast<const float*>(y.data());
        bool ok = true;
        for (std::size_t i = 0; i < M * N; ++i) {
            ok &= std::fabs(yp[i] - ref[i]) <= 1e-5F + 1e-5F * std::fabs(ref[i]);
        }
        expect(ok, "matmulInt8Weights " + std::to_string(M) + "x" + std::to_string(K) + "x" +
                       std::to_string(N) + " within 1e-5 of the CPU path");
        expectThrows<std::invalid_argument>(
            [&] { tb.matmulInt8Weights(dx.view(), dq.view(), {0.003F, -3}, dx.view()); },
            "INT8 matmul output cannot alias an input");
    }
    {
        auto dx = tb.allocateTensor(Shape{2, 8}, DType::FP32);
        auto dq = tb.allocateTensor(Shape{9, 4}, DType::INT8);
        auto dy = tb.allocateTensor(Shape{2, 4}, DType::FP32);
        expectThrows<std::invalid_argument>(
            [&] { tb.matmulInt8Weights(dx.view(), dq.view(), {1.0F, 0}, dy.view()); },
            "INT8 matmul dimension mismatch");
    }

    // FP32 matmul vs the oracle's sequential float loop (tolerance: the
    // device sums in another order)
    {
        const std::size_t M = 7, K = 300, N = 45;
        std::vector<float> a(M * K), w(K * N), ref(M * N);
        hm_synth_normal(3, 900, (int64_t)a.size(), 0.0F, 1.0F, a.data());
        hm_synth_normal(3, 901, (int64_t)w.size(), 0.0F, 0.02F, w.data());
        hmo_matmul_f32(a.data(), w.data(), ref.data(), (int64_t)M, (int64_t)K, (int64_t)N);
        auto da = tb.allocateTensor(Shape{M, K}, DType::FP32);
        auto dw = tb.allocateTensor(Shape{K, N}, DType::FP32);
        auto dy = tb.allocateTensor(Shape{M, N}, DType::FP32);
        hip->copyToDevice(da.data(), a.data(), a.size() * 4);
        hip->copyToDevice(dw.data(), w.data(), w.size() * 4);
        tb.matmul(da.view(), dw.view(), dy.view());
        tb.synchronizeExecution();
        std::vector<float> y(M * N);
        hip->copyFromDevice(y.data(), dy.data(), y.size() * 4);
        float maxd = 0, maxr = 0;
        for (std::size_t i = 0; i < y.size(); ++i) {
            maxd = std::max(maxd, std::fabs(y[i] - ref[i]));
            maxr = std::max(maxr, std::fabs(ref[i]));
        }
        expect(maxd <= 1e-5F * maxr, "FP32 matmul normwise within 1e-5");
    }

    // add / mul: one rounding each, bit-exact against the host
    {
        const std::size_t n = 1000;
        std::vector<float> a(n), b(n), s(n), p(n);
        hm_synth_normal(4, 1, (int64_t)n, 0.0F, 1.0F, a.data());
        hm_synth_normal(4, 2, (int64_t)n, 0.0F, 1.0F, b.data());
        auto da = tb.allocateTensor(Shape{n}, DType::FP32);
        auto db = tb.allocateTensor(Shape{n}, DType::FP32);
        auto dc = tb.allocateTensor(Shape{n}, DType::FP32);
        auto dd = tb.allocateTensor(Shape{n}, DType::FP32);
        hip->copyToDevice(da.data(), a.data(), n * 4);
        hip->copyToDevice(db.data(), b.data(), n * 4);
        tb.add(da.view(), db.view(), dc.view());
        tb.mul(da.view(), db.view(), dd.view());
        tb.synchronizeExecution();
        hip->copyFromDevice(s.data(), dc.data(), n * 4);
        hip->copyFromDevice(p.data(), dd.data(), n * 4);
        bool ok = true;
        for (std::size_t i = 0; i < n; ++i) {
            volatile float ss = a[i] + b[i], pp = a[i] * b[i];
            ok &= bits(ss) == bits(s[i]) && bits(pp) == bits(p[i]);
        }
        expect(ok, "add/mul bit-exact");
        auto small = tb.allocateTensor(Shape{n - 1}, DType::FP32);
        expectThrows<std::invalid_argument>([&] { tb.add(da.view(), small.view(), dc.view()); },
                                            "add shape mismatch");
    }
}

struct SynthLayer {
    std::vector<std::byte> payload;
    std::vector<float> scale;
    std::vector<int32_t> zp;
    std::vector<ExpertQuantization> q;
};

SynthLayer synthLayer(uint64_t seed, std::size_t E, std::size_t H, std::size_t I, bool int8) {
    SynthLayer s;
    s.payload.resize(E * 3 * H * I * (int8 ? 1 : 4));
    s.scale.resize(E * 3);
    s.zp.resize(E * 3);
    hm_synth_layer(seed, 0, (int64_t)E, (int64_t)H, (int64_t)I, 0.02F, int8 ? 1 : 0,
                   s.payload.data(), s.scale.data(), s.zp.data(), 8);
    if (int8) {
        for (std::size_t e = 0; e < E; ++e) {
            s.q.push_back({{s.scale[3 * e], s.zp[3 * e]},
                           {s.scale[3 * e + 1], s.zp[3 * e + 1]},
                           {s.scale[3 * e + 2], s.zp[3 * e + 2]}});
        }
    }
    return s;
}

void blockTests(const std::shared_ptr<backend::HipBackend>& hip) {
    tensor::HipTensorBackend tb(hip);
    const std::size_t T = 37, H = 512, E = 16, I = 256, k = 4;
    auto L = synthLayer(21, E, H, I, true);
    auto layer = DeviceExpertLayer::fromPayload(hip, L.payload, E, H, I, DType::INT8, L.q);
    std::vector<float> raw(T * H), h(T * H), w(H * E), gamma(H, 1.0F);
    hm_synth_normal(21, 1, (int64_t)raw.size(), 0.0F, 1.0F, raw.data());
    hmo_rmsnorm(raw.data(), gamma.data(), h.data(), (int64_t)T, (int64_t)H, 1e-6F);
    hm_synth_normal(21, 1000, (int64_t)w.size(), 0.0F, 0.02F, w.data());
    auto dh = tb.allocateTensor(Shape{T, H}, DType::FP32);
    auto dw = tb.allocateTensor(Shape{H, E}, DType::FP32);
    hip->copyToDevice(dh.data(), h.data(), h.size() * 4);
    hip->copyToDevice(dw.data(), w.data(), w.size() * 4);

    HipMoEBlock block(hip, {E, k, router::RoutingNormalization::Softmax, true});
    block.addLayer(7, layer);
    auto res = block.executeBatch(7, dh.view(), dw.view());

    hmo_layer ol{(int64_t)E, (int64_t)H, (int64_t)I, 1, L.payload.data(), L.scale.data(),
                 L.zp.data()};
    std::vector<float> lout(T * H), lsc(T * k);
    std::vector<uint32_t> lids(T * k);
    hmo_moe_block_limbs(&ol, h.data(), w.data(), (int64_t)T, (int32_t)k, 1, 1, 2, 3, lout.data(),
                        lids.data(), lsc.data());
    bool idsOk = res.routing.tokens.size() == T && res.routing.layerId == 7;
    for (std::size_t t = 0; t < T && idsOk; ++t) {
        const auto& d = res.routing.tokens[t];
        idsOk &= d.layerId == 7 && d.selectedExpertIds.size() == k;
        for (std::size_t r = 0; r < k && idsOk; ++r) {
            idsOk &= d.selectedExpertIds[r] == lids[t * k + r] &&
                     bits(d.routingScores[r]) == bits(lsc[t * k + r]);
        }
    }
    expect(idsOk, "routing ids and scores bit-exact vs the oracle");
    std::vector<float> out(T * H);
    hip->copyFromDevice(out.data(), res.output.data(), out.size() * 4);
    std::size_t first = 0;
    expect(bitexact(out.data(), lout.data(), out.size(), &first),
           "block output bit-exact vs the limb oracle (first diff " + std::to_string(first) + ")");
    std::vector<float> rout(T * H);
    hmo_moe_block(&ol, h.data(), w.data(), (int64_t)T, (int32_t)k, 1, 1, rout.data(), nullptr,
                  nullptr);
    float maxd = 0, maxr = 0;
    for (std::size_t i = 0; i < out.size(); ++i) {
        maxd = std::max(maxd, std::fabs(out[i] - rout[i]));
        maxr = std::max(maxr, std::fabs(rout[i]));
    }
    expect(maxd <= 1e-4F * maxr, "block output within 1e-4 of the reference W8A32 path");

    // groups: ascending expert id, tokens ascending, sizes sum to T*k
    std::size_t total = 0;
    bool groupsOk = res.expertBatches.size() == res.routing.expertGroups.size() &&
                    res.expertOutputs.size() == res.expertBatches.size();
    for (std::size_t g = 0; g < res.expertBatches.size() && groupsOk; ++g) {
        const auto& b = res.expertBatches[g];
        groupsOk &= b.layerId == 7 && (g == 0 || res.expertBatches[g - 1].expertId < b.expertId);
        groupsOk &= std::is_sorted(b.tokenIndices.begin(), b.tokenIndices.end());
        groupsOk &= res.expertOutputs[g].shape() == Shape({b.size(), H});
        for (std::size_t i = 0; i < b.size(); ++i) {
            const auto& d = res.routing.tokens[b.tokenIndices[i]];
            const auto it = std::find(d.selectedExpertIds.begin(), d.selectedExpertIds.end(),
                                      b.expertId);
            groupsOk &= it != d.selectedExpertIds.end() &&
                        bits(d.routingScores[it - d.selectedExpertIds.begin()]) ==
                            bits(b.routingWeights[i]);
        }
        total += b.size();
    }
    expect(groupsOk && total == T * k, "expert batches are the stable grouping of the routing");
    expect(res.execution.expertAssignments == T * k &&
               res.execution.uniqueExperts == res.expertBatches.size() &&
               res.execution.expertPayloadBytes == res.execution.uniqueExperts * 3 * H * I &&
               res.execution.expertExecutionTime.count() > 0,
           "execution metadata");

    // expert outputs: the combine of the per-expert outputs is the output
    {
        std::vector<float> comb(T * H, 0.0F);
        std::vector<float> ye;
        for (std::size_t g = 0; g < res.expertBatches.size(); ++g) {
            const auto& b = res.expertBatches[g];
            ye.resize(b.size() * H);
            hip->copyFromDevice(ye.data(), res.expertOutputs[g].data(), ye.size() * 4);
            for (std::size_t i = 0; i < b.size(); ++i) {
                for (std::size_t c = 0; c < H; ++c) {
                    volatile float prod = b.routingWeights[i] * ye[i * H + c];
                    comb[b.tokenIndices[i] * H + c] += prod;
                }
            }
        }
        expect(bitexact(comb.data(), out.data(), comb.size()),
               "ascending-expert combine of expertOutputs reproduces the output");
    }

    // residual: out = residual + MoE(h), the add last (TransformerBlock.cpp:101-104)
    {
        std::vector<float> resid(T * H);
        hm_synth_normal(21, 77, (int64_t)resid.size(), 0.0F, 1.0F, resid.data());
        auto dr = tb.allocateTensor(Shape{T, H}, DType::FP32);
        hip->copyToDevice(dr.data(), resid.data(), resid.size() * 4);
        auto res2 = block.executeBatch(7, dh.view(), dw.view(), dr.view());
        std::vector<float> out2(T * H);
        hip->copyFromDevice(out2.data(), res2.output.data(), out2.size() * 4);
        bool ok = true;
        for (std::size_t i = 0; i < out2.size(); ++i) {
            volatile float s = resid[i] + out[i];
            ok &= bits(s) == bits(out2[i]);
        }
        expect(ok, "residual variant adds the residual last");

        // launchBatch: two calls queued with no synchronisation inside,
        // their results taken in reverse order, each equal to the
        // executeBatch result of the same inputs
        const auto syncs0 = hip->stats().synchronizationCount;
        auto p1 = block.launchBatch(7, dh.view(), dw.view());
        auto p2 = block.launchBatch(7, dh.view(), dw.view(), dr.view());
        expect(hip->stats().synchronizationCount == syncs0,
               "launchBatch queues the call without a stream synchronisation");
        const void* out1 = p1.output().data();
        auto sameRouting = [&](const BatchLayerExecutionResult& a, const BatchLayerExecutionResult& b) {
            bool same = a.routing.tokens.size() == b.routing.tokens.size() &&
                        a.expertBatches.size() == b.expertBatches.size();
            for (std::size_t t = 0; t < a.routing.tokens.size() && same; ++t) {
                same &= a.routing.tokens[t].selectedExpertIds == b.routing.tokens[t].selectedExpertIds;
                for (std::size_t r = 0; r < k && same; ++r)
                    same &= bits(a.routing.tokens[t].routingScores[r]) ==
                            bits(b.routing.tokens[t].routingScores[r]);
            }
            for (std::size_t g = 0; g < a.expertBatches.size() && same; ++g) {
                same &= a.expertBatches[g].expertId == b.expertBatches[g].expertId &&
                        a.expertBatches[g].tokenIndices == b.expertBatches[g].tokenIndices;
                for (std::size_t i = 0; i < a.expertBatches[g].size() && same; ++i)
                    same &= bits(a.expertBatches[g].routingWeights[i]) ==
                            bits(b.expertBatches[g].routingWeights[i]);
            }
            return same;
        };
        auto r2 = p2.get();
        auto r1 = p1.get();
        expect(sameRouting(r1, res) && sameRouting(r2, res2),
               "launched results' routing equals executeBatch's");
        std::vector<float> o1(T * H), o2(T * H);
        hip->copyFromDevice(o1.data(), r1.output.data(), o1.size() * 4);
        hip->copyFromDevice(o2.data(), r2.output.data(), o2.size() * 4);
        expect(bitexact(o1.data(), out.data(), o1.size()) && bitexact(o2.data(), out2.data(), o2.size()),
               "launched results' outputs equal executeBatch's");
        expect(r1.output.data() == out1, "the pending output is the result's output");
        expectThrows<std::logic_error>([&] { (void)p1.get(); }, "a pending result is taken once");

        // a released output buffer is reused by the next call of the same
        // shape; a pending result dropped without get() leaves the block usable
        r1 = BatchLayerExecutionResult{};
        {
            auto p3 = block.launchBatch(7, dh.view(), dw.view());
            expect(p3.output().data() == out1, "released output buffer reused");
        }
        auto r4 = block.executeBatch(7, dh.view(), dw.view());
        std::vector<float> o4(T * H);
        hip->copyFromDevice(o4.data(), r4.output.data(), o4.size() * 4);
        expect(sameRouting(r4, res) && bitexact(o4.data(), out.data(), o4.size()),
               "a call after a dropped pending result is unchanged");
    }

    // argument errors
    auto hostH = tensor::allocateHostTensor(Shape{T, H}, DType::FP32);
    expectThrows<std::invalid_argument>([&] { (void)block.executeBatch(7, hostH.view(), dw.view()); },
                                        "hidden states must be on the device");
    auto narrow = tb.allocateTensor(Shape{T, H / 2}, DType::FP32);
    expectThrows<std::invalid_argument>([&] { (void)block.executeBatch(7, narrow.view(), dw.view()); },
                                        "hidden width must match the layer");
    expectThrows<std::out_of_range>([&] { (void)block.executeBatch(8, dh.view(), dw.view()); },
                                    "unknown layer");
    expectThrows<std::invalid_argument>([&] { (void)block.executeBatch(7, dh.view(), dh.view()); },
                                        "router weights shape");

    // FP32 experts (C1-like shape, small): within 1e-3 of the reference
    {
        const std::size_t E2 = 8, k2 = 2, T2 = 9;
        auto L2 = synthLayer(5, E2, H, I, false);
        auto layer2 = DeviceExpertLayer::fromPayload(hip, L2.payload, E2, H, I, DType::FP32);
        std::vector<float> w2(H * E2);
        hm_synth_normal(5, 1000, (int64_t)w2.size(), 0.0F, 0.02F, w2.data());
        auto dw2 = tb.allocateTensor(Shape{H, E2}, DType::FP32);
        auto dh2 = tb.allocateTensor(Shape{T2, H}, DType::FP32);
        hip->copyToDevice(dw2.data(), w2.data(), w2.size() * 4);
        hip->copyToDevice(dh2.data(), h.data(), T2 * H * 4);
        HipMoEBlock b2(hip, {E2, k2, router::RoutingNormalization::Softmax, true});
        b2.addLayer(0, layer2);
        auto r2 = b2.executeBatch(0, dh2.view(), dw2.view());
        hmo_layer ol2{(int64_t)E2, (int64_t)H, (int64_t)I, 0, L2.payload.data(), nullptr, nullptr};
        std::vector<float> ref(T2 * H), got(T2 * H);
        hmo_moe_block(&ol2, h.data(), w2.data(), (int64_t)T2, (int32_t)k2, 1, 1, ref.data(),
                      nullptr, nullptr);
        hip->copyFromDevice(got.data(), r2.output.data(), got.size() * 4);
        bool ok = true;
        for (std::size_t i = 0; i < got.size(); ++i) {
            ok &= std::fabs(got[i] - ref[i]) <= 1e-3F + 1e-3F * std::fabs(ref[i]);
        }
        expect(ok, "FP32 block within 1e-3 of the reference");
    }
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        if (mode == "cpu") {
            cpuTests();
        } else if (mode == "gpu") {
            auto hip = std::make_shared<backend::HipBackend>(0);
            expect(hip->isAvailable(), "a HIP device is available");
            if (hip->isAvailable()) {
                std::printf("[cpp] backend\n");
                std::fflush(stdout);
                backendTests(hip);
                std::printf("[cpp] tensor backend\n");
                std::fflush(stdout);
                tensorBackendTests(hip);
                std::printf("[cpp] moe block\n");
                std::fflush(stdout);
                blockTests(hip);
            }
        } else {
            std::fprintf(stderr, "usage: test_host cpu|gpu\n");
            return 2;
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: uncaught exception: %s\n", e.what());
        ++g_failures;
    }
    std::printf("%s: %d checks, %d failures\n", mode.c_str(), g_checks, g_failures);
    return g_failures == 0 ? 0 : 1;
}
