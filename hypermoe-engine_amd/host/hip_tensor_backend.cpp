// hip_tensor_backend.cpp -- tensors and HipTensorBackend, the TensorBackend
// surface (src/tensor/backend/TensorBackend.hpp:11-39) on the HIP kernels.
// Argument checks and messages follow CpuTensorBackend.cpp:25-220.
#include "hm_tensor.hpp"
#include "hm_moe.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <new>
#include <stdexcept>
#include <string>
#include <utility>

namespace hm::tensor {

// ---- Shape / Tensor / TensorView --------------------------------------------

Shape::Shape(std::initializer_list<std::size_t> dimensions) : dims_(dimensions) { validate(); }
Shape::Shape(std::vector<std::size_t> dimensions) : dims_(std::move(dimensions)) { validate(); }

void Shape::validate() {
    if (dims_.empty()) throw std::invalid_argument("tensor shape must have rank >= 1");
    std::size_t n = 1;
    for (const auto d : dims_) {
        if (d == 0) throw std::invalid_argument("tensor dimensions must be nonzero");
        if (n > std::numeric_limits<std::size_t>::max() / d) {
            throw std::overflow_error("tensor element count overflow");
        }
        n *= d;
    }
    count_ = n;
}

std::size_t tensorBytes(const Shape& shape, DType dtype) {
    const auto elem = sizeOf(dtype);
    if (elem == 0) throw std::invalid_argument("unsupported tensor dtype");
    if (shape.elementCount() > std::numeric_limits<std::size_t>::max() / elem) {
        throw std::overflow_error("tensor allocation byte size overflow");
    }
    return shape.elementCount() * elem;
}

Tensor Tensor::fromStorage(Shape shape, DType dtype, Device device, void* data,
                           std::size_t storageBytes, std::shared_ptr<void> owner) {
    if (data == nullptr || !owner) throw std::invalid_argument("tensor storage is null");
    if (tensorBytes(shape, dtype) > storageBytes) {
        throw std::invalid_argument("tensor storage is smaller than its shape");
    }
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.device_ = device;
    t.data_ = data;
    t.storageBytes_ = storageBytes;
    t.owner_ = std::move(owner);
    return t;
}

Tensor Tensor::fromDeviceBuffer(Shape shape, DType dtype, Device device,
                                std::shared_ptr<backend::DeviceBuffer> buffer) {
    if (!buffer || !*buffer) throw std::invalid_argument("tensor device buffer is empty");
    void* data = buffer->data();
    const auto size = buffer->size();
    return fromStorage(std::move(shape), dtype, device, data, size, std::move(buffer));
}

std::size_t Tensor::bytes() const noexcept {
    return shape_.elementCount() * sizeOf(dtype_);
}

Tensor Tensor::reshape(Shape shape) const {
    if (shape.elementCount() != shape_.elementCount()) {
        throw std::invalid_argument("tensor reshape changes the element count");
    }
    Tensor t = *this;
    t.shape_ = std::move(shape);
    return t;
}

TensorView Tensor::view() & { return TensorView(*this); }
TensorView Tensor::view() const& { return TensorView(*this); }

TensorView::TensorView(Tensor& tensor)
    : shape_(tensor.shape_), dtype_(tensor.dtype_), device_(tensor.device_), data_(tensor.data_),
      mutable_(tensor.data_), storageBytes_(tensor.storageBytes_), lifetime_(tensor.owner_) {}

TensorView::TensorView(const Tensor& tensor)
    : shape_(tensor.shape_), dtype_(tensor.dtype_), device_(tensor.device_), data_(tensor.data_),
      mutable_(nullptr), storageBytes_(tensor.storageBytes_), lifetime_(tensor.owner_) {}

std::size_t TensorView::bytes() const noexcept { return shape_.elementCount() * sizeOf(dtype_); }

TensorView TensorView::reshape(Shape shape) const {
    if (shape.elementCount() != shape_.elementCount()) {
        throw std::invalid_argument("tensor view reshape changes the element count");
    }
    TensorView v = *this;
    v.shape_ = std::move(shape);
    return v;
}

TensorView TensorView::readOnly() const {
    TensorView v = *this;
    v.mutable_ = nullptr;
    return v;
}

namespace quantization {

void validateInt8Parameters(const QuantizationParameters& parameters) {
    if (!std::isfinite(parameters.scale) || parameters.scale <= 0.0F) {
        throw std::invalid_argument("quantization scale must be finite and positive");
    }
    if (parameters.zeroPoint < -128 || parameters.zeroPoint > 127) {
        throw std::invalid_argument("8-bit zero point is outside [-128, 127]");
    }
}

}  // namespace quantization

Tensor allocateHostTensor(const Shape& shape, DType dtype) {
    const auto n = tensorBytes(shape, dtype);
    auto owner = std::shared_ptr<void>(::operator new(n, std::align_val_t{64}),
                                       [](void* p) { ::operator delete(p, std::align_val_t{64}); });
    void* data = owner.get();
    return Tensor::fromStorage(shape, dtype, Device::cpu(), data, n, std::move(owner));
}

// ---- HipTensorBackend ---------------------------------------------------------

namespace {

std::shared_ptr<void> pin(const TensorView& t, const char* op) {
    auto owner = t.lockOwner();
    if (!owner) throw std::invalid_argument(std::string(op) + " received expired tensor storage");
    return owner;
}

void requireHip(const TensorView& t, const Device& dev, const char* op) {
    if (!t || t.device() != dev) {
        throw std::invalid_argument(std::string(op) + " requires a contiguous HIP tensor");
    }
}

void validateElementwise(const TensorView& l, const TensorView& r, const TensorView& o,
                         const Device& dev, const char* op) {
    requireHip(l, dev, op);
    requireHip(r, dev, op);
    requireHip(o, dev, op);
    if (l.dtype() != DType::FP32 || r.dtype() != DType::FP32 || o.dtype() != DType::FP32 ||
        l.shape() != r.shape() || l.shape() != o.shape() || !o.writable()) {
        throw std::invalid_argument(std::string(op) + " requires equal-shape FP32 tensors");
    }
}

struct GemmDims {
    std::size_t rows, inner, columns;
};

GemmDims validateGemm(const TensorView& l, const TensorView& r, const TensorView& o,
                      DType rightType, const Device& dev, const char* op) {
    requireHip(l, dev, op);
    requireHip(r, dev, op);
    requireHip(o, dev, op);
    if (l.dtype() != DType::FP32 || r.dtype() != rightType || o.dtype() != DType::FP32 ||
        l.shape().rank() != 2 || r.shape().rank() != 2 || o.shape().rank() != 2 ||
        !o.writable()) {
        throw std::invalid_argument(std::string(op) +
                                    (rightType == DType::INT8
                                         ? " requires FP32 input/output and rank-2 INT8 weights"
                                         : " requires contiguous rank-2 FP32 tensors"));
    }
    const GemmDims d{l.shape()[0], l.shape()[1], r.shape()[1]};
    if (r.shape()[0] != d.inner || o.shape()[0] != d.rows || o.shape()[1] != d.columns) {
        throw std::invalid_argument(std::string(op) + " dimensions are incompatible");
    }
    if (l.data() == o.data() || r.data() == o.data()) {
        throw std::invalid_argument(std::string(op) + " output cannot alias an input");
    }
    return d;
}

}  // namespace

HipTensorBackend::HipTensorBackend(std::shared_ptr<backend::HipBackend> backend)
    : backend_(std::move(backend)) {
    if (!backend_) throw std::invalid_argument("HIP tensor backend requires a HIP backend");
}

HipTensorBackend::~HipTensorBackend() {
    try {
        if (backend_->isAvailable()) synchronizeExecution();
    } catch (...) {
    }
}

Device HipTensorBackend::device() const noexcept { return Device::hip(backend_->deviceOrdinal()); }
bool HipTensorBackend::available() const noexcept { return backend_->isAvailable(); }

Tensor HipTensorBackend::allocateTensor(const Shape& shape, DType dtype) {
    auto buffer = std::make_shared<backend::DeviceBuffer>(backend_, tensorBytes(shape, dtype));
    return Tensor::fromDeviceBuffer(shape, dtype, device(), std::move(buffer));
}

void HipTensorBackend::retain(std::initializer_list<std::shared_ptr<void>> owners) {
    constexpr std::size_t kMaxInflightOwners = 4096;
    bool drain = false;
    {
        std::scoped_lock lock(mutex_);
        for (const auto& o : owners) inflight_.push_back(o);
        drain = inflight_.size() > kMaxInflightOwners;
    }
    if (drain) synchronizeExecution();  // bounds the retained set
}

void* HipTensorBackend::scratch(std::size_t bytes) {
    std::scoped_lock lock(mutex_);
    if (!scratch_ || scratch_->size() < bytes) {
        if (scratch_) {
            // the old pool may still be read by launched work
            (void)hm_stream_synchronize(backend_->computeStream());
        }
        scratch_ = std::make_shared<backend::DeviceBuffer>(backend_, bytes);
    }
    return scratch_->data();
}

void HipTensorBackend::copyTensor(TensorView source, TensorView destination) {
    const char* op = "HIP tensor copy";
    auto so = pin(source, op);
    auto dso = pin(destination, op);
    if (source.dtype() != destination.dtype() || source.shape() != destination.shape() ||
        !destination.writable()) {
        throw std::invalid_argument("HIP tensor copy metadata mismatch");
    }
    const auto n = source.bytes();
    const bool srcDev = source.device().type == DeviceType::HIP;
    const bool dstDev = destination.device().type == DeviceType::HIP;
    if ((srcDev && source.device() != device()) || (dstDev && destination.device() != device())) {
        throw std::invalid_argument("HIP tensor copy across devices");
    }
    auto s = backend_->computeStream();
    if (srcDev && dstDev) {
        backend_->copyOnDevice(destination.mutableData(), source.data(), n, s);
        retain({so, dso});
    } else if (dstDev) {
        // pageable host source: complete before the caller may reuse it
        backend_->copyToDevice(destination.mutableData(), source.data(), n, s);
        backend_->synchronize(s);
    } else if (srcDev) {
        backend_->copyFromDevice(destination.mutableData(), source.data(), n, s);
        backend_->synchronize(s);
    } else {
        std::memmove(destination.mutableData(), source.data(), n);
    }
}

void HipTensorBackend::matmul(TensorView left, TensorView right, TensorView output) {
    const char* op = "HIP matmul";
    auto lo = pin(left, op), ro = pin(right, op), oo = pin(output, op);
    const auto d = validateGemm(left, right, output, DType::FP32, device(), op);
    backend::throwOnStatus(
        hm_matmul_f32(static_cast<const float*>(left.data()),
                      static_cast<const float*>(right.data()),
                      static_cast<float*>(output.mutableData()), (int64_t)d.rows,
                      (int64_t)d.inner, (int64_t)d.columns, backend_->computeStream()),
        op);
    retain({lo, ro, oo});
}

void HipTensorBackend::matmulInt8Weights(TensorView left, TensorView right,
                                         const quantization::QuantizationParameters& parameters,
                                         TensorView output) {
    const char* op = "HIP INT8 weight matmul";
    auto lo = pin(left, op), ro = pin(right, op), oo = pin(output, op);
    quantization::validateInt8Parameters(parameters);
    const auto d = validateGemm(left, right, output, DType::INT8, device(), op);
    hm_int8_gemm_plan plan{};
    backend::throwOnStatus(hm_plan_int8_gemm((int64_t)d.rows, (int64_t)d.inner,
                                             (int64_t)d.columns, 0, &plan),
                           op);
    std::size_t scratchBytes = 0;
    float* scratchPtr = nullptr;
    if (plan.scratch_elements > 0) {
        scratchBytes = (std::size_t)plan.scratch_elements * sizeof(float);
        scratchPtr = static_cast<float*>(scratch(scratchBytes));
    }
    backend::throwOnStatus(
        hm_matmul_w8a32(static_cast<const float*>(left.data()),
                        static_cast<const int8_t*>(right.data()), parameters.scale,
                        parameters.zeroPoint, static_cast<float*>(output.mutableData()),
                        (int64_t)d.rows, (int64_t)d.inner, (int64_t)d.columns, 0, scratchPtr,
                        scratchBytes, backend_->computeStream()),
        op);
    retain({lo, ro, oo});
}

void HipTensorBackend::add(TensorView left, TensorView right, TensorView output) {
    const char* op = "HIP add";
    auto lo = pin(left, op), ro = pin(right, op), oo = pin(output, op);
    validateElementwise(left, right, output, device(), op);
    backend::throwOnStatus(hm_add(static_cast<const float*>(left.data()),
                                  static_cast<const float*>(right.data()),
                                  static_cast<float*>(output.mutableData()),
                                  (int64_t)left.shape().elementCount(), backend_->computeStream()),
                           op);
    retain({lo, ro, oo});
}

void HipTensorBackend::mul(TensorView left, TensorView right, TensorView output) {
    const char* op = "HIP multiply";
    auto lo = pin(left, op), ro = pin(right, op), oo = pin(output, op);
    validateElementwise(left, right, output, device(), op);
    backend::throwOnStatus(hm_mul(static_cast<const float*>(left.data()),
                                  static_cast<const float*>(right.data()),
                                  static_cast<float*>(output.mutableData()),
                                  (int64_t)left.shape().elementCount(), backend_->computeStream()),
                           op);
    retain({lo, ro, oo});
}

Tensor HipTensorBackend::reshape(const Tensor& tensor, Shape shape) {
    return tensor.reshape(std::move(shape));
}

void HipTensorBackend::synchronize() {
    backend_->synchronize(nullptr);
    std::scoped_lock lock(mutex_);
    inflight_.clear();
}

void HipTensorBackend::synchronizeExecution() {
    backend_->synchronize(backend_->computeStream());
    std::scoped_lock lock(mutex_);
    inflight_.clear();
}

}  // namespace hm::tensor
