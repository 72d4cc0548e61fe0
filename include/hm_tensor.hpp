// hm_tensor.hpp -- tensors and the HIP tensor backend.
//
// The TensorBackend surface of the reference
// (src/tensor/backend/TensorBackend.hpp:11-39) with its value types
// (DType src/tensor/DType.hpp:9-14, Shape src/tensor/Shape.hpp, Tensor /
// TensorView src/tensor/Tensor.hpp, src/tensor/TensorView.hpp,
// QuantizationParameters src/tensor/quantization/Quantization.hpp:19-25).
// HipTensorBackend runs every op as a HIP kernel through the C ABI:
//   matmul             hm_matmul_f32     (CpuTensorBackend.cpp:87-131)
//   matmulInt8Weights  hm_matmul_w8a32   (CpuTensorBackend.cpp:133-190)
//   add / mul          hm_add / hm_mul   (CpuTensorBackend.cpp:192-220)
// with the reference's argument checks and error categories.
//
// Shapes here are dense row-major (the reference's strided shapes are not
// used on the MoE path).  A TensorView never extends storage lifetime; each
// op locks the owners for the duration of the call and, because launches are
// asynchronous, until the compute stream has finished with them
// (synchronizeExecution()).
#pragma once

#include "hm_backend.hpp"

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <memory>
#include <mutex>
#include <string_view>
#include <vector>

namespace hm::tensor {

enum class DType : std::uint32_t {
    FP32 = 0,
    FP16 = 1,
    BF16 = 2,
    INT8 = 3,
};

[[nodiscard]] constexpr std::size_t sizeOf(DType dtype) noexcept {
    switch (dtype) {
    case DType::FP32: return 4;
    case DType::FP16:
    case DType::BF16: return 2;
    case DType::INT8: return 1;
    }
    return 0;
}

enum class DeviceType : std::uint8_t {
    CPU = 0,
    HIP = 1,
};

struct Device {
    DeviceType type{DeviceType::CPU};
    int ordinal{};

    [[nodiscard]] static constexpr Device cpu() noexcept { return {}; }
    [[nodiscard]] static constexpr Device hip(int ordinal = 0) noexcept {
        return {DeviceType::HIP, ordinal};
    }
    [[nodiscard]] constexpr bool operator==(const Device&) const noexcept = default;
};

// Dense row-major shape.  Zero-sized dimensions are rejected and the element
// count is overflow-checked (std::overflow_error), as in the reference.
class Shape {
public:
    Shape() = default;
    Shape(std::initializer_list<std::size_t> dimensions);
    explicit Shape(std::vector<std::size_t> dimensions);

    [[nodiscard]] const std::vector<std::size_t>& dimensions() const noexcept { return dims_; }
    [[nodiscard]] std::size_t rank() const noexcept { return dims_.size(); }
    [[nodiscard]] std::size_t elementCount() const noexcept { return count_; }
    [[nodiscard]] std::size_t operator[](std::size_t i) const { return dims_.at(i); }
    [[nodiscard]] bool operator==(const Shape& other) const noexcept {
        return dims_ == other.dims_;
    }

private:
    void validate();
    std::vector<std::size_t> dims_;
    std::size_t count_{0};
};

// Bytes for `shape` elements of `dtype`, overflow-checked.
[[nodiscard]] std::size_t tensorBytes(const Shape& shape, DType dtype);

class TensorView;

class Tensor {
public:
    Tensor() = default;

    // Wraps existing storage; `owner` keeps it alive.
    [[nodiscard]] static Tensor fromStorage(Shape shape, DType dtype, Device device, void* data,
                                            std::size_t storageBytes,
                                            std::shared_ptr<void> owner);
    [[nodiscard]] static Tensor fromDeviceBuffer(Shape shape, DType dtype, Device device,
                                                 std::shared_ptr<backend::DeviceBuffer> buffer);

    [[nodiscard]] const Shape& shape() const noexcept { return shape_; }
    [[nodiscard]] DType dtype() const noexcept { return dtype_; }
    [[nodiscard]] Device device() const noexcept { return device_; }
    [[nodiscard]] void* data() noexcept { return data_; }
    [[nodiscard]] const void* data() const noexcept { return data_; }
    [[nodiscard]] std::size_t bytes() const noexcept;
    [[nodiscard]] std::size_t storageBytes() const noexcept { return storageBytes_; }
    [[nodiscard]] bool valid() const noexcept { return data_ != nullptr && owner_ != nullptr; }
    [[nodiscard]] explicit operator bool() const noexcept { return valid(); }
    [[nodiscard]] const std::shared_ptr<void>& owner() const noexcept { return owner_; }
    [[nodiscard]] Tensor reshape(Shape shape) const;
    [[nodiscard]] TensorView view() &;
    [[nodiscard]] TensorView view() const&;
    TensorView view() && = delete;

private:
    friend class TensorView;
    Shape shape_;
    DType dtype_{DType::FP32};
    Device device_{};
    void* data_{};
    std::size_t storageBytes_{};
    std::shared_ptr<void> owner_;
};

// Non-owning view (src/tensor/TensorView.hpp:10-11): holds a weak reference
// to the storage owner and never extends its lifetime.
class TensorView {
public:
    TensorView() = default;
    TensorView(Tensor& tensor);
    TensorView(const Tensor& tensor);
    TensorView(Tensor&&) = delete;

    [[nodiscard]] const Shape& shape() const noexcept { return shape_; }
    [[nodiscard]] DType dtype() const noexcept { return dtype_; }
    [[nodiscard]] Device device() const noexcept { return device_; }
    [[nodiscard]] const void* data() const noexcept { return data_; }
    [[nodiscard]] void* mutableData() const noexcept { return mutable_; }
    [[nodiscard]] std::size_t bytes() const noexcept;
    [[nodiscard]] std::size_t storageBytes() const noexcept { return storageBytes_; }
    [[nodiscard]] bool writable() const noexcept { return mutable_ != nullptr; }
    [[nodiscard]] bool valid() const noexcept { return data_ != nullptr && !lifetime_.expired(); }
    [[nodiscard]] explicit operator bool() const noexcept { return valid(); }
    [[nodiscard]] std::shared_ptr<void> lockOwner() const noexcept { return lifetime_.lock(); }
    [[nodiscard]] TensorView reshape(Shape shape) const;
    [[nodiscard]] TensorView readOnly() const;

private:
    Shape shape_;
    DType dtype_{DType::FP32};
    Device device_{};
    const void* data_{};
    void* mutable_{};
    std::size_t storageBytes_{};
    std::weak_ptr<void> lifetime_;
};

namespace quantization {

struct QuantizationParameters {
    float scale{1.0F};
    std::int32_t zeroPoint{};

    friend bool operator==(const QuantizationParameters&,
                           const QuantizationParameters&) = default;
};

// validateParameters for INT8 (src/tensor/quantization/Quantization.cpp:24-43):
// scale finite and positive, zero point in [-128, 127].
void validateInt8Parameters(const QuantizationParameters& parameters);

}  // namespace quantization

class TensorBackend {
public:
    virtual ~TensorBackend() = default;

    [[nodiscard]] virtual std::string_view name() const noexcept = 0;
    [[nodiscard]] virtual Device device() const noexcept = 0;
    [[nodiscard]] virtual bool available() const noexcept = 0;
    [[nodiscard]] virtual Tensor allocateTensor(const Shape& shape, DType dtype) = 0;
    virtual void copyTensor(TensorView source, TensorView destination) = 0;
    virtual void matmul(TensorView left, TensorView right, TensorView output) = 0;
    virtual void matmulInt8Weights(TensorView left, TensorView right,
                                   const quantization::QuantizationParameters& parameters,
                                   TensorView output) = 0;
    virtual void add(TensorView left, TensorView right, TensorView output) = 0;
    virtual void mul(TensorView left, TensorView right, TensorView output) = 0;
    [[nodiscard]] virtual Tensor reshape(const Tensor& tensor, Shape shape) = 0;
    virtual void synchronize() = 0;
    // Completes only the execution dependency chain.
    virtual void synchronizeExecution() { synchronize(); }
};

// Host tensors for staging and results (pageable memory, CPU device).
[[nodiscard]] Tensor allocateHostTensor(const Shape& shape, DType dtype);

class HipTensorBackend final : public TensorBackend {
public:
    explicit HipTensorBackend(std::shared_ptr<backend::HipBackend> backend);
    ~HipTensorBackend() override;

    [[nodiscard]] std::string_view name() const noexcept override { return "HIP tensor backend"; }
    [[nodiscard]] Device device() const noexcept override;
    [[nodiscard]] bool available() const noexcept override;
    [[nodiscard]] Tensor allocateTensor(const Shape& shape, DType dtype) override;
    // Any direction between CPU and HIP tensors of equal shape and dtype.
    void copyTensor(TensorView source, TensorView destination) override;
    void matmul(TensorView left, TensorView right, TensorView output) override;
    // The reference's W8A32 arithmetic, acc += x * (float(q - zp) * scale), on
    // the device with its bounded split-K plan (hm_plan_int8_gemm); split-K
    // scratch comes from a grow-only pool owned by this backend.
    void matmulInt8Weights(TensorView left, TensorView right,
                           const quantization::QuantizationParameters& parameters,
                           TensorView output) override;
    void add(TensorView left, TensorView right, TensorView output) override;
    void mul(TensorView left, TensorView right, TensorView output) override;
    [[nodiscard]] Tensor reshape(const Tensor& tensor, Shape shape) override;
    void synchronize() override;
    void synchronizeExecution() override;

    [[nodiscard]] const std::shared_ptr<backend::HipBackend>& hipBackend() const noexcept {
        return backend_;
    }

private:
    void* scratch(std::size_t bytes);
    // Keeps the owners of an asynchronous op alive until the next
    // synchronizeExecution() (the role of GpuEventQueue::begin's owners).
    void retain(std::initializer_list<std::shared_ptr<void>> owners);

    std::shared_ptr<backend::HipBackend> backend_;
    std::mutex mutex_;
    std::shared_ptr<backend::DeviceBuffer> scratch_;
    std::vector<std::shared_ptr<void>> inflight_;
};

}  // namespace hm::tensor
