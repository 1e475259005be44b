// Move-only device tensor view: raw device pointer + dtype + shape.
// Mirrors Aila's Tensor (src/core/Tensor.hpp:15-132: allocate / view,
// data(), shape(i), numel(), size_bytes(), valid()) with a plain dtype enum
// in place of dnnl::memory::data_type.
#pragma once

#include <cstdint>
#include <functional>
#include <numeric>
#include <vector>

#include "Context.hpp"

namespace aila {

enum class DType { f32, bf16, f16, s8, u8, s32, f64 };

inline size_t dtype_size(DType t) {
  switch (t) {
    case DType::f32: case DType::s32: return 4;
    case DType::bf16: case DType::f16: return 2;
    case DType::s8: case DType::u8: return 1;
    case DType::f64: return 8;
  }
  return 0;
}

class Tensor {
 public:
  Tensor() = default;
  static Tensor allocate(Context& ctx, const std::vector<int64_t>& shape, DType dt = DType::bf16) {
    Tensor t;
    t.shape_ = shape;
    t.dtype_ = dt;
    t.ctx_ = &ctx;
    t.owns_ = true;
    t.data_ = ctx.alloc_device(t.size_bytes());
    return t;
  }
  static Tensor view(Context& ctx, void* ptr, const std::vector<int64_t>& shape, DType dt = DType::bf16) {
    Tensor t;
    t.shape_ = shape;
    t.dtype_ = dt;
    t.ctx_ = &ctx;
    t.owns_ = false;
    t.data_ = ptr;
    return t;
  }
  ~Tensor() { release(); }
  Tensor(Tensor&& o) noexcept { *this = std::move(o); }
  Tensor& operator=(Tensor&& o) noexcept {
    if (this != &o) {
      release();
      shape_ = std::move(o.shape_);
      dtype_ = o.dtype_;
      data_ = o.data_;
      ctx_ = o.ctx_;
      owns_ = o.owns_;
      o.data_ = nullptr;
      o.owns_ = false;
    }
    return *this;
  }
  Tensor(const Tensor&) = delete;
  Tensor& operator=(const Tensor&) = delete;

  void* data() { return data_; }
  const void* data() const { return data_; }
  template <typename T> T* data_as() { return static_cast<T*>(data_); }
  const std::vector<int64_t>& shape() const { return shape_; }
  int64_t shape(int d) const { return shape_[d]; }
  int ndim() const { return static_cast<int>(shape_.size()); }
  DType dtype() const { return dtype_; }
  Context* context() const { return ctx_; }
  bool valid() const { return data_ != nullptr; }
  int64_t numel() const {
    if (shape_.empty()) return 0;
    return std::accumulate(shape_.begin(), shape_.end(), int64_t{1}, std::multiplies<int64_t>());
  }
  size_t element_size() const { return dtype_size(dtype_); }
  size_t size_bytes() const { return static_cast<size_t>(numel()) * element_size(); }

 private:
  void release() {
    if (owns_ && data_ && ctx_) ctx_->free_device(data_);
    data_ = nullptr;
    owns_ = false;
  }
  std::vector<int64_t> shape_;
  DType dtype_ = DType::bf16;
  void* data_ = nullptr;
  Context* ctx_ = nullptr;
  bool owns_ = false;
};

}  // namespace aila

// The reference's Tensor is a global class (src/core/Tensor.hpp:15).
using aila::DType;
using aila::Tensor;
