// HIP runtime context for the ops:: host layer: one in-order HIP stream on
// the current device plus device allocation with byte accounting.
// Mirrors Aila's Context (src/core/Context.hpp:16-78: in-order sycl::queue,
// USM alloc/free with current/peak accounting, blocking and async copies,
// synchronize) with a hipStream_t in place of the SYCL queue.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>
#include <string>
#include <unordered_map>

namespace aila {

inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

class Context {
 public:
  Context() { hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate"); }
  // Wrap an existing stream (not owned).
  explicit Context(hipStream_t s) : stream_(s), owns_stream_(false) {}
  ~Context() {
    if (owns_stream_ && stream_) (void)hipStreamDestroy(stream_);   // nothing to report from a destructor
  }
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;

  hipStream_t stream() const { return stream_; }

  void* alloc_device(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess || !p)
      throw std::runtime_error("GPU memory allocation failed: " + std::to_string(bytes) + " bytes");
    alloc_bytes_[p] = bytes;
    current_ += bytes;
    if (current_ > peak_) peak_ = current_;
    return p;
  }
  void free_device(void* p) {
    if (!p) return;
    auto it = alloc_bytes_.find(p);
    if (it != alloc_bytes_.end()) {
      current_ = current_ >= it->second ? current_ - it->second : 0;
      alloc_bytes_.erase(it);
    }
    (void)hipFree(p);   // free errors surface at the next synchronising call
  }
  void memcpy_h2d(void* dst, const void* src, size_t bytes) {
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_), "memcpy_h2d");
    synchronize();
  }
  void memcpy_d2h(void* dst, const void* src, size_t bytes) {
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream_), "memcpy_d2h");
    synchronize();
  }
  void memcpy_h2d_async(void* dst, const void* src, size_t bytes) {
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_), "memcpy_h2d_async");
  }
  void memcpy_d2h_async(void* dst, const void* src, size_t bytes) {
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream_), "memcpy_d2h_async");
  }
  void synchronize() { hip_check(hipStreamSynchronize(stream_), "synchronize"); }

  size_t current_allocated_bytes() const { return current_; }
  size_t peak_allocated_bytes() const { return peak_; }

 private:
  hipStream_t stream_ = nullptr;
  bool owns_stream_ = true;
  std::unordered_map<void*, size_t> alloc_bytes_;
  size_t current_ = 0, peak_ = 0;
};

}  // namespace aila

// The reference's Context is a global class (src/core/Context.hpp:14).
using aila::Context;
