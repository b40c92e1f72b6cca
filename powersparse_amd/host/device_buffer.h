// RAII device allocation over the C ABI (ps_malloc / ps_free).
#pragma once

#include <cstddef>
#include <utility>
#include <vector>

#include "matrix_utils.h"

namespace PowerSparse {

template <typename T>
class DeviceArray {
 public:
  DeviceArray() = default;
  explicit DeviceArray(size_t count) { Allocate(count); }
  // Frees synchronise the device first: buffers here are handed to enqueued
  // preprocessing kernels, and freeing one must not race them.
  ~DeviceArray() { Reset(); }
  DeviceArray(const DeviceArray&) = delete;
  DeviceArray& operator=(const DeviceArray&) = delete;
  DeviceArray(DeviceArray&& o) noexcept : data_(o.data_), count_(o.count_) {
    o.data_ = nullptr;
    o.count_ = 0;
  }
  DeviceArray& operator=(DeviceArray&& o) noexcept {
    std::swap(data_, o.data_);
    std::swap(count_, o.count_);
    return *this;
  }

  void Allocate(size_t count) {
    Reset();
    if (count > size_t(-1) / sizeof(T)) throw std::overflow_error("Device allocation size overflow");
    void* p = nullptr;
    ThrowOnError(ps_malloc(&p, count * sizeof(T)));
    data_ = static_cast<T*>(p);
    count_ = count;
  }
  void Reset() {
    if (data_) ps_device_synchronize();
    ps_free(data_);
    data_ = nullptr;
    count_ = 0;
  }
  // Hands ownership to the caller (who frees with ps_free).
  T* Release() {
    T* p = data_;
    data_ = nullptr;
    count_ = 0;
    return p;
  }
  void Upload(const T* host, size_t count) {
    if (count > count_) throw std::invalid_argument("Upload size mismatch");
    ThrowOnError(ps_memcpy_htod(data_, host, count * sizeof(T)));
  }
  void Download(T* host, size_t count) const {
    if (count > count_) throw std::invalid_argument("Download size mismatch");
    ThrowOnError(ps_memcpy_dtoh(host, data_, count * sizeof(T)));
  }
  void Zero(ps_stream_t stream) { ThrowOnError(ps_memset_async(data_, 0, count_ * sizeof(T), stream)); }

  T* data() const { return data_; }
  size_t size() const { return count_; }

 private:
  T* data_ = nullptr;
  size_t count_ = 0;
};

}  // namespace PowerSparse
