// HIP helpers of the host surface: the reference's error and ownership
// conventions (device.hpp:16-77) over the voxcpm_amd C ABI.
#ifndef VOXCPM_AMD_HOST_DEVICE_HPP_
#define VOXCPM_AMD_HOST_DEVICE_HPP_

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <stdexcept>
#include <string>
#include <utility>

#include "voxcpm_amd.h"

namespace gufo::models::voxcpm {

/// A failed device call (device.hpp:16-19).
class GpuError : public std::runtime_error {
public:
  using std::runtime_error::runtime_error;
};

inline void Check(hipError_t status, const char* what) {
  if (status != hipSuccess)
    throw GpuError(std::string(what) + ": " + hipGetErrorString(status));
}

/// Throws GpuError for a failed vx_status, with the library's message.
inline void CheckVx(int status, const char* what) {
  if (status != VX_OK)
    throw GpuError(std::string(what) + ": " + vx_last_error());
}

/// A device allocation of `count` elements of T (device.hpp:33-77).
template<typename T>
class DeviceBuffer {
public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(std::size_t count) { Resize(count); }
  ~DeviceBuffer() { Release(); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& other) noexcept
      : data_(std::exchange(other.data_, nullptr)),
        count_(std::exchange(other.count_, 0)) {}
  DeviceBuffer& operator=(DeviceBuffer&& other) noexcept {
    Release();
    data_ = std::exchange(other.data_, nullptr);
    count_ = std::exchange(other.count_, 0);
    return *this;
  }

  /// Reallocates when `count` exceeds the capacity; contents are lost.
  void Reserve(std::size_t count) {
    if (count > count_)
      Resize(count);
  }

  [[nodiscard]] T* get() const { return data_; }
  [[nodiscard]] std::size_t size() const { return count_; }

private:
  void Resize(std::size_t count) {
    Release();
    Check(hipMalloc(reinterpret_cast<void**>(&data_),
                    std::max<std::size_t>(count, 1) * sizeof(T)),
          "hipMalloc");
    count_ = count;
  }
  void Release() noexcept {
    if (data_ != nullptr)
      (void)hipFree(data_);
    data_ = nullptr;
    count_ = 0;
  }

  T* data_ = nullptr;
  std::size_t count_ = 0;
};

}  // namespace gufo::models::voxcpm

#endif  // VOXCPM_AMD_HOST_DEVICE_HPP_
