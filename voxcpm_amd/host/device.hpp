// HIP helpers of the host surface: the reference's error and ownership
// conventions (device.hpp:16-77) over the voxcpm_amd C ABI.
#ifndef VOXCPM_AMD_HOST_DEVICE_HPP_
#define VOXCPM_AMD_HOST_DEVICE_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <memory>
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

/// The deleter of DeviceBuffer's allocation.
struct DeviceFree {
  void operator()(void* pointer) const noexcept { (void)hipFree(pointer); }
};

/// Uninitialised device storage for elements of T with one owner: moved,
/// never copied, freed with its owner (the ownership of device.hpp:33-77).
/// The allocation is a unique_ptr with a hipFree deleter, so moves and
/// destruction come from it; the element count travels beside it and
/// counts only while an allocation is held.
template<typename T>
class DeviceBuffer {
public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(std::size_t count) : memory_(Allocate(count)), count_(count) {}

  /// Ensures room for `count` elements. A larger request frees the old
  /// allocation before making the new one (the contents are not kept); a
  /// smaller one keeps what is held.
  void Reserve(std::size_t count) {
    if (count <= size())
      return;
    memory_.reset();
    memory_.reset(Allocate(count));
    count_ = count;
  }

  [[nodiscard]] T* get() const { return memory_.get(); }
  [[nodiscard]] std::size_t size() const { return memory_ ? count_ : 0; }

private:
  /// hipMalloc of `count` elements; a zero count still takes one element,
  /// so that every held buffer has a valid device address.
  static T* Allocate(std::size_t count) {
    void* pointer = nullptr;
    Check(hipMalloc(&pointer, (count == 0 ? 1 : count) * sizeof(T)), "hipMalloc");
    return static_cast<T*>(pointer);
  }

  std::unique_ptr<T, DeviceFree> memory_;
  std::size_t count_ = 0;
};

}  // namespace gufo::models::voxcpm

#endif  // VOXCPM_AMD_HOST_DEVICE_HPP_
