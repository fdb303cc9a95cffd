#pragma once
// Device handle: backend registration key + ordinal. There is no device-type enum: a backend is identified
// only by its registry string (reference: include/frame/core/device.h:12-24). "hip" is the MI355X backend of
// this library.

#include <cstdint>
#include <string_view>

namespace frame {

inline constexpr std::string_view kCpuBackendName = "cpu";
inline constexpr std::string_view kCudaBackendName = "cuda";
inline constexpr std::string_view kIntelGpuBackendName = "intel_gpu";
inline constexpr std::string_view kIntelNpuBackendName = "intel_npu";
inline constexpr std::string_view kAscendBackendName = "ascend";
inline constexpr std::string_view kHipBackendName = "hip";

struct Device {
  std::string_view backend;
  int32_t index = 0;
  constexpr bool operator==(const Device&) const = default;
};

constexpr Device cpu_device(int32_t index = 0) { return Device{kCpuBackendName, index}; }

}  // namespace frame
