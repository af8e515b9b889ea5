#pragma once
// Device descriptor (mirrors include/ctd/device.h of the reference).
// The GPU enumerator keeps the reference's value 1 under a HIP spelling:
// DeviceType::kHIP / kHIP0 / is_hip() are the reference's kCUDA / kCUDA0 / is_cuda().

#include <cstdint>

namespace ctd {

enum class DeviceType : uint8_t {
  kCPU = 0,
  kHIP = 1,
};

struct Device {
  DeviceType type = DeviceType::kCPU;
  int index = 0;

  constexpr Device() = default;
  constexpr Device(DeviceType t, int i = 0) : type(t), index(i) {}

  bool is_cpu() const { return type == DeviceType::kCPU; }
  bool is_hip() const { return type == DeviceType::kHIP; }

  bool operator==(const Device& o) const { return type == o.type && index == o.index; }
  bool operator!=(const Device& o) const { return !(*this == o); }
};

constexpr Device kCPU{DeviceType::kCPU, 0};
constexpr Device kHIP0{DeviceType::kHIP, 0};

}  // namespace ctd
