#pragma once
// Devices (API of include/vectorcore/device.hpp) with the MI355X `hip` device
// added next to `cpu`. METAL is kept so code written for the reference still
// compiles; there is no Metal backend here, and it reports itself unavailable.
#include <string>

namespace vectorcore {

enum class DeviceType { CPU, METAL, HIP };

struct Device {
    DeviceType type{DeviceType::CPU};

    constexpr Device() = default;
    constexpr explicit Device(DeviceType value) : type(value) {}
    [[nodiscard]] std::string str() const;

    friend constexpr bool operator==(Device a, Device b) { return a.type == b.type; }
    friend constexpr bool operator!=(Device a, Device b) { return !(a == b); }

    static constexpr Device cpu() { return Device(DeviceType::CPU); }
    static constexpr Device metal() { return Device(DeviceType::METAL); }
    static constexpr Device hip() { return Device(DeviceType::HIP); }
};

}  // namespace vectorcore
