#pragma once
// The reference's Apple Metal device is not implemented here; these keep its
// free functions (include/vectorcore/metal_backend.hpp:58-63) with the
// behaviour the reference has on a machine without Metal.
#include <string>

namespace vectorcore {

[[nodiscard]] bool metal_available();
[[nodiscard]] std::string metal_device_name();
// Waits for all queued device work (the HIP stream) and surfaces any device
// error. Reading a tensor's values (item(), to_vector(), to(cpu)) does this.
void synchronize();

}  // namespace vectorcore
