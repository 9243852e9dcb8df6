#pragma once
// The reference's Apple Metal device is not implemented here; these keep its
// free functions (include/vectorcore/metal_backend.hpp:58-63) with the
// behaviour the reference has on a machine without Metal.
#include <string>

namespace vectorcore {

[[nodiscard]] bool metal_available();
[[nodiscard]] std::string metal_device_name();
// Waits for all queued device work (the HIP stream) and surfaces any device
// error. Reading a tensor's values (to_vector(), to(cpu), at(), repr()) does
// this too. item() on the one-element result of a loss or a full sum waits
// only for the kernel that produced it: it reports an error the stream has
// already recorded, but a fault in work enqueued before the item() call and
// still running surfaces at the next full read or synchronize().
void synchronize();

}  // namespace vectorcore
