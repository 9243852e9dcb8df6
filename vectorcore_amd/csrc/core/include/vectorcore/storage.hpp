#pragma once
// Storage with the in-place version counter (API of include/vectorcore/storage.hpp).
#include "vectorcore/device.hpp"

#include <cstddef>
#include <cstdint>
#include <memory>

namespace vectorcore {

class Storage {
public:
    virtual ~Storage() = default;
    [[nodiscard]] virtual Device device() const noexcept = 0;
    [[nodiscard]] virtual std::size_t size() const noexcept = 0;
    // Host-addressable data; device storages throw std::runtime_error.
    [[nodiscard]] virtual const float* data() const;
    [[nodiscard]] virtual float* mutable_data();

    // Shared by every view of the storage. Autograd records it when a tensor
    // is saved for backward and rejects the backward if it changed.
    [[nodiscard]] std::uint64_t version() const noexcept { return version_; }
    void bump_version() noexcept { ++version_; }

private:
    std::uint64_t version_{0};
};

std::shared_ptr<Storage> make_cpu_storage(std::size_t elements);
std::shared_ptr<Storage> make_cpu_storage(const float* values, std::size_t elements);

}  // namespace vectorcore
