#include "vectorcore/storage.hpp"

#include <algorithm>
#include <stdexcept>

namespace vectorcore {

const float* Storage::data() const { throw std::runtime_error("storage is not directly CPU-addressable"); }
float* Storage::mutable_data() { throw std::runtime_error("storage is not directly CPU-addressable"); }

namespace {

// Host buffer; left uninitialised because every kernel writes its whole output.
class HostStorage final : public Storage {
public:
    explicit HostStorage(std::size_t n) : values_(n ? new float[n] : nullptr), n_(n) {}
    [[nodiscard]] Device device() const noexcept override { return Device::cpu(); }
    [[nodiscard]] std::size_t size() const noexcept override { return n_; }
    [[nodiscard]] const float* data() const override { return values_.get(); }
    [[nodiscard]] float* mutable_data() override { return values_.get(); }
private:
    std::unique_ptr<float[]> values_;
    std::size_t n_;
};

}  // namespace

std::shared_ptr<Storage> make_cpu_storage(std::size_t elements) { return std::make_shared<HostStorage>(elements); }

std::shared_ptr<Storage> make_cpu_storage(const float* values, std::size_t elements) {
    if (!values && elements) throw std::invalid_argument("null storage source");
    auto s = std::make_shared<HostStorage>(elements);
    if (elements) std::copy(values, values + elements, s->mutable_data());
    return s;
}

}  // namespace vectorcore
