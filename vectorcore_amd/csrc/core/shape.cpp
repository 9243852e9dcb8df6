#include "vectorcore/shape.hpp"

#include <algorithm>
#include <limits>
#include <sstream>
#include <stdexcept>

namespace vectorcore {

std::size_t numel(const Shape& shape) {
    std::size_t n = 1;
    for (std::size_t d : shape) {
        if (d != 0 && n > std::numeric_limits<std::size_t>::max() / d)
            throw std::overflow_error("tensor element count overflows size_t");
        n *= d;
    }
    return n;
}

Strides contiguous_strides(const Shape& shape) {
    Strides s(shape.size());
    std::size_t step = 1;
    for (std::size_t i = shape.size(); i-- > 0;) {
        s[i] = step;
        step *= shape[i];
    }
    return s;
}

bool is_contiguous(const Shape& shape, const Strides& strides) { return strides == contiguous_strides(shape); }

Shape broadcast_shape(const Shape& a, const Shape& b) {
    const std::size_t rank = std::max(a.size(), b.size());
    Shape out(rank);
    for (std::size_t i = 0; i < rank; ++i) {
        // Align from the trailing axis; missing leading axes act as 1.
        const std::size_t da = i + a.size() >= rank ? a[i + a.size() - rank] : 1;
        const std::size_t db = i + b.size() >= rank ? b[i + b.size() - rank] : 1;
        if (da != db && da != 1 && db != 1)
            throw std::invalid_argument("cannot broadcast shapes " + shape_string(a) + " and " + shape_string(b));
        out[i] = da == 1 ? db : da;
    }
    return out;
}

std::string shape_string(const Shape& shape) {
    std::ostringstream s;
    s << '[';
    for (std::size_t i = 0; i < shape.size(); ++i) s << (i ? ", " : "") << shape[i];
    s << ']';
    return s.str();
}

}  // namespace vectorcore
