#pragma once
// Host thread pool for the `cpu` device kernels.
#include <cstddef>
#include <functional>

namespace vectorcore::cpu {

// Calls body(begin, end) for the chunks [i*grain, min((i+1)*grain, count)).
// The chunking depends only on count and grain, so per-chunk partial results
// combined in chunk order do not depend on how many threads ran them. Calls
// from inside a running body execute inline.
void parallel_for(std::size_t count, std::size_t grain, const std::function<void(std::size_t, std::size_t)>& body);

}  // namespace vectorcore::cpu
