// Instantiates the vc_hip_map launchers for VC_MAP_NIN inputs (the build
// compiles this file once per input count, 1 to 8).
#include "fused_map.hpp"

#ifndef VC_MAP_NIN
#error "compile with -DVC_MAP_NIN=<inputs>"
#endif

namespace vchip {
namespace fmap {

template void launch_flat<VC_MAP_NIN>(Device&, const Program&, int64_t, bool);
template void launch_columns<VC_MAP_NIN>(Device&, const Program&, int64_t, int64_t, bool, double*);

}  // namespace fmap
}  // namespace vchip
