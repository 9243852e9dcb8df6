// One pass of a small elementwise program over same-shape contiguous
// operands (vc_hip_map): the gradient expressions that the backward rules of
// a chain of elementwise ops build one kernel at a time, evaluated together,
// each element read once and each result written once, with the column sums
// of up to two program values accumulated on the way.
//
// The program is straight-line code over 16 value slots: the inputs sit in
// slots [0, n_inputs) (reloaded for every element), the constants in the
// next n_constants slots, and each instruction writes one slot. A slot is an
// element of a 16-wide vector register per component, indexed with the
// instruction's operand numbers: these are uniform across the wavefront, so
// the hardware's relative register addressing reads and writes them without
// touching memory. The instruction words are kernel arguments, read into
// scalar registers once per kernel; programs of at most 16 instructions run a
// kernel unrolled to 16, which keeps the decoded words in scalar registers.
// Every operation is the single fp32 operation that the unfused kernel of the
// same rule performs (contraction is off), so each result has the same bits as
// the chain of kernels it replaces.
//
// Every element is read and written once, so loads and stores are
// non-temporal (streamed past the caches). Measured on MI355X at 4096 x 4096
// with four inputs, one output and one column sum: 60 us for 268 MB read and
// 67 MB written (5.6 TB/s).
#include "fused_map.hpp"
#include "reduce_common.hpp"

#include <string>

namespace vchip {
namespace fmap {

// Instantiated in fused_map_inputs.hip, one translation unit per input count.
#define VC_MAP_EXTERN(N)                                                                  \
    extern template void launch_flat<N>(Device&, const Program&, int64_t, bool);         \
    extern template void launch_columns<N>(Device&, const Program&, int64_t, int64_t, bool, double*);
VC_MAP_EXTERN(1)
VC_MAP_EXTERN(2)
VC_MAP_EXTERN(3)
VC_MAP_EXTERN(4)
VC_MAP_EXTERN(5)
VC_MAP_EXTERN(6)
VC_MAP_EXTERN(7)
VC_MAP_EXTERN(8)
#undef VC_MAP_EXTERN

namespace {

template <template <int> class F, typename... Args>
void by_inputs(int n_in, Args&&... args) {
    switch (n_in) {
        case 1: F<1>::go(args...); break;
        case 2: F<2>::go(args...); break;
        case 3: F<3>::go(args...); break;
        case 4: F<4>::go(args...); break;
        case 5: F<5>::go(args...); break;
        case 6: F<6>::go(args...); break;
        case 7: F<7>::go(args...); break;
        default: F<8>::go(args...); break;
    }
}
template <int N>
struct FlatLaunch {
    static void go(Device& d, const Program& P, int64_t count, bool vec) { launch_flat<N>(d, P, count, vec); }
};
template <int N>
struct ColumnLaunch {
    static void go(Device& d, const Program& P, int64_t rows, int64_t cols, bool vec, double* part) {
        launch_columns<N>(d, P, rows, cols, vec, part);
    }
};

// Checks the program on the host: operand and destination slots in range,
// every slot read after it is written (inputs and constants count as
// written), constants never overwritten, opcodes known.
void validate(const vc_hip_map_program& p) {
    auto bad = [](const std::string& why) { fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_map: " + why); };
    if (p.n_inputs < 1 || p.n_inputs > size_t(kInputs)) bad("needs 1 to 8 inputs");
    if (p.n_constants > size_t(kConsts)) bad("at most 8 constants");
    if (p.n_inputs + p.n_constants > size_t(kSlots)) bad("inputs and constants exceed the 16 slots");
    if (p.n_code > size_t(kCode)) bad("at most 32 instructions");
    if (p.n_outputs > size_t(kOutputs) || p.n_sums > size_t(kSums)) bad("at most 4 outputs and 2 column sums");
    if (p.n_outputs + p.n_sums == 0) bad("nothing to compute");
    for (size_t j = 0; j < p.n_inputs; ++j)
        if (!p.inputs[j]) bad("null input");
    for (size_t j = 0; j < p.n_outputs; ++j)
        if (!p.outputs[j]) bad("null output");
    for (size_t j = 0; j < p.n_sums; ++j)
        if (!p.sums[j]) bad("null column-sum output");
    const size_t first_temp = p.n_inputs + p.n_constants;
    uint32_t written = (1u << first_temp) - 1u;
    for (size_t k = 0; k < p.n_code; ++k) {
        const uint32_t w = p.code[k];
        const unsigned op = w & 255u, a = (w >> 8) & 255u, b = (w >> 16) & 255u, dst = w >> 24;
        if (op > VC_MAP_STEP) bad("unknown opcode at instruction " + std::to_string(k));
        if (a >= unsigned(kSlots) || b >= unsigned(kSlots) || dst >= unsigned(kSlots))
            bad("slot out of range at instruction " + std::to_string(k));
        if (!(written >> a & 1u) || !(written >> b & 1u))
            bad("instruction " + std::to_string(k) + " reads a slot before it is written");
        if (dst >= p.n_inputs && dst < first_temp) bad("instruction " + std::to_string(k) + " overwrites a constant");
        written |= 1u << dst;
    }
    for (size_t j = 0; j < p.n_outputs; ++j)
        if (p.output_slots[j] >= kSlots || !(written >> p.output_slots[j] & 1u)) bad("output slot never written");
    for (size_t j = 0; j < p.n_sums; ++j)
        if (p.sum_slots[j] >= kSlots || !(written >> p.sum_slots[j] & 1u)) bad("column-sum slot never written");
}

}  // namespace
}  // namespace fmap
}  // namespace vchip

using namespace vchip;
using namespace vchip::fmap;

using namespace vchip;

extern "C" {

int vc_hip_map(const vc_hip_map_program* program) {
    return guard([&] {
        Device& d = require_device();
        if (!program) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_map: null program");
        const vc_hip_map_program& p = *program;
        validate(p);
        if (p.cols != 0 && p.rows > SIZE_MAX / p.cols) fail(VC_HIP_ERR_OVERFLOW, "vc_hip_map: element count overflows");
        const size_t count = p.rows * p.cols;
        if (count > size_t(INT64_MAX) / 8) fail(VC_HIP_ERR_OVERFLOW, "vc_hip_map: too many elements");
        if (p.n_sums > 0 && count == 0) {  // an empty column: its sum is 0
            for (size_t s = 0; s < p.n_sums; ++s) {
                const int status = p.cols ? vc_hip_fill(p.sums[s], p.cols, 0.0f) : VC_HIP_OK;
                if (status != VC_HIP_OK) fail(status, vc_hip_last_error());
            }
            return;
        }
        if (count == 0) return;

        Program P{};
        for (size_t j = 0; j < p.n_inputs; ++j) P.in[j] = p.inputs[j];
        for (size_t j = 0; j < p.n_outputs; ++j) {
            P.out[j] = p.outputs[j];
            P.out_slot[j] = p.output_slots[j];
        }
        for (size_t j = 0; j < p.n_constants; ++j) P.konst[j] = p.constants[j];
        for (size_t k = 0; k < p.n_code; ++k) P.code[k] = p.code[k];
        for (size_t s = 0; s < p.n_sums; ++s) P.sum_slot[s] = p.sum_slots[s];
        P.n_code = int(p.n_code);
        P.n_const = int(p.n_constants);
        P.n_out = int(p.n_outputs);
        P.n_sum = int(p.n_sums);

        bool vec = true;
        for (size_t j = 0; j < p.n_inputs; ++j) vec = vec && aligned16(p.inputs[j]);
        for (size_t j = 0; j < p.n_outputs; ++j) vec = vec && aligned16(p.outputs[j]);
        const double bytes = 4.0 * double(count) * double(p.n_inputs + p.n_outputs);
        const int n_in = int(p.n_inputs);
        if (p.n_sums == 0) {
            Profiled prof("fused_map", 0.0, bytes);
            by_inputs<FlatLaunch>(n_in, d, P, int64_t(count), vec);
            after_launch("fused_map");
            prof.done();
            return;
        }
        const int64_t rows = int64_t(p.rows), cols = int64_t(p.cols);
        vec = vec && cols % 4 == 0;
        const ColumnGrid g = column_grid(rows, cols, vec ? 4 : 1);
        Scratch part(sizeof(double) * size_t(p.n_sums) * size_t(g.gy) * size_t(cols));
        {
            Profiled prof("fused_map_columns", 0.0, bytes + 8.0 * double(p.n_sums) * double(g.gy * cols));
            by_inputs<ColumnLaunch>(n_in, d, P, rows, cols, vec, part.as<double>());
            after_launch("fused_map_columns");
            prof.done();
        }
        Profiled prof("column_sum_combine", 0.0,
                      8.0 * double(p.n_sums) * double(g.gy * cols) + 4.0 * double(p.n_sums * cols));
        for (size_t s = 0; s < p.n_sums; ++s) {
            launch(red::column_partials_kernel, dim3(unsigned((cols + 63) / 64)), dim3(64 * red::kCombineWaves), 0,
                   d.stream, part.as<double>() + int64_t(s) * g.gy * cols, g.gy, cols, p.sums[s]);
            after_launch("column_sum_combine");
        }
        prof.done();
    });
}

}  // extern "C"
