// Kernels of vc_hip_map (fused elementwise programs), shared by the
// translation units that instantiate them: fused_map_inputs.hip is compiled
// once per input count (VC_MAP_NIN = 1..8) so that the unrolled
// interpreters compile in parallel; fused_map.hip holds the C ABI.
#pragma once

#include "vc_hip_internal.hpp"

namespace vchip {
namespace fmap {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kSlots = VC_HIP_MAP_SLOTS;
constexpr int kCode = VC_HIP_MAP_CODE;
constexpr int kShortCode = 16;
constexpr int kInputs = VC_HIP_MAP_INPUTS;
constexpr int kOutputs = VC_HIP_MAP_OUTPUTS;
constexpr int kSums = VC_HIP_MAP_SUMS;
constexpr int kConsts = VC_HIP_MAP_CONSTANTS;
constexpr unsigned kMapBlock = 256;
static_assert(kSlots == 16, "a slot is one element of a 16-wide register vector");

struct Program {
    const float* in[kInputs];
    float* out[kOutputs];
    float konst[kConsts];
    uint32_t code[kCode];  // op | a << 8 | b << 16 | dst << 24
    int n_code, n_const, n_out, n_sum;
    uint8_t out_slot[kOutputs];
    uint8_t sum_slot[kSums];
};

// W values per slot: one element (W = 1) or four consecutive ones (W = 4).
template <int W>
struct Regs {
    f16v c[W];
};
template <int W>
struct Vals {
    float v[W];
};

template <int W>
__device__ inline Vals<W> get(const Regs<W>& r, int slot) {
    Vals<W> o;
#pragma unroll
    for (int j = 0; j < W; ++j) o.v[j] = r.c[j][slot];
    return o;
}
template <int W>
__device__ inline void put(Regs<W>& r, int slot, const Vals<W>& v) {
#pragma unroll
    for (int j = 0; j < W; ++j) r.c[j][slot] = v.v[j];
}

template <int W>
__device__ inline Vals<W> load(const float* __restrict__ p) {
    Vals<W> o;
    if constexpr (W == 4) {
        const f4 x = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
        o.v[0] = x.x;
        o.v[1] = x.y;
        o.v[2] = x.z;
        o.v[3] = x.w;
    } else {
        o.v[0] = __builtin_nontemporal_load(p);
    }
    return o;
}
template <int W>
__device__ inline void store(float* __restrict__ p, const Vals<W>& v) {
    if constexpr (W == 4) {
        __builtin_nontemporal_store(f4{v.v[0], v.v[1], v.v[2], v.v[3]}, reinterpret_cast<f4*>(p));
    } else {
        __builtin_nontemporal_store(v.v[0], p);
    }
}

// The first Code instructions (Code >= n_code), unrolled so that every word
// is a kernel-argument scalar.
template <int Code, int W>
__device__ inline void run(Regs<W>& r, const Program& P) {
#pragma unroll
    for (int k = 0; k < Code; ++k) {
        if (k >= P.n_code) continue;  // uniform: the rest of the loop is skipped
        const uint32_t word = P.code[k];
        const int op = int(word & 255u), ia = int((word >> 8) & 255u), ib = int((word >> 16) & 255u),
                  id = int(word >> 24);
        const Vals<W> a = get(r, ia), b = get(r, ib);
        Vals<W> v;
        switch (op) {
            case VC_MAP_ADD:
#pragma unroll
                for (int j = 0; j < W; ++j) v.v[j] = a.v[j] + b.v[j];
                break;
            case VC_MAP_SUB:
#pragma unroll
                for (int j = 0; j < W; ++j) v.v[j] = a.v[j] - b.v[j];
                break;
            case VC_MAP_MUL:
#pragma unroll
                for (int j = 0; j < W; ++j) v.v[j] = a.v[j] * b.v[j];
                break;
            case VC_MAP_DIV:
#pragma unroll
                for (int j = 0; j < W; ++j) v.v[j] = a.v[j] / b.v[j];
                break;
            case VC_MAP_NEG:
#pragma unroll
                for (int j = 0; j < W; ++j) v.v[j] = -a.v[j];
                break;
            default:  // VC_MAP_STEP
#pragma unroll
                for (int j = 0; j < W; ++j) v.v[j] = a.v[j] > 0.0f ? 1.0f : 0.0f;
                break;
        }
        put(r, id, v);
    }
}

template <int W>
__device__ inline void set_constants(Regs<W>& r, const Program& P, int n_in) {
#pragma nounroll
    for (int c = 0; c < P.n_const; ++c) {
        Vals<W> v;
#pragma unroll
        for (int j = 0; j < W; ++j) v.v[j] = P.konst[c];
        put(r, n_in + c, v);
    }
}

// Loads element group e (W consecutive values) of every input into its slot.
// (Loading the next group ahead of the computation measured no faster: the
// other waves of the CU hide the latency.)
template <int NIn, int W>
__device__ inline void load_inputs(Regs<W>& r, const Program& P, int64_t e) {
    Vals<W> v[NIn];
#pragma unroll
    for (int j = 0; j < NIn; ++j) v[j] = load<W>(P.in[j] + e);
#pragma unroll
    for (int j = 0; j < NIn; ++j) put(r, j, v[j]);
}

template <int W>
__device__ inline void store_outputs(const Regs<W>& r, const Program& P, int64_t e) {
#pragma unroll
    for (int j = 0; j < kOutputs; ++j)
        if (j < P.n_out) store<W>(P.out[j] + e, get(r, P.out_slot[j]));
}

// Elements [0, count) in groups of W: thread t takes groups t, t + threads, ...
template <int NIn, int W, int Code>
__global__ __launch_bounds__(kMapBlock) void map_flat_kernel(Program P, int64_t groups) {
    Regs<W> r;
    set_constants(r, P, NIn);
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t g = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; g < groups; g += stride) {
        load_inputs<NIn, W>(r, P, g * W);
        run<Code>(r, P);
        store_outputs(r, P, g * W);
    }
}

// A [rows, cols] view, with the column sums of P.sum_slot[s] for s < NSum.
// Workgroup (x, y) of a grid (col_blocks, gy) takes columns
// [x * 64 W, (x + 1) * 64 W): lane l holds W consecutive columns, and wave w
// the rows w + 4 y, w + 4 y + 4 gy, w + 4 y + 8 gy, ... (at any moment the
// grid streams a contiguous band of rows). Each lane adds its values in double
// in row order; the four waves' sums are added in wave order and written as
// partial row y: part[s][y][col]. column_partials_kernel then adds the gy
// partial rows in a fixed order.
template <int NIn, int W, int Code, int NSum>
__global__ __launch_bounds__(kMapBlock) void map_columns_kernel(Program P, int64_t rows, int64_t cols,
                                                                double* __restrict__ part) {
    __shared__ double wave_part[NSum][4][64 * W];
    const int lane = int(threadIdx.x) & 63, w = int(threadIdx.x) >> 6;
    const int64_t col = (int64_t(blockIdx.x) * 64 + lane) * W;
    const int64_t step = 4 * int64_t(gridDim.y);
    Regs<W> r;
    set_constants(r, P, NIn);
    double acc[NSum][W];
#pragma unroll
    for (int s = 0; s < NSum; ++s)
#pragma unroll
        for (int j = 0; j < W; ++j) acc[s][j] = 0.0;
    if (col < cols) {
        for (int64_t row = int64_t(blockIdx.y) * 4 + w; row < rows; row += step) {
            const int64_t e = row * cols + col;
            load_inputs<NIn, W>(r, P, e);
            run<Code>(r, P);
            store_outputs(r, P, e);
#pragma unroll
            for (int s = 0; s < NSum; ++s) {
                if (s < P.n_sum) {
                    const Vals<W> v = get(r, P.sum_slot[s]);
#pragma unroll
                    for (int j = 0; j < W; ++j) acc[s][j] += double(v.v[j]);
                }
            }
        }
    }
#pragma unroll
    for (int s = 0; s < NSum; ++s)
#pragma unroll
        for (int j = 0; j < W; ++j) wave_part[s][w][lane * W + j] = acc[s][j];
    __syncthreads();
    if (w == 0 && col < cols) {
        for (int s = 0; s < P.n_sum; ++s) {
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const int i = lane * W + j;
                const double t = ((wave_part[s][0][i] + wave_part[s][1][i]) + wave_part[s][2][i]) + wave_part[s][3][i];
                if (col + j < cols) part[(int64_t(s) * gridDim.y + blockIdx.y) * cols + col + j] = t;
            }
        }
    }
}

// Flat launches: at most 4096 workgroups (16 per CU), each thread looping.
constexpr unsigned kFlatBlocks = 4096;

template <int NIn>
void launch_flat(Device& d, const Program& P, int64_t count, bool vec) {
    if (vec) {
        const int64_t groups = count / 4;
        if (groups > 0) {
            const dim3 grid(grid_1d(size_t(groups), kMapBlock, kFlatBlocks));
            if (P.n_code <= kShortCode)
                launch(map_flat_kernel<NIn, 4, kShortCode>, grid, dim3(kMapBlock), 0, d.stream, P, groups);
            else
                launch(map_flat_kernel<NIn, 4, kCode>, grid, dim3(kMapBlock), 0, d.stream, P, groups);
        }
        const int64_t done = groups * 4;
        if (done < count) {  // the last count % 4 elements
            Program tail = P;
            for (int j = 0; j < NIn; ++j) tail.in[j] += done;
            for (int j = 0; j < P.n_out; ++j) tail.out[j] += done;
            launch(map_flat_kernel<NIn, 1, kCode>, dim3(1), dim3(kMapBlock), 0, d.stream, tail, count - done);
        }
    } else {
        launch(map_flat_kernel<NIn, 1, kCode>, dim3(grid_1d(size_t(count), kMapBlock, kFlatBlocks)), dim3(kMapBlock), 0,
               d.stream, P, count);
    }
}

// The column traversal's grid: about 2048 workgroups, with gy (the number of
// partial rows) at most rows / 4. A function of the shape only, so the order
// of every column sum is too.
struct ColumnGrid {
    int64_t col_blocks, gy;
};
inline ColumnGrid column_grid(int64_t rows, int64_t cols, int w) {
    ColumnGrid g{};
    g.col_blocks = (cols + 64 * w - 1) / (64 * w);
    g.gy = (2048 + g.col_blocks - 1) / g.col_blocks;
    const int64_t max_gy = (rows + 3) / 4;
    if (g.gy > max_gy) g.gy = max_gy;
    if (g.gy < 1) g.gy = 1;
    return g;
}

template <int NIn>
void launch_columns(Device& d, const Program& P, int64_t rows, int64_t cols, bool vec, double* part) {
    const ColumnGrid g = column_grid(rows, cols, vec ? 4 : 1);
    const dim3 grid(unsigned(g.col_blocks), unsigned(g.gy));
    if (vec && P.n_code <= kShortCode && P.n_sum == 1)  // the common case: a short program, one sum
        launch(map_columns_kernel<NIn, 4, kShortCode, 1>, grid, dim3(kMapBlock), 0, d.stream, P, rows, cols, part);
    else if (vec)
        launch(map_columns_kernel<NIn, 4, kCode, kSums>, grid, dim3(kMapBlock), 0, d.stream, P, rows, cols, part);
    else
        launch(map_columns_kernel<NIn, 1, kCode, kSums>, grid, dim3(kMapBlock), 0, d.stream, P, rows, cols, part);
}

}  // namespace fmap
}  // namespace vchip
