// Batched fp32 GEMM on gfx950 matrix cores:  C[z] = sum_r op(A[z,r]) @ op(B[z,r])
//
// Covers the three products of a linear layer's forward and backward
// (src/ops.cpp:244-262): NN (y = x W), NT (dA = dY B^T, B read as stored
// [n, k]) and TN (dB = A^T dY, A read as stored [k, m]); transposed operands
// are read in place. The r-sum is the batch reduction that a batch-broadcast
// operand's gradient needs (one fixed order, no atomics).
//
// Tiling: a 256-thread workgroup computes a 128 x 128 tile of C; each of its
// four waves owns a 64 x 64 quadrant as 2 x 2 blocks of
// V_MFMA_F32_32X32X2_F32 (A: lane l holds A[l%32][k], B: B[k][l%32], k = l/32;
// D: 16 values per lane, row 8(v/4) + 4(l/32) + v%4, column l%32 — checked on
// the device). K advances in slices of 32: while the waves run the 64 MFMAs of
// one slice from LDS, every thread already holds the next slice's global loads
// in registers.
//
// LDS layout follows each operand's contiguous axis, so no transposing stores:
//  - k-contiguous operand (A in NN/NT, B in NT): [128][32 + 4] floats; a lane
//    reads 4 consecutive k with one ds_read_b128, feeding 4 MFMA steps. The
//    +4 padding makes the 8-lane phases of those reads conflict-free.
//  - m/n-contiguous operand (A in TN, B in NN/TN): [32][128 + 8] floats; a
//    lane reads one value per MFMA step (ds_read_b32); +8 keeps the two
//    half-waves (k and k+4) on different banks.
// Within each group of 8 k, half-wave 0 of a step takes k = 8g + s and
// half-wave 1 takes k = 8g + 4 + s (s = 0..3): a fixed permutation of the
// summation index applied identically to A and B.
//
// Tile order: workgroups are dispatched round-robin over the 8 XCDs, each with
// its own L2. Consecutive tile ids are remapped onto one XCD and walked in
// groups of 8 tile-rows, so tiles sharing A rows or B columns share an L2.
#include "vc_hip_internal.hpp"

#include <algorithm>
#include <limits>
#include <vector>

namespace vchip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int kThreads = 256;
constexpr int kPadK = 4;   // k-contiguous LDS row padding
constexpr int kPadMN = 8;  // m/n-contiguous LDS row padding
constexpr int kLdsK = BM * (BK + kPadK);   // floats, k-contiguous tile
constexpr int kLdsMN = BK * (BM + kPadMN); // floats, m/n-contiguous tile
constexpr int kLdsTile = kLdsK > kLdsMN ? kLdsK : kLdsMN;
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

struct GemmArgs {
    const float* a;
    const float* b;
    float* c;
    int M, N, K;
    int lda, ldb;                  // row stride of A and B as stored
    int64_t batch;                 // output matrices
    int64_t a_bstride, b_bstride;  // element offset per output batch (affine mode)
    const int64_t* table;          // per-batch (a, b) offsets, or null for affine mode
    int64_t reduce;                // products summed into each output
    int64_t a_rstride, b_rstride;
    int tiles_m, tiles_n;
};

// Tile id -> (tile_m, tile_n) with the XCD remap and grouped order.
__device__ inline void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    const int whole = total / kXcds * kXcds;
    if (pid < whole) {
        const int per_xcd = whole / kXcds;
        pid = (pid % kXcds) * per_xcd + pid / kXcds;
    }
    const int in_group = kGroupM * tiles_n;
    const int group = pid / in_group;
    const int first_m = group * kGroupM;
    const int group_rows = min(tiles_m - first_m, kGroupM);
    const int local = pid % in_group;
    tm = first_m + local % group_rows;
    tn = local / group_rows;
}

// Buffer resource over `base` (gfx9 descriptor word 3). Offsets at or above
// kOutOfRange fall outside num_records: loads return 0, stores are dropped.
// The raw buffer builtins move 32-bit integers; values are bit-cast.
constexpr uint32_t kOutOfRange = 0x80000000u;
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), short(0), int(kOutOfRange - 1), 0x00020000);
}

// Global -> register loader for one operand tile (128 along m/n, BK along k).
// The tile origin is uniform (scalar registers); each thread keeps 32-bit byte
// offsets of its four 16-byte slots, their k position and whether their m/n
// row is inside the matrix. Edges are masked by pointing a slot out of range.
// KC: operand contiguous along k.
template <bool KC, bool Vec>
struct TileLoader {
    const float* origin;  // element (mn0, 0) of this operand
    int64_t step;         // elements per BK slice
    int K;
    uint32_t boff[4];
    int kpos[4];
    int mn_ok;
    int ld, mn_lim;       // scalar path: row stride, rows left in the matrix

    __device__ void init(const float* base, int ld_, int mn0, int MN, int K_) {
        K = K_;
        ld = ld_;
        mn_lim = MN - mn0;
        origin = KC ? base + int64_t(mn0) * ld : base + mn0;
        step = KC ? int64_t(BK) : int64_t(BK) * ld;
        mn_ok = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = threadIdx.x + q * kThreads;
            int mn_local, k_local;
            if (KC) {  // 128 rows x 8 vectors along k
                mn_local = idx / (BK / 4);
                k_local = (idx % (BK / 4)) * 4;
                boff[q] = uint32_t(mn_local * ld + k_local) * 4u;
            } else {  // 32 k-rows x 32 vectors along m/n
                k_local = idx / (BM / 4);
                mn_local = (idx % (BM / 4)) * 4;
                boff[q] = uint32_t(k_local * ld + mn_local) * 4u;
            }
            if (mn_local < mn_lim) mn_ok |= 1 << q;
            kpos[q] = k_local;
        }
    }

    __device__ void load(int kt, f4 (&reg)[4]) const {
        const int k0 = kt * BK;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(origin + int64_t(kt) * step);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (Vec) {
                const bool ok = ((mn_ok >> q) & 1) && (k0 + kpos[q] < K);
                reg[q] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? boff[q] : kOutOfRange, 0, 0));
            } else {
                const int idx = threadIdx.x + q * kThreads;
                f4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int mn, k;
                    if (KC) {
                        mn = idx / (BK / 4);
                        k = (idx % (BK / 4)) * 4 + e;
                    } else {
                        k = idx / (BM / 4);
                        mn = (idx % (BM / 4)) * 4 + e;
                    }
                    const bool ok = mn < mn_lim && k0 + k < K;
                    const uint32_t off = uint32_t(KC ? mn * ld + k : k * ld + mn) * 4u;
                    v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? off : kOutOfRange, 0, 0));
                }
                reg[q] = v;
            }
        }
    }
};

template <bool KC>
__device__ inline void store_slice(float* __restrict__ lds, const f4 (&reg)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int idx = threadIdx.x + q * kThreads;
        if (KC) {
            const int row = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
            *reinterpret_cast<f4*>(lds + row * (BK + kPadK) + c) = reg[q];
        } else {
            const int row = idx / (BM / 4), c = (idx % (BM / 4)) * 4;
            *reinterpret_cast<f4*>(lds + row * (BM + kPadMN) + c) = reg[q];
        }
    }
}

// Fragment values of 4 MFMA steps (k-group g) for the 32-row block at `off`.
template <bool KC>
__device__ inline f4 read_frag(const float* __restrict__ lds, int off, int g, int lane) {
    const int r = off + (lane & 31);
    const int kb = g * 8 + 4 * (lane >> 5);
    if (KC) return *reinterpret_cast<const f4*>(lds + r * (BK + kPadK) + kb);
    f4 v;
#pragma unroll
    for (int s = 0; s < 4; ++s) v[s] = lds[(kb + s) * (BM + kPadMN) + r];
    return v;
}

template <bool TA, bool TB, bool Vec>
__global__ __launch_bounds__(kThreads, 2) void gemm_mfma_kernel(GemmArgs p) {
    __shared__ __attribute__((aligned(16))) float As[kLdsTile];
    __shared__ __attribute__((aligned(16))) float Bs[kLdsTile];
    constexpr bool AKC = !TA;  // A contiguous along k
    constexpr bool BKC = TB;   // B contiguous along k
    int tm, tn;
    tile_coords(int(blockIdx.x), p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int kt_count = (p.K + BK - 1) / BK;

    for (int64_t z = blockIdx.y; z < p.batch; z += gridDim.y) {
        int64_t aoff, boff;
        if (p.table) {
            aoff = p.table[2 * z];
            boff = p.table[2 * z + 1];
        } else {
            aoff = z * p.a_bstride;
            boff = z * p.b_bstride;
        }
        f16v acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

        for (int64_t r = 0; r < p.reduce; ++r) {
            TileLoader<AKC, Vec> la;
            TileLoader<BKC, Vec> lb;
            la.init(p.a + aoff + r * p.a_rstride, p.lda, m0, p.M, p.K);
            lb.init(p.b + boff + r * p.b_rstride, p.ldb, n0, p.N, p.K);
            f4 ra[4], rb[4];
            if (kt_count > 0) {
                la.load(0, ra);
                lb.load(0, rb);
            }
            for (int kt = 0; kt < kt_count; ++kt) {
                __syncthreads();  // the previous slice is no longer read
                store_slice<AKC>(As, ra);
                store_slice<BKC>(Bs, rb);
                __syncthreads();
                if (kt + 1 < kt_count) {  // next slice in flight during the MFMAs
                    la.load(kt + 1, ra);
                    lb.load(kt + 1, rb);
                }
#pragma unroll
                for (int g = 0; g < BK / 8; ++g) {
                    f4 fa[2], fb[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) fa[i] = read_frag<AKC>(As, wm + 32 * i, g, lane);
#pragma unroll
                    for (int j = 0; j < 2; ++j) fb[j] = read_frag<BKC>(Bs, wn + 32 * j, g, lane);
#pragma unroll
                    for (int s = 0; s < 4; ++s)
#pragma unroll
                        for (int i = 0; i < 2; ++i)
#pragma unroll
                            for (int j = 0; j < 2; ++j)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
                }
            }
        }
        // Epilogue: buffer stores relative to the tile origin; rows/columns
        // outside C are pointed out of range and dropped by the hardware.
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.c + z * int64_t(p.M) * p.N + int64_t(m0) * p.N + n0);
        const int row_lim = p.M - m0, col_lim = p.N - n0;
        const int row0 = wm + 4 * (lane >> 5);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = wn + 32 * j + (lane & 31);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int row = row0 + 32 * i + 8 * (v >> 2) + (v & 3);
                    const bool ok = row < row_lim && col < col_lim;
                    const float value = acc[i][j][v];  // element first: bit-casting the subscript takes lane 0
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), rc,
                                                          ok ? uint32_t(row * p.N + col) * 4u : kOutOfRange,
                                                          0, 0);
                }
            }
    }
}

// Portable LDS-tiled FMA kernel (VECTORCORE_HIP_GEMM=simple): 16 x 16 outputs
// per 256-thread workgroup, one per thread.
template <bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm_simple_kernel(GemmArgs p) {
    __shared__ float as[16][17];
    __shared__ float bs[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t row = int64_t(blockIdx.x / p.tiles_n) * 16 + ty;
    const int64_t col = int64_t(blockIdx.x % p.tiles_n) * 16 + tx;
    for (int64_t z = blockIdx.y; z < p.batch; z += gridDim.y) {
        const int64_t aoff = p.table ? p.table[2 * z] : z * p.a_bstride;
        const int64_t boff = p.table ? p.table[2 * z + 1] : z * p.b_bstride;
        float acc = 0.0f;
        for (int64_t r = 0; r < p.reduce; ++r) {
            const float* A = p.a + aoff + r * p.a_rstride;
            const float* B = p.b + boff + r * p.b_rstride;
            for (int64_t k0 = 0; k0 < p.K; k0 += 16) {
                const int64_t ar = int64_t(blockIdx.x / p.tiles_n) * 16 + ty, ak = k0 + tx;
                as[ty][tx] = (ar < p.M && ak < p.K) ? (TA ? A[ak * p.lda + ar] : A[ar * p.lda + ak]) : 0.0f;
                const int64_t bk = k0 + ty, bc = int64_t(blockIdx.x % p.tiles_n) * 16 + tx;
                bs[ty][tx] = (bk < p.K && bc < p.N) ? (TB ? B[bc * p.ldb + bk] : B[bk * p.ldb + bc]) : 0.0f;
                __syncthreads();
                for (int kk = 0; kk < 16; ++kk) acc += as[ty][kk] * bs[kk][tx];
                __syncthreads();
            }
        }
        if (row < p.M && col < p.N) p.c[z * p.M * p.N + row * p.N + col] = acc;
    }
}

template <bool TA, bool TB>
void launch_variant(const GemmArgs& args, bool vec, bool simple, dim3 grid, hipStream_t stream) {
    if (simple) {
        hipLaunchKernelGGL((gemm_simple_kernel<TA, TB>), grid, dim3(256), 0, stream, args);
    } else if (vec) {
        hipLaunchKernelGGL((gemm_mfma_kernel<TA, TB, true>), grid, dim3(kThreads), 0, stream, args);
    } else {
        hipLaunchKernelGGL((gemm_mfma_kernel<TA, TB, false>), grid, dim3(kThreads), 0, stream, args);
    }
}

const char* variant_label(bool ta, bool tb) {
    return ta ? (tb ? "gemm_tt" : "gemm_tn") : (tb ? "gemm_nt" : "gemm_nn");
}

// offsets: nullptr for the affine mode (a_bstride / b_bstride).
void gemm(const float* a, const float* b, float* c, int64_t M, int64_t N, int64_t K, int64_t batch, int64_t a_bstride,
          int64_t b_bstride, const std::vector<int64_t>* offsets, int64_t reduce, int64_t a_rstride, int64_t b_rstride,
          bool ta, bool tb) {
    Device& d = require_device();
    if (M < 0 || N < 0 || K < 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "negative matrix dimension");
    if (M == 0 || N == 0 || batch == 0) return;
    if (!a || !b || !c) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul: null buffer");
    const int64_t tiles_m_simple = (M + 15) / 16, tiles_n_simple = (N + 15) / 16;
    const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const bool simple = d.simple_gemm;
    const int64_t tiles = simple ? tiles_m_simple * tiles_n_simple : tiles_m * tiles_n;
    if (tiles > std::numeric_limits<int>::max() / 2) fail(VC_HIP_ERR_OVERFLOW, "matmul output has too many tiles");
    // Byte offsets relative to a tile origin are 32-bit: 128 rows of any
    // operand or of C must span less than 2 GiB.
    const int64_t kMax = int64_t(1) << 29;
    const int64_t widest = std::max({ta ? M : K, tb ? K : N, N});
    if (M >= kMax || N >= kMax || K >= kMax || widest * 128 >= kMax)
        fail(VC_HIP_ERR_OVERFLOW, "matmul operands exceed the 2 GiB per-matrix addressing of the HIP kernels");

    GemmArgs args{};
    args.a = a;
    args.b = b;
    args.c = c;
    args.M = int(M);
    args.N = int(N);
    args.K = int(K);
    args.lda = int(ta ? M : K);
    args.ldb = int(tb ? K : N);
    args.batch = batch;
    args.a_bstride = a_bstride;
    args.b_bstride = b_bstride;
    args.reduce = reduce;
    args.a_rstride = a_rstride;
    args.b_rstride = b_rstride;
    args.tiles_m = int(simple ? tiles_m_simple : tiles_m);
    args.tiles_n = int(simple ? tiles_n_simple : tiles_n);

    // 16-byte vector loads need every row start and batch offset on a 4-float boundary.
    bool vec = aligned16(a) && aligned16(b) && args.lda % 4 == 0 && args.ldb % 4 == 0 && a_rstride % 4 == 0 &&
               b_rstride % 4 == 0;
    Scratch table(offsets ? offsets->size() * sizeof(int64_t) : 8);
    if (offsets) {
        for (int64_t v : *offsets) vec = vec && v % 4 == 0;
        const int rc = vc_hip_upload(table.as<void>(), offsets->data(), offsets->size() * sizeof(int64_t));
        if (rc != VC_HIP_OK) fail(rc, "matmul offset table upload failed");
        args.table = table.as<int64_t>();
    } else {
        vec = vec && a_bstride % 4 == 0 && b_bstride % 4 == 0;
    }
    const dim3 grid(unsigned(tiles), unsigned(std::min<int64_t>(batch, 65535)));
    const char* label = variant_label(ta, tb);
    const double flops = 2.0 * double(M) * double(N) * double(K) * double(batch) * double(reduce);
    const double bytes = 4.0 * (double(M * K + K * N) * double(reduce) + double(M * N)) * double(batch);
    Profiled prof(label, flops, bytes);
    if (ta && tb) launch_variant<true, true>(args, vec, simple, grid, d.stream);
    else if (ta) launch_variant<true, false>(args, vec, simple, grid, d.stream);
    else if (tb) launch_variant<false, true>(args, vec, simple, grid, d.stream);
    else launch_variant<false, false>(args, vec, simple, grid, d.stream);
    after_launch(label);
    prof.done();
}

}  // namespace
}  // namespace vchip

using namespace vchip;

extern "C" {

int vc_hip_matmul(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, const size_t* a_offsets,
                  const size_t* b_offsets, size_t batch, int trans_a, int trans_b) {
    return guard([&] {
        if (batch == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul needs one A and B offset per batch");
        if (!a_offsets || !b_offsets) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul: null offsets");
        // Affine offsets (the common batched and broadcast cases) go as strides.
        const int64_t sa = batch > 1 ? int64_t(a_offsets[1]) - int64_t(a_offsets[0]) : 0;
        const int64_t sb = batch > 1 ? int64_t(b_offsets[1]) - int64_t(b_offsets[0]) : 0;
        bool affine = a_offsets[0] == 0 && b_offsets[0] == 0;
        for (size_t z = 0; affine && z < batch; ++z)
            affine = int64_t(a_offsets[z]) == int64_t(z) * sa && int64_t(b_offsets[z]) == int64_t(z) * sb;
        if (affine) {
            gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), int64_t(batch), sa, sb, nullptr, 1, 0, 0, trans_a != 0,
                 trans_b != 0);
        } else {
            std::vector<int64_t> table(2 * batch);
            for (size_t z = 0; z < batch; ++z) {
                table[2 * z] = int64_t(a_offsets[z]);
                table[2 * z + 1] = int64_t(b_offsets[z]);
            }
            gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), int64_t(batch), 0, 0, &table, 1, 0, 0, trans_a != 0,
                 trans_b != 0);
        }
    });
}

int vc_hip_matmul_reduce(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, size_t count,
                         size_t a_stride, size_t b_stride, int trans_a, int trans_b) {
    return guard([&] {
        if (count == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_reduce needs at least one product");
        gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), 1, 0, 0, nullptr, int64_t(count), int64_t(a_stride),
             int64_t(b_stride), trans_a != 0, trans_b != 0);
    });
}

}  // extern "C"
