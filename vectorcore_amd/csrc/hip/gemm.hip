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
// the device). K advances in slices of 32 through two LDS stages with one
// barrier per slice (the pipeline is described at gemm_mfma_kernel). Outputs
// with few tiles and a long K split K into ranges whose partial products are
// summed in range order by a second pass. Products of a few dozen such tiles
// at most run on 32 x 32 tiles instead, K split over a workgroup's eight waves
// (gemm_small_kernel), and tiny ones on the FMA kernel (gemm_simple_kernel).
//
// Each operand tile sits in LDS as it is laid out in memory, so it is stored
// as loaded. A k-contiguous operand (A in NN/NT, B in NT/TT) is [128][32 + 4]
// floats: a lane reads 4 consecutive k with one ds_read_b128, feeding 4 MFMA
// steps (the +4 padding keeps those reads conflict-free). An m/n-contiguous
// operand (A in TN/TT, B in NN/TN) is [32][128]: a lane reads two adjacent
// rows (columns) at one k with one ds_read_b64, feeding that step's MFMAs of
// both 32-row blocks, so its blocks interleave (block b holds rows 2d + b of
// the wave's 64). Within each group of 8 k, half-wave 0 of a step takes
// k = 8g + s and half-wave 1 takes k = 8g + 4 + s (s = 0..3), in either
// layout: a fixed permutation of the summation index applied identically to
// A and B, so every C element adds its products in the same order whatever
// the operands' layouts.
//
// Tile order: workgroups are dispatched round-robin over the 8 XCDs, each with
// its own L2. Consecutive tile ids are remapped onto one XCD and walked in
// groups of 8 tile-rows, so tiles sharing A rows or B columns share an L2.
#include "reduce_common.hpp"
#include "vc_hip_internal.hpp"

#include <algorithm>
#include <cstdlib>
#include <limits>
#include <optional>
#include <string>
#include <type_traits>
#include <vector>

namespace vchip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

// (A 64-deep slice, with the 139 KB of two stages holding one workgroup per
// CU, measured 2-7% slower on every product shape of the workloads.)
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int kSlots = BK / 8;                 // 16-byte global loads per thread per operand slice
constexpr int kKcRowsPerSlot = 4 * 256 / BK;   // k-contiguous rows one slot of 256 threads covers
constexpr int kThreads = 256;
constexpr int kPadK = 4;                     // LDS row padding
constexpr int kLdsTile = BM * (BK + kPadK);  // floats per operand tile stage: [128][32 + 4] k-contiguous
constexpr int kMnRow = BM;                   // an m/n-contiguous tile is [32][128] (fits in kLdsTile)
static_assert(BK * kMnRow <= kLdsTile, "m/n-contiguous tile larger than a stage");
constexpr int kGroupM = 8;
#ifndef VC_NN_VIA_NT_MIN_ROWS
#define VC_NN_VIA_NT_MIN_ROWS 4096
#endif
constexpr int64_t kNnViaNtMinRows = VC_NN_VIA_NT_MIN_ROWS;
constexpr int64_t kTinyTiles = 8;  // outputs of at most this many tiles split K finely
constexpr double kTinyMacs = 1048576.0;
constexpr int64_t kSimpleMaxK = 1024;  // and K up to this run on the FMA kernel
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
    int splits;                    // work split into this many ranges (partials summed afterwards):
    int kt_per_split;              //   reduce == 1: BK slices of K per split
    int64_t r_per_split;           //   reduce > 1: products r per split
    const float* relu_mask;        // null, or [batch][M][N]: C *= [relu_mask > 0] (fused ReLU backward)
    const float* bias;             // null, or [N]: C += bias[column] (fused row-bias add)
    int relu;                      // nonzero: C = C > 0 ? C : 0 after the bias (fused ReLU forward)
    double* col_part;              // null, or partial rows of C's column sums (batch 1, no split), in
                                   //   double: MFMA kernel 2 tiles_m rows (one per 64 rows of a tile),
                                   //   FMA kernel tiles_m rows (one per 16-row tile)
    // ReLU bitmasks (gemm_big_kernel with A k-contiguous, batch 1, no split):
    // bit r % 32 of word (r / 32) N + c stands for element (r, c).
    const uint32_t* relu_bits;     // null, or the fused ReLU backward's mask as such bits: C *= [bit]
    uint32_t* relu_bits_out;       // null, or receives the bits of [C > 0] after the forward epilogue
};

// The forward epilogue, in the order of the unfused ops: the row-broadcast add
// (a + b in fp32), then relu (x > 0 ? x : 0).
__device__ inline float bias_relu(float value, float bias, bool relu) {
    value = value + bias;
    return relu ? (value > 0.0f ? value : 0.0f) : value;
}

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

// f(std::integral_constant<int, i>) for i = 0 .. N - 1, in order, with i a
// constant expression inside f.
template <int N, typename F, int I = 0>
__device__ inline void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, F, I + 1>(static_cast<F&&>(f));
    }
}

__device__ inline int64_t uniform64(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(uint64_t(v)));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(uint64_t(v) >> 32));
    return int64_t((uint64_t(hi) << 32) | lo);
}

// Buffer resource over `base` (gfx9 descriptor word 3). Offsets at or above
// kOutOfRange fall outside num_records: loads return 0, stores are dropped.
// The raw buffer builtins move 32-bit integers; values are bit-cast.
constexpr uint32_t kOutOfRange = 0x80000000u;
// s_waitcnt immediate (gfx9 encoding) that waits for every vector memory
// operation (vmcnt 0) and no other counter: loads that write LDS directly
// must land before the barrier that hands their stage to the other waves.
constexpr int kWaitVmcnt0 = 0x0F70;
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), short(0), int(kOutOfRange - 1), 0x00020000);
}

// Global -> register loader for one operand tile (128 along m/n, BK along k),
// in four 16-byte slots per thread. Slot q of a k-contiguous operand is row
// mn0 + 32 q, k k0..k0+3 (8 threads per 32-float row). Slot q of an
// m/n-contiguous operand is k-row k0 + 8 q, columns mn0..mn0+3 (32 threads
// per 128-float row): a load instruction reads two whole 512-byte row
// segments, and the LDS store of a slot writes one LDS row per 32 lanes (no
// bank conflicts). Each thread keeps
// one byte offset (slot 0); slots step by a uniform amount passed as the
// instruction's scalar offset. The tile origin is uniform (scalar registers).
// Edges are masked by pointing a slot out of range.
// KC: operand contiguous along k.
template <bool KC, bool Vec>
struct TileLoader {
    const float* origin;  // element (mn0, 0) of this operand
    int64_t step;         // elements per BK slice
    int K, mn_lim;        // k extent; rows/columns left in the matrix from the tile origin
    uint32_t qstep;       // bytes between slots
    uint32_t ld4;         // bytes per stored row
    uint32_t voff;        // this thread's byte offset of slot 0 within a slice
    int mn0, k0;          // this thread's slot-0 coordinates within the tile

    __device__ void init(const float* base, int ld, int mn_origin, int MN, int K_) {
        K = K_;
        mn_lim = MN - mn_origin;
        origin = KC ? base + int64_t(mn_origin) * ld : base + mn_origin;
        step = KC ? int64_t(BK) : int64_t(BK) * ld;
        ld4 = uint32_t(ld) * 4u;
        const int t = threadIdx.x;
        if (KC) {
            mn0 = t / (BK / 4);
            k0 = (t % (BK / 4)) * 4;
            qstep = uint32_t(kKcRowsPerSlot) * ld4;
        } else {  // 32 threads cover one 128-float row along m/n
            k0 = t / (BM / 4);
            mn0 = (t % (BM / 4)) * 4;
            qstep = 8u * ld4;
        }
        voff = KC ? uint32_t(mn0) * ld4 + uint32_t(k0) * 4u : uint32_t(k0) * ld4 + uint32_t(mn0) * 4u;
    }

    __device__ __amdgpu_buffer_rsrc_t slice(int kt) const { return make_rsrc(origin + int64_t(kt) * step); }

    // Slot q of slice kt. Slices past K read as zeros without touching memory.
    __device__ f4 load(__amdgpu_buffer_rsrc_t rs, int kt, int q) const {
        const int k = kt * BK + k0 + (KC ? 0 : 8 * q);
        const int mn = mn0 + (KC ? kKcRowsPerSlot * q : 0);
        const uint32_t soff = uint32_t(q) * qstep;
        if (Vec) {
            const bool ok = mn < mn_lim && k < K;
            return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? voff : kOutOfRange, soff, 0));
        }
        f4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool ok = KC ? (mn < mn_lim && k + e < K) : (mn + e < mn_lim && k < K);
            v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? voff + 4u * e : kOutOfRange,
                                                                                    soff, 0));
        }
        return v;
    }

    // Byte offset in an LDS stage of this thread's first 16-byte store
    // (m/n mn0, k k0); store q adds q * lds_qstep.
    __device__ uint32_t lds_off() const {
        return KC ? uint32_t(mn0 * (BK + kPadK) + k0) * 4u : uint32_t(k0 * kMnRow + mn0) * 4u;
    }
    static constexpr uint32_t lds_qstep = KC ? uint32_t(kKcRowsPerSlot) * (BK + kPadK) * 4u : 8u * kMnRow * 4u;
};

// Store q (0..3) of this thread's slice registers into an LDS stage (`off`
// from TileLoader::lds_off): every slot goes as loaded, in either layout.
template <bool KC, bool Vec>
__device__ inline void store_slot(char* __restrict__ lds, uint32_t off, const f4 (&v)[kSlots], int q) {
    *reinterpret_cast<f4*>(lds + off + q * TileLoader<KC, Vec>::lds_qstep) = v[q];
}

typedef float f2 __attribute__((ext_vector_type(2)));

// One operand's MFMA fragments of one k-group for the wave's two 32-row
// blocks: at(b, s) is block b's value for MFMA step s. A k-contiguous tile
// gives each block's 4 steps with one ds_read_b128; an m/n-contiguous tile
// gives each step's 2 blocks (interleaved rows) with one ds_read_b64.
template <bool KC>
struct Frag;
template <>
struct Frag<true> {
    f4 v[2];
    __device__ float at(int b, int s) const { return v[b][s]; }
};
template <>
struct Frag<false> {
    f2 v[4];
    __device__ float at(int b, int s) const { return v[s][b]; }
};

// Part s (0..3) of the fragments of k-group g for the wave's 64 rows at `off`.
// A k-contiguous tile issues block b's read at part first + b (A uses parts
// 0-1, B parts 2-3); an m/n-contiguous tile issues step s's read at part s.
template <bool KC>
__device__ inline void read_part(const float* __restrict__ lds, int off, int g, int lane, int s, int first,
                                 Frag<KC>& frag) {
    const int kb = g * 8 + 4 * (lane >> 5);
    if constexpr (KC) {
        const int b = s - first;
        if (b == 0 || b == 1)
            frag.v[b] = *reinterpret_cast<const f4*>(lds + (off + (lane & 31) + 32 * b) * (BK + kPadK) + kb);
    } else {
        frag.v[s] = *reinterpret_cast<const f2*>(lds + (kb + s) * kMnRow + off + 2 * (lane & 31));
    }
}

// Vector-load variants fit two workgroups per CU (<= 256 VGPRs). The scalar-load
// variants (misaligned operands only) keep 32 element loads and their masks
// in flight, so they get the register file of one workgroup per CU rather
// than spilling.
template <bool TA, bool TB, bool Vec>
__global__ __launch_bounds__(kThreads, Vec ? 2 : 1) void gemm_mfma_kernel(GemmArgs p) {
    // Two LDS stages. Step kt multiplies out of stage cur while its second
    // k-group also stores slice kt + 1 (in registers since step kt - 1) into
    // the other stage and issues the global loads of slice kt + 2, each slot
    // right after its store. Storing in the second group rather than the
    // first lets a tile's first step run a group of MFMAs while slice 1, loaded
    // just before it, is still arriving. Fragments are read one k-group ahead;
    // after the third group's MFMAs one barrier makes stage cur ^ 1 complete
    // and stage cur free, and the fourth group's MFMAs overlap the reads of the
    // next step's first group.
    __shared__ __attribute__((aligned(16))) float As[2][kLdsTile];
    __shared__ __attribute__((aligned(16))) float Bs[2][kLdsTile];
    constexpr bool AKC = !TA;  // A contiguous along k
    constexpr bool BKC = TB;   // B contiguous along k
    int tm, tn;
    tile_coords(int(blockIdx.x), p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int kt_total = (p.K + BK - 1) / BK;
    const int64_t jobs = p.batch * p.splits;

    for (int64_t job = blockIdx.y; job < jobs; job += gridDim.y) {
        // Per-job values are workgroup-uniform; saying so keeps the buffer
        // descriptors in scalar registers (a 64-bit division or a table read
        // would otherwise leave them in vector registers and every buffer
        // access would become a per-lane loop).
        const int64_t z = uniform64(job / p.splits);
        const int split = __builtin_amdgcn_readfirstlane(int(job - z * p.splits));
        int kt_begin = 0, kt_end = kt_total;
        int64_t r_begin = 0, r_end = p.reduce;
        if (p.reduce > 1) {
            r_begin = split * p.r_per_split;
            r_end = min(p.reduce, r_begin + p.r_per_split);
        } else {
            kt_begin = split * p.kt_per_split;
            kt_end = min(kt_total, kt_begin + p.kt_per_split);
        }
        const int64_t aoff = uniform64(p.table ? p.table[2 * z] : z * p.a_bstride);
        const int64_t boff = uniform64(p.table ? p.table[2 * z + 1] : z * p.b_bstride);
        f16v acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

        for (int64_t r = r_begin; r < r_end && kt_begin < kt_end; ++r) {
            TileLoader<AKC, Vec> la;
            TileLoader<BKC, Vec> lb;
            la.init(p.a + aoff + r * p.a_rstride, p.lda, m0, p.M, p.K);
            lb.init(p.b + boff + r * p.b_rstride, p.ldb, n0, p.N, p.K);
            f4 ra[kSlots], rb[kSlots];
            char* const lds_a = reinterpret_cast<char*>(As[0]);
            char* const lds_b = reinterpret_cast<char*>(Bs[0]);
            const uint32_t a_st = la.lds_off(), b_st = lb.lds_off();
            {
                const __amdgpu_buffer_rsrc_t sa = la.slice(kt_begin), sb = lb.slice(kt_begin);
#pragma unroll
                for (int q = 0; q < kSlots; ++q) {
                    ra[q] = la.load(sa, kt_begin, q);
                    rb[q] = lb.load(sb, kt_begin, q);
                }
#pragma unroll
                for (int q = 0; q < kSlots; ++q) {
                    store_slot<AKC, Vec>(lds_a, a_st, ra, q);
                    store_slot<BKC, Vec>(lds_b, b_st, rb, q);
                }
                const __amdgpu_buffer_rsrc_t na = la.slice(kt_begin + 1), nb = lb.slice(kt_begin + 1);
#pragma unroll
                for (int q = 0; q < kSlots; ++q) {
                    ra[q] = la.load(na, kt_begin + 1, q);
                    rb[q] = lb.load(nb, kt_begin + 1, q);
                }
            }
            __syncthreads();
            Frag<AKC> fa[2];  // [k-group parity]
            Frag<BKC> fb[2];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                read_part<AKC>(As[0], wm, 0, lane, s, 0, fa[0]);
                read_part<BKC>(Bs[0], wn, 0, lane, s, 2, fb[0]);
            }
            for (int kt = kt_begin; kt < kt_end; ++kt) {
                const int cur = (kt - kt_begin) & 1;
                const float* as = As[cur];
                const float* bs = Bs[cur];
                float* as_next = As[cur ^ 1];
                float* bs_next = Bs[cur ^ 1];
                char* const st_a = lds_a + (cur ^ 1) * kLdsTile * 4;
                char* const st_b = lds_b + (cur ^ 1) * kLdsTile * 4;
                // Past the end of the range the stores and loads below are idle
                // work (slices past K are masked), kept so each step is straight-line.
                const __amdgpu_buffer_rsrc_t sa = la.slice(kt + 2), sb = lb.slice(kt + 2);
#pragma unroll
                for (int g = 0; g < BK / 8; ++g) {
                    const int cb = g & 1;
                    if (g == BK / 8 - 1) __syncthreads();
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        // Store q of the next stage at step q of k-group 1,
                        // then reload slot q right away (a store reads its
                        // own slot only, in either layout).
                        if (g >= 1 && g <= kSlots / 4) {
                            const int q = 4 * (g - 1) + s;
                            store_slot<AKC, Vec>(st_a, a_st, ra, q);
                            store_slot<BKC, Vec>(st_b, b_st, rb, q);
                            ra[q] = la.load(sa, kt + 2, q);
                            rb[q] = lb.load(sb, kt + 2, q);
                        }
                        if (g + 1 < BK / 8) {
                            read_part<AKC>(as, wm, g + 1, lane, s, 0, fa[cb ^ 1]);
                            read_part<BKC>(bs, wn, g + 1, lane, s, 2, fb[cb ^ 1]);
                        } else {
                            read_part<AKC>(as_next, wm, 0, lane, s, 0, fa[cb ^ 1]);
                            read_part<BKC>(bs_next, wn, 0, lane, s, 2, fb[cb ^ 1]);
                        }
#pragma unroll
                        for (int i = 0; i < 2; ++i)
#pragma unroll
                            for (int j = 0; j < 2; ++j)
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[cb].at(i, s), fb[cb].at(j, s),
                                                                                 acc[i][j], 0, 0, 0);
                        // Keep this order: the scheduler would otherwise sink
                        // each LDS read to just before its first use.
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
            // The last step's look-ahead reads touched the other stage.
            __syncthreads();
        }
        // Epilogue: buffer stores relative to the tile origin; rows/columns
        // outside C are pointed out of range and dropped by the hardware. With a
        // split K each split writes its own partial matrix.
        // The fused ReLU mask (g * [x > 0], the backward rule's arithmetic) is
        // applied here unless K was split, in which case split_sum_kernel does.
        float* C = p.c + (p.splits > 1 ? job : z) * int64_t(p.M) * p.N;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(C + int64_t(m0) * p.N + n0);
        const bool masked = p.relu_mask && p.splits == 1;
        const __amdgpu_buffer_rsrc_t rm =
            make_rsrc((masked ? p.relu_mask + z * int64_t(p.M) * p.N : C) + int64_t(m0) * p.N + n0);
        const int row_lim = p.M - m0, col_lim = p.N - n0;
        // Tile coordinates of accumulator value v of block (i, j) on this
        // lane (D row d = 8 (v / 4) + 4 (lane / 32) + v % 4, column lane % 32):
        // a k-contiguous operand's blocks are 32 consecutive rows (columns),
        // an m/n-contiguous one's interleave (block b holds 2 d + b).
        // (The two forms below keep every variant within 256 registers: the
        // register allocation of the masked epilogue, 64 mask loads in flight,
        // follows how these indices are written.)
        const int row0 = wm + 4 * (lane >> 5), col0 = wn + (lane & 31);
        const auto crow = [&](int i, int v) {
            return AKC ? row0 + 32 * i + 8 * (v >> 2) + (v & 3) : wm + 2 * (8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) + i;
        };
        const auto ccol = [&](int j) { return BKC ? col0 + 32 * j : wn + 2 * (lane & 31) + j; };
        if (masked) {  // all 64 mask loads in flight before the first use
            f16v x[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = ccol(j);
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int row = crow(i, v);
                        const bool ok = row < row_lim && col < col_lim;
                        x[i][j][v] = __builtin_bit_cast(
                            float, __builtin_amdgcn_raw_buffer_load_b32(
                                       rm, ok ? uint32_t(row * p.N + col) * 4u : kOutOfRange, 0, 0));
                    }
                }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const float xv = x[i][j][v];
                        const float value = acc[i][j][v];
                        acc[i][j][v] = value * (xv > 0.0f ? 1.0f : 0.0f);
                    }
        }
        if (p.splits == 1 && (p.bias || p.relu)) {  // forward epilogue: + bias[column], then ReLU
            float bias[2] = {0.0f, 0.0f};
            if (p.bias) {
                const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.bias + n0);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = ccol(j);
                    bias[j] = __builtin_bit_cast(
                        float, __builtin_amdgcn_raw_buffer_load_b32(rb, col < col_lim ? uint32_t(col) * 4u : kOutOfRange,
                                                                    0, 0));
                }
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const float value = acc[i][j][v];
                        acc[i][j][v] = bias_relu(value, bias[j], p.relu != 0);
                    }
        }
        if (p.col_part) {
            // Column sums of the tile's final values, in double, one partial
            // row per wave row (64 rows): each lane adds its 32 rows of a
            // column (i, then v), then the two half-waves (rows 4 apart) are
            // joined. Partial row 2 tm + wm / 64. In a last, partial tile the
            // rows past M are left out (their values are not C's: a zero row
            // of A times an infinite B is NaN).
            const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.col_part + (int64_t(2 * tm) + (wm >> 6)) * p.N + n0);
            const bool whole = row_lim >= BM;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                double sum = 0.0;
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const float value = acc[i][j][v];
                        const int row = crow(i, v);
                        sum += whole || row < row_lim ? double(value) : 0.0;
                    }
                sum += __shfl_xor(sum, 32, 64);
                const int col = ccol(j);
                const uint64_t bits = __builtin_bit_cast(uint64_t, sum);
                const uint32_t off = lane < 32 && col < col_lim ? uint32_t(col) * 8u : kOutOfRange;
                __builtin_amdgcn_raw_buffer_store_b32(uint32_t(bits), rp, off, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b32(uint32_t(bits >> 32), rp, off + 4u, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = ccol(j);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int row = crow(i, v);
                    const bool ok = row < row_lim && col < col_lim;
                    const float value = acc[i][j][v];  // element first: bit-casting the subscript takes lane 0
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), rc,
                                                          ok ? uint32_t(row * p.N + col) * 4u : kOutOfRange,
                                                          0, 0);
                }
            }
    }
}

// ---- 256 x 256 tiles: one workgroup per CU, a 128 x 128 quadrant per wave ----
//
// Large products run on 256 x 256 tiles. Each of the four waves owns a
// 128 x 128 quadrant as 2 x 2 blocks of 64 x 64, and computes each of them
// exactly as gemm_mfma_kernel's wave computes its 64 x 64 (the same MFMA
// blocks, the same lane layouts and the same k order), so C, the fused
// epilogues and the column-sum partial rows (one per 64 rows) are the same
// bits as on the 128 x 128 tiles. What changes is the work between barriers:
// a wave issues 256 MFMAs per 32-deep slice instead of 64, and every LDS
// fragment read feeds twice the MFMAs. One workgroup, so one wave per SIMD,
// per CU; the accumulators (256 per lane) live in the accumulation registers.
// With one wave per SIMD nothing hides an instruction that holds up the
// MFMAs, so operand slices go from memory straight into LDS (16-byte buffer
// loads with the LDS destination: no staging registers, no LDS store
// instructions; those stores alone cost 3% of the K loop), and the loop holds
// no vector ALU work. Two stages of two unpadded 32 KiB tiles: 128 KiB of
// LDS. Vector (16-byte) loads only; misaligned operands stay on the 128 x 128
// tiles.
constexpr int BT = 256;                   // tile rows (M); tile columns BN_ = 256 or 128
constexpr int kBigLdsTile = BT * BK;       // floats per operand stage at most (32 KiB)

// LDS pointer for the loads that write LDS directly.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Memory -> LDS loader of an EXT (m/n; 256 or 128) x 32 (k) operand slice:
// EXT / 32 loads per thread, each writing its wave's 1 KiB contiguously
// (lane t at byte 16 t of the load's LDS destination, which is uniform per
// wave; load q of wave w lands at byte 1024 w + 4096 q of the stage).
// - k-contiguous operand ([EXT][32] in LDS): load q of wave w covers rows
//   32 q + 8 w .. + 7, 8 lanes per 32-float row. Lane t writes 16-byte chunk
//   t % 8 of its row r and fetches into it the row's chunk (t % 8) ^ (r / 2 % 8)
//   (k = 4 x chunk): chunk c of row r lies at c ^ (r / 2 % 8), so the
//   fragment reads (16 consecutive rows at one k) hit 16 different bank groups.
// - m/n-contiguous operand ([32][EXT]): load q of wave w covers the 256 / EXT
//   k-rows from (1024 / EXT) q + (256 / EXT) w, lane t column 4 t mod EXT.
// Edges: rows (columns) past the matrix, and k past K, point out of range;
// such lanes write zeros into LDS.
template <bool KC, int EXT>
struct BigLoader {
    static constexpr int kSlots = EXT / 32;        // loads per thread per slice
    static constexpr int kRowsPerLoad = 1024 / EXT;  // k-rows of an m/n-contiguous operand per load round
    const float* origin;
    int64_t step;
    int K, mn_lim, wave;
    uint32_t qstep, voff;  // soffset step per load; this lane's byte offset of load 0 in a slice
    int mn0, k0;           // this lane's row (column) and k of load 0, from the slice origin

    __device__ void init(const float* base, int ld, int mn_origin, int MN, int K_, int wave_, int lane) {
        K = K_;
        mn_lim = MN - mn_origin;
        wave = wave_;
        origin = KC ? base + int64_t(mn_origin) * ld : base + mn_origin;
        step = KC ? int64_t(BK) : int64_t(BK) * ld;
        const uint32_t ld4 = uint32_t(ld) * 4u;
        if (KC) {
            mn0 = 8 * wave + lane / 8;
            k0 = 4 * ((lane % 8) ^ ((mn0 >> 1) & 7));
            qstep = 32u * ld4;
        } else {
            k0 = (256 / EXT) * wave + lane / (EXT / 4);
            mn0 = 4 * (lane % (EXT / 4));
            qstep = uint32_t(kRowsPerLoad) * ld4;
        }
        voff = KC ? uint32_t(mn0) * ld4 + uint32_t(k0) * 4u : uint32_t(k0) * ld4 + uint32_t(mn0) * 4u;
    }

    __device__ __amdgpu_buffer_rsrc_t slice(int kt) const { return make_rsrc(origin + int64_t(kt) * step); }

    // Load q's offset in slice kt, every edge masked.
    __device__ uint32_t masked_off(int kt, int q) const {
        const int k = kt * BK + k0 + (KC ? 0 : kRowsPerLoad * q);
        const int mn = mn0 + (KC ? 32 * q : 0);
        return mn < mn_lim && k < K ? voff : kOutOfRange;
    }
    // Load q's offset in a slice whose k all lie inside K: only rows
    // (columns) past the matrix point out of range.
    __device__ uint32_t full_slice_off(int q) const { return mn0 + (KC ? 32 * q : 0) < mn_lim ? voff : kOutOfRange; }

    // Issue load q of the slice at rs into the LDS stage at `stage`. Written
    // as inline assembly so that the compiler does not see an LDS write: it
    // cannot always tell which LDS array such a load writes, and would then
    // wait for every load in flight before unrelated LDS reads. The loads are
    // waited for explicitly (kWaitVmcnt0) before the barrier that publishes
    // their stage; the compiler's own vmcnt waits only ever wait for more.
    // The LDS destination is this wave's base in the stage plus a constant
    // per load, added in the statement itself, so that one base per stage is
    // kept rather than one address per load.
    template <int Q>
    __device__ void load(__amdgpu_buffer_rsrc_t rs, float* stage, uint32_t off) const {
        constexpr uint32_t dst_q = 4096u * Q;
        const uint32_t base = uint32_t(reinterpret_cast<uintptr_t>((lds_ptr_t)stage)) + 1024u * uint32_t(wave);
        asm volatile("s_add_u32 m0, %0, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                     :
                     : "s"(base), "v"(off), "s"(rs), "s"(uint32_t(Q) * qstep), "i"(dst_q)
                     : "memory", "m0", "scc");
    }
};

// One operand's fragments of one k-group for the wave's 128 rows: at(p, b, s)
// is the value of 64-row half p, block b, for MFMA step s (as Frag, per half).
template <bool KC>
struct BigFrag;
template <>
struct BigFrag<true> {
    f4 v[2][2];  // [half][block]
    __device__ float at(int p, int b, int s) const { return v[p][b][s]; }
};
template <>
struct BigFrag<false> {
    f2 v[2][4];  // [half][step]
    __device__ float at(int p, int b, int s) const { return v[p][s][b]; }
};

// Part s (0..3) of the fragments of k-group g for the wave's NP 64-row halves
// at `off` of a tile EXT wide along m/n: a k-contiguous tile reads block
// (s / 2, s % 2) with one ds_read_b128 (k 8 g + 4 h .. + 3 for half-wave h:
// chunk 2 g + h, found at (2 g + h) ^ (row / 2 % 8), and row / 2 % 8 =
// lane / 2 % 8 here), an m/n-contiguous tile step s of each half with one
// ds_read_b64. Each half holds what read_part gives a wave's 64 rows.
template <bool KC, int EXT, int NP>
__device__ inline void big_read_part(const float* __restrict__ lds, int off, int g, int lane, int s,
                                     BigFrag<KC>& frag) {
    if constexpr (KC) {
        const int p = s >> 1, b = s & 1;
        const int chunk = (2 * g + (lane >> 5)) ^ ((lane >> 1) & 7);
        if (p < NP)
            frag.v[p][b] = *reinterpret_cast<const f4*>(lds + (off + 64 * p + 32 * b + (lane & 31)) * BK + 4 * chunk);
    } else {
        const int kb = g * 8 + 4 * (lane >> 5);
#pragma unroll
        for (int p = 0; p < NP; ++p)
            frag.v[p][s] = *reinterpret_cast<const f2*>(lds + (kb + s) * EXT + off + 64 * p + 2 * (lane & 31));
    }
}

// The lane index, computed where it is used (mbcnt) and passed through an
// empty asm statement, so that neither it nor the per-element offsets derived
// from it are kept across the K loop, where they would take registers the
// loop needs.
__device__ inline int epilogue_lane() {
    int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(lane));
    return lane;
}

// Tile coordinates of accumulator value v of block (i, j) of the 64 x 64
// block at tile rows wm.., columns wn.. (D row d = 8 (v / 4) + 4 (lane / 32)
// + v % 4, column lane % 32; a k-contiguous operand's blocks are 32
// consecutive rows (columns), an m/n-contiguous one's interleave).
template <bool AKC, bool BKC>
struct BlockCoords {
    int wm, wn, lane;
    __device__ int row(int i, int v) const {
        return AKC ? wm + 4 * (lane >> 5) + 32 * i + 8 * (v >> 2) + (v & 3)
                   : wm + 2 * (8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) + i;
    }
    __device__ int col(int j) const { return BKC ? wn + (lane & 31) + 32 * j : wn + 2 * (lane & 31) + j; }
};

// Issues the loads of the ReLU mask under the 64 x 64 block at tile rows
// wm.., columns wn.. (one per accumulator value; outside C they read 0).
template <bool AKC, bool BKC>
__device__ inline void big_mask_load(const GemmArgs& p, int64_t z, int m0, int n0, int wm, int wn,
                                     f16v (&x)[2][2]) {
    const BlockCoords<AKC, BKC> bc{wm, wn, epilogue_lane()};
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(p.relu_mask + z * int64_t(p.M) * p.N + int64_t(m0) * p.N + n0);
    const int row_lim = p.M - m0, col_lim = p.N - n0;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = bc.col(j);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = bc.row(i, v);
                const bool ok = row < row_lim && col < col_lim;
                x[i][j][v] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rm, ok ? uint32_t(row * p.N + col) * 4u : kOutOfRange, 0, 0));
            }
        }
}

// The epilogue of one 64 x 64 block of C at tile rows wm.., columns wn..:
// gemm_mfma_kernel's epilogue for one wave (ReLU mask, bias + ReLU, the
// block's column-sum partial row `part_row`, the store), in the same order.
// The mask values come loaded (big_mask_load) when the product has one.
template <bool AKC, bool BKC>
__device__ inline void big_epilogue(const GemmArgs& p, f16v (&acc)[2][2], const f16v (&mask)[2][2], int64_t z,
                                    int64_t job, int m0, int n0, int wm, int wn, int part_row) {
    const BlockCoords<AKC, BKC> bc{wm, wn, epilogue_lane()};
    const int lane = bc.lane;
    float* C = p.c + (p.splits > 1 ? job : z) * int64_t(p.M) * p.N;
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(C + int64_t(m0) * p.N + n0);
    const bool masked = p.relu_mask && p.splits == 1;
    const int row_lim = p.M - m0, col_lim = p.N - n0;
    if (masked) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float xv = mask[i][j][v];
                    const float value = acc[i][j][v];
                    acc[i][j][v] = value * (xv > 0.0f ? 1.0f : 0.0f);
                }
    }
    // A lane's 16 values of a 32-row group of one column (rows as bc.row
    // with A k-contiguous) are bits 4 (lane / 32) + 8 (v / 4) + v % 4 of that
    // column's word for the group; rows wm + 32 i .. of the tile are group
    // (m0 + wm) / 32 + i.
    const int bit_base = 4 * (lane >> 5);
    if (AKC && p.relu_bits && p.splits == 1) {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.relu_bits + int64_t((m0 + wm) / 32) * p.N + n0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = bc.col(j);
                const bool ok = wm + 32 * i < row_lim && col < col_lim;
                const uint32_t word =
                    __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? uint32_t(i * p.N + col) * 4u : kOutOfRange, 0, 0) >>
                    bit_base;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float keep = float((word >> (8 * (v >> 2) + (v & 3))) & 1u);
                    const float value = acc[i][j][v];
                    acc[i][j][v] = value * keep;
                }
            }
    }
    if (p.splits == 1 && (p.bias || p.relu)) {
        float bias[2] = {0.0f, 0.0f};
        if (p.bias) {
            const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.bias + n0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = bc.col(j);
                bias[j] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rb, col < col_lim ? uint32_t(col) * 4u : kOutOfRange, 0, 0));
            }
        }
        if (AKC && p.relu_bits_out && p.relu) {
            // bias_relu with the ReLU bitmask of its results: the compare that
            // picks a value also sets its bit. Each half-wave holds half of a
            // column's 32 rows: the two halves' bits are joined, and lanes
            // 0-31 write the words of their columns.
            const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.relu_bits_out + int64_t((m0 + wm) / 32) * p.N + n0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    uint32_t bits = 0;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const float value = acc[i][j][v] + bias[j];
                        const bool positive = value > 0.0f;
                        acc[i][j][v] = positive ? value : 0.0f;
                        bits |= positive ? 1u << (8 * (v >> 2) + (v & 3)) : 0u;
                    }
                    bits <<= bit_base;
                    bits |= uint32_t(__shfl_xor(int(bits), 32, 64));
                    const int col = bc.col(j);
                    const bool ok = lane < 32 && wm + 32 * i < row_lim && col < col_lim;
                    __builtin_amdgcn_raw_buffer_store_b32(bits, rw, ok ? uint32_t(i * p.N + col) * 4u : kOutOfRange, 0,
                                                          0);
                }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const float value = acc[i][j][v];
                        acc[i][j][v] = bias_relu(value, bias[j], p.relu != 0);
                    }
        }
    }
    // Partial rows past the 2 ceil(M / 128) that the 128 x 128 tiles write
    // (and the caller allocates) lie wholly below C and are not written.
    if (p.col_part && part_row < 2 * ((p.M + BM - 1) / BM)) {
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.col_part + int64_t(part_row) * p.N + n0);
        const bool whole = row_lim >= wm + 64;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            double sum = 0.0;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float value = acc[i][j][v];
                    const int row = bc.row(i, v);
                    sum += whole || row < row_lim ? double(value) : 0.0;
                }
            sum += __shfl_xor(sum, 32, 64);
            const int col = bc.col(j);
            const uint64_t bits = __builtin_bit_cast(uint64_t, sum);
            const uint32_t off = lane < 32 && col < col_lim ? uint32_t(col) * 8u : kOutOfRange;
            __builtin_amdgcn_raw_buffer_store_b32(uint32_t(bits), rp, off, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b32(uint32_t(bits >> 32), rp, off + 4u, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = bc.col(j);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = bc.row(i, v);
                const bool ok = row < row_lim && col < col_lim;
                const float value = acc[i][j][v];
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), rc,
                                                      ok ? uint32_t(row * p.N + col) * 4u : kOutOfRange, 0, 0);
            }
        }
}

template <bool TA, bool TB, int BN_>
__global__ __launch_bounds__(kThreads, 1) void gemm_big_kernel(GemmArgs p) {
    // Step kt multiplies out of stage cur while k-groups 0 and 1 issue the
    // loads of slice kt + 1 into the other stage (free since the previous
    // step's barrier), four per operand each; fragments are read one k-group
    // ahead; before the fourth k-group the loads are waited for and one
    // barrier makes the other stage complete, and the fourth k-group's MFMAs
    // overlap the reads of its first fragments.
    __shared__ __attribute__((aligned(16))) float A0[kBigLdsTile];
    __shared__ __attribute__((aligned(16))) float A1[kBigLdsTile];
    __shared__ __attribute__((aligned(16))) float B0[BN_ * BK];
    __shared__ __attribute__((aligned(16))) float B1[BN_ * BK];
    constexpr bool AKC = !TA;
    constexpr bool BKC = TB;
    constexpr int QN = BN_ / 128;  // 64-column halves per wave
    using LoaderA = BigLoader<AKC, BT>;
    using LoaderB = BigLoader<BKC, BN_>;
    int tm, tn;
    tile_coords(int(blockIdx.x), p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BT, n0 = tn * BN_;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * (BN_ / 2);
    const int kt_total = (p.K + BK - 1) / BK;
    // One job (output matrix, or split of one) per workgroup row of the grid:
    // loops around the K loop here would make the register allocator spill.
    // A batch reduction is split one product per split (the host sees to
    // it), which the 128 x 128 tiles do too when they split one: split s
    // multiplies product s over the whole K.
    {
        const int64_t job = blockIdx.y;
        const int64_t z = uniform64(job / p.splits);
        const int split = __builtin_amdgcn_readfirstlane(int(job - z * p.splits));
        const bool per_product = p.reduce > 1;
        const int kt_begin = per_product ? 0 : split * p.kt_per_split;
        const int kt_end = per_product ? kt_total : min(kt_total, kt_begin + p.kt_per_split);
        const int64_t aoff = uniform64((p.table ? p.table[2 * z] : z * p.a_bstride) +
                                       (per_product ? split * p.a_rstride : 0));
        const int64_t boff = uniform64((p.table ? p.table[2 * z + 1] : z * p.b_bstride) +
                                       (per_product ? split * p.b_rstride : 0));
        const bool masked = p.relu_mask && p.splits == 1;
        f16v mk[2][2][2];       // fused ReLU mask of a block of C: [block parity][i][j]
        f16v acc[2][QN][2][2];  // [A half][B half][block i][block j]
#pragma unroll
        for (int ph = 0; ph < 2; ++ph)
#pragma unroll
            for (int qh = 0; qh < QN; ++qh)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int v = 0; v < 16; ++v) acc[ph][qh][i][j][v] = 0.0f;

        if (kt_begin < kt_end) {
            LoaderA la;
            LoaderB lb;
            la.init(p.a + aoff, p.lda, m0, p.M, p.K, wave, lane);
            lb.init(p.b + boff, p.ldb, n0, p.N, p.K, wave, lane);
            {
                const __amdgpu_buffer_rsrc_t sa = la.slice(kt_begin), sb = lb.slice(kt_begin);
                static_for<LoaderA::kSlots>([&](auto qc) {
                    constexpr int q = decltype(qc)::value;
                    la.template load<q>(sa, A0, la.masked_off(kt_begin, q));
                    if constexpr (q < LoaderB::kSlots) lb.template load<q>(sb, B0, lb.masked_off(kt_begin, q));
                });
            }
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            __syncthreads();
            BigFrag<AKC> fa[2];  // [k-group parity]
            BigFrag<BKC> fb[2];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                big_read_part<AKC, BT, 2>(A0, wm, 0, lane, s, fa[0]);
                big_read_part<BKC, BN_, QN>(B0, wn, 0, lane, s, fb[0]);
            }
            // Per-load offsets of full slices (every k inside K): only the
            // rows past the matrix are masked, once per tile. Steps whose
            // loads are full slices use them, so their loop holds no vector
            // ALU work; the last steps mask every load.
            uint32_t a_off[LoaderA::kSlots], b_off[LoaderB::kSlots];
#pragma unroll
            for (int q = 0; q < LoaderA::kSlots; ++q) a_off[q] = la.full_slice_off(q);
#pragma unroll
            for (int q = 0; q < LoaderB::kSlots; ++q) b_off[q] = lb.full_slice_off(q);
            // One step. kFast: its loads (slice kt + 1) are a full slice of the
            // range. kCur: the stage multiplied out of, 0 or 1 (known here, so
            // every LDS address is a fixed offset from a per-lane base), or -1
            // (from kt).
            const auto step = [&](auto fast_c, auto cur_c, int kt) {
                constexpr bool kFast = decltype(fast_c)::value;
                constexpr int kCur = decltype(cur_c)::value;
                const int cur = kCur >= 0 ? kCur : (kt - kt_begin) & 1;
                const float* as = cur ? A1 : A0;
                const float* bs = cur ? B1 : B0;
                float* const as_next = cur ? A0 : A1;
                float* const bs_next = cur ? B0 : B1;
                const bool more = kFast || kt + 1 < kt_end;
                const __amdgpu_buffer_rsrc_t sa = la.slice(kt + 1), sb = lb.slice(kt + 1);
                static_for<BK / 8>([&](auto gc) {
                    constexpr int g = decltype(gc)::value;
                    const int cb = g & 1;
                    if (g == BK / 8 - 1) {
                        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
                        __syncthreads();
                    }
                    static_for<4>([&](auto sc) {
                        constexpr int s = decltype(sc)::value;
                        if constexpr (g <= 1) {
                            constexpr int q = 4 * g + s;
                            if (more) {
                                la.template load<q>(sa, as_next, kFast ? a_off[q] : la.masked_off(kt + 1, q));
                                if constexpr (q < LoaderB::kSlots)
                                    lb.template load<q>(sb, bs_next, kFast ? b_off[q] : lb.masked_off(kt + 1, q));
                            }
                        }
                        if (g + 1 < BK / 8) {
                            big_read_part<AKC, BT, 2>(as, wm, g + 1, lane, s, fa[cb ^ 1]);
                            big_read_part<BKC, BN_, QN>(bs, wn, g + 1, lane, s, fb[cb ^ 1]);
                        } else {
                            big_read_part<AKC, BT, 2>(as_next, wm, 0, lane, s, fa[cb ^ 1]);
                            big_read_part<BKC, BN_, QN>(bs_next, wn, 0, lane, s, fb[cb ^ 1]);
                        }
#pragma unroll
                        for (int ph = 0; ph < 2; ++ph)
#pragma unroll
                            for (int qh = 0; qh < QN; ++qh)
#pragma unroll
                                for (int i = 0; i < 2; ++i)
#pragma unroll
                                    for (int j = 0; j < 2; ++j)
                                        acc[ph][qh][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                            fa[cb].at(ph, i, s), fb[cb].at(qh, j, s), acc[ph][qh][i][j], 0, 0, 0);
                        __builtin_amdgcn_sched_barrier(0);
                    });
                });
            };
            // Pairs of steps whose loads are full slices of the range, then the
            // rest one at a time. A pair starts on stage 0.
            const int fast_end = min(kt_end, p.K / BK);
            int kt = kt_begin;
            for (; kt + 2 < fast_end; kt += 2) {
                step(std::true_type{}, std::integral_constant<int, 0>{}, kt);
                step(std::true_type{}, std::integral_constant<int, 1>{}, kt + 1);
            }
            for (; kt < kt_end; ++kt) step(std::false_type{}, std::integral_constant<int, -1>{}, kt);
            __syncthreads();
        }
        // Each 64 x 64 block as gemm_mfma_kernel's wave finishes it; its
        // column-sum partial row is the block's 64-row index in C. A fused
        // ReLU mask is loaded one block ahead (two register sets), so only the
        // first block waits for its whole load latency.
        if (masked) big_mask_load<AKC, BKC>(p, z, m0, n0, wm, wn, mk[0]);
#pragma unroll
        for (int ph = 0; ph < 2; ++ph)
#pragma unroll
            for (int qh = 0; qh < QN; ++qh) {
                const int blk = QN * ph + qh;
                if (masked && blk + 1 < 2 * QN)
                    big_mask_load<AKC, BKC>(p, z, m0, n0, wm + 64 * ((blk + 1) / QN), wn + 64 * ((blk + 1) % QN),
                                            mk[(blk + 1) & 1]);
                // One block at a time: its 64 values are copied out of the
                // accumulation registers here (the empty asm pins the copy), so
                // the epilogue's branches join vector registers, not the
                // accumulators of the blocks still waiting.
                f16v c[2][2];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        c[i][j] = acc[ph][qh][i][j];
                        asm volatile("" : "+v"(c[i][j]));
                    }
                big_epilogue<AKC, BKC>(p, c, mk[blk & 1], z, job, m0, n0, wm + 64 * ph, wn + 64 * qh,
                                       (m0 + wm + 64 * ph) / 64);
            }
    }
}

// Split combine: c[z][i] = sum over s of part[z][s][i], in split order, then
// the fused ReLU mask or the forward epilogue when there is one.
__global__ __launch_bounds__(256) void split_sum_kernel(const float* __restrict__ part, float* __restrict__ c,
                                                        int64_t batch, int64_t mn, int64_t n, int splits,
                                                        const float* __restrict__ relu_mask,
                                                        const float* __restrict__ bias, int relu) {
    const int64_t total = batch * mn;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
        const int64_t z = t / mn, i = t % mn;
        const float* src = part + z * splits * mn + i;
        float acc = src[0];
        for (int s = 1; s < splits; ++s) acc += src[int64_t(s) * mn];
        if (relu_mask) acc = acc * (relu_mask[t] > 0.0f ? 1.0f : 0.0f);
        if (bias || relu) acc = bias_relu(acc, bias ? bias[i % n] : 0.0f, relu != 0);
        c[t] = acc;
    }
}

// The float mask [bit] of a ReLU bitmask (bit r % 32 of word (r / 32) n + c
// for element (r, c)), for a product that does not take gemm_big_kernel.
__global__ __launch_bounds__(256) void relu_bits_expand_kernel(const uint32_t* __restrict__ bits,
                                                               float* __restrict__ mask, int64_t m, int64_t n) {
    const int64_t total = m * n;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < total; t += stride) {
        const int64_t r = t / n, col = t % n;
        mask[t] = float((bits[(r / 32) * n + col] >> (r % 32)) & 1u);
    }
}

// out [cols][rows] = in [rows][cols] transposed, both row-major with rows and
// cols multiples of 4: 64 x 64 tiles through LDS, 16-byte loads and stores.
// The padded row (65 floats) keeps both LDS passes free of bank conflicts.
__global__ __launch_bounds__(256) void transpose64_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                          int64_t rows, int64_t cols) {
    __shared__ float tile[64][65];
    const int64_t r0 = int64_t(blockIdx.y) * 64, c0 = int64_t(blockIdx.x) * 64;
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = (t >> 4) + 16 * i, c = (t & 15) * 4;
        if (r0 + r < rows && c0 + c < cols) {
            const f4 v = *reinterpret_cast<const f4*>(in + (r0 + r) * cols + c0 + c);
            tile[r][c] = v.x;
            tile[r][c + 1] = v.y;
            tile[r][c + 2] = v.z;
            tile[r][c + 3] = v.w;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = (t >> 4) + 16 * i, r = (t & 15) * 4;
        if (c0 + c < cols && r0 + r < rows) {
            const f4 v{tile[r][c], tile[r + 1][c], tile[r + 2][c], tile[r + 3][c]};
            *reinterpret_cast<f4*>(out + (c0 + c) * rows + r0 + r) = v;
        }
    }
}

// Portable FMA kernel (VECTORCORE_HIP_GEMM=simple or
// vc_hip_set_gemm_kernel("simple"), and small products): 16 x 16 outputs per
// 256-thread workgroup, one per thread, each the sum over k in order. K goes
// through LDS in slices of KS (16, 64 or 256, the smallest that holds K, up
// to 256): each thread issues its share of a slice's loads together (one
// memory round trip per slice), and the next slice's loads are in flight
// while the current slice is summed.
//
// Thread t's share of a slice, element i (0 .. KS / 16 - 1), ordered so that
// consecutive threads read consecutive addresses of the operand as stored
// (R = 256 / KS):
//   A, 16 rows x KS: stored [M][K]: row t / KS + R i, k t % KS; stored [K][M]: row t % 16, k t / 16 + 16 i;
//   B, KS x 16 columns: stored [K][N]: k t / 16 + 16 i, column t % 16; stored [N][K]: k t % KS, column t / KS + R i.
// Only elements inside the operand are read; the rest of the slice is 0.
template <int KS>
struct SimpleSlice {
    static constexpr int kLoads = KS / 16;  // elements of each operand per thread
    static constexpr int kStep = 256 / KS;  // rows (columns) between a thread's elements, [M][K] A and [N][K] B
    static constexpr int kAStride = KS + 4; // A slice row stride: 16-byte rows for float4 reads
};

template <bool TA, bool TB, int KS>
__device__ inline void simple_load(const GemmArgs& p, const float* A, const float* B, int64_t row0, int64_t col0,
                                   int64_t k0, float (&ra)[KS / 16], float (&rb)[KS / 16]) {
    using S = SimpleSlice<KS>;
    const int t = threadIdx.x, lo = t % 16, hi = t / 16;
    if (TA) {
        const bool row_ok = row0 + lo < p.M;
        const int64_t base = (k0 + hi) * p.lda + row0 + lo, step = int64_t(16) * p.lda;
#pragma unroll
        for (int i = 0; i < S::kLoads; ++i)
            ra[i] = (row_ok && k0 + hi + 16 * i < p.K) ? A[base + i * step] : 0.0f;
    } else {
        const int64_t k = k0 + t % KS, r = row0 + t / KS;
        const int64_t base = r * p.lda + k, step = int64_t(S::kStep) * p.lda;
#pragma unroll
        for (int i = 0; i < S::kLoads; ++i)
            ra[i] = (k < p.K && r + S::kStep * i < p.M) ? A[base + i * step] : 0.0f;
    }
    if (TB) {
        const int64_t k = k0 + t % KS, c = col0 + t / KS;
        const int64_t base = c * p.ldb + k, step = int64_t(S::kStep) * p.ldb;
#pragma unroll
        for (int i = 0; i < S::kLoads; ++i)
            rb[i] = (k < p.K && c + S::kStep * i < p.N) ? B[base + i * step] : 0.0f;
    } else {
        const bool col_ok = col0 + lo < p.N;
        const int64_t base = (k0 + hi) * p.ldb + col0 + lo, step = int64_t(16) * p.ldb;
#pragma unroll
        for (int i = 0; i < S::kLoads; ++i)
            rb[i] = (col_ok && k0 + hi + 16 * i < p.K) ? B[base + i * step] : 0.0f;
    }
}

template <bool TA, bool TB, int KS>
__device__ inline void simple_store(float (*as)[SimpleSlice<KS>::kAStride], float (*bs)[17], const float (&ra)[KS / 16],
                                    const float (&rb)[KS / 16]) {
    using S = SimpleSlice<KS>;
    const int t = threadIdx.x, lo = t % 16, hi = t / 16;
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
        if (TA) as[lo][hi + 16 * i] = ra[i];
        else as[t / KS + S::kStep * i][t % KS] = ra[i];
        if (TB) bs[t % KS][t / KS + S::kStep * i] = rb[i];
        else bs[hi + 16 * i][lo] = rb[i];
    }
}

template <bool TA, bool TB, int KS>
__global__ __launch_bounds__(256) void gemm_simple_kernel(GemmArgs p) {
    using S = SimpleSlice<KS>;
    __shared__ __align__(16) float as[16][S::kAStride];
    __shared__ float bs[KS][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t row0 = int64_t(blockIdx.x / p.tiles_n) * 16, col0 = int64_t(blockIdx.x % p.tiles_n) * 16;
    const int64_t row = row0 + ty, col = col0 + tx;
    for (int64_t z = blockIdx.y; z < p.batch; z += gridDim.y) {
        const int64_t aoff = p.table ? p.table[2 * z] : z * p.a_bstride;
        const int64_t boff = p.table ? p.table[2 * z + 1] : z * p.b_bstride;
        float acc = 0.0f;
        for (int64_t r = 0; r < p.reduce; ++r) {
            const float* A = p.a + aoff + r * p.a_rstride;
            const float* B = p.b + boff + r * p.b_rstride;
            float ra[S::kLoads], rb[S::kLoads];
            simple_load<TA, TB, KS>(p, A, B, row0, col0, 0, ra, rb);
            for (int64_t k0 = 0; k0 < p.K; k0 += KS) {
                simple_store<TA, TB, KS>(as, bs, ra, rb);
                __syncthreads();
                if (k0 + KS < p.K) simple_load<TA, TB, KS>(p, A, B, row0, col0, k0 + KS, ra, rb);
                // Sixteen k per step, every LDS read issued before the first
                // product, so the reads' latency is paid once per step.
                const int kc = int(std::min<int64_t>(KS, p.K - k0));
                int kk = 0;
                for (; kk + 16 <= kc; kk += 16) {
                    f4 a4[4];
                    float b1[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) a4[q] = *reinterpret_cast<const f4*>(&as[ty][kk + 4 * q]);
#pragma unroll
                    for (int j = 0; j < 16; ++j) b1[j] = bs[kk + j][tx];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        acc += a4[q].x * b1[4 * q];
                        acc += a4[q].y * b1[4 * q + 1];
                        acc += a4[q].z * b1[4 * q + 2];
                        acc += a4[q].w * b1[4 * q + 3];
                    }
                }
                for (; kk < kc; ++kk) acc += as[ty][kk] * bs[kk][tx];
                __syncthreads();
            }
        }
        const bool inside = row < p.M && col < p.N;
        if (inside) {
            const int64_t t = z * p.M * p.N + row * p.N + col;
            if (p.relu_mask) acc = acc * (p.relu_mask[t] > 0.0f ? 1.0f : 0.0f);
            if (p.bias || p.relu) acc = bias_relu(acc, p.bias ? p.bias[col] : 0.0f, p.relu != 0);
            p.c[t] = acc;
        }
        if (p.col_part) {  // batch 1: the tile's 16 rows of each column, in row order, in double
            __shared__ double tile_rows[16][16];
            tile_rows[ty][tx] = inside ? double(acc) : 0.0;
            __syncthreads();
            if (ty == 0 && col < p.N) {
                double sum = 0.0;
#pragma unroll
                for (int r = 0; r < 16; ++r) sum += tile_rows[r][tx];
                p.col_part[(row0 / 16) * p.N + col] = sum;
            }
            __syncthreads();
        }
    }
}

// Small products (a few 128 x 128 tiles, K too long for the FMA kernel): a
// workgroup of W = kSmallWaves waves computes one 32 x 32 tile of C as one
// V_MFMA_F32_32X32X2_F32 block per wave, wave w taking the 32-deep K chunks
// w, w + W, ..., and the W partial tiles are added in wave order through
// LDS, so one launch finishes the product in a fixed order. Operands go from
// memory straight into the MFMA operand layout, no LDS staging: in chunk c,
// half-wave h of MFMA step j takes k = 32 c + 16 h + j (a fixed permutation of
// the summation index, identical for A and B), lane l row (A) or column (B)
// l % 32. A k-contiguous operand is read as four 16-byte loads per lane and
// chunk (vec), an m/n-contiguous one as 16 loads of 32 consecutive floats per
// half-wave. The next chunk's loads are issued before this chunk's MFMAs.
// col_part: one partial row per 32-row tile.
constexpr int kSmallTile = 32;
// Element `elem` of a buffer (4 floats from it: small_ld4), or 0 when !ok.
__device__ inline float small_ld1(__amdgpu_buffer_rsrc_t rs, uint32_t elem, bool ok) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? elem * 4u : kOutOfRange, 0, 0));
}
__device__ inline f4 small_ld4(__amdgpu_buffer_rsrc_t rs, uint32_t elem, bool ok) {
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? elem * 4u : kOutOfRange, 0, 0));
}

template <bool TA, bool TB, bool Vec>
struct SmallChunk {
    float a[16], b[16];
    // The 16 k from k0 of A (row `row` of op(A)) and B (column `col` of
    // op(B)); elements outside op(A) / op(B) read as 0.
    __device__ void load(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, const GemmArgs& p, int row, int col,
                         int k0) {
        const bool row_ok = row < p.M, col_ok = col < p.N;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = k0 + 4 * q;
            if constexpr (!TA && Vec) {  // A [M][K]: 16 consecutive k of one row
                const f4 v = small_ld4(ra, uint32_t(row * p.lda + k), row_ok && k < p.K);
                a[4 * q] = v.x, a[4 * q + 1] = v.y, a[4 * q + 2] = v.z, a[4 * q + 3] = v.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    a[4 * q + e] = small_ld1(ra, TA ? uint32_t((k + e) * p.lda + row) : uint32_t(row * p.lda + k + e),
                                             row_ok && k + e < p.K);
            }
            if constexpr (TB && Vec) {  // B [N][K]: 16 consecutive k of one column
                const f4 v = small_ld4(rb, uint32_t(col * p.ldb + k), col_ok && k < p.K);
                b[4 * q] = v.x, b[4 * q + 1] = v.y, b[4 * q + 2] = v.z, b[4 * q + 3] = v.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    b[4 * q + e] = small_ld1(rb, TB ? uint32_t(col * p.ldb + k + e) : uint32_t((k + e) * p.ldb + col),
                                             col_ok && k + e < p.K);
            }
        }
    }
};

// Eight waves measured 5-18% faster than four on the products this kernel
// takes (1024^3: 38.1 against 42.5 us; 512 x 8192 x 512: 62.5 against 75.8);
// sixteen spill registers.
constexpr int kSmallWaves = 8;  // waves (K shares) per 32 x 32 tile
constexpr int kSmallThreads = 64 * kSmallWaves;

template <bool TA, bool TB, bool Vec>
__global__ __launch_bounds__(kSmallThreads) void gemm_small_kernel(GemmArgs p) {
    __shared__ float part[kSmallWaves][16][64];         // [wave][accumulator v][lane]
    __shared__ float tile[kSmallTile][kSmallTile + 1];  // final values, for the column sums
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tm = int(blockIdx.x) / p.tiles_n, tn = int(blockIdx.x) % p.tiles_n;
    const int m0 = tm * kSmallTile, n0 = tn * kSmallTile;
    const int half = lane >> 5;
    const int chunks = (p.K + 31) / 32;
    for (int64_t z = blockIdx.y; z < p.batch; z += gridDim.y) {
        const int64_t aoff = uniform64(p.table ? p.table[2 * z] : z * p.a_bstride);
        const int64_t boff = uniform64(p.table ? p.table[2 * z + 1] : z * p.b_bstride);
        f16v acc;
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
        for (int64_t r = 0; r < p.reduce; ++r) {
            const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a + aoff + r * p.a_rstride);
            const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.b + boff + r * p.b_rstride);
            const int row = m0 + (lane & 31), col = n0 + (lane & 31);
            SmallChunk<TA, TB, Vec> cur, next;
            if (wave < chunks) cur.load(ra, rb, p, row, col, 32 * wave + 16 * half);
            for (int c = wave; c < chunks; c += kSmallWaves) {
                const bool more = c + kSmallWaves < chunks;
                if (more) next.load(ra, rb, p, row, col, 32 * (c + kSmallWaves) + 16 * half);
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.a[j], cur.b[j], acc, 0, 0, 0);
                if (more) cur = next;
            }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) part[wave][v][lane] = acc[v];
        __syncthreads();
        // Thread t finishes accumulator slots (v, l) = t / 64 + W i, t % 64
        // (W waves): the waves' partials in wave order, then the epilogue.
        float* C = p.c + z * int64_t(p.M) * p.N;
#pragma unroll
        for (int i = 0; i < 16 / kSmallWaves; ++i) {
            const int v = int(threadIdx.x) / 64 + kSmallWaves * i, l = int(threadIdx.x) % 64;
            float value = part[0][v][l];
#pragma unroll
            for (int w = 1; w < kSmallWaves; ++w) value += part[w][v][l];
            const int tr = 8 * (v / 4) + 4 * (l / 32) + v % 4, tc = l % 32;  // the MFMA's D layout
            const int row = m0 + tr, col = n0 + tc;
            const bool inside = row < p.M && col < p.N;
            const int64_t t = int64_t(row) * p.N + col;
            if (inside) {
                if (p.relu_mask) value = value * (p.relu_mask[z * int64_t(p.M) * p.N + t] > 0.0f ? 1.0f : 0.0f);
                if (p.bias || p.relu) value = bias_relu(value, p.bias ? p.bias[col] : 0.0f, p.relu != 0);
                C[t] = value;
            }
            tile[tr][tc] = inside ? value : 0.0f;
        }
        if (p.col_part) {  // batch 1: the tile's 32 rows of each column, in row order, in double
            __syncthreads();
            if (threadIdx.x < kSmallTile && n0 + int(threadIdx.x) < p.N) {
                double sum = 0.0;
                for (int rr = 0; rr < kSmallTile; ++rr) sum += double(tile[rr][threadIdx.x]);
                p.col_part[int64_t(tm) * p.N + n0 + threadIdx.x] = sum;
            }
        }
        __syncthreads();
    }
}

template <bool TA, bool TB>
void launch_variant(const GemmArgs& args, bool vec, bool simple, bool small, int big_n, dim3 grid,
                    hipStream_t stream) {
    if (big_n == 256) {
        launch((gemm_big_kernel<TA, TB, 256>), grid, dim3(kThreads), 0, stream, args);
    } else if (big_n == 128) {
        launch((gemm_big_kernel<TA, TB, 128>), grid, dim3(kThreads), 0, stream, args);
    } else if (small) {
        if (vec) launch((gemm_small_kernel<TA, TB, true>), grid, dim3(kSmallThreads), 0, stream, args);
        else launch((gemm_small_kernel<TA, TB, false>), grid, dim3(kSmallThreads), 0, stream, args);
    } else if (simple) {
        if (args.K <= 16) launch((gemm_simple_kernel<TA, TB, 16>), grid, dim3(256), 0, stream, args);
        else if (args.K <= 64) launch((gemm_simple_kernel<TA, TB, 64>), grid, dim3(256), 0, stream, args);
        else launch((gemm_simple_kernel<TA, TB, 256>), grid, dim3(256), 0, stream, args);
    } else if (vec) {
        launch((gemm_mfma_kernel<TA, TB, true>), grid, dim3(kThreads), 0, stream, args);
    } else {
        launch((gemm_mfma_kernel<TA, TB, false>), grid, dim3(kThreads), 0, stream, args);
    }
}

const char* variant_label(bool ta, bool tb) {
    return ta ? (tb ? "gemm_tt" : "gemm_tn") : (tb ? "gemm_nt" : "gemm_nn");
}

// Whether a product takes gemm_small_kernel rather than the 128 x 128 tiles
// (tiles128 of them, times `products` matrices) or the FMA kernel (tiny).
// Measured on MI355X with four waves per 32 x 32 tile (eight are faster
// still): the 32 x 32 tiles run at up to ~60 TFLOP/s, while 9 to 64 tiles of
// 128 x 128 leave most CUs idle (1024^3: 37.8 against 68.2 us;
// 512 x 8192 x 512: 86 against 145 us). Up to 8 tiles and K above 2048, the
// larger tiles split K 32 ways and win (256 x 4096 x 256: 27 against 42 us);
// from 128 tiles they are as fast or faster (2048 x 1024^2: 69 against 72 us;
// 2048^2 x 1024: 80 against 133 us). Among tiny products, weight gradients
// (A transposed, K the batch, at least 128) gain from the waves' K split
// (256 x 300 x 64: 6.1 against 12.1 us); the others stay on the FMA kernel.
bool small_tiles(int64_t K, int64_t products, int64_t tiles128, bool tiny, bool ta, bool tb) {
    if (tiny) return ta && !tb && K >= 128;
    const int64_t work = tiles128 * products;
    if (work <= 64 && K <= 2048) return true;
    return work > 8 && work <= 32;
}

// The tile width of gemm_big_kernel (256 or 128 columns of 256 rows) for a
// product under the automatic setting, or 0 for the other kernels, from
// measurements on MI355X against the 128 x 128 tiles:
// - a full round of 256 x 256 tiles (one workgroup per CU) and at least 32 K
//   slices: 256 (8192 x 4096 x 4096 NT 1914 -> 1807 us, 4096^2 x 8192 TN
//   1958 -> 1807, 8192 x 4096 x 1024 NN 495 -> 477);
// - else a full round of 256 x 128 tiles: 128 (8192 x 1000 x 4096 NN 485 ->
//   458; 8 x 1024^3 NT 128 -> 124, TN 134 -> 127);
// - where the 128 x 128 tiles would split K (fewer than two workgroups per
//   CU): 256 x 128 tiles split in two (4096 x 1000 x 8192 TN 504 -> 469,
//   1024 x 4096 x 8192 TN 504 -> 469; 256 x 256 tiles split in four took
//   482 and 485), or 256 x 256 tiles split in four.
// A fused float ReLU mask adds its loads to the epilogue, which with one
// workgroup per CU nothing overlaps and every CU reaches at once: masked
// products need 64 slices (8192 x 4096 x 4096 masked NT 1915 -> 1846 us;
// 8192 x 4096 x 1000 508 -> 518, so it stays). A mask given as ReLU bits (one
// load per 32 values) takes the unmasked rule (8192 x 4096 x 1000: 512 us on
// the 128 x 128 tiles with the float mask, 487 on the 256 x 256 with the bits).
int big_tiles(int64_t M, int64_t N, int64_t K, int64_t batch, int64_t reduce, int cu_count, bool masked) {
    const int64_t tiles = ((M + BT - 1) / BT) * ((N + BT - 1) / BT) * batch;
    const int64_t tiles_half = ((M + BT - 1) / BT) * ((N + 127) / 128) * batch;
    const int64_t tiles128 = ((M + BM - 1) / BM) * ((N + BN - 1) / BN) * batch;
    const int64_t slices = (K + BK - 1) / BK;
    if (reduce > 1)  // one product per split, at least half a round of 256 x 128 tiles
        return tiles_half * reduce <= cu_count && 2 * tiles_half * reduce >= cu_count && slices >= 32 ? 128 : 0;
    if (masked && slices < 64) return 0;
    if (tiles >= cu_count && slices >= 32) return 256;
    if (tiles_half >= cu_count && slices >= 32) return 128;
    if (tiles128 < 2 * int64_t(cu_count) && 2 * tiles_half >= cu_count && slices >= 64) return 128;
    if (tiles128 < 2 * int64_t(cu_count) && 4 * tiles >= cu_count && slices >= 128) return 256;
    return 0;
}

// offsets: nullptr for the affine mode (a_bstride / b_bstride).
void gemm(const float* a, const float* b, float* c, int64_t M, int64_t N, int64_t K, int64_t batch, int64_t a_bstride,
          int64_t b_bstride, const std::vector<int64_t>* offsets, int64_t reduce, int64_t a_rstride, int64_t b_rstride,
          bool ta, bool tb, const float* relu_mask = nullptr, const float* bias = nullptr, bool relu = false,
          bool in_caller_scope = false, float* column_sum = nullptr, vc_hip_colsum** pending = nullptr,
          const uint32_t* relu_bits = nullptr, uint32_t* relu_bits_out = nullptr, bool* bits_written = nullptr) {
    Device& d = require_device();
    if (M < 0 || N < 0 || K < 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "negative matrix dimension");
    if (pending) *pending = nullptr;
    if (bits_written) *bits_written = false;
    if (relu_mask && relu_bits) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul: a ReLU mask and ReLU bits at once");
    if (column_sum && (batch != 1 || reduce != 1))
        fail(VC_HIP_ERR_INVALID_ARGUMENT, "a fused column sum needs a single product");
    if (pending && !column_sum) fail(VC_HIP_ERR_INVALID_ARGUMENT, "pending column sums need a column-sum buffer");
    if (M == 0 || N == 0 || batch == 0) return;
    if (!a || !b || !c) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul: null buffer");
    const int mode = d.gemm_mode.load();  // the kernel setting in force for this call
    const bool force_simple = mode == kGemmSimple;
    // A single large NN product runs as NT on a transposed copy of B: the
    // 128 x 128 tiles are ~3.5% faster when both operands are contiguous along
    // k, which outweighs the copy (2 K N floats of traffic) once M >= 4096. The
    // LDS tiles, and so the bits, are those of the NN kernel. (K is bounded by
    // the transpose's grid: 65535 tiles of 64 rows.) On the 256 x 256 tiles NN
    // is as fast as NT, and from K = 2048 on the copy no longer pays
    // (8192 x 4096 x 4096: 1886 us with the copy, 1872 without; at K = 1024
    // the copy still wins, 490 against 495).
    const bool big_nn = (mode == kGemmTiles256 || mode == kGemmTiles256x128 ||
                         (mode == kGemmAuto && K >= 2048 && big_tiles(M, N, K, batch, reduce, d.cu_count, false))) &&
                        std::max(K, N) * BT < (int64_t(1) << 29);
    if (!ta && !tb && batch == 1 && reduce == 1 && !force_simple && M >= kNnViaNtMinRows && N % 4 == 0 &&
        K % 4 == 0 && K <= int64_t(65535) * 64 && aligned16(a) && aligned16(b) && !relu_mask && !relu_bits &&
        !big_nn) {
        Profiled prof("gemm_nn", 2.0 * double(M) * double(N) * double(K),
                      4.0 * double(M * K + 2 * K * N + M * N) + (bias ? 4.0 * double(N) : 0.0));
        Scratch bt(size_t(K * N) * sizeof(float));
        launch(transpose64_kernel, dim3(unsigned((N + 63) / 64), unsigned((K + 63) / 64)), dim3(256), 0, d.stream, b,
               bt.as<float>(), K, N);
        after_launch("gemm_nn");
        // Inside this scope: the transpose and the product are timed together.
        gemm(a, bt.as<float>(), c, M, N, K, 1, 0, 0, nullptr, 1, 0, 0, false, true, nullptr, bias, relu, true,
             column_sum, pending, nullptr, relu_bits_out, bits_written);
        prof.done();
        return;
    }
    const int64_t tiles_m_simple = (M + 15) / 16, tiles_n_simple = (N + 15) / 16;
    const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    // Small products (<= 2^20 multiply-adds, K <= 1024) run on the FMA kernel:
    // a 128 x 128 MFMA tile there is mostly padding, and its fixed latency
    // (~8 us, plus a second pass when K is split) is several times the FMA
    // kernel's whole run (one memory round trip per 256 k).
    const bool tiny = double(M) * double(N) * double(K) * double(batch) * double(reduce) <= kTinyMacs &&
                      K <= kSimpleMaxK;
    const int64_t tiles_m32 = (M + kSmallTile - 1) / kSmallTile, tiles_n32 = (N + kSmallTile - 1) / kSmallTile;
    // A product of a few 128 x 128 tiles takes 32 x 32 tiles with K split over
    // the workgroup's eight waves (gemm_small_kernel): one launch, no split pass.
    // Its operand offsets are 32-bit from the operand's origin.
    const bool small_fits = M * K < (int64_t(1) << 29) && K * N < (int64_t(1) << 29) && M * N < (int64_t(1) << 29);
    const bool automatic = mode == kGemmAuto;
    bool small = automatic && small_fits && small_tiles(K, batch * reduce, tiles_m * tiles_n, tiny, ta, tb);
    bool simple = force_simple || (automatic && !small && tiny);
    // Byte offsets relative to a tile origin are 32-bit: 128 rows of any
    // operand or of C must span less than 2 GiB (256 rows for the 256 x 256 tiles).
    const int64_t kMax = int64_t(1) << 29;
    const int64_t widest = std::max({ta ? M : K, tb ? K : N, N});
    if (M >= kMax || N >= kMax || K >= kMax || widest * 128 >= kMax)
        fail(VC_HIP_ERR_OVERFLOW, "matmul operands exceed the 2 GiB per-matrix addressing of the HIP kernels");
    // 16-byte vector loads need every row start and batch offset on a 4-float boundary.
    bool vec = aligned16(a) && aligned16(b) && (ta ? M : K) % 4 == 0 && (tb ? K : N) % 4 == 0 && a_rstride % 4 == 0 &&
               b_rstride % 4 == 0;
    if (offsets) {
        for (int64_t v : *offsets) vec = vec && v % 4 == 0;
    } else {
        vec = vec && a_bstride % 4 == 0 && b_bstride % 4 == 0;
    }
    // A batch reduction takes the 256-row tiles only when it splits one
    // product per split (r_per_split 1 below): output tiles times products
    // within one workgroup per CU.
    const auto reduce_fits = [&](int64_t width) {
        return reduce == 1 || ((M + BT - 1) / BT) * ((N + width - 1) / width) * batch * reduce <= d.cu_count;
    };
    const bool big_fits = vec && widest * BT < kMax && batch <= 65535 / 32;
    const int big_n = !big_fits                                        ? 0
                      : mode == kGemmTiles256                          ? (reduce_fits(256) ? 256 : 0)
                      : mode == kGemmTiles256x128                      ? (reduce_fits(128) ? 128 : 0)
                      : automatic && !small && !simple && reduce_fits(128)
                          ? big_tiles(M, N, K, batch, reduce, d.cu_count, relu_mask != nullptr)
                          : 0;
    const bool big = big_n != 0;
    if (big) small = simple = false;
    const int64_t tiles_m256 = (M + BT - 1) / BT, tiles_n256 = big ? (N + big_n - 1) / big_n : 0;
    const int64_t tiles = big     ? tiles_m256 * tiles_n256
                          : small ? tiles_m32 * tiles_n32
                          : simple ? tiles_m_simple * tiles_n_simple
                                   : tiles_m * tiles_n;
    if (tiles > std::numeric_limits<int>::max() / 2) fail(VC_HIP_ERR_OVERFLOW, "matmul output has too many tiles");

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
    args.tiles_m = int(big ? tiles_m256 : small ? tiles_m32 : simple ? tiles_m_simple : tiles_m);
    args.tiles_n = int(big ? tiles_n256 : small ? tiles_n32 : simple ? tiles_n_simple : tiles_n);

    Scratch table(offsets ? offsets->size() * sizeof(int64_t) : 8);
    if (offsets) {
        const int rc = vc_hip_upload(table.as<void>(), offsets->data(), offsets->size() * sizeof(int64_t));
        if (rc != VC_HIP_OK) fail(rc, "matmul offset table upload failed");
        args.table = table.as<int64_t>();
    }
    // Split the work when the output has fewer tiles than workgroup slots
    // (two per CU on the 128 x 128 tiles, one on the 256 x 256): a batch reduction (reduce > 1) splits into ranges of r, a long K into
    // ranges of at least 32 slices (16 for 65 to 128 tiles; at most 4 ranges), and the K of a tiny output
    // (<= kTinyTiles tiles) into up to 32 ranges. Each split accumulates into
    // its own partial matrix and a second pass sums the partials in split
    // order (deterministic). No split range is empty.
    const int kt_total = int((K + BK - 1) / BK);
    int splits = 1;
    int64_t r_per_split = reduce;
    const int64_t slots = (big ? 1 : 2) * int64_t(d.cu_count);
    const int64_t want = (slots + tiles * batch - 1) / (tiles * batch);
    if (!simple && !small && tiles * batch < slots) {
        if (reduce > 1) {
            r_per_split = (reduce + std::min(want, reduce) - 1) / std::min(want, reduce);
            splits = int((reduce + r_per_split - 1) / r_per_split);
        } else if (tiles * batch <= kTinyTiles && kt_total >= 4) {
            // A handful of output tiles: one workgroup's K loop is a chain of
            // ~1.7 us steps, so split K as far as 32 ways (one slice or more each).
            splits = std::min(kt_total, 32);
        } else if (kt_total >= 64) {
            splits = int(std::min<int64_t>(want, 4));
            splits = std::min(splits, kt_total / 32);
        } else if (4 * tiles * batch <= slots && kt_total >= 32) {
            // 65 to 128 tiles (fewer take the 32 x 32 tiles) with K of 1024
            // to 2047 fill at most a quarter of the workgroup slots: ranges of
            // at least 16 slices fill them (2048 x 1024 x 1024: 72 -> 50 us;
            // splitting 256 tiles this way measured slower, 81 -> 90 us).
            splits = int(std::min<int64_t>(want, 4));
            splits = std::min(splits, kt_total / 16);
        }
    }
    if (reduce == 1 && splits > 1)  // drop the ranges that ceil(kt_total / splits) slices each would leave empty
        splits = (kt_total + (kt_total + splits - 1) / splits - 1) / ((kt_total + splits - 1) / splits);
    if (batch * splits > std::numeric_limits<int>::max()) fail(VC_HIP_ERR_OVERFLOW, "matmul batch too large");
    args.splits = splits;
    args.kt_per_split = (kt_total + splits - 1) / splits;
    args.r_per_split = r_per_split;
    Scratch partials(splits > 1 ? size_t(batch * splits) * size_t(M * N) * sizeof(float) : 4);
    if (splits > 1) args.c = partials.as<float>();
    const dim3 grid(unsigned(tiles), unsigned(std::min<int64_t>(batch * splits, 65535)));
    const char* label = variant_label(ta, tb);
    const double flops = 2.0 * double(M) * double(N) * double(K) * double(batch) * double(reduce);
    // ReLU bitmasks go with gemm_big_kernel's epilogue for one product with A
    // k-contiguous and no split. Elsewhere a consumer's bits are expanded into
    // a float mask first (below), and a producer writes none.
    const bool bits_here = big && !ta && batch == 1 && reduce == 1 && splits == 1;
    Scratch expanded(relu_bits && !bits_here ? size_t(M * N) * sizeof(float) : 4);
    const uint32_t* expand_from = nullptr;
    if (relu_bits && !bits_here) {
        expand_from = relu_bits;
        relu_bits = nullptr;
        relu_mask = expanded.as<float>();
    }
    args.relu_mask = relu_mask;
    args.relu_bits = relu_bits;
    args.relu_bits_out = bits_here && relu && relu_bits_out ? relu_bits_out : nullptr;
    if (bits_written) *bits_written = args.relu_bits_out != nullptr;
    args.bias = bias;
    args.relu = relu ? 1 : 0;
    // The column sums of C (a bias gradient) come from partial rows that the
    // epilogue keeps when one launch writes C (the MFMA kernel one per 64 rows
    // of a tile, the FMA kernel one per 16-row tile): column_partials_kernel
    // adds them next, or they are handed to the caller as pending sums. A
    // split product's C is summed again afterwards instead.
    ColsumPtr sums;
    if (column_sum && splits == 1) sums = new_colsum(small ? tiles_m32 : simple ? tiles_m_simple : 2 * tiles_m, N);
    if (sums) args.col_part = sums->part;
    const double bytes =
        4.0 * (double(M * K + K * N) * double(reduce) + double(M * N) * (relu_mask ? 2.0 : 1.0)) * double(batch) +
        (bias ? 4.0 * double(N) : 0.0) + (relu_bits || args.relu_bits_out ? double(M * N) / 8.0 : 0.0);
    std::optional<Profiled> prof;
    if (!in_caller_scope) prof.emplace(label, flops, bytes);
    if (expand_from) {
        launch(relu_bits_expand_kernel, dim3(unsigned(std::min<int64_t>((M * N + 255) / 256, int64_t(d.cu_count) * 16))),
               dim3(256), 0, d.stream, expand_from, expanded.as<float>(), M, N);
        after_launch("relu_bits_expand");
    }
    if (ta && tb) launch_variant<true, true>(args, vec, simple, small, big_n, grid, d.stream);
    else if (ta) launch_variant<true, false>(args, vec, simple, small, big_n, grid, d.stream);
    else if (tb) launch_variant<false, true>(args, vec, simple, small, big_n, grid, d.stream);
    else launch_variant<false, false>(args, vec, simple, small, big_n, grid, d.stream);
    if (splits > 1) {
        after_launch(label);
        const int64_t total = batch * M * N;
        launch(split_sum_kernel, dim3(unsigned(std::min<int64_t>((total + 255) / 256, int64_t(d.cu_count) * 16))),
                           dim3(256), 0, d.stream, partials.as<float>(), c, batch, M * N, N, splits, relu_mask, bias,
                           args.relu);
    }
    after_launch(label);
    if (prof) prof->done();
    if (sums) {
        if (pending) *pending = sums.release();
        else finish_colsum(*sums, column_sum);
    } else if (column_sum) {
        const int rc = vc_hip_reduce_axis(c, column_sum, 1, size_t(M), size_t(N), VC_REDUCE_SUM);
        if (rc != VC_HIP_OK) fail(rc, std::string("column sum of a product: ") + vc_hip_last_error());
    }
}

// Per-batch offsets as the reference passes them: affine ones (the common
// batched and broadcast cases) go as strides, anything else as a table.
void matmul_offsets(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, const size_t* a_offsets,
                    const size_t* b_offsets, size_t batch, int trans_a, int trans_b, const float* relu_mask) {
    if (batch == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul needs one A and B offset per batch");
    if (!a_offsets || !b_offsets) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul: null offsets");
    const int64_t sa = batch > 1 ? int64_t(a_offsets[1]) - int64_t(a_offsets[0]) : 0;
    const int64_t sb = batch > 1 ? int64_t(b_offsets[1]) - int64_t(b_offsets[0]) : 0;
    bool affine = a_offsets[0] == 0 && b_offsets[0] == 0;
    for (size_t z = 0; affine && z < batch; ++z)
        affine = int64_t(a_offsets[z]) == int64_t(z) * sa && int64_t(b_offsets[z]) == int64_t(z) * sb;
    if (affine) {
        gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), int64_t(batch), sa, sb, nullptr, 1, 0, 0, trans_a != 0,
             trans_b != 0, relu_mask);
    } else {
        std::vector<int64_t> table(2 * batch);
        for (size_t z = 0; z < batch; ++z) {
            table[2 * z] = int64_t(a_offsets[z]);
            table[2 * z + 1] = int64_t(b_offsets[z]);
        }
        gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), int64_t(batch), 0, 0, &table, 1, 0, 0, trans_a != 0,
             trans_b != 0, relu_mask);
    }
}

}  // namespace
}  // namespace vchip

using namespace vchip;

extern "C" {

int vc_hip_matmul(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, const size_t* a_offsets,
                  const size_t* b_offsets, size_t batch, int trans_a, int trans_b) {
    return guard([&] { matmul_offsets(a, b, c, m, k, n, a_offsets, b_offsets, batch, trans_a, trans_b, nullptr); });
}

int vc_hip_matmul_relu_mask(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                            const size_t* a_offsets, const size_t* b_offsets, size_t batch, int trans_a, int trans_b,
                            const float* mask) {
    return guard([&] {
        if (!mask) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_relu_mask: null mask");
        matmul_offsets(a, b, c, m, k, n, a_offsets, b_offsets, batch, trans_a, trans_b, mask);
    });
}

}  // extern "C"

namespace {
void relu_mask_colsum(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, int trans_a,
                      int trans_b, const float* mask, float* column_sum, vc_hip_colsum** pending,
                      const uint32_t* bits = nullptr) {
    if (pending) *pending = nullptr;
    if ((!mask && !bits) || !column_sum)
        fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_relu_mask_colsum: null mask or column sum");
    if (n == 0) return;
    if (m == 0) {  // an empty column sum is zero
        const int rc = vc_hip_fill(column_sum, n, 0.0f);
        if (rc != VC_HIP_OK) fail(rc, vc_hip_last_error());
        return;
    }
    if (k == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_relu_mask_colsum needs k > 0");
    gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), 1, 0, 0, nullptr, 1, 0, 0, trans_a != 0, trans_b != 0, mask,
         nullptr, false, false, column_sum, pending, bits);
}
}  // namespace

extern "C" {

int vc_hip_matmul_relu_mask_colsum(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                   int trans_a, int trans_b, const float* mask, float* column_sum) {
    return guard([&] { relu_mask_colsum(a, b, c, m, k, n, trans_a, trans_b, mask, column_sum, nullptr); });
}

int vc_hip_matmul_relu_mask_colsum_pending(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                           int trans_a, int trans_b, const float* mask, float* column_sum,
                                           vc_hip_colsum** pending) {
    return guard([&] {
        if (!pending) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_relu_mask_colsum_pending: null handle pointer");
        relu_mask_colsum(a, b, c, m, k, n, trans_a, trans_b, mask, column_sum, pending);
    });
}

int vc_hip_matmul_bias_relu(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                            const float* bias, int relu) {
    return guard([&] {
        if (m == 0 || n == 0) return;
        if (k == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_bias_relu needs k > 0");
        gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), 1, 0, 0, nullptr, 1, 0, 0, false, false, nullptr, bias,
             relu != 0);
    });
}

int vc_hip_matmul_bias_relu_bits(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                 const float* bias, uint32_t* relu_bits, int* bits_written) {
    return guard([&] {
        if (!relu_bits || !bits_written) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_bias_relu_bits: null bits or flag");
        *bits_written = 0;
        if (m == 0 || n == 0) return;
        if (k == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_bias_relu_bits needs k > 0");
        bool written = false;
        gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), 1, 0, 0, nullptr, 1, 0, 0, false, false, nullptr, bias, true,
             false, nullptr, nullptr, nullptr, relu_bits, &written);
        *bits_written = written ? 1 : 0;
    });
}

int vc_hip_matmul_relu_bits(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, int trans_a,
                            int trans_b, const uint32_t* relu_bits) {
    return guard([&] {
        if (!relu_bits) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_relu_bits: null bits");
        gemm(a, b, c, int64_t(m), int64_t(n), int64_t(k), 1, 0, 0, nullptr, 1, 0, 0, trans_a != 0, trans_b != 0,
             nullptr, nullptr, false, false, nullptr, nullptr, relu_bits);
    });
}

int vc_hip_matmul_relu_bits_colsum_pending(const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                                           int trans_a, int trans_b, const uint32_t* relu_bits, float* column_sum,
                                           vc_hip_colsum** pending) {
    return guard([&] {
        if (!pending) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_relu_bits_colsum_pending: null handle pointer");
        if (!relu_bits) fail(VC_HIP_ERR_INVALID_ARGUMENT, "matmul_relu_bits_colsum_pending: null bits");
        relu_mask_colsum(a, b, c, m, k, n, trans_a, trans_b, nullptr, column_sum, pending, relu_bits);
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
