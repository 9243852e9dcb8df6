// Fused softmax cross-entropy loss node (the hip path of src/nn.cpp:31-53).
//
// The reference composes the loss from ~10 tensor ops over [rows, classes]:
//   m = max(x, 1) (detached), shifted = x - m, s = sum(exp(shifted), 1)
//   (double accumulation), logsm = shifted - log(s),
//   loss = -(sum(logsm * onehot)) / rows                    (src/ops.cpp:378-384)
// and its backward walks the same graph in reverse. With c = g / rows that
// backward evaluates, per element,
//   dx_ij = ((c / s_i) * exp(x_ij - m_i)) + (j == t_i ? -c : -0.0)
// (div -> negate -> sum -> mul -> sub/log/sum/exp rules of src/ops.cpp). These
// kernels compute those fp32 operations in that order, reading the logits
// once per pass: one wavefront per row, lanes striding the classes, row
// statistics combined with cross-lane exchanges. The one operation that is
// not the reference's is exp (row_exp below: the hardware exp2, where the
// reference calls the C library's expf), within ~1e-6 relative of it on the
// terms that carry a row's sum.
//
// The reference's masked sum also turns any non-finite non-target log-prob
// into NaN (inf * 0); the forward reproduces that.
#include "reduce_common.hpp"
#include "vc_hip_internal.hpp"

#include <algorithm>
#include <limits>

namespace vchip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr unsigned kBlock = 256;
constexpr int kRowsPerBlock = kBlock / kWave;
constexpr int64_t kXentBlocksPerCu = 8;  // workgroups per CU of the register-held forward

__device__ inline f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }

using red::Best;
using red::kNone;

// exp of a shifted logit s = x - m (s <= 0 unless the row holds NaN or
// +inf): the hardware exp2 (V_EXP_F32, 1 ulp) of s * log2(e). Rounding the
// product adds up to |s| 2^-24 relative error: at most ~1e-6 on the terms that
// carry a row's sum (s > -16), ~5e-6 just above the underflow at s = -87.3,
// below which the result is 0. Every kernel here takes its exponentials from
// this one function, so a row's statistics and gradient have the same bits
// whichever path (register-held or streaming) it takes.
__device__ inline float row_exp(float s) { return __expf(s); }

// The row's maximum as the reference's max() takes it, and (in .i) its
// argmax: the first strict maximum of an ascending scan, element 0 when that
// is NaN or when no element is above -inf.
__device__ inline Best row_max(const float* row, int64_t len, int lane, bool vec) {
    Best b = red::no_best();
    if (vec) {
        for (int64_t a = int64_t(lane) * 4; a < len; a += kWave * 4) {
            const f4 v = ld4(row + a);
            red::consider_ordered(b, v.x, int(a));
            red::consider_ordered(b, v.y, int(a + 1));
            red::consider_ordered(b, v.z, int(a + 2));
            red::consider_ordered(b, v.w, int(a + 3));
        }
    } else {
        for (int64_t a = lane; a < len; a += kWave) red::consider_ordered(b, row[a], int(a));
    }
    b = red::wave_best(b);
    const float first = row[0];
    if (first != first) return Best{first, 0};  // max() keeps a NaN first element (src/cpu/cpu_backend.cpp:443-452)
    return Best{b.v, b.i == kNone ? 0 : b.i};
}

// Lane 0: the row's statistics (max, exp-sum) and its loss term
// shifted_t - log(s) (x_t the target's logit), NaN when a non-target log-prob
// is not finite or the target is outside the row (never with checked
// targets). Returns the term.
__device__ inline float write_row(int64_t r, int64_t len, int t, float x_t, float m, double acc, int bad,
                                  float* __restrict__ stats) {
    const float s = float(acc);
    const float L = logf(s);
    float term;
    if (t < 0 || int64_t(t) >= len) {
        term = __builtin_nanf("");
    } else {
        const float shifted = x_t - m;
        term = bad ? __builtin_nanf("") : shifted - L;
    }
    stats[2 * r] = m;
    stats[2 * r + 1] = s;
    return term;
}

// Largest value over the wavefront (inputs never NaN). Lanes can disagree
// only on the sign of a zero maximum, which the caller decides exactly.
__device__ inline float wave_max(float v) {
    const int lane = red::lane_id();
    float o = red::partner<0>(v, lane);
    v = o > v ? o : v;
    o = red::partner<1>(v, lane);
    v = o > v ? o : v;
    o = red::partner<2>(v, lane);
    v = o > v ? o : v;
    o = red::partner<3>(v, lane);
    v = o > v ? o : v;
    o = red::partner<4>(v, lane);
    v = o > v ? o : v;
    o = red::partner<5>(v, lane);
    return o > v ? o : v;
}

// Largest unsigned value over the wavefront.
__device__ inline uint32_t wave_umax(uint32_t v) {
    const int lane = red::lane_id();
    v = max(v, red::partner<0>(v, lane));
    v = max(v, red::partner<1>(v, lane));
    v = max(v, red::partner<2>(v, lane));
    v = max(v, red::partner<3>(v, lane));
    v = max(v, red::partner<4>(v, lane));
    return max(v, red::partner<5>(v, lane));
}

__device__ inline uint32_t bits_of(float v) { return __builtin_bit_cast(uint32_t, v); }

// Smallest value over the wavefront (Steps 6) or each half-wave (Steps 5).
template <int Steps>
__device__ inline int lanes_min(int v) {
    const int lane = red::lane_id();
    v = min(v, red::partner<0>(v, lane));
    v = min(v, red::partner<1>(v, lane));
    v = min(v, red::partner<2>(v, lane));
    v = min(v, red::partner<3>(v, lane));
    v = min(v, red::partner<4>(v, lane));
    if constexpr (Steps == 6) v = min(v, red::partner<5>(v, lane));
    return v;
}

// The reference's argmax of a row (src/cpu/cpu_backend.cpp:443-457), from the
// row's maximum m as the statistics take it: the first strict maximum of an
// ascending scan is the first element equal to the largest non-NaN value (a
// tie, ±0 included, never replaces the running best), and a NaN element 0 is
// never replaced (m is then that NaN and no element equals it). So: the
// smallest index holding a value == m, else 0. v holds NV float4 per lane,
// element a = base + Stride u + component (padding past the row holds -inf,
// which equals m only when a real element does, at a smaller index). Returns
// this lane's smallest such index, kNone if none; the caller takes the
// minimum over the row's lanes.
template <int NV, int Stride>
__device__ inline int first_equal(const f4 (&v)[NV], float m, int base) {
    int idx = kNone;
#pragma unroll
    for (int u = NV - 1; u >= 0; --u) {  // descending, so the smallest index is written last
        const int a = base + Stride * u;
        idx = v[u].w == m ? a + 3 : idx;
        idx = v[u].z == m ? a + 2 : idx;
        idx = v[u].y == m ? a + 1 : idx;
        idx = v[u].x == m ? a : idx;
    }
    return idx;
}

__device__ inline float argmax_value(int idx) { return float(idx == kNone ? 0 : idx); }

// Row statistics and loss term of one row from values in registers (NV
// float4 per lane; element a = 4 lane + 256 u + component, a row of at most
// 256 NV classes; elements past the row hold -inf). Each lane visits its
// elements in ascending order, as the streaming path does, so both give the
// same bits. Returns the loss term on lane 0.
template <bool Vec, int NV>
__device__ inline float finish_row(const f4 (&v)[NV], int64_t r, int64_t len, int t, int lane,
                                   float* __restrict__ stats, float* __restrict__ amax) {
    // The reference's max is the first strict maximum, skipping NaN after
    // element 0. Its value is the largest non-NaN element, whichever index
    // holds it (fmaxf ignores NaN too), except for the sign of a zero maximum
    // (the first zero wins) and a NaN element 0, both settled below. The
    // largest bit pattern of the row (padding left out) tells whether any
    // element is -inf, whose shifted value is the one non-finite case the
    // exp-sum does not show: as unsigned integers, -inf (0xff800000) and the
    // negative NaNs are above every other float. (An integer maximum needs no
    // NaN handling, which a float minimum costs an instruction per element.)
    float mx = -__builtin_inff();
    uint32_t hi = 0;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        mx = __builtin_fmaxf(__builtin_fmaxf(mx, v[u].x), __builtin_fmaxf(__builtin_fmaxf(v[u].y, v[u].z), v[u].w));
        // Padding past the row is left out: whole float4s of it (Vec: the row
        // is a multiple of 4), or single elements.
        const int a = lane * 4 + u * kWave * 4, n = int(len);
        if constexpr (Vec) {
            const uint32_t b = max(max(bits_of(v[u].x), bits_of(v[u].y)), max(bits_of(v[u].z), bits_of(v[u].w)));
            hi = a < n ? max(hi, b) : hi;
        } else {
            const uint32_t b = max(max(a < n ? bits_of(v[u].x) : 0u, a + 1 < n ? bits_of(v[u].y) : 0u),
                                   max(a + 2 < n ? bits_of(v[u].z) : 0u, a + 3 < n ? bits_of(v[u].w) : 0u));
            hi = max(hi, b);
        }
    }
    mx = wave_max(mx);
    const float first = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v[0].x)));
    float m;
    if (first != first) {
        m = first;  // max() keeps a NaN first element (src/cpu/cpu_backend.cpp:443-452)
    } else if (mx == 0.0f) {  // rare: which zero comes first
        Best b = red::no_best();
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int a = lane * 4 + u * kWave * 4;
            if (a < len) {
                red::consider_ordered(b, v[u].x, a);
                red::consider_ordered(b, v[u].y, a + 1);
                red::consider_ordered(b, v[u].z, a + 2);
                red::consider_ordered(b, v[u].w, a + 3);
            }
        }
        m = red::wave_best(b).v;
    } else {
        m = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, mx)));
    }
    if (amax) {
        const int idx = lanes_min<6>(first_equal<NV, kWave * 4>(v, m, lane * 4));
        if (lane == 0) amax[r] = argmax_value(idx);
    }
    // Elements past the row give exp(-inf - m) = 0 (or NaN when m is -inf or
    // NaN, and then every real element's term is NaN too): adding them leaves
    // the sum unchanged.
    // Four chains per lane, one per float4 component: each adds up to four
    // terms (float4s u = 4q .. 4q + 3) in fp32, then that partial in double;
    // the chains are joined in component order, the lanes in double. A
    // partial of at most four positive terms is within 3 * 2^-24 of its exact
    // sum, so the row's sum keeps that relative accuracy before its final
    // rounding to float (a double add per term measured slower: the forward
    // is bound by instruction issue).
    double c0 = 0.0, c1 = 0.0, c2 = 0.0, c3 = 0.0;
#pragma unroll
    for (int q = 0; q < NV; q += 4) {
        float f0 = 0.0f, f1 = 0.0f, f2 = 0.0f, f3 = 0.0f;
#pragma unroll
        for (int u = q; u < q + 4 && u < NV; ++u) {
            f0 += row_exp(v[u].x - m);
            f1 += row_exp(v[u].y - m);
            f2 += row_exp(v[u].z - m);
            f3 += row_exp(v[u].w - m);
        }
        c0 += double(f0);
        c1 += double(f1);
        c2 += double(f2);
        c3 += double(f3);
    }
    const double acc = red::wave_sum(((c0 + c1) + c2) + c3);
    // Some shifted value is not finite exactly when m is not finite, an
    // element is -inf, or the sum is NaN (a NaN or +inf element makes its own
    // term, or every term, NaN).
    const bool nonfinite = !isfinite(m) || wave_umax(hi) >= 0xff800000u || acc != acc;
    int bad = 0;  // a non-target log-prob that is not finite
    if (nonfinite) {  // rare: decide exactly, leaving the target out
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int a = lane * 4 + u * kWave * 4;
            if (a < len) {
                const float s0 = v[u].x - m, s1 = v[u].y - m, s2 = v[u].z - m, s3 = v[u].w - m;
                if constexpr (Vec) {  // whole float4s of the row
                    bad |= (a != t && !isfinite(s0)) | (a + 1 != t && !isfinite(s1)) | (a + 2 != t && !isfinite(s2)) |
                           (a + 3 != t && !isfinite(s3));
                } else {
                    const int n = int(len);
                    bad |= (a != t && !isfinite(s0)) | (a + 1 < n && a + 1 != t && !isfinite(s1)) |
                           (a + 2 < n && a + 2 != t && !isfinite(s2)) | (a + 3 < n && a + 3 != t && !isfinite(s3));
                }
            }
        }
    }
    bad = red::wave_or(bad);
    // The target's logit from the registers of the lane holding it (t is
    // wave-uniform): element t is component t % 4 of v[t / 256] on lane
    // (t / 4) % 64.
    float x_t = 0.0f;
    if (t >= 0 && int64_t(t) < len) {
        const int tu = t >> 8, tc = t & 3, owner = (t >> 2) & 63;
        float mine = 0.0f;
#pragma unroll
        for (int u = 0; u < NV; ++u)
            if (u == tu) mine = tc == 0 ? v[u].x : tc == 1 ? v[u].y : tc == 2 ? v[u].z : v[u].w;
        x_t = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), owner));
    }
    return lane == 0 ? write_row(r, len, t, x_t, m, acc, bad, stats) : 0.0f;
}

// Loads a row into registers, -inf past its end. Vec: 16-byte loads (len a
// multiple of 4, row 16-byte aligned); otherwise four scalar loads per float4,
// the same values in the same places.
template <bool Vec, int NV>
__device__ inline void load_row(f4 (&v)[NV], const float* __restrict__ row, int64_t len, int lane) {
    const float pad = -__builtin_inff();
    const int64_t full = len / (kWave * 4);  // float4 slots inside the row on every lane (wave-uniform)
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int64_t a = int64_t(lane) * 4 + int64_t(u) * kWave * 4;
        if (u < full) {  // no padding to set: a uniform branch instead of per-lane selects
            if constexpr (Vec) v[u] = ld4(row + a);
            else v[u] = f4{row[a], row[a + 1], row[a + 2], row[a + 3]};
        } else if constexpr (Vec) {
            v[u] = a < len ? ld4(row + a) : f4{pad, pad, pad, pad};
        } else {
            v[u] = f4{a < len ? row[a] : pad, a + 1 < len ? row[a + 1] : pad, a + 2 < len ? row[a + 2] : pad,
                      a + 3 < len ? row[a + 3] : pad};
        }
    }
}

// Rows held in registers. Each wavefront walks rows r, r + W, ... (W
// wavefronts in the grid); the other wavefronts in flight on the SIMD hide a
// row's load latency. The loss terms are summed on the way: each wavefront in
// row order, then the block's wavefronts in order, into one double per block.
//
// The block that finishes last also finishes the loss, so the forward is one
// launch (red::count_in and red::finish_partials: the partials are added in
// one fixed order whichever block is last).

// ---- two rows per wavefront: lanes 0-31 hold one row, lanes 32-63 the next --
// For rows of at most 1024 classes. A row's cross-lane reductions then take
// five exchange steps instead of six, and one instruction serves both rows:
// the per-row work that does not scale with the row length halves. The row's
// values are dead after the exp-sum (the target's logit and the rare exact
// non-finite check read memory again), which keeps the kernel at five waves
// per SIMD without spilling.
__device__ inline float half_max(float v) {
    const int lane = red::lane_id();
    float o = red::partner<0>(v, lane);
    v = o > v ? o : v;
    o = red::partner<1>(v, lane);
    v = o > v ? o : v;
    o = red::partner<2>(v, lane);
    v = o > v ? o : v;
    o = red::partner<3>(v, lane);
    v = o > v ? o : v;
    o = red::partner<4>(v, lane);
    return o > v ? o : v;
}

// Sum over the half-wave in a fixed order; every lane of the half gets the same bits.
__device__ inline double half_sum(double v) {
    const int lane = red::lane_id();
    v += red::partner<0>(v, lane);
    v += red::partner<1>(v, lane);
    v += red::partner<2>(v, lane);
    v += red::partner<3>(v, lane);
    v += red::partner<4>(v, lane);
    return v;
}

__device__ inline uint32_t half_umax(uint32_t v) {
    const int lane = red::lane_id();
    v = max(v, red::partner<0>(v, lane));
    v = max(v, red::partner<1>(v, lane));
    v = max(v, red::partner<2>(v, lane));
    v = max(v, red::partner<3>(v, lane));
    return max(v, red::partner<4>(v, lane));
}

__device__ inline int half_or(int v) {
    const int lane = red::lane_id();
    v |= red::partner<0>(v, lane);
    v |= red::partner<1>(v, lane);
    v |= red::partner<2>(v, lane);
    v |= red::partner<3>(v, lane);
    v |= red::partner<4>(v, lane);
    return v;
}

__device__ inline Best half_best(Best b) {
    const int lane = red::lane_id();
    b = red::combine_partner<0>(b, lane);
    b = red::combine_partner<1>(b, lane);
    b = red::combine_partner<2>(b, lane);
    b = red::combine_partner<3>(b, lane);
    return red::combine_partner<4>(b, lane);
}

// A row of at most 128 NV classes into the registers of one half-wave: lane
// hl of the half holds element a = 4 hl + 128 u + component (-inf past the row).
template <bool Vec, int NV>
__device__ inline void load_half_row(f4 (&v)[NV], const float* __restrict__ row, int64_t len, int hl) {
    const float pad = -__builtin_inff();
    const int64_t full = len / 128;  // slots inside the row on every lane (wave-uniform)
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int64_t a = int64_t(hl) * 4 + int64_t(u) * 128;
        if (u < full) {
            if constexpr (Vec) v[u] = ld4(row + a);
            else v[u] = f4{row[a], row[a + 1], row[a + 2], row[a + 3]};
        } else if constexpr (Vec) {
            v[u] = a < len ? ld4(row + a) : f4{pad, pad, pad, pad};
        } else {
            v[u] = f4{a < len ? row[a] : pad, a + 1 < len ? row[a + 1] : pad, a + 2 < len ? row[a + 2] : pad,
                      a + 3 < len ? row[a + 3] : pad};
        }
    }
}

// finish_row for the row (at `row` in memory, index r) held by this lane's
// half-wave; t is its target, the same on the half's 32 lanes. valid false:
// a padding row past the batch, whose results are not written. Returns the
// loss term on the half's lane 0, as the same arithmetic as finish_row does
// with a half-wave's lanes.
template <bool Vec, int NV>
__device__ inline float finish_half_row(const f4 (&v)[NV], int64_t r, bool valid, const float* __restrict__ row,
                                        int64_t len, int t, int lane, float* __restrict__ stats,
                                        float* __restrict__ amax) {
    const int hl = lane & 31;
    const bool t_in_row = t >= 0 && int64_t(t) < len;
    const float x_t = t_in_row ? row[t] : 0.0f;  // loaded now, used at the end
    float mx = -__builtin_inff();
    uint32_t hi = 0;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        mx = __builtin_fmaxf(__builtin_fmaxf(mx, v[u].x), __builtin_fmaxf(__builtin_fmaxf(v[u].y, v[u].z), v[u].w));
        const int a = hl * 4 + u * 128, n = int(len);
        if constexpr (Vec) {
            const uint32_t b = max(max(bits_of(v[u].x), bits_of(v[u].y)), max(bits_of(v[u].z), bits_of(v[u].w)));
            hi = a < n ? max(hi, b) : hi;
        } else {
            const uint32_t b = max(max(a < n ? bits_of(v[u].x) : 0u, a + 1 < n ? bits_of(v[u].y) : 0u),
                                   max(a + 2 < n ? bits_of(v[u].z) : 0u, a + 3 < n ? bits_of(v[u].w) : 0u));
            hi = max(hi, b);
        }
    }
    mx = half_max(mx);
    // Element 0 of each half's row is on that half's lane 0.
    const float f0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[0].x), 0));
    const float f1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[0].x), 32));
    const float first = lane >= 32 ? f1 : f0;
    float m;
    if (first != first) {
        m = first;  // max() keeps a NaN first element (src/cpu/cpu_backend.cpp:443-452)
    } else if (mx == 0.0f) {  // rare: which zero comes first
        Best b = red::no_best();
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int a = hl * 4 + u * 128;
            if (a < len) {
                red::consider_ordered(b, v[u].x, a);
                red::consider_ordered(b, v[u].y, a + 1);
                red::consider_ordered(b, v[u].z, a + 2);
                red::consider_ordered(b, v[u].w, a + 3);
            }
        }
        m = half_best(b).v;
    } else {
        m = mx;
    }
    if (amax) {
        const int idx = lanes_min<5>(first_equal<NV, 128>(v, m, hl * 4));
        if (hl == 0 && valid) amax[r] = argmax_value(idx);
    }
    double c0 = 0.0, c1 = 0.0, c2 = 0.0, c3 = 0.0;  // as in finish_row
#pragma unroll
    for (int q = 0; q < NV; q += 4) {
        float g0 = 0.0f, g1 = 0.0f, g2 = 0.0f, g3 = 0.0f;
#pragma unroll
        for (int u = q; u < q + 4 && u < NV; ++u) {
            g0 += row_exp(v[u].x - m);
            g1 += row_exp(v[u].y - m);
            g2 += row_exp(v[u].z - m);
            g3 += row_exp(v[u].w - m);
        }
        c0 += double(g0);
        c1 += double(g1);
        c2 += double(g2);
        c3 += double(g3);
    }
    const double acc = half_sum(((c0 + c1) + c2) + c3);
    const bool nonfinite = !isfinite(m) || half_umax(hi) >= 0xff800000u || acc != acc;
    int bad = 0;  // a non-target log-prob that is not finite
    if (nonfinite) {  // rare: decide exactly from memory, leaving the target out
        for (int64_t a = hl; a < len; a += 32) bad |= (a != t && !isfinite(row[a] - m));
    }
    bad = half_or(bad);
    return (hl == 0 && valid) ? write_row(r, len, t, x_t, m, acc, bad, stats) : 0.0f;
}

// loss = -(float)(sum of row terms) / (float)rows: negate, then divide, as
// -(...).sum() / batch evaluates (src/nn.cpp:52).
struct NegateDivide {
    float rows;
    __device__ float operator()(float sum) const {
        const float negated = -sum;
        return negated / rows;
    }
};

// The end of a one-launch forward: each wavefront's loss terms are in
// wave_terms. Wavefront 0 adds them in wave order into the block's partial
// (the block's other wavefronts leave); the block that finishes last adds all
// partials in red::finish_partials' order (red::count_in) and writes the loss.
// With host_loss (pinned host memory), the loss is also written there, for a
// reader that waits for this kernel's completion only.
__device__ inline void finish_loss(double* wave_terms, double* __restrict__ part, int64_t rows,
                                   float* __restrict__ loss, float* __restrict__ host_loss) {
    __syncthreads();
    if (threadIdx.x >= kWave) return;
    double sum = 0.0;
    if (threadIdx.x == 0) {
        sum = wave_terms[0];
        for (int w = 1; w < kRowsPerBlock; ++w) sum += wave_terms[w];
    }
    if (!red::count_in(sum, part)) return;
    const double total = red::finish_partials(part);
    if (threadIdx.x == 0) {
        const float value = NegateDivide{float(rows)}(float(total));
        loss[0] = value;
        if (host_loss) host_loss[0] = value;
    }
}

// Rows of 1025 to 4096 classes, one row per wavefront at a time. The row
// takes NV float4 per lane (32 registers at NV 8, 64 at NV 16) and the
// allocation is left to the compiler (132 and 229 registers: three and two
// waves per SIMD; a minimum of waves per SIMD made it spill). The waves in
// flight hide the loads: loading the next row while finishing this one took a
// second register set, left three and one waves per SIMD, and measured 6% (2000
// classes) and 26% (4096 classes) slower over 32768 rows.
template <int NV, bool Vec>
__global__ __launch_bounds__(kBlock) void xent_rows_cached_kernel(const float* __restrict__ x,
                                                                  const int* __restrict__ targets, int64_t rows,
                                                                  int64_t len, float* __restrict__ stats,
                                                                  float* __restrict__ amax, double* __restrict__ part,
                                                                  float* __restrict__ loss,
                                                                  float* __restrict__ host_loss) {
    __shared__ double wave_terms[kRowsPerBlock];
    const int lane = threadIdx.x % kWave;
    const int64_t first = int64_t(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
    const int64_t waves = int64_t(gridDim.x) * kRowsPerBlock;
    double total = 0.0;  // lane 0: this wavefront's terms, in row order
    // The target is loaded before the row, so waiting for it never waits for
    // the row loads.
    for (int64_t r = first; r < rows; r += waves) {
        const int t = __builtin_amdgcn_readfirstlane(targets[r]);
        f4 cur[NV];
        load_row<Vec>(cur, x + r * len, len, lane);
        total += double(finish_row<Vec>(cur, r, len, t, lane, stats, amax));
    }
    if (lane == 0) wave_terms[threadIdx.x / kWave] = total;
    finish_loss(wave_terms, part, rows, loss, host_loss);
}

// Rows of at most 1024 classes, two per wavefront (finish_half_row): wave w
// takes row pairs p = w, w + W, ... (rows 2p and 2p + 1). The loss terms are
// summed per half in row order, then the wavefront's lower half before its
// upper half, then as xent_rows_cached_kernel does (its last block finishes
// the loss). With 16-byte loads five waves per SIMD (96 registers) fit without
// spilling and measured faster than six (which spill) or loading the next pair
// ahead (three waves): 32768 x 1000 in 22.8 us against 25.8 us for a row per
// wavefront. The scalar-load variant (rows not a multiple of 4 classes, or
// misaligned) needs a few more registers at NV 8 and runs four waves.
template <int NV, bool Vec>
__global__ __launch_bounds__(kBlock, Vec || NV < 8 ? 5 : 4) void xent_half_rows_kernel(
    const float* __restrict__ x, const int* __restrict__ targets, int64_t rows, int64_t len, float* __restrict__ stats,
    float* __restrict__ amax, double* __restrict__ part, float* __restrict__ loss, float* __restrict__ host_loss) {
    __shared__ double wave_terms[kRowsPerBlock];
    const int lane = threadIdx.x % kWave, h = lane >> 5;
    const int64_t wave_id = int64_t(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
    const int64_t waves = int64_t(gridDim.x) * kRowsPerBlock;
    double total = 0.0;  // lanes 0 and 32: their half's terms
    for (int64_t pair = wave_id; 2 * pair < rows; pair += waves) {
        const int64_t r = 2 * pair + h;
        const int64_t rr = r < rows ? r : rows - 1;  // the upper half of a last, odd pair repeats row rows - 1
        const int t = targets[rr];
        f4 v[NV];
        load_half_row<Vec>(v, x + rr * len, len, lane & 31);
        total += double(finish_half_row<Vec>(v, rr, r < rows, x + rr * len, len, t, lane, stats, amax));
    }
    const uint64_t tb = __builtin_bit_cast(uint64_t, total);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(tb)), 32));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(tb >> 32)), 32));
    const double upper = __builtin_bit_cast(double, uint64_t(lo) | (uint64_t(hi) << 32));
    if (lane == 0) wave_terms[threadIdx.x / kWave] = total + upper;
    finish_loss(wave_terms, part, rows, loss, host_loss);
}

// One wavefront per row, streaming the row twice (rows too long for
// registers, or not 16-byte aligned).
template <bool Vec>
__global__ __launch_bounds__(kBlock) void xent_rows_kernel(const float* __restrict__ x, const int* __restrict__ targets,
                                                           int64_t rows, int64_t len, float* __restrict__ stats,
                                                           float* __restrict__ amax, float* __restrict__ terms) {
    const int lane = threadIdx.x % kWave;
    const int64_t r = int64_t(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
    if (r >= rows) return;
    const float* row = x + r * len;
    const int t = targets[r];
    const Best best = row_max(row, len, lane, Vec);
    const float m = best.v;
    if (amax && lane == 0) amax[r] = float(best.i);
    double acc = 0.0;
    int bad = 0;  // a non-target log-prob that is not finite
    if (Vec) {  // four component chains, joined in order, as the register-held path adds
        double c0 = 0.0, c1 = 0.0, c2 = 0.0, c3 = 0.0;
        for (int64_t a = int64_t(lane) * 4; a < len; a += kWave * 4) {
            const f4 v = ld4(row + a);
            const float s0 = v.x - m, s1 = v.y - m, s2 = v.z - m, s3 = v.w - m;
            c0 += double(row_exp(s0));
            c1 += double(row_exp(s1));
            c2 += double(row_exp(s2));
            c3 += double(row_exp(s3));
            bad |= (a != t && !isfinite(s0)) | (a + 1 != t && !isfinite(s1)) | (a + 2 != t && !isfinite(s2)) |
                   (a + 3 != t && !isfinite(s3));
        }
        acc = ((c0 + c1) + c2) + c3;
    } else {
        for (int64_t a = lane; a < len; a += kWave) {
            const float s = row[a] - m;
            acc += double(row_exp(s));
            bad |= (a != t && !isfinite(s));
        }
    }
    acc = red::wave_sum(acc);
    bad = red::wave_or(bad);
    if (lane == 0) {
        const bool in_row = t >= 0 && int64_t(t) < len;
        terms[r] = write_row(r, len, t, in_row ? row[t] : 0.0f, m, acc, bad, stats);
    }
}

template <bool Vec>
__global__ __launch_bounds__(kBlock) void xent_backward_kernel(const float* __restrict__ x, const int* __restrict__ targets,
                                                               const float* __restrict__ stats,
                                                               const float* __restrict__ grad_loss, float grad_value,
                                                               int64_t rows, int64_t len, float* __restrict__ dx) {
    const int lane = threadIdx.x % kWave;
    const int64_t r = int64_t(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
    if (r >= rows) return;
    const float c = (grad_loss ? grad_loss[0] : grad_value) / float(rows);
    const float m = stats[2 * r], s = stats[2 * r + 1];
    const float scale = c / s;
    const float neg_c = -c;
    const int t = targets[r];
    const float* row = x + r * len;
    float* out = dx + r * len;
    if (Vec) {
        for (int64_t a = int64_t(lane) * 4; a < len; a += kWave * 4) {
            const f4 v = ld4(row + a);
            f4 g;
            g.x = scale * row_exp(v.x - m) + (a == t ? neg_c : -0.0f);
            g.y = scale * row_exp(v.y - m) + (a + 1 == t ? neg_c : -0.0f);
            g.z = scale * row_exp(v.z - m) + (a + 2 == t ? neg_c : -0.0f);
            g.w = scale * row_exp(v.w - m) + (a + 3 == t ? neg_c : -0.0f);
            *reinterpret_cast<f4*>(out + a) = g;
        }
    } else {
        for (int64_t a = lane; a < len; a += kWave) out[a] = scale * row_exp(row[a] - m) + (a == t ? neg_c : -0.0f);
    }
}

// The backward above, also leaving the column sums of dx (the gradient of a
// bias added to the logits): a workgroup takes kColRows consecutive rows,
// wave w the rows w, w + 4, ... of them, each held in registers as in the
// forward (NV float4 per lane, the next row loaded before the current one is
// finished). Each lane adds its columns' values over its rows in double;
// the four waves are joined in wave order through LDS into one partial row
// per workgroup, which red::column_partials_kernel then adds up. dx has the
// same bits as xent_backward_kernel's.
constexpr int kColRows = 16;

template <int NV, bool Vec>
__global__ __launch_bounds__(kBlock) void xent_backward_colsum_kernel(const float* __restrict__ x,
                                                                      const int* __restrict__ targets,
                                                                      const float* __restrict__ stats,
                                                                      const float* __restrict__ grad_loss,
                                                                      float grad_value, int64_t rows, int64_t len,
                                                                      float* __restrict__ dx, double* __restrict__ part) {
    __shared__ double joined[kRowsPerBlock - 1][NV * kWave * 4];
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    const float c = (grad_loss ? grad_loss[0] : grad_value) / float(rows);
    const float neg_c = -c;
    double acc[NV][4];
#pragma unroll
    for (int u = 0; u < NV; ++u) acc[u][0] = acc[u][1] = acc[u][2] = acc[u][3] = 0.0;
    const int64_t first = int64_t(blockIdx.x) * kColRows + w;
    const int64_t last = std::min<int64_t>(rows, int64_t(blockIdx.x + 1) * kColRows);
    if (first < last) {
        f4 cur[NV], next[NV];
        // The next row's statistics and target are loaded before its values
        // and read after this row is stored, so waiting for them never waits
        // for the row loads in flight.
        float m = stats[2 * first], s = stats[2 * first + 1];
        int t = targets[first];
        load_row<Vec>(cur, x + first * len, len, lane);
        for (int64_t r = first; r < last; r += kRowsPerBlock) {
            float mn = 0.0f, sn = 1.0f;
            int tn = 0;
            if (r + kRowsPerBlock < last) {
                mn = stats[2 * (r + kRowsPerBlock)];
                sn = stats[2 * (r + kRowsPerBlock) + 1];
                tn = targets[r + kRowsPerBlock];
                load_row<Vec>(next, x + (r + kRowsPerBlock) * len, len, lane);
            }
            const float scale = c / s;
            float* out = dx + r * len;
#pragma unroll
            for (int u = 0; u < NV; ++u) {
                const int a = lane * 4 + u * kWave * 4;
                if (a < len) {
                    f4 g;
                    g.x = scale * row_exp(cur[u].x - m) + (a == t ? neg_c : -0.0f);
                    g.y = scale * row_exp(cur[u].y - m) + (a + 1 == t ? neg_c : -0.0f);
                    g.z = scale * row_exp(cur[u].z - m) + (a + 2 == t ? neg_c : -0.0f);
                    g.w = scale * row_exp(cur[u].w - m) + (a + 3 == t ? neg_c : -0.0f);
                    if constexpr (Vec) {
                        *reinterpret_cast<f4*>(out + a) = g;
                    } else {
                        out[a] = g.x;
                        if (a + 1 < len) out[a + 1] = g.y;
                        if (a + 2 < len) out[a + 2] = g.z;
                        if (a + 3 < len) out[a + 3] = g.w;
                    }
                    // past the row: exp(-inf - m) * scale + -0.0 = +0.0 (or NaN with a NaN m, never stored)
                    acc[u][0] += double(g.x);
                    acc[u][1] += double(a + 1 < len ? g.y : 0.0f);
                    acc[u][2] += double(a + 2 < len ? g.z : 0.0f);
                    acc[u][3] += double(a + 3 < len ? g.w : 0.0f);
                }
            }
#pragma unroll
            for (int u = 0; u < NV; ++u) cur[u] = next[u];
            m = mn;
            s = sn;
            t = tn;
        }
    }
    if (w > 0) {
#pragma unroll
        for (int u = 0; u < NV; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) joined[w - 1][u * kWave * 4 + lane * 4 + e] = acc[u][e];
    }
    __syncthreads();
    if (w == 0) {
#pragma unroll
        for (int u = 0; u < NV; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int a = lane * 4 + u * kWave * 4 + e;
                double total = acc[u][e];
#pragma unroll
                for (int k = 0; k < kRowsPerBlock - 1; ++k) total += joined[k][u * kWave * 4 + lane * 4 + e];
                if (a < len) part[int64_t(blockIdx.x) * len + a] = total;
            }
    }
}

void xent_backward(const float* logits, const int32_t* targets, const float* row_stats, const float* grad_loss,
                   float grad_value, size_t rows, size_t classes, float* grad_logits) {
    Device& d = require_device();
    if (rows == 0 || classes == 0) return;
    if (classes > size_t(std::numeric_limits<int>::max())) fail(VC_HIP_ERR_OVERFLOW, "too many classes");
    const int64_t R = int64_t(rows), C = int64_t(classes);
    const bool vec = C % 4 == 0 && aligned16(logits) && aligned16(grad_logits);
    const unsigned grid = unsigned((R + kRowsPerBlock - 1) / kRowsPerBlock);
    Profiled p("xent_backward", 0.0, 8.0 * double(R * C) + 12.0 * double(R));
    if (vec)
        launch(xent_backward_kernel<true>, dim3(grid), dim3(kBlock), 0, d.stream, logits, targets, row_stats, grad_loss,
               grad_value, R, C, grad_logits);
    else
        launch(xent_backward_kernel<false>, dim3(grid), dim3(kBlock), 0, d.stream, logits, targets, row_stats,
               grad_loss, grad_value, R, C, grad_logits);
    after_launch("xent_backward");
    p.done();
}

// Workgroups of xent_rows_cached_kernel<NV, Vec> resident on one CU at once
// (its register use sets it; queried once per process).
template <int NV, bool Vec>
int64_t cached_resident_blocks() {
    static const int64_t blocks = [] {
        int b = 0;
        const bool ok =
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, xent_rows_cached_kernel<NV, Vec>, kBlock, 0) == hipSuccess;
        return ok && b > 0 ? int64_t(b) : int64_t(1);
    }();
    return blocks;
}

// The forward. With `publish`, the loss is also copied into that mirror's
// host slot: by the finishing block of a register-held row kernel, whose
// dispatch then carries the mirror's completion event (recorded on the stream
// right after the dispatch when the profiler holds the dispatch's events), or,
// when the rows are streamed, by a copy launched after the forward. With
// row_argmax, every path also writes each row's argmax (as a float index)
// from the row it already holds.
void xent_forward(const float* logits, const int32_t* targets, size_t rows, size_t classes, float* row_stats,
                  float* loss, float* row_argmax, vc_hip_mirror* publish) {
    Device& d = require_device();
    if (rows == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "cross_entropy of an empty batch is undefined");
    if (classes == 0) fail(VC_HIP_ERR_INVALID_ARGUMENT, "cross_entropy needs at least one class");
    if (classes > size_t(std::numeric_limits<int>::max())) fail(VC_HIP_ERR_OVERFLOW, "too many classes");
    const int64_t R = int64_t(rows), C = int64_t(classes);
    Scratch terms(rows * sizeof(float));
    const bool vec = C % 4 == 0 && aligned16(logits);
    const unsigned grid = unsigned((R + kRowsPerBlock - 1) / kRowsPerBlock);
    Profiled p("xent_forward", 0.0,
               4.0 * double(R * C) + 4.0 * double(R) + 8.0 * double(R) + (row_argmax ? 4.0 * double(R) : 0.0));
    // Rows are held in registers: up to 1024 classes two rows per wavefront,
    // up to 4096 one row per wavefront (NV float4 per lane). At most 8
    // workgroups per CU walk the two-row kernel's rows (3 to 12 per CU
    // measured within 3%); the one-row kernel takes as many as are resident
    // at once (two or three per CU), so no workgroup waits for a CU to free up
    // (8 per CU measured 5-40% slower). Longer rows are streamed.
    const int64_t nv = (C + kWave * 4 - 1) / (kWave * 4);
    const int64_t nh = (C + 127) / 128;  // float4s per lane with a half-wave per row
    int64_t row_blocks = 0;              // grid of the register-held row kernel
    if (nh <= 8) {
        row_blocks = std::min<int64_t>({(R + 2 * kRowsPerBlock - 1) / (2 * kRowsPerBlock),
                                        int64_t(d.cu_count) * kXentBlocksPerCu, int64_t(red::kMaxFinishBlocks)});
    } else if (nv <= 16) {
        const int64_t resident = nv <= 8 ? (vec ? cached_resident_blocks<8, true>() : cached_resident_blocks<8, false>())
                                         : (vec ? cached_resident_blocks<16, true>() : cached_resident_blocks<16, false>());
        row_blocks = std::min<int64_t>({(R + kRowsPerBlock - 1) / kRowsPerBlock,
                                        int64_t(d.cu_count) * std::min(kXentBlocksPerCu, resident),
                                        int64_t(red::kMaxFinishBlocks)});
    }
    Scratch part(size_t(std::max<int64_t>(row_blocks, (R + red::sum_chunk(R) - 1) / red::sum_chunk(R))) *
                 sizeof(double));
    // Register-held rows (nv <= 16) write the loss's host copy from their
    // finishing block, the dispatch signalling the mirror; when the profiler
    // holds the dispatch's events, the mirror's event is recorded after it.
    float* host_loss = nullptr;
    hipEvent_t published = nullptr;
    bool record_published = false;
    if (publish && nv <= 16) {
        host_loss = publish->host;
        if (p.stop_event()) record_published = true;
        else published = publish->done;
    }
    auto row_launch = [&](auto kernel, unsigned blocks) {
        if (published)
            hipExtLaunchKernelGGL(kernel, dim3(blocks), dim3(kBlock), 0, d.stream, nullptr, published, 0u, logits,
                                  targets, R, C, row_stats, row_argmax, part.as<double>(), loss, host_loss);
        else
            launch(kernel, dim3(blocks), dim3(kBlock), 0, d.stream, logits, targets, R, C, row_stats, row_argmax,
                   part.as<double>(), loss, host_loss);
    };
    if (nh <= 8) {
        // Rows of at most 1024 classes: two per wavefront.
#define VC_XENT_HALF(NV) \
    row_launch(vec ? xent_half_rows_kernel<NV, true> : xent_half_rows_kernel<NV, false>, unsigned(row_blocks))
        if (nh <= 1) VC_XENT_HALF(1);
        else if (nh <= 2) VC_XENT_HALF(2);
        else if (nh <= 4) VC_XENT_HALF(4);
        else VC_XENT_HALF(8);
#undef VC_XENT_HALF
    } else if (nv > 16) {
        // Row terms, then the shared deterministic full sum (one launch).
        launch((vec ? xent_rows_kernel<true> : xent_rows_kernel<false>), dim3(grid), dim3(kBlock), 0, d.stream,
               logits, targets, R, C, row_stats, row_argmax, terms.as<float>());
        after_launch("xent_forward");
        const int64_t chunk = red::sum_chunk(R);
        const int64_t blocks = (R + chunk - 1) / chunk;
        launch(red::sum_finish_kernel<true, NegateDivide>, dim3(unsigned(blocks)), dim3(kBlock), 0, d.stream,
               terms.as<float>(), part.as<double>(), loss, R, chunk, NegateDivide{float(R)});
    } else {
        // Register-held rows; the row kernel sums the terms per block and
        // its last block finishes the loss.
#define VC_XENT_ROWS(NV) \
    row_launch(vec ? xent_rows_cached_kernel<NV, true> : xent_rows_cached_kernel<NV, false>, unsigned(row_blocks))
        if (nv <= 8) VC_XENT_ROWS(8);  // rows of more than 1024 classes: nv >= 5
        else VC_XENT_ROWS(16);
#undef VC_XENT_ROWS
    }
    after_launch("xent_forward");
    if (record_published) {
        const hipError_t e = hipEventRecord(publish->done, d.stream);
        if (e != hipSuccess)
            fail(VC_HIP_ERR_RUNTIME, std::string("xent_forward: event record failed: ") + hipGetErrorString(e));
    }
    if (publish && !host_loss) launch_mirror(publish, loss);
    p.done();
}

// Runs forward(m) with a mirror taken for it, handed to *mirror on success.
template <class F>
void with_mirror(vc_hip_mirror** mirror, const char* name, F&& forward) {
    if (!mirror) fail(VC_HIP_ERR_INVALID_ARGUMENT, std::string(name) + ": null mirror");
    require_device();
    vc_hip_mirror* m = take_mirror();
    try {
        forward(m);
    } catch (...) {
        give_mirror(m);
        throw;
    }
    *mirror = m;
}

// The backward with the column sums of dx (vc_hip_xent_backward_colsum):
// for rows of at most 2048 classes the kernel keeps one partial row per
// kColRows rows, finished next by column_partials_kernel or, with `pending`,
// handed to the caller; longer rows run the plain backward and a separate
// reduction of dx.
void xent_backward_colsum(const float* logits, const int32_t* targets, const float* row_stats, const float* grad_loss,
                          float grad_loss_value, size_t rows, size_t classes, float* grad_logits, float* column_sum,
                          vc_hip_colsum** pending) {
    Device& d = require_device();
    if (pending) *pending = nullptr;
    if (!column_sum) fail(VC_HIP_ERR_INVALID_ARGUMENT, "xent_backward_colsum: null column sum");
    if (classes == 0) return;
    if (classes > size_t(std::numeric_limits<int>::max())) fail(VC_HIP_ERR_OVERFLOW, "too many classes");
    const int64_t R = int64_t(rows), C = int64_t(classes);
    const int64_t nv = (C + kWave * 4 - 1) / (kWave * 4);
    const bool fused = rows > 0 && nv <= 8;
    const bool vec = C % 4 == 0 && aligned16(logits) && aligned16(grad_logits);
    if (!fused) {  // the plain backward, then a separate reduction of dx
        xent_backward(logits, targets, row_stats, grad_loss, grad_loss_value, rows, classes, grad_logits);
        const int rc = vc_hip_reduce_axis(grad_logits, column_sum, 1, rows, classes, VC_REDUCE_SUM);
        if (rc != VC_HIP_OK) fail(rc, std::string("column sum of the cross-entropy gradient: ") + vc_hip_last_error());
        return;
    }
    const int64_t blocks = (R + kColRows - 1) / kColRows;
    if (blocks > std::numeric_limits<int>::max()) fail(VC_HIP_ERR_OVERFLOW, "too many rows");
    ColsumPtr sums = new_colsum(blocks, C);
    {
        Profiled p("xent_backward", 0.0, 8.0 * double(R * C) + 12.0 * double(R) + 8.0 * double(blocks * C));
#define VC_XENT_BWD_COLSUM(NV)                                                                               \
    launch(vec ? xent_backward_colsum_kernel<NV, true> : xent_backward_colsum_kernel<NV, false>,               \
           dim3(unsigned(blocks)), dim3(kBlock), 0, d.stream, logits, targets, row_stats, grad_loss,           \
           grad_loss_value, R, C, grad_logits, sums->part)
        if (nv <= 1) VC_XENT_BWD_COLSUM(1);
        else if (nv <= 2) VC_XENT_BWD_COLSUM(2);
        else if (nv <= 4) VC_XENT_BWD_COLSUM(4);
        else VC_XENT_BWD_COLSUM(8);
#undef VC_XENT_BWD_COLSUM
        after_launch("xent_backward");
        p.done();
    }
    if (pending) *pending = sums.release();
    else finish_colsum(*sums, column_sum);
}

}  // namespace
}  // namespace vchip

using namespace vchip;

extern "C" {

int vc_hip_xent_forward(const float* logits, const int32_t* targets, size_t rows, size_t classes, float* row_stats,
                        float* loss) {
    return guard([&] { xent_forward(logits, targets, rows, classes, row_stats, loss, nullptr, nullptr); });
}


int vc_hip_xent_forward_published(const float* logits, const int32_t* targets, size_t rows, size_t classes,
                                  float* row_stats, float* loss, vc_hip_mirror** mirror) {
    return guard([&] {
        with_mirror(mirror, "vc_hip_xent_forward_published", [&](vc_hip_mirror* m) {
            xent_forward(logits, targets, rows, classes, row_stats, loss, nullptr, m);
        });
    });
}

int vc_hip_xent_forward_argmax(const float* logits, const int32_t* targets, size_t rows, size_t classes,
                               float* row_stats, float* loss, float* row_argmax, vc_hip_mirror** mirror) {
    return guard([&] {
        if (!row_argmax) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_xent_forward_argmax: null row_argmax");
        if (!mirror) {
            xent_forward(logits, targets, rows, classes, row_stats, loss, row_argmax, nullptr);
            return;
        }
        with_mirror(mirror, "vc_hip_xent_forward_argmax", [&](vc_hip_mirror* m) {
            xent_forward(logits, targets, rows, classes, row_stats, loss, row_argmax, m);
        });
    });
}

int vc_hip_xent_backward(const float* logits, const int32_t* targets, const float* row_stats, const float* grad_loss,
                         size_t rows, size_t classes, float* grad_logits) {
    return guard([&] {
        if (!grad_loss) fail(VC_HIP_ERR_INVALID_ARGUMENT, "xent_backward: null grad_loss");
        xent_backward(logits, targets, row_stats, grad_loss, 0.0f, rows, classes, grad_logits);
    });
}

int vc_hip_xent_backward_value(const float* logits, const int32_t* targets, const float* row_stats, float grad_loss,
                               size_t rows, size_t classes, float* grad_logits) {
    return guard([&] { xent_backward(logits, targets, row_stats, nullptr, grad_loss, rows, classes, grad_logits); });
}

int vc_hip_xent_backward_colsum(const float* logits, const int32_t* targets, const float* row_stats,
                                const float* grad_loss, float grad_loss_value, size_t rows, size_t classes,
                                float* grad_logits, float* column_sum) {
    return guard([&] {
        xent_backward_colsum(logits, targets, row_stats, grad_loss, grad_loss_value, rows, classes, grad_logits,
                             column_sum, nullptr);
    });
}

int vc_hip_xent_backward_colsum_pending(const float* logits, const int32_t* targets, const float* row_stats,
                                        const float* grad_loss, float grad_loss_value, size_t rows, size_t classes,
                                        float* grad_logits, float* column_sum, vc_hip_colsum** pending) {
    return guard([&] {
        if (!pending) fail(VC_HIP_ERR_INVALID_ARGUMENT, "xent_backward_colsum_pending: null handle pointer");
        xent_backward_colsum(logits, targets, row_stats, grad_loss, grad_loss_value, rows, classes, grad_logits,
                             column_sum, pending);
    });
}

}  // extern "C"
