// Internal plumbing shared by the HIP translation units of libvc_hip.so:
// the device singleton (one in-order stream), status/error reporting, launch
// checks and the optional per-launch event profiler.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "vc_hip.h"

// A pinned host slot and the event that completes when a value has been
// copied into it (vc_hip_mirror_scalar).
struct vc_hip_mirror {
    float* host;
    hipEvent_t done;
};

// Column sums left pending by the kernel that wrote a matrix: `rows` partial
// rows of n doubles (every row of the matrix counted in exactly one) in a
// pool buffer, added in red::combine_waves' order by whichever kernel
// finishes them (vc_hip_colsum_finish, vc_hip_axpy_batch_colsum).
struct vc_hip_colsum {
    double* part;
    int64_t rows;
    int64_t n;
};

namespace vchip {

// An error carrying the C-ABI status it maps to.
struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string& message) : std::runtime_error(message), status(s) {}
};

[[noreturn]] inline void fail(int status, const std::string& message) { throw Error(status, message); }

inline void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fail(e == hipErrorOutOfMemory ? VC_HIP_ERR_OUT_OF_MEMORY : VC_HIP_ERR_RUNTIME,
             std::string(what) + ": " + hipGetErrorString(e));
    }
}

void set_last_error(const std::string& message);

// Runs `body` and converts exceptions into a status + thread-local message.
template <typename F>
int guard(F&& body) {
    try {
        body();
        return VC_HIP_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.status;
    } catch (const std::bad_alloc&) {
        set_last_error("host allocation failed");
        return VC_HIP_ERR_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return VC_HIP_ERR_RUNTIME;
    }
}

struct Device {
    bool ready = false;
    std::string error;  // why the device is unavailable
    std::string name;
    int ordinal = 0;
    int cu_count = 0;
    hipStream_t stream = nullptr;
    bool sync_each_launch = false;  // VECTORCORE_HIP_SYNC_EACH=1 (fault localisation)
    std::atomic<int> gemm_mode{0};  // a GemmMode: VECTORCORE_HIP_GEMM or vc_hip_set_gemm_kernel
};

// GEMM kernel selection (vc_hip_set_gemm_kernel names in brackets): automatic
// ("mfma": the FMA kernel for tiny products, 32 x 32, 128 x 128 or 256 x 256
// matrix-core tiles by shape), the portable FMA kernel for every product
// ("simple"), the 128 x 128 tiles for every product ("mfma128"), or the
// 256 x 256 ("mfma256") or 256 x 128 ("mfma256x128") tiles for every product
// whose operands allow them, the 128 x 128 tiles for the rest.
enum GemmMode : int { kGemmAuto = 0, kGemmSimple = 1, kGemmTiles128 = 2, kGemmTiles256 = 3, kGemmTiles256x128 = 4 };
const char* gemm_mode_name(int mode);

// Initialises once (thread-safe) and makes the device current on this thread.
Device& device();
// device() plus a thrown VC_HIP_ERR_UNAVAILABLE when there is no usable GPU.
Device& require_device();

// Call right after every kernel launch on the library stream.
void after_launch(const char* label);

// Pool-backed device scratch for multi-pass kernels. Released to the pool when
// the object dies; stream order keeps the enqueued passes safe.
void* pool_alloc(size_t bytes);
void pool_release(void* p) noexcept;

// Scalar mirrors (runtime.hip): a pinned host slot and its completion event,
// taken from and given back to the library's free list; launch_mirror copies
// a device value into the slot in stream order, the copy's dispatch carrying
// the event.
vc_hip_mirror* take_mirror();
void give_mirror(vc_hip_mirror* m) noexcept;
void launch_mirror(vc_hip_mirror* m, const float* device_value);

// Pending column sums (reduce.hip): a handle owning a pool buffer of
// rows * n doubles, released in stream order; finish_colsum enqueues
// column_partials_kernel into out (n floats) under the "column_sum_combine"
// profiler label.
struct ColsumRelease {
    void operator()(vc_hip_colsum* h) const noexcept;
};
using ColsumPtr = std::unique_ptr<vc_hip_colsum, ColsumRelease>;
ColsumPtr new_colsum(int64_t rows, int64_t n);
void finish_colsum(const vc_hip_colsum& h, float* out);
class Scratch {
public:
    explicit Scratch(size_t bytes) : p_(pool_alloc(bytes)) {}
    ~Scratch() { pool_release(p_); }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    template <typename T>
    T* as() const { return static_cast<T*>(p_); }
private:
    void* p_;
};

// --- profiler --------------------------------------------------------------
// Usage around one launch:  Profiled p("label", flops, bytes);  kernel<<<...>>>;
// p.done();  Both are no-ops unless profiling is enabled.
// One labelled unit of work (an entry point's kernels) under the optional
// profiler. Its timing comes from the kernels' own dispatch-packet timestamps:
// launch() hands the first kernel of the scope the start event and every
// kernel the stop event (hipExtLaunchKernelGGL), so profiling adds no marker
// packets, and no bubbles, between kernels. Scopes nest per thread.
class Profiled {
public:
    Profiled(const char* label, double flops, double bytes);
    ~Profiled();
    Profiled(const Profiled&) = delete;
    Profiled& operator=(const Profiled&) = delete;
    void done();  // records the scope if any kernel carried its events
    hipEvent_t start_event() {
        if (label_ < 0 || started_) return nullptr;
        started_ = true;
        return start_;
    }
    hipEvent_t stop_event() const { return label_ < 0 ? nullptr : stop_; }
    static Profiled* current();

private:
    int label_ = -1;
    bool started_ = false;
    bool popped_ = false;
    hipEvent_t start_ = nullptr, stop_ = nullptr;
    double flops_ = 0, bytes_ = 0;
    Profiled* outer_ = nullptr;
};

// Every kernel of the library is launched through here, on `stream`.
template <typename F, typename... Args>
inline void launch(F kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t stream, Args... args) {
    Profiled* p = Profiled::current();
    hipEvent_t start = p ? p->start_event() : nullptr;
    hipEvent_t stop = p ? p->stop_event() : nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, start, stop, 0u, args...);
}

// --- launch-shape checks -----------------------------------------------------
inline unsigned grid_1d(size_t items, unsigned block, unsigned max_blocks) {
    size_t blocks = (items + block - 1) / block;
    if (blocks == 0) blocks = 1;
    if (blocks > max_blocks) blocks = max_blocks;
    return static_cast<unsigned>(blocks);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Shape metadata for broadcasting kernels (rank <= 8), passed by value.
constexpr int kMaxRank = 8;
struct Bcast {
    int rank;
    int64_t out_shape[kMaxRank];
    int64_t a_stride[kMaxRank];  // 0 on broadcast axes
    int64_t b_stride[kMaxRank];
};

// Builds collapsed broadcast metadata; throws VC_HIP_ERR_INVALID_ARGUMENT for
// a rank above 8 or incompatible shapes.
Bcast make_bcast(const size_t* a_shape, const size_t* a_strides, size_t a_rank, const size_t* b_shape,
                 const size_t* b_strides, size_t b_rank, const size_t* out_shape, size_t out_rank);

}  // namespace vchip
