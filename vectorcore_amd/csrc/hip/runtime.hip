// Device, memory and measurement entry points of libvc_hip.so.
//
// Execution model: one in-order, default-priority stream per process. Every
// kernel, upload and device copy is enqueued on it, so a buffer returned to
// the pool can be handed out again immediately: any later use is ordered
// after every earlier one. The host waits only in vc_hip_download and
// vc_hip_synchronize (and, rarely, when the pinned staging ring or the pool
// needs memory back), and in vc_hip_mirror_read, which waits for one point of
// the stream only.
#include "vc_hip_internal.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <memory>
#include <unordered_map>

namespace vchip {

namespace {

thread_local std::string t_last_error;

bool env_is(const char* name, const char* value) {
    const char* v = std::getenv(name);
    return v && std::strcmp(v, value) == 0;
}

Device& device_singleton() {
    static Device dev;
    return dev;
}

void init_device(Device& d) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) {
        d.error = std::string("no HIP device visible (") + (e != hipSuccess ? hipGetErrorString(e) : "0 devices") + ")";
        return;
    }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, d.ordinal);
    if (e != hipSuccess) {
        d.error = std::string("hipGetDeviceProperties failed: ") + hipGetErrorString(e);
        return;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        d.error = std::string("kernels are built for gfx950 (MI355X); device 0 is ") + prop.gcnArchName;
        return;
    }
    e = hipSetDevice(d.ordinal);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        d.error = std::string("HIP stream creation failed: ") + hipGetErrorString(e);
        return;
    }
    d.name = prop.name[0] ? prop.name : "AMD Instinct MI355X";
    d.name += std::string(" (") + prop.gcnArchName + ")";
    d.cu_count = prop.multiProcessorCount;
    d.sync_each_launch = env_is("VECTORCORE_HIP_SYNC_EACH", "1");
    for (int mode : {kGemmSimple, kGemmTiles128, kGemmTiles256, kGemmTiles256x128})
        if (env_is("VECTORCORE_HIP_GEMM", gemm_mode_name(mode))) d.gemm_mode = mode;
    d.ready = true;
}

// ---- pool ---------------------------------------------------------------------

class Pool {
public:
    // Powers of two from 256 B to 4 MiB, then whole 2 MiB steps.
    static size_t size_class(size_t bytes) {
        constexpr size_t kMin = 256, kPow2Limit = size_t(4) << 20, kStep = size_t(2) << 20;
        if (bytes <= kMin) return kMin;
        if (bytes <= kPow2Limit) {
            size_t c = kMin;
            while (c < bytes) c <<= 1;
            return c;
        }
        return (bytes + kStep - 1) / kStep * kStep;
    }

    void* alloc(size_t bytes) {
        Device& d = require_device();
        const size_t cls = size_class(bytes);
        {
            std::lock_guard<std::mutex> lock(mu_);
            auto it = free_.find(cls);
            if (it != free_.end() && !it->second.empty()) {
                void* p = it->second.back();
                it->second.pop_back();
                pooled_bytes_ -= cls;
                live_[p] = cls;
                live_bytes_ += cls;
                ++reuses_;
                return p;
            }
        }
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, cls);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            trim();
            e = hipMalloc(&p, cls);
        }
        if (e != hipSuccess) {
            (void)hipGetLastError();
            fail(VC_HIP_ERR_OUT_OF_MEMORY, "HIP allocation of " + std::to_string(cls) + " bytes failed on " + d.name +
                                               ": " + hipGetErrorString(e));
        }
        std::lock_guard<std::mutex> lock(mu_);
        live_[p] = cls;
        live_bytes_ += cls;
        ++allocs_;
        return p;
    }

    void release(void* p) {
        if (!p) return;
        std::lock_guard<std::mutex> lock(mu_);
        auto it = live_.find(p);
        if (it == live_.end()) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_release: buffer was not allocated by vc_hip_alloc");
        const size_t cls = it->second;
        live_.erase(it);
        live_bytes_ -= cls;
        free_[cls].push_back(p);
        pooled_bytes_ += cls;
    }

    void trim() {
        Device& d = require_device();
        check_hip(hipStreamSynchronize(d.stream), "hipStreamSynchronize");
        std::lock_guard<std::mutex> lock(mu_);
        for (auto& [cls, list] : free_) {
            for (void* p : list) (void)hipFree(p);
            list.clear();
        }
        pooled_bytes_ = 0;
    }

    vc_hip_pool_stats stats() {
        std::lock_guard<std::mutex> lock(mu_);
        return vc_hip_pool_stats{allocs_, reuses_, live_bytes_, pooled_bytes_};
    }

private:
    std::mutex mu_;
    std::unordered_map<size_t, std::vector<void*>> free_;
    std::unordered_map<void*, size_t> live_;
    uint64_t allocs_ = 0, reuses_ = 0, live_bytes_ = 0, pooled_bytes_ = 0;
};

Pool& pool() {
    static Pool p;
    return p;
}

// ---- pinned staging ring for uploads --------------------------------------------

class Staging {
public:
    static constexpr size_t kCapacity = size_t(64) << 20;
    static constexpr size_t kChunk = size_t(16) << 20;

    void upload(void* dst, const void* src, size_t bytes) {
        Device& d = require_device();
        std::lock_guard<std::mutex> lock(mu_);
        if (!base_) check_hip(hipHostMalloc(reinterpret_cast<void**>(&base_), kCapacity, hipHostMallocDefault),
                              "hipHostMalloc (staging ring)");
        const char* s = static_cast<const char*>(src);
        char* t = static_cast<char*>(dst);
        while (bytes) {
            const size_t n = std::min(bytes, kChunk);
            char* slot = reserve(n);
            std::memcpy(slot, s, n);
            check_hip(hipMemcpyAsync(t, slot, n, hipMemcpyHostToDevice, d.stream), "hipMemcpyAsync (upload)");
            hipEvent_t ev = take_event();
            check_hip(hipEventRecord(ev, d.stream), "hipEventRecord");
            inflight_.push_back(Segment{static_cast<size_t>(slot - base_), static_cast<size_t>(slot - base_) + n, ev});
            s += n;
            t += n;
            bytes -= n;
        }
    }

    // Everything enqueued so far has completed: all slots are free again.
    void on_synchronized() {
        std::lock_guard<std::mutex> lock(mu_);
        for (auto& seg : inflight_) spare_.push_back(seg.event);
        inflight_.clear();
    }

private:
    struct Segment {
        size_t begin, end;
        hipEvent_t event;
    };

    char* reserve(size_t n) {
        if (head_ + n > kCapacity) head_ = 0;
        const size_t b = head_, e = head_ + n;
        for (auto it = inflight_.begin(); it != inflight_.end();) {
            if (it->begin < e && b < it->end) {
                check_hip(hipEventSynchronize(it->event), "hipEventSynchronize (staging)");
                spare_.push_back(it->event);
                it = inflight_.erase(it);
            } else {
                ++it;
            }
        }
        head_ = e;
        return base_ + b;
    }

    hipEvent_t take_event() {
        if (!spare_.empty()) {
            hipEvent_t ev = spare_.back();
            spare_.pop_back();
            return ev;
        }
        hipEvent_t ev;
        check_hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "hipEventCreate");
        return ev;
    }

    std::mutex mu_;
    char* base_ = nullptr;
    size_t head_ = 0;
    std::deque<Segment> inflight_;
    std::vector<hipEvent_t> spare_;
};

Staging& staging() {
    static Staging s;
    return s;
}

// ---- scalar mirrors ---------------------------------------------------------------
// A one-element device value copied, in stream order, into a pinned host slot by
// a one-thread kernel whose dispatch carries a completion event. Reading the
// value waits for that event only, not for the work enqueued after it.

__global__ void mirror_kernel(const float* __restrict__ src, float* __restrict__ dst) {
    if (threadIdx.x == 0) dst[0] = src[0];
}

class Mirrors {
public:
    vc_hip_mirror* take() {
        std::lock_guard<std::mutex> lock(mu_);
        if (free_.empty()) grow();
        vc_hip_mirror* m = free_.back();
        free_.pop_back();
        return m;
    }
    void give(vc_hip_mirror* m) {
        std::lock_guard<std::mutex> lock(mu_);
        free_.push_back(m);
    }

private:
    static constexpr size_t kSlots = 256;
    void grow() {
        float* slab = nullptr;
        check_hip(hipHostMalloc(reinterpret_cast<void**>(&slab), kSlots * sizeof(float), hipHostMallocDefault),
                  "hipHostMalloc (scalar mirrors)");
        auto block = std::make_unique<vc_hip_mirror[]>(kSlots);
        for (size_t i = 0; i < kSlots; ++i) {
            block[i].host = slab + i;
            check_hip(hipEventCreate(&block[i].done), "hipEventCreate");
            free_.push_back(&block[i]);
        }
        blocks_.push_back(std::move(block));  // slots and events live until the process ends
    }

    std::mutex mu_;
    std::vector<vc_hip_mirror*> free_;
    std::vector<std::unique_ptr<vc_hip_mirror[]>> blocks_;
};

Mirrors& mirrors() {
    static Mirrors m;
    return m;
}

}  // namespace

vc_hip_mirror* take_mirror() { return mirrors().take(); }

void give_mirror(vc_hip_mirror* m) noexcept {
    try {
        mirrors().give(m);
    } catch (...) {  // a slot that cannot be listed again stays unused
    }
}

void launch_mirror(vc_hip_mirror* m, const float* device_value) {
    hipExtLaunchKernelGGL(mirror_kernel, dim3(1), dim3(64), 0, device().stream, nullptr, m->done, 0u, device_value,
                          m->host);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) fail(VC_HIP_ERR_RUNTIME, std::string("launch of mirror_kernel failed: ") + hipGetErrorString(e));
}

namespace {

// ---- profiler -----------------------------------------------------------------

struct ProfRecord {
    int label;
    hipEvent_t start, stop;
    double flops, bytes;
};

struct ProfAggregate {
    std::string label;
    uint64_t launches = 0;
    double ms = 0, flops = 0, bytes = 0;
};

struct Profiler {
    std::mutex mu;
    bool enabled = false;
    std::vector<std::string> only;  // empty: every label
    std::vector<std::string> labels;
    std::unordered_map<std::string, int> ids;
    std::vector<ProfRecord> done;
    std::vector<hipEvent_t> spare;
    std::vector<ProfAggregate> summary;

    hipEvent_t event() {
        if (!spare.empty()) {
            hipEvent_t e = spare.back();
            spare.pop_back();
            return e;
        }
        hipEvent_t e;
        check_hip(hipEventCreate(&e), "hipEventCreate");
        return e;
    }
};

Profiler& profiler() {
    static Profiler p;
    return p;
}

}  // namespace

void set_last_error(const std::string& message) { t_last_error = message; }

void* pool_alloc(size_t bytes) { return pool().alloc(bytes ? bytes : 4); }

void pool_release(void* p) noexcept {
    try {
        pool().release(p);
    } catch (...) {
    }
}

const char* gemm_mode_name(int mode) {
    switch (mode) {
        case kGemmSimple: return "simple";
        case kGemmTiles128: return "mfma128";
        case kGemmTiles256: return "mfma256";
        case kGemmTiles256x128: return "mfma256x128";
        default: return "mfma";
    }
}

Device& device() {
    static std::once_flag once;
    Device& d = device_singleton();
    std::call_once(once, [&] { init_device(d); });
    if (d.ready) {
        thread_local bool current = false;
        if (!current) {
            (void)hipSetDevice(d.ordinal);
            current = true;
        }
    }
    return d;
}

Device& require_device() {
    Device& d = device();
    if (!d.ready) fail(VC_HIP_ERR_UNAVAILABLE, "HIP backend unavailable: " + d.error);
    return d;
}

void after_launch(const char* label) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) fail(VC_HIP_ERR_RUNTIME, std::string("launch of ") + label + " failed: " + hipGetErrorString(e));
    Device& d = device();
    if (d.sync_each_launch) {
        e = hipStreamSynchronize(d.stream);
        if (e != hipSuccess) fail(VC_HIP_ERR_RUNTIME, std::string(label) + " failed on the device: " + hipGetErrorString(e));
    }
}

namespace {
thread_local Profiled* t_profiled = nullptr;
}

Profiled* Profiled::current() { return t_profiled; }

Profiled::Profiled(const char* label, double flops, double bytes) {
    outer_ = t_profiled;
    t_profiled = this;
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    if (!p.enabled) return;
    if (!p.only.empty() && std::find(p.only.begin(), p.only.end(), label) == p.only.end()) return;
    auto it = p.ids.find(label);
    if (it == p.ids.end()) {
        label_ = static_cast<int>(p.labels.size());
        p.labels.emplace_back(label);
        p.ids.emplace(label, label_);
    } else {
        label_ = it->second;
    }
    start_ = p.event();
    stop_ = p.event();
    flops_ = flops;
    bytes_ = bytes;
}

Profiled::~Profiled() {
    if (!popped_) t_profiled = outer_;
    if (label_ >= 0) {  // abandoned (an error before done()): return the events unused
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        p.spare.push_back(start_);
        p.spare.push_back(stop_);
    }
}

void Profiled::done() {
    if (!popped_) {
        t_profiled = outer_;
        popped_ = true;
    }
    if (label_ < 0) return;
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    if (started_) {
        p.done.push_back(ProfRecord{label_, start_, stop_, flops_, bytes_});
    } else {
        p.spare.push_back(start_);
        p.spare.push_back(stop_);
    }
    label_ = -1;
}

Bcast make_bcast(const size_t* a_shape, const size_t* a_strides, size_t a_rank, const size_t* b_shape,
                 const size_t* b_strides, size_t b_rank, const size_t* out_shape, size_t out_rank) {
    if (out_rank > kMaxRank || a_rank > kMaxRank || b_rank > kMaxRank)
        fail(VC_HIP_ERR_INVALID_ARGUMENT, "HIP broadcasting supports at most 8 dimensions");
    if (a_rank > out_rank || b_rank > out_rank) fail(VC_HIP_ERR_INVALID_ARGUMENT, "operand rank exceeds output rank");
    int64_t shp[kMaxRank], sa[kMaxRank], sb[kMaxRank];
    int r = 0;
    for (size_t ax = 0; ax < out_rank; ++ax) {
        const int64_t od = static_cast<int64_t>(out_shape[ax]);
        int64_t as = 0, bs = 0;
        if (ax >= out_rank - a_rank) {
            const size_t i = ax - (out_rank - a_rank);
            if (a_shape[i] != 1) {
                if (a_shape[i] != out_shape[ax]) fail(VC_HIP_ERR_INVALID_ARGUMENT, "operand does not broadcast to the output shape");
                as = static_cast<int64_t>(a_strides[i]);
            }
        }
        if (ax >= out_rank - b_rank) {
            const size_t i = ax - (out_rank - b_rank);
            if (b_shape[i] != 1) {
                if (b_shape[i] != out_shape[ax]) fail(VC_HIP_ERR_INVALID_ARGUMENT, "operand does not broadcast to the output shape");
                bs = static_cast<int64_t>(b_strides[i]);
            }
        }
        if (od == 1) continue;  // size-1 output axes carry no index
        shp[r] = od;
        sa[r] = as;
        sb[r] = bs;
        ++r;
    }
    Bcast m{};
    if (r == 0) {
        m.rank = 1;
        m.out_shape[0] = 1;
        m.a_stride[0] = 0;
        m.b_stride[0] = 0;
        return m;
    }
    // Merge an axis into the next inner one when both operands continue
    // contiguously across the boundary (or both stay broadcast).
    int64_t cs[kMaxRank], ca[kMaxRank], cb[kMaxRank];
    int n = 0;
    cs[0] = shp[r - 1];
    ca[0] = sa[r - 1];
    cb[0] = sb[r - 1];
    n = 1;
    for (int ax = r - 2; ax >= 0; --ax) {
        const int64_t inner = cs[n - 1];
        if (sa[ax] == ca[n - 1] * inner && sb[ax] == cb[n - 1] * inner) {
            cs[n - 1] *= shp[ax];
        } else {
            cs[n] = shp[ax];
            ca[n] = sa[ax];
            cb[n] = sb[ax];
            ++n;
        }
    }
    m.rank = n;
    for (int i = 0; i < n; ++i) {  // back to outermost-first order
        m.out_shape[i] = cs[n - 1 - i];
        m.a_stride[i] = ca[n - 1 - i];
        m.b_stride[i] = cb[n - 1 - i];
    }
    return m;
}

}  // namespace vchip

using namespace vchip;

extern "C" {

int vc_hip_available(void) { return device().ready ? 1 : 0; }

const char* vc_hip_device_name(void) {
    Device& d = device();
    return d.ready ? d.name.c_str() : "unavailable";
}

const char* vc_hip_last_error(void) {
    if (!t_last_error.empty()) return t_last_error.c_str();
    Device& d = device();
    return d.ready ? "" : d.error.c_str();
}

const char* vc_hip_gemm_kernel(void) {
    Device& d = device();
    if (!d.ready) return "unavailable";
    return gemm_mode_name(d.gemm_mode.load());
}

int vc_hip_set_gemm_kernel(const char* name) {
    return guard([&] {
        Device& d = require_device();
        for (int mode : {kGemmAuto, kGemmSimple, kGemmTiles128, kGemmTiles256, kGemmTiles256x128})
            if (name && std::strcmp(name, gemm_mode_name(mode)) == 0) {
                d.gemm_mode = mode;
                return;
            }
        fail(VC_HIP_ERR_INVALID_ARGUMENT, std::string("unknown GEMM kernel '") + (name ? name : "(null)") +
                                              "': expected \"mfma\", \"simple\", \"mfma128\", \"mfma256\" or "
                                              "\"mfma256x128\"");
    });
}

int vc_hip_alloc(size_t bytes, void** out) {
    return guard([&] {
        if (!out) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_alloc: null output pointer");
        *out = pool().alloc(bytes ? bytes : 4);
    });
}

int vc_hip_release(void* buffer) {
    return guard([&] { pool().release(buffer); });
}

int vc_hip_upload(void* dst, const void* src, size_t bytes) {
    return guard([&] {
        if (bytes == 0) return;
        if (!dst || !src) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_upload: null pointer");
        staging().upload(dst, src, bytes);
    });
}

int vc_hip_download(void* dst, const void* src, size_t bytes) {
    return guard([&] {
        Device& d = require_device();
        if (bytes) {
            if (!dst || !src) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_download: null pointer");
            check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, d.stream), "hipMemcpyAsync (download)");
        }
        check_hip(hipStreamSynchronize(d.stream), "HIP command failed");
        staging().on_synchronized();
    });
}

int vc_hip_mirror_scalar(const float* device_value, vc_hip_mirror** out) {
    return guard([&] {
        Device& d = require_device();
        if (!device_value || !out) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_mirror_scalar: null pointer");
        vc_hip_mirror* m = take_mirror();
        try {
            launch_mirror(m, device_value);
        } catch (...) {
            give_mirror(m);
            throw;
        }
        *out = m;
    });
}

int vc_hip_mirror_read(vc_hip_mirror* mirror, float* value) {
    return guard([&] {
        if (!mirror || !value) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_mirror_read: null pointer");
        check_hip(hipEventSynchronize(mirror->done), "HIP command failed");
        // Report an error the stream has already recorded (work enqueued
        // before this point that failed), without waiting for the rest.
        const hipError_t state = hipStreamQuery(device().stream);
        if (state != hipSuccess && state != hipErrorNotReady) check_hip(state, "HIP command failed");
        *value = *static_cast<volatile float*>(mirror->host);
    });
}

int vc_hip_mirror_release(vc_hip_mirror* mirror) {
    return guard([&] {
        if (mirror) mirrors().give(mirror);
    });
}

int vc_hip_copy(void* dst, const void* src, size_t bytes) {
    return guard([&] {
        Device& d = require_device();
        if (bytes == 0) return;
        check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, d.stream), "hipMemcpyAsync (device copy)");
    });
}

int vc_hip_synchronize(void) {
    return guard([&] {
        Device& d = device();
        if (!d.ready) return;  // like the reference: a no-op without a device
        check_hip(hipStreamSynchronize(d.stream), "HIP command failed");
        staging().on_synchronized();
    });
}

int vc_hip_stream_idle(int* idle) {
    return guard([&] {
        if (!idle) fail(VC_HIP_ERR_INVALID_ARGUMENT, "vc_hip_stream_idle: null pointer");
        Device& d = device();
        if (!d.ready) {
            *idle = 1;
            return;
        }
        const hipError_t state = hipStreamQuery(d.stream);
        if (state != hipSuccess && state != hipErrorNotReady) check_hip(state, "HIP command failed");
        *idle = state == hipSuccess ? 1 : 0;
    });
}

int vc_hip_pool_stats_get(vc_hip_pool_stats* out) {
    return guard([&] {
        if (!out) fail(VC_HIP_ERR_INVALID_ARGUMENT, "null stats pointer");
        *out = pool().stats();
    });
}

int vc_hip_pool_trim(void) {
    return guard([&] { pool().trim(); });
}

int vc_hip_profile_enable(int enable) {
    return guard([&] {
        require_device();
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        p.enabled = enable != 0;
    });
}

int vc_hip_profile_labels(const char* labels) {
    return guard([&] {
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        p.only.clear();
        if (!labels) return;
        std::string item;
        for (const char* c = labels;; ++c) {
            if (*c == ',' || *c == '\0') {
                if (!item.empty()) p.only.push_back(item);
                item.clear();
                if (*c == '\0') break;
            } else if (*c != ' ') {
                item.push_back(*c);
            }
        }
    });
}

int vc_hip_profile_reset(void) {
    return guard([&] {
        Device& d = require_device();
        check_hip(hipStreamSynchronize(d.stream), "HIP command failed");
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        for (auto& r : p.done) {
            p.spare.push_back(r.start);
            p.spare.push_back(r.stop);
        }
        p.done.clear();
        p.summary.clear();
    });
}

int vc_hip_profile_count(size_t* labels) {
    return guard([&] {
        Device& d = require_device();
        check_hip(hipStreamSynchronize(d.stream), "HIP command failed");
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        p.summary.assign(p.labels.size(), ProfAggregate{});
        for (size_t i = 0; i < p.labels.size(); ++i) p.summary[i].label = p.labels[i];
        for (const auto& r : p.done) {
            float ms = 0;
            check_hip(hipEventElapsedTime(&ms, r.start, r.stop), "hipEventElapsedTime");
            auto& s = p.summary[r.label];
            s.launches += 1;
            s.ms += ms;
            s.flops += r.flops;
            s.bytes += r.bytes;
        }
        *labels = p.summary.size();
    });
}

int vc_hip_profile_entry(size_t i, const char** label, uint64_t* launches, double* milliseconds, double* flops,
                         double* bytes) {
    return guard([&] {
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        if (i >= p.summary.size()) fail(VC_HIP_ERR_OUT_OF_RANGE, "profile entry index out of range");
        const auto& s = p.summary[i];
        *label = s.label.c_str();
        *launches = s.launches;
        *milliseconds = s.ms;
        *flops = s.flops;
        *bytes = s.bytes;
    });
}

}  // extern "C"
