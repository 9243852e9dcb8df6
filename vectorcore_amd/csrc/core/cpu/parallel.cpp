#include "parallel.hpp"

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <condition_variable>
#include <exception>
#include <mutex>
#include <thread>
#include <vector>

namespace vectorcore::cpu {

namespace {

thread_local bool t_in_body = false;

// Workers sleep until a job is posted; the posting thread works too. Chunks
// are claimed from an atomic counter.
class Workers {
public:
    Workers() {
        const unsigned n = std::max(1U, std::thread::hardware_concurrency());
        for (unsigned i = 1; i < n; ++i) threads_.emplace_back([this] { loop(); });
    }
    ~Workers() {
        {
            std::lock_guard<std::mutex> g(m_);
            quit_ = true;
        }
        cv_.notify_all();
        for (auto& t : threads_) t.join();
    }
    std::size_t size() const { return threads_.size() + 1; }

    void run(std::size_t count, std::size_t grain, const std::function<void(std::size_t, std::size_t)>& body) {
        std::lock_guard<std::mutex> one_job(job_);
        {
            std::lock_guard<std::mutex> g(m_);
            body_ = &body;
            count_ = count;
            grain_ = grain;
            chunks_ = (count + grain - 1) / grain;
            next_.store(0);
            busy_ = threads_.size();
            error_ = nullptr;
            ++epoch_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> g(m_);
        done_cv_.wait(g, [&] { return busy_ == 0; });
        body_ = nullptr;
        if (error_) std::rethrow_exception(error_);
    }

private:
    void work() {
        const bool outer = t_in_body;
        t_in_body = true;
        for (std::size_t c; (c = next_.fetch_add(1)) < chunks_;) {
            try {
                (*body_)(c * grain_, std::min(count_, (c + 1) * grain_));
            } catch (...) {
                std::lock_guard<std::mutex> g(m_);
                if (!error_) error_ = std::current_exception();
                next_.store(chunks_);
            }
        }
        t_in_body = outer;
    }
    void loop() {
        std::uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> g(m_);
                cv_.wait(g, [&] { return quit_ || epoch_ != seen; });
                if (quit_) return;
                seen = epoch_;
            }
            work();
            {
                std::lock_guard<std::mutex> g(m_);
                --busy_;
            }
            done_cv_.notify_one();
        }
    }

    std::vector<std::thread> threads_;
    std::mutex job_, m_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(std::size_t, std::size_t)>* body_ = nullptr;
    std::size_t count_ = 0, grain_ = 1, chunks_ = 0, busy_ = 0;
    std::atomic<std::size_t> next_{0};
    std::uint64_t epoch_ = 0;
    bool quit_ = false;
    std::exception_ptr error_;
};

Workers& workers() {
    static Workers w;
    return w;
}

}  // namespace

void parallel_for(std::size_t count, std::size_t grain, const std::function<void(std::size_t, std::size_t)>& body) {
    if (count == 0) return;
    grain = std::max<std::size_t>(grain, 1);
    if (count <= grain || t_in_body || workers().size() == 1) {
        for (std::size_t b = 0; b < count; b += grain) body(b, std::min(count, b + grain));
        return;
    }
    workers().run(count, grain, body);
}

}  // namespace vectorcore::cpu
