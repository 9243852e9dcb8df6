#include "parallel.hpp"

// A job queue served by a fixed set of worker threads.
//
// Each parallel_for call posts one Job (it lives on the caller's stack) to
// the queue and then helps run it. Any idle worker that finds the job at the
// head of the queue joins in. Chunks are claimed one at a time from the job's
// counter, so the chunk boundaries are those of the serial loop whatever the
// number of threads. The caller returns once every chunk has finished and no
// worker still holds the job; the pool lock guards both the queue and each
// job's count of workers inside it. Several threads may run jobs at once: the
// queue serves them in posting order.
//
// Errors: every chunk runs even when one throws, and the caller rethrows the
// exception of the lowest-numbered chunk that threw, so the error a caller
// sees does not depend on thread timing either.

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <exception>
#include <limits>
#include <mutex>
#include <thread>
#include <vector>

namespace vectorcore::cpu {

namespace {

using Body = std::function<void(std::size_t, std::size_t)>;

// Nonzero while this thread executes a chunk body: a nested parallel_for
// then runs inline instead of waiting on workers that may all be busy.
thread_local int t_chunk_depth = 0;

class Job {
public:
    Job(const Body& body, std::size_t count, std::size_t grain)
        : body_(body), count_(count), grain_(grain), chunks_((count + grain - 1) / grain) {}

    // Claims and runs chunks until none is left.
    void help() {
        ++t_chunk_depth;
        for (std::size_t c = claim_.fetch_add(1, std::memory_order_relaxed); c < chunks_;
             c = claim_.fetch_add(1, std::memory_order_relaxed)) {
            const std::size_t begin = c * grain_;
            try {
                body_(begin, std::min(count_, begin + grain_));
            } catch (...) {
                record_failure(c, std::current_exception());
            }
            finished_.fetch_add(1, std::memory_order_acq_rel);
        }
        --t_chunk_depth;
    }

    [[nodiscard]] bool unclaimed_left() const { return claim_.load(std::memory_order_relaxed) < chunks_; }
    [[nodiscard]] bool all_finished() const { return finished_.load(std::memory_order_acquire) == chunks_; }

    void rethrow_first_failure() {
        std::lock_guard<std::mutex> lock(failure_mutex_);
        if (failure_) std::rethrow_exception(failure_);
    }

    int helpers = 0;  // workers inside help(); guarded by the pool lock

private:
    void record_failure(std::size_t chunk, std::exception_ptr e) {
        std::lock_guard<std::mutex> lock(failure_mutex_);
        if (chunk < failed_chunk_) {
            failed_chunk_ = chunk;
            failure_ = std::move(e);
        }
    }

    const Body& body_;
    const std::size_t count_, grain_, chunks_;
    std::atomic<std::size_t> claim_{0};
    std::atomic<std::size_t> finished_{0};
    std::mutex failure_mutex_;
    std::size_t failed_chunk_ = std::numeric_limits<std::size_t>::max();
    std::exception_ptr failure_;
};

class Pool {
public:
    Pool() {
        const unsigned threads = std::max(1U, std::thread::hardware_concurrency());
        for (unsigned t = 1; t < threads; ++t) workers_.emplace_back([this] { serve(); });
    }

    ~Pool() {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            closing_ = true;
        }
        posted_.notify_all();
        for (auto& w : workers_) w.join();
    }

    [[nodiscard]] std::size_t threads() const { return workers_.size() + 1; }

    void run(Job& job) {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            queue_.push_back(&job);
        }
        posted_.notify_all();
        job.help();
        {
            std::unique_lock<std::mutex> lock(mutex_);
            finished_.wait(lock, [&] { return job.all_finished() && job.helpers == 0; });
            // Nobody can pick the job up any more once it leaves the queue.
            auto it = std::find(queue_.begin(), queue_.end(), &job);
            if (it != queue_.end()) queue_.erase(it);
        }
        job.rethrow_first_failure();
    }

private:
    void serve() {
        std::unique_lock<std::mutex> lock(mutex_);
        for (;;) {
            posted_.wait(lock, [&] { return closing_ || !queue_.empty(); });
            if (closing_) return;
            Job* job = queue_.front();
            if (!job->unclaimed_left()) {  // its remaining chunks are already running
                queue_.pop_front();
                continue;
            }
            ++job->helpers;
            lock.unlock();
            job->help();
            lock.lock();
            --job->helpers;
            finished_.notify_all();
        }
    }

    std::vector<std::thread> workers_;
    std::mutex mutex_;
    std::condition_variable posted_;    // a job was queued, or the pool closes
    std::condition_variable finished_;  // a worker left a job
    std::deque<Job*> queue_;
    bool closing_ = false;
};

Pool& pool() {
    static Pool p;
    return p;
}

}  // namespace

void parallel_for(std::size_t count, std::size_t grain, const Body& body) {
    if (count == 0) return;
    grain = std::max<std::size_t>(grain, 1);
    if (count <= grain || t_chunk_depth > 0 || pool().threads() == 1) {
        for (std::size_t begin = 0; begin < count; begin += grain) body(begin, std::min(count, begin + grain));
        return;
    }
    Job job(body, count, grain);
    pool().run(job);
}

}  // namespace vectorcore::cpu
