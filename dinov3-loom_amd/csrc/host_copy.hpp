// Host-side copies of the pipelined forward (Model::forward): a memcpy split
// over host threads, and a copier thread that runs such copies one after
// another in the order they are submitted. Host code only, with no HIP
// calls, so it also builds on its own for the thread-sanitizer test
// (tests/host_copy_check.cpp).
#pragma once
#include <condition_variable>
#include <cstdint>
#include <deque>
#include <mutex>
#include <thread>

namespace dhx {

// memcpy split over up to 16 host threads; never throws (what no thread can
// be started for is copied on the calling thread).
void parallel_copy(void* dst, const void* src, uint64_t n) noexcept;

// Copies between pageable and pinned memory, run on a thread of their own in
// submission order. It never calls the HIP runtime: HIP calls from another
// thread beside a graph launch were measured to slow the launch down, so the
// thread that launches keeps every HIP call and hands the copies over.
class Copier {
public:
    // threaded = false: submit() copies at once on the calling thread (one
    // chunk has nothing to overlap, and a thread would only add its start).
    explicit Copier(bool threaded);
    // Runs every queued copy before returning: their buffers outlive the
    // caller's scope, also when the caller is unwinding an exception.
    ~Copier();
    Copier(const Copier&) = delete;
    Copier& operator=(const Copier&) = delete;

    // Queues dst <- src (n bytes); returns the copy's ticket (0, 1, 2, ...).
    uint64_t submit(void* dst, const void* src, uint64_t n);
    // Waits until the copy with this ticket (and every earlier one) is done.
    void wait(uint64_t ticket);

private:
    struct Job {
        void* dst;
        const void* src;
        uint64_t n;
    };
    void run();
    std::mutex m_;
    std::condition_variable work_, done_cv_;
    std::deque<Job> jobs_;
    uint64_t submitted_ = 0, done_ = 0;
    bool stop_ = false;
    std::thread worker_;  // started (if threaded) in the constructor's body, once the members above exist
};

}  // namespace dhx
