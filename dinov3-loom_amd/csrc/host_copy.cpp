// Host-side copies of the pipelined forward; see host_copy.hpp.
#include "host_copy.hpp"

#include <algorithm>
#include <cstring>
#include <vector>

namespace dhx {

void parallel_copy(void* dst, const void* src, uint64_t n) noexcept {
    constexpr uint64_t kChunk = 4ull << 20;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned threads = (unsigned)std::min<uint64_t>(std::min(16u, hw), (n + kChunk - 1) / kChunk);
    if (threads <= 1) {
        if (n) std::memcpy(dst, src, n);
        return;
    }
    // Never throws: a thread that cannot be started leaves its part (and the
    // parts after it) to the calling thread.
    std::vector<std::thread> pool;
    const uint64_t per = (n + threads - 1) / threads;
    uint64_t handed = 0;  // bytes [0, handed) belong to started threads
    try {
        pool.reserve(threads);
        for (unsigned t = 0; t < threads; ++t) {
            const uint64_t a = t * per, b = std::min(n, a + per);
            if (a >= b) break;
            pool.emplace_back([=] { std::memcpy(static_cast<char*>(dst) + a, static_cast<const char*>(src) + a, b - a); });
            handed = b;
        }
    } catch (...) {
    }
    if (handed < n) std::memcpy(static_cast<char*>(dst) + handed, static_cast<const char*>(src) + handed, n - handed);
    for (auto& th : pool) th.join();
}

Copier::Copier(bool threaded) {
    if (threaded) worker_ = std::thread([this] { run(); });
}

Copier::~Copier() {
    if (!worker_.joinable()) return;
    {
        std::lock_guard<std::mutex> lock(m_);
        stop_ = true;
    }
    work_.notify_all();
    worker_.join();
}

uint64_t Copier::submit(void* dst, const void* src, uint64_t n) {
    std::lock_guard<std::mutex> lock(m_);
    if (!worker_.joinable()) {
        parallel_copy(dst, src, n);
        ++done_;
        return submitted_++;
    }
    jobs_.push_back(Job{dst, src, n});
    work_.notify_all();
    return submitted_++;
}

void Copier::wait(uint64_t ticket) {
    std::unique_lock<std::mutex> lock(m_);
    done_cv_.wait(lock, [&] { return done_ > ticket; });
}

void Copier::run() {
    std::unique_lock<std::mutex> lock(m_);
    for (;;) {
        work_.wait(lock, [&] { return stop_ || !jobs_.empty(); });
        if (jobs_.empty()) return;  // stopping, nothing left
        const Job j = jobs_.front();
        jobs_.pop_front();
        lock.unlock();
        parallel_copy(j.dst, j.src, j.n);
        lock.lock();
        ++done_;
        done_cv_.notify_all();
    }
}

}  // namespace dhx
