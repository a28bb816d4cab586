// Cumulative prefix-cache and copy-on-write work counters; durations only
// when timing is enabled (reference: miniprefix/include/miniprefix/cost_stats.h:6-17).
#pragma once
#include <chrono>
#include <cstdint>

namespace miniprefix {

struct CostStats {
    std::uint64_t lookup_calls = 0, lookup_ns = 0, publish_calls = 0, publish_ns = 0;
    std::uint64_t cow_pages = 0, cow_bytes = 0, cow_copy_ns = 0, cow_timed_copies = 0;
};

// Adds the elapsed steady-clock nanoseconds to `total` on destruction when
// enabled; does nothing otherwise.
class CostTimer {
public:
    CostTimer(bool enabled, std::uint64_t& total) : total_(enabled ? &total : nullptr) {
        if (total_) start_ = std::chrono::steady_clock::now();
    }
    ~CostTimer() {
        if (total_)
            *total_ += static_cast<std::uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                                      std::chrono::steady_clock::now() - start_)
                                                      .count());
    }
    CostTimer(const CostTimer&) = delete;
    CostTimer& operator=(const CostTimer&) = delete;

private:
    std::uint64_t* total_;
    std::chrono::steady_clock::time_point start_;
};

}  // namespace miniprefix
