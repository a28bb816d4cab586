// Admission and the stable decode-first order of one iteration (reference:
// miniprefix/include/miniprefix/scheduler.h:6-32).
#pragma once
#include <cstddef>
#include <vector>

namespace miniprefix {

enum class SchedulePhase { Prefill, Decode };
struct ScheduledRequest {
    std::size_t active_index;
    SchedulePhase phase;
};
struct SchedulerConfig {
    int max_batch_size = 2, token_budget = 32, prefill_chunk = 16;
};

class SchedulePlan {
    friend class Scheduler;
    SchedulePlan(const std::vector<SchedulePhase>& phases, const SchedulerConfig& config);

public:
    const std::vector<ScheduledRequest>& order() const { return order_; }
    bool has_budget() const { return remaining_ != 0; }
    // Input length for the next request of the order: one token to decode, or
    // a prefill chunk bounded by the remaining budget.
    std::size_t take_input(SchedulePhase phase, std::size_t unprefilled_tokens);

private:
    std::vector<ScheduledRequest> order_;
    std::size_t remaining_, chunk_;
};

class Scheduler {
public:
    explicit Scheduler(SchedulerConfig config);
    std::size_t admission_count(std::size_t active, std::size_t waiting) const;
    SchedulePlan plan(const std::vector<SchedulePhase>& active_phases) const {
        return SchedulePlan(active_phases, config_);
    }

private:
    SchedulerConfig config_;
};

}  // namespace miniprefix
