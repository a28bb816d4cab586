// Request lifecycle over a ModelRunner (reference interface:
// miniprefix/include/miniprefix/engine.h:8-36). When the runner also
// implements StagedRunner, a step's appends go to the device as batches;
// the KV metadata sequence and the emitted events are those of the
// per-request loop.
#pragma once
#include "model.h"
#include "scheduler.h"
#include <deque>
#include <set>

namespace miniprefix {

struct EngineConfig {
    int max_batch_size = 2, token_budget = 32, prefill_chunk = 16, context = 512;
};
struct EngineStepStats {
    std::size_t prefix_reused_tokens = 0, prefill_tokens = 0, decode_tokens = 0;
};

class Engine {
public:
    Engine(std::unique_ptr<ModelRunner>, EngineConfig);
    ~Engine();
    void submit(Request);
    bool step();
    std::vector<GenerationEvent> poll_events();
    void cancel(const RequestId&);
    void shutdown();
    bool idle() const { return jobs_.empty(); }
    bool failed() const { return failed_; }
    ModelRunner& runner() { return *runner_; }
    const EngineStepStats& last_step_stats() const { return step_stats_; }
    // Batched stepping can be turned off to run the reference's per-request loop.
    void set_batching(bool enabled) { batching_ = enabled; }

private:
    struct Job {
        Request request;
        std::size_t prefilled = 0;  // prompt tokens with committed KV
        std::vector<TokenId> output;
        bool admitted = false, resident = false, finished = false;
    };
    class Executor;
    enum class Cleanup { Release, RunnerOwned };

    bool admit();
    void execute(SchedulePlan& plan);
    void restore_prefix(Job& job);
    void finish(Job& job, FinishReason reason, std::optional<TokenId> token = std::nullopt,
                const std::string& error = "", Cleanup cleanup = Cleanup::Release);
    void emit_token(Job& job, TokenId token);
    void account(Job& job, std::size_t tokens, bool prefill);
    void drop_finished();
    void fail_all(const std::string& message);

    std::unique_ptr<ModelRunner> runner_;
    EngineConfig config_;
    Scheduler scheduler_;
    // Unfinished requests in submission order. Admission takes the oldest
    // waiting request, so the admitted ones are always the first `admitted_`.
    std::deque<Job> jobs_;
    std::size_t admitted_ = 0;
    std::set<RequestId> seen_;
    std::vector<GenerationEvent> events_;
    bool failed_ = false;
    bool batching_ = true;
    EngineStepStats step_stats_;
};

}  // namespace miniprefix
