// Engine with the observable behaviour of the reference
// (miniprefix/src/engine/engine.cpp:13-140): the same admission, order of
// runner calls, events, error messages and failure handling.
//
// Design: one queue of unfinished jobs in submission order, whose first
// `admitted_` entries are the admitted ones, and one executor that carries
// out a step's appends in plan order. The executor either appends each
// request at once (ModelRunner::append, the reference's loop) or, with a
// StagedRunner and batching on, stages the appends and runs them as device
// batches. A batch is run early when a later append must observe its
// effects:
//  - sampling a job that may finish releases its pages, which the next
//    append's reservation must see (the per-request loop releases them
//    before the next append);
//  - a job that maps cached pages written by a queued forward (a prefix
//    published earlier in the same step) must not read or copy them before
//    that forward has written them.
#include "miniprefix/engine.h"

#include "staged_runner.h"

#include <algorithm>
#include <cmath>

namespace miniprefix {
namespace {

SchedulerConfig scheduler_config(const EngineConfig& c) {
    if (c.max_batch_size < 1 || c.token_budget < 1 || c.prefill_chunk < 1)
        throw std::invalid_argument("invalid engine configuration");
    return {c.max_batch_size, c.token_budget, c.prefill_chunk};
}

TokenId greedy(const std::vector<float>& logits) {
    return static_cast<TokenId>(std::max_element(logits.begin(), logits.end()) - logits.begin());
}

}  // namespace

class Engine::Executor {
public:
    explicit Executor(Engine& engine)
        : engine_(engine),
          staged_(engine.batching_ ? dynamic_cast<StagedRunner*>(engine.runner_.get()) : nullptr) {}
    ~Executor() {
        if (staged_ && !queue_.empty()) staged_->discard_staged();  // unwinding
    }

    // After `job` mapped cached pages: they may hold tokens a queued forward
    // has not written yet.
    void mapped(const Job& job) {
        if (staged_ && !queue_.empty() && staged_->shares_staged_pages(job.request.id)) run_queue();
    }

    void append(Job& job, const std::vector<TokenId>& input, bool prefill) {
        ModelRunner& runner = *engine_.runner_;
        const RequestId& id = job.request.id;
        if (staged_) {
            // A queued item that may finish in this step (EOS possible, or
            // its last token) releases its sequence when the queue runs. In
            // the per-request order that release precedes every later append
            // of the step; it changes what a later append gets only if that
            // append takes pages from the pool or publishes into a prefix
            // cache, so only such an append runs the queue first.
            const bool samples =
                !prefill || job.prefilled + input.size() >= job.request.prompt_token_ids.size();
            if (may_release_ && staged_->stage_touches_pool(id, input.size(), samples)) run_queue();
            staged_->stage(id, input);
            engine_.account(job, input.size(), prefill);
            queue_.push_back({&job, samples});
            if (!samples) return;
            runner.cache_prefix(id);
            if (may_finish(job)) may_release_ = true;
            return;
        }
        const std::vector<float> logits = runner.append(id, input);
        engine_.account(job, input.size(), prefill);
        if (!prompt_done(job)) return;
        if (logits.size() != static_cast<std::size_t>(runner.config().vocabulary))
            throw std::runtime_error("invalid logits arity");
        for (const float v : logits)
            if (!std::isfinite(v)) throw std::runtime_error("nonfinite model result");
        // Publish the committed history before sampling: the sampled token has no KV yet.
        runner.cache_prefix(id);
        engine_.emit_token(job, greedy(logits));
    }

    void run_queue() {
        may_release_ = false;  // the queue's finishes release in order below
        if (queue_.empty()) return;
        const std::vector<StagedResult> results = staged_->run_staged();
        std::vector<Queued> batch;
        batch.swap(queue_);
        if (results.size() != batch.size()) throw std::runtime_error("invalid staged result count");
        for (std::size_t i = 0; i < batch.size(); ++i) {
            if (!results[i].finite) throw std::runtime_error("nonfinite model result");
            if (batch[i].samples) engine_.emit_token(*batch[i].job, results[i].argmax);
        }
    }

private:
    struct Queued {
        Job* job;
        bool samples;
    };
    static bool prompt_done(const Job& job) { return job.prefilled >= job.request.prompt_token_ids.size(); }
    static bool may_finish(const Job& job) {
        const GenerationOptions& g = job.request.generation;
        return g.eos_token_id.has_value() || job.output.size() + 1 == g.max_new_tokens;
    }

    Engine& engine_;
    StagedRunner* staged_;
    std::vector<Queued> queue_;
    bool may_release_ = false;  // a queued item may finish when the queue runs
};

Engine::Engine(std::unique_ptr<ModelRunner> runner, EngineConfig config)
    : runner_(std::move(runner)), config_(config), scheduler_(scheduler_config(config)) {
    if (!runner_ || config.context < 1 || config.context > runner_->config().context ||
        config.context > runner_->context_limit())
        throw std::invalid_argument("invalid engine configuration");
}

Engine::~Engine() {
    try {
        shutdown();
    } catch (...) {
    }
}

void Engine::submit(Request request) {
    if (failed_) throw std::runtime_error("engine failed; create a new engine");
    const std::vector<TokenId>& prompt = request.prompt_token_ids;
    const std::uint64_t length = prompt.size() + std::uint64_t(request.generation.max_new_tokens);
    if (request.id.empty() || seen_.count(request.id) || prompt.empty() || request.generation.max_new_tokens < 1 ||
        length > std::uint64_t(config_.context))
        throw std::invalid_argument("invalid request, duplicate ID or context overflow");
    const int vocabulary = runner_->config().vocabulary;
    if (std::any_of(prompt.begin(), prompt.end(), [&](TokenId t) { return t < 0 || t >= vocabulary; }))
        throw std::invalid_argument("invalid prompt token");
    const std::optional<TokenId>& eos = request.generation.eos_token_id;
    if (eos && (*eos < 0 || *eos >= vocabulary)) throw std::invalid_argument("invalid EOS");
    seen_.insert(request.id);
    Job job;
    job.request = std::move(request);
    jobs_.push_back(std::move(job));
}

void Engine::finish(Job& job, FinishReason reason, std::optional<TokenId> token, const std::string& error,
                    Cleanup cleanup) {
    if (job.finished) return;
    // After a fatal error the runner's clear() owns the sequences; otherwise
    // the job's sequence is released first (a throw leaves it unfinished).
    if (job.resident && cleanup == Cleanup::Release) runner_->release(job.request.id);
    runner_->release_reservation(job.request.id);
    job.resident = false;
    events_.push_back({job.request.id, token, reason, error});
    job.finished = true;
}

void Engine::emit_token(Job& job, TokenId token) {
    const GenerationOptions& g = job.request.generation;
    job.output.push_back(token);
    if (g.eos_token_id && token == *g.eos_token_id) finish(job, FinishReason::Eos, token);
    else if (job.output.size() == g.max_new_tokens) finish(job, FinishReason::Length, token);
    else events_.push_back({job.request.id, token, std::nullopt, {}});
}

void Engine::account(Job& job, std::size_t tokens, bool prefill) {
    if (prefill) {
        job.prefilled += tokens;
        step_stats_.prefill_tokens += tokens;
    } else {
        step_stats_.decode_tokens += tokens;
    }
}

void Engine::drop_finished() {
    jobs_.erase(std::remove_if(jobs_.begin(), jobs_.end(), [](const Job& j) { return j.finished; }), jobs_.end());
    admitted_ = static_cast<std::size_t>(std::count_if(jobs_.begin(), jobs_.end(), [](const Job& j) { return j.admitted; }));
}

void Engine::restore_prefix(Job& job) {
    const Request& r = job.request;
    runner_->create(r.id);
    job.resident = true;
    const std::size_t reused = runner_->reuse_prefix(r.id, r.prompt_token_ids);
    // The runner keeps no logits: at least one prompt token must be left to
    // append. A reusable prefix may end inside a page.
    const std::size_t block_tokens = runner_->stats().kv_block_tokens;
    if (reused >= r.prompt_token_ids.size() || (reused && !block_tokens))
        throw std::runtime_error("invalid reusable prefix range");
    job.prefilled = reused;
    step_stats_.prefix_reused_tokens += reused;
}

bool Engine::admit() {
    bool progressed = false;
    std::size_t slots = scheduler_.admission_count(admitted_, jobs_.size() - admitted_);
    while (slots && admitted_ < jobs_.size()) {
        Job& job = jobs_[admitted_];
        const Request& r = job.request;
        // The last sampled token is delivered, never appended to the KV.
        const std::size_t tokens = r.prompt_token_ids.size() + std::size_t(r.generation.max_new_tokens) - 1;
        const KvAdmission admission = runner_->reserve_request(r.id, tokens);
        if (admission == KvAdmission::Wait && admitted_) break;
        progressed = true;
        if (admission != KvAdmission::Ready) {
            finish(job, FinishReason::Error, std::nullopt,
                   admission == KvAdmission::Impossible ? "request exceeds total KV capacity"
                                                        : "KV capacity unavailable without active requests to make progress");
            jobs_.erase(jobs_.begin() + static_cast<std::ptrdiff_t>(admitted_));
            continue;
        }
        job.admitted = true;
        ++admitted_;
        --slots;
    }
    return progressed;
}

void Engine::execute(SchedulePlan& plan) {
    Executor executor(*this);
    for (const ScheduledRequest& work : plan.order()) {
        if (!plan.has_budget()) break;
        Job& job = jobs_[work.active_index];
        const std::vector<TokenId>& prompt = job.request.prompt_token_ids;
        try {
            if (!job.resident) {
                restore_prefix(job);
                executor.mapped(job);
            }
            const bool prefill = work.phase == SchedulePhase::Prefill;
            const std::size_t count = plan.take_input(work.phase, prompt.size() - job.prefilled);
            std::vector<TokenId> input;
            if (prefill) {
                const auto first = prompt.begin() + static_cast<std::ptrdiff_t>(job.prefilled);
                input.assign(first, first + static_cast<std::ptrdiff_t>(count));
            } else {
                input.push_back(job.output.back());
            }
            executor.append(job, input, prefill);
        } catch (const KvCapacityError& error) {
            // Request-scoped: earlier requests' results come first, as in
            // the per-request loop.
            executor.run_queue();
            finish(job, FinishReason::Error, std::nullopt, error.what());
        }
    }
    executor.run_queue();
}

void Engine::fail_all(const std::string& cause) {
    // Poison first: the runner's ownership must survive a failed cleanup.
    failed_ = true;
    std::string message = cause;
    try {
        runner_->clear();
    } catch (const std::exception& cleanup) {
        message += "; cleanup failed: ";
        message += cleanup.what();
    } catch (...) {
        message += "; cleanup failed: unknown exception";
    }
    for (Job& job : jobs_) finish(job, FinishReason::Error, std::nullopt, message, Cleanup::RunnerOwned);
    drop_finished();
}

bool Engine::step() {
    step_stats_ = {};
    if (failed_) throw std::runtime_error("engine failed");
    try {
        const bool progressed = admit();
        if (!admitted_) return progressed;
        std::vector<SchedulePhase> phases(admitted_);
        for (std::size_t i = 0; i < admitted_; ++i)
            phases[i] = jobs_[i].output.empty() ? SchedulePhase::Prefill : SchedulePhase::Decode;
        SchedulePlan plan = scheduler_.plan(phases);
        execute(plan);
        drop_finished();
    } catch (const std::exception& error) {
        fail_all(error.what());
    }
    return true;
}

std::vector<GenerationEvent> Engine::poll_events() {
    std::vector<GenerationEvent> out;
    out.swap(events_);
    return out;
}

void Engine::cancel(const RequestId& id) {
    const auto it = std::find_if(jobs_.begin(), jobs_.end(),
                                 [&](const Job& j) { return !j.finished && j.request.id == id; });
    if (it == jobs_.end()) throw std::invalid_argument("request is unknown or already terminal");
    finish(*it, FinishReason::Cancelled);
    drop_finished();
}

void Engine::shutdown() {
    try {
        for (Job& job : jobs_) finish(job, FinishReason::Cancelled);
    } catch (...) {
        drop_finished();
        throw;
    }
    drop_finished();
    runner_->clear();
}

}  // namespace miniprefix
