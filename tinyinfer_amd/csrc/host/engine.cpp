// Engine (reference semantics: miniprefix/src/engine/engine.cpp:13-140).
//
// With a StagedRunner the per-request loop of one step is kept, but each
// append is staged (its KV transaction commits immediately, in plan order)
// and the staged forwards run as one device batch. The batch is flushed
// before any staged request could finish: finishing releases pages, and the
// reference releases them before the next request's append reserves pages.
#include "miniprefix/engine.h"

#include <algorithm>
#include <cmath>

namespace miniprefix {
namespace {
SchedulerConfig scheduler_config(const EngineConfig& c) {
    if (c.max_batch_size < 1 || c.token_budget < 1 || c.prefill_chunk < 1)
        throw std::invalid_argument("invalid engine configuration");
    return {c.max_batch_size, c.token_budget, c.prefill_chunk};
}
}  // namespace

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
    const auto& p = request.prompt_token_ids;
    if (request.id.empty() || seen_.count(request.id) || p.empty() || request.generation.max_new_tokens < 1 ||
        p.size() + std::uint64_t(request.generation.max_new_tokens) > std::uint64_t(config_.context))
        throw std::invalid_argument("invalid request, duplicate ID or context overflow");
    const int vocabulary = runner_->config().vocabulary;
    for (const TokenId t : p)
        if (t < 0 || t >= vocabulary) throw std::invalid_argument("invalid prompt token");
    const auto& eos = request.generation.eos_token_id;
    if (eos && (*eos < 0 || *eos >= vocabulary)) throw std::invalid_argument("invalid EOS");
    State state;
    state.request = std::move(request);
    seen_.insert(state.request.id);
    waiting_.push_back(std::move(state));
}

void Engine::terminal(State& state, FinishReason reason, std::optional<TokenId> token, const std::string& error,
                      TerminalCleanup cleanup) {
    if (state.finished) return;
    // Normal endings release the sequence; after a fatal error the runner's
    // clear() owns cleanup, so no per-request release is attempted.
    if (state.resident && cleanup == TerminalCleanup::ReleaseSequence) runner_->release(state.request.id);
    runner_->release_reservation(state.request.id);
    state.resident = false;
    events_.push_back({state.request.id, token, reason, error});
    state.finished = true;
}

void Engine::remove_finished(bool include_waiting) {
    const auto done = [](const State& s) { return s.finished; };
    active_.erase(std::remove_if(active_.begin(), active_.end(), done), active_.end());
    if (include_waiting) waiting_.erase(std::remove_if(waiting_.begin(), waiting_.end(), done), waiting_.end());
}

void Engine::restore_prefix(State& state) {
    const Request& request = state.request;
    runner_->create(request.id);
    state.resident = true;
    const std::size_t reused = runner_->reuse_prefix(request.id, request.prompt_token_ids);
    // The runner returns no cached logits: at least one prompt token must
    // remain to append. A reusable prefix may end inside a page.
    const std::size_t block_tokens = runner_->stats().kv_block_tokens;
    if (reused >= request.prompt_token_ids.size() || (reused && !block_tokens))
        throw std::runtime_error("invalid reusable prefix range");
    state.kv_block_tokens = block_tokens;
    state.prefilled = reused;
    step_stats_.prefix_reused_tokens += reused;
}

void Engine::sample(State& s, TokenId token) {
    const Request& r = s.request;
    s.output.push_back(token);
    std::optional<FinishReason> finish;
    if (r.generation.eos_token_id && token == *r.generation.eos_token_id) finish = FinishReason::Eos;
    else if (s.output.size() == r.generation.max_new_tokens) finish = FinishReason::Length;
    if (finish) terminal(s, *finish, token);
    else events_.push_back({r.id, token, std::nullopt, {}});
}

void Engine::run_plan_sequential(SchedulePlan& plan) {
    for (const auto& work : plan.order()) {
        if (!plan.has_budget()) break;
        State& s = active_[work.active_index];
        const Request& r = s.request;
        try {
            if (!s.resident) restore_prefix(s);
            const bool prefilling = work.phase == SchedulePhase::Prefill;
            const std::size_t count = plan.take_input(work.phase, r.prompt_token_ids.size() - s.prefilled);
            std::vector<TokenId> input;
            if (!prefilling) input = {s.output.back()};
            else input.assign(r.prompt_token_ids.begin() + static_cast<std::ptrdiff_t>(s.prefilled),
                              r.prompt_token_ids.begin() + static_cast<std::ptrdiff_t>(s.prefilled + count));
            const std::vector<float> logits = runner_->append(r.id, input);
            if (prefilling) {
                s.prefilled += input.size();
                step_stats_.prefill_tokens += input.size();
            } else {
                step_stats_.decode_tokens += input.size();
            }
            if (s.prefilled < r.prompt_token_ids.size()) continue;
            if (logits.size() != static_cast<std::size_t>(runner_->config().vocabulary))
                throw std::runtime_error("invalid logits arity");
            for (const float v : logits)
                if (!std::isfinite(v)) throw std::runtime_error("nonfinite model result");
            // Publish before sampling: the new output token has no KV yet.
            runner_->cache_prefix(r.id);
            sample(s, static_cast<TokenId>(std::max_element(logits.begin(), logits.end()) - logits.begin()));
        } catch (const KvCapacityError& error) {
            terminal(s, FinishReason::Error, std::nullopt, error.what());
        }
    }
}

void Engine::run_plan_staged(SchedulePlan& plan, StagedRunner& staged) {
    struct Item {
        std::size_t index;
        bool samples;
    };
    std::vector<Item> items;
    auto flush = [&]() {
        if (items.empty()) return;
        const std::vector<StagedResult> results = staged.run_staged();
        if (results.size() != items.size()) throw std::runtime_error("invalid staged result count");
        for (std::size_t i = 0; i < items.size(); ++i) {
            if (!results[i].finite) throw std::runtime_error("nonfinite model result");
            if (items[i].samples) sample(active_[items[i].index], results[i].argmax);
        }
        items.clear();
    };
    try {
        for (const auto& work : plan.order()) {
            if (!plan.has_budget()) break;
            State& s = active_[work.active_index];
            const Request& r = s.request;
            try {
                if (!s.resident) restore_prefix(s);
                const bool prefilling = work.phase == SchedulePhase::Prefill;
                const std::size_t count = plan.take_input(work.phase, r.prompt_token_ids.size() - s.prefilled);
                std::vector<TokenId> input;
                if (!prefilling) input = {s.output.back()};
                else input.assign(r.prompt_token_ids.begin() + static_cast<std::ptrdiff_t>(s.prefilled),
                                  r.prompt_token_ids.begin() + static_cast<std::ptrdiff_t>(s.prefilled + count));
                staged.stage(r.id, input);
                if (prefilling) {
                    s.prefilled += input.size();
                    step_stats_.prefill_tokens += input.size();
                } else {
                    step_stats_.decode_tokens += input.size();
                }
                const bool samples = s.prefilled >= r.prompt_token_ids.size();
                items.push_back({work.active_index, samples});
                if (!samples) continue;
                runner_->cache_prefix(r.id);
                // A request that may finish now releases its pages when
                // sampled; later appends must see that release first.
                const bool may_finish = r.generation.eos_token_id.has_value() ||
                                        s.output.size() + 1 == r.generation.max_new_tokens;
                if (may_finish) flush();
            } catch (const KvCapacityError& error) {
                // Deliver the events of earlier staged requests first, so the
                // event order is the reference's plan order.
                flush();
                terminal(s, FinishReason::Error, std::nullopt, error.what());
            }
        }
        flush();
    } catch (...) {
        staged.discard_staged();
        throw;
    }
}

bool Engine::step() {
    step_stats_ = {};
    if (failed_) throw std::runtime_error("engine failed");
    bool progressed = false;
    try {
        std::size_t slots = scheduler_.admission_count(active_.size(), waiting_.size());
        while (slots && !waiting_.empty()) {
            State& state = waiting_.front();
            const Request& request = state.request;
            // The final sampled token is delivered, never appended to KV.
            const std::size_t tokens =
                request.prompt_token_ids.size() + std::size_t(request.generation.max_new_tokens) - 1;
            const KvAdmission admission = runner_->reserve_request(request.id, tokens);
            if (admission == KvAdmission::Wait && !active_.empty()) break;
            if (admission != KvAdmission::Ready) {
                terminal(state, FinishReason::Error, std::nullopt,
                         admission == KvAdmission::Impossible
                             ? "request exceeds total KV capacity"
                             : "KV capacity unavailable without active requests to make progress");
                waiting_.pop_front();
                progressed = true;
                continue;
            }
            active_.push_back(std::move(state));
            waiting_.pop_front();
            --slots;
            progressed = true;
        }
        if (active_.empty()) return progressed;
        std::vector<SchedulePhase> phases;
        phases.reserve(active_.size());
        for (const State& s : active_) phases.push_back(s.output.empty() ? SchedulePhase::Prefill : SchedulePhase::Decode);
        SchedulePlan plan = scheduler_.plan(phases);
        StagedRunner* staged = batching_ ? dynamic_cast<StagedRunner*>(runner_.get()) : nullptr;
        if (staged) run_plan_staged(plan, *staged);
        else run_plan_sequential(plan);
        remove_finished();
    } catch (const std::exception& error) {
        // Poison first: backend ownership must survive a failed cleanup.
        failed_ = true;
        std::string message = error.what();
        try {
            runner_->clear();
        } catch (const std::exception& cleanup) {
            message += "; cleanup failed: ";
            message += cleanup.what();
        } catch (...) {
            message += "; cleanup failed: unknown exception";
        }
        for (State& s : active_) terminal(s, FinishReason::Error, std::nullopt, message, TerminalCleanup::RunnerManaged);
        for (State& s : waiting_) terminal(s, FinishReason::Error, std::nullopt, message, TerminalCleanup::RunnerManaged);
        remove_finished(true);
    }
    return true;
}

std::vector<GenerationEvent> Engine::poll_events() {
    std::vector<GenerationEvent> out = std::move(events_);
    events_.clear();
    return out;
}

void Engine::cancel(const RequestId& id) {
    for (State& s : waiting_)
        if (s.request.id == id && !s.finished) {
            terminal(s, FinishReason::Cancelled);
            remove_finished(true);
            return;
        }
    for (State& s : active_)
        if (s.request.id == id && !s.finished) {
            terminal(s, FinishReason::Cancelled);
            remove_finished();
            return;
        }
    throw std::invalid_argument("request is unknown or already terminal");
}

void Engine::shutdown() {
    try {
        for (State& s : active_) terminal(s, FinishReason::Cancelled);
        for (State& s : waiting_) terminal(s, FinishReason::Cancelled);
    } catch (...) {
        remove_finished(true);
        throw;
    }
    remove_finished(true);
    runner_->clear();
}

}  // namespace miniprefix
