// Engine behaviour restated from the reference's engine tests, compiled
// against this repository's host runtime and against the reference's own
// sources; both builds must pass.
//
//  - miniprefix/tests/engine_prefill_test.cpp:86-310 (capacity admission,
//    runner context limits, chunk positions and budgets, small budgets and
//    cancel, invalid prefix hits and logits, failure cleanup, same-step
//    publish/reuse, decode-first order), without the part that needs the
//    reference's CPU model runner (:155-167);
//  - miniprefix/tests/engine_history_test.cpp:46-116 (publication history,
//    page boundaries, cancellation/EOS/failure, concurrent fork).
//    engine_history_test.cpp:55 expects 4 reused tokens for an aligned
//    8-token prompt; the reference's prefix cache returns 7 (a partial match
//    inside the second page counts, prefix_cache.cpp:124-135), and that
//    assertion fails on the reference's own sources. It is restated here
//    with 7, the value the reference code produces.
#include <miniprefix/engine.h>
#include <miniprefix/kv_manager.h>

#include <cstdio>
#include <cstdlib>
#include <limits>
#include <map>
#include <string>

using namespace miniprefix;

#define CHECK(cond)                                                                       \
    do {                                                                                  \
        if (!(cond)) {                                                                    \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

namespace {

template <class E, class F>
bool throws_as(F&& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

Request make(const std::string& id, std::vector<TokenId> prompt, unsigned max_new = 2) {
    Request r;
    r.id = id;
    r.prompt_token_ids = std::move(prompt);
    r.generation.max_new_tokens = max_new;
    return r;
}
// Prompt 1, 2, ..., length.
Request counting(const std::string& id, int length, unsigned max_new = 2) {
    std::vector<TokenId> p;
    for (int i = 1; i <= length; ++i) p.push_back(i);
    return make(id, p, max_new);
}

std::vector<float> one_hot(TokenId at) {
    std::vector<float> logits(128, 0.0f);
    logits[static_cast<std::size_t>(at % 128)] = 1.0f;
    return logits;
}

// A runner without KV storage that records every append and answers
// prefix lookups from a table (engine_prefill_test.cpp:26-60).
class Recorder final : public ModelRunner {
public:
    struct Call {
        RequestId id;
        std::size_t position;
        std::vector<TokenId> input;
    };
    std::map<RequestId, std::size_t> hit, at, restores, publishes;
    std::vector<Call> calls;
    RequestId fail_on;
    bool nan_logits = false, reuse_after_publish = false;
    int cleanup_failure = 0, clears = 0, releases = 0, limit = 128;

    Recorder() {
        cfg_.context = 128;
        cfg_.vocabulary = 128;
    }
    const ModelConfig& config() const override { return cfg_; }
    int context_limit() const override { return limit; }
    void create(const RequestId& id) override {
        CHECK(!at.count(id));
        at[id] = 0;
    }
    std::size_t reuse_prefix(const RequestId& id, const std::vector<TokenId>& prompt) override {
        if (reuse_after_publish && !publishes.empty() && prompt.size() > 4) hit[id] = 4;
        ++restores[id];
        return at[id] = hit[id];
    }
    void cache_prefix(const RequestId& id) override { ++publishes[id]; }
    std::vector<float> append(const RequestId& id, const std::vector<TokenId>& tokens) override {
        CHECK(!tokens.empty());
        calls.push_back({id, at.at(id), tokens});
        at[id] += tokens.size();
        if (id == fail_on) throw std::runtime_error("forward failed");
        std::vector<float> logits = one_hot(tokens.back() + 1);
        if (nan_logits) logits[0] = std::numeric_limits<float>::quiet_NaN();
        return logits;
    }
    void release(const RequestId& id) override {
        ++releases;
        CHECK(at.erase(id) == 1);
    }
    void clear() override {
        ++clears;
        if (cleanup_failure == 1) throw std::runtime_error("stream synchronization failed");
        if (cleanup_failure == 2) throw 42;
        at.clear();
    }
    RunnerStats stats() const override {
        RunnerStats s;
        s.kv_block_tokens = 4;
        s.live_sequences = at.size();
        return s;
    }

private:
    ModelConfig cfg_;
};

// A runner over a real KVManager (engine_prefill_test.cpp:65-85 and
// engine_history_test.cpp:8-33): appends commit metadata only, logits are a
// one-hot of the last token + 1.
class KvBacked final : public ModelRunner {
public:
    KVManager kv;
    std::vector<std::vector<TokenId>> published;
    bool capacity_error_once = false, fail_publish = false, nan_logits = false;

    KvBacked(KvCacheConfig c) : kv(c, 1, 1, 128, 128) {
        cfg_.context = 128;
        cfg_.vocabulary = 128;
    }
    const ModelConfig& config() const override { return cfg_; }
    int context_limit() const override { return 128; }
    KvAdmission reserve_request(const RequestId& id, std::size_t n) override { return kv.reserve_request(id, n); }
    void release_reservation(const RequestId& id) noexcept override { kv.release_reservation(id); }
    void create(const RequestId& id) override { kv.create(id); }
    std::size_t reuse_prefix(const RequestId& id, const std::vector<TokenId>& p) override { return kv.reuse_prefix(id, p); }
    void cache_prefix(const RequestId& id) override {
        if (fail_publish) throw std::runtime_error("publish failed");
        published.push_back(kv.sequence(id).tokens);
        kv.cache_prefix(id);
    }
    std::vector<float> append(const RequestId& id, const std::vector<TokenId>& t) override {
        if (capacity_error_once) {
            capacity_error_once = false;
            throw KvCapacityError("injected capacity");
        }
        auto tx = kv.prepare_append(id, t);
        tx.copy_shared_tail([](std::size_t, std::size_t, std::size_t) {});
        tx.commit();
        std::vector<float> logits = one_hot(t.back() + 1);
        if (nan_logits) logits[0] = std::numeric_limits<float>::quiet_NaN();
        return logits;
    }
    void release(const RequestId& id) override { kv.release(id); }
    void clear() override { kv.clear(); }
    RunnerStats stats() const override {
        RunnerStats s;
        s.update_kv_stats(kv.stats());
        return s;
    }

private:
    ModelConfig cfg_;
};

struct Tally {
    std::vector<GenerationEvent> events;
    std::vector<TokenId> tokens;
    int terminal = 0;
};
Tally drain(Engine& e) {
    Tally t;
    for (auto& ev : e.poll_events()) {
        if (ev.token_id) t.tokens.push_back(*ev.token_id);
        if (ev.finish_reason) ++t.terminal;
        t.events.push_back(ev);
    }
    return t;
}
// Steps until idle (at most `limit` steps) and returns what was emitted.
Tally run_out(Engine& e, int limit = 128) {
    Tally all = drain(e);
    for (int i = 0; i < limit && !e.idle(); ++i) {
        e.step();
        Tally t = drain(e);
        all.events.insert(all.events.end(), t.events.begin(), t.events.end());
        all.tokens.insert(all.tokens.end(), t.tokens.begin(), t.tokens.end());
        all.terminal += t.terminal;
    }
    CHECK(e.idle());
    return all;
}

// ------------------------------------------------ engine_prefill_test.cpp
void capacity_admission() {
    {
        auto owned = std::make_unique<KvBacked>(KvCacheConfig{2, 2, 2});
        KvBacked* r = owned.get();
        Engine e(std::move(owned), {2, 1, 1, 128});
        e.submit(counting("first", 1, 1));
        e.submit(counting("reserved-only", 1, 1));
        e.step();
        CHECK(!r->kv.contains("reserved-only"));  // reserved, never given budget
        e.cancel("reserved-only");
        e.poll_events();
        e.submit(counting("full-pool", 4, 1));  // 4 KV tokens: every page
        const Tally t = run_out(e, 8);
        CHECK(!e.failed() && t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Length);
    }
    auto owned = std::make_unique<KvBacked>(KvCacheConfig{2, 2, 2});
    KvBacked* r = owned.get();
    Engine e(std::move(owned), {2, 2, 1, 128});
    e.submit(counting("large", 5, 1));  // 3 pages of 2: never fits
    e.submit(counting("a", 2, 3));
    e.submit(counting("b", 2, 3));
    std::map<std::string, int> tokens, finished;
    for (int i = 0; i < 20 && !e.idle(); ++i) {
        e.step();
        for (const auto& ev : e.poll_events()) {
            if (ev.request_id == "large") CHECK(ev.finish_reason == FinishReason::Error && !ev.token_id);
            else CHECK(ev.finish_reason != FinishReason::Error);
            if (ev.token_id) ++tokens[ev.request_id];
            if (ev.finish_reason) ++finished[ev.request_id];
        }
        CHECK(!e.failed() && r->kv.stats().live_sequences <= 1);
    }
    CHECK(e.idle() && tokens["a"] == 3 && tokens["b"] == 3);
    CHECK(finished["large"] == 1 && finished["a"] == 1 && finished["b"] == 1);
    // A reservation is held before the request gets any budget.
    e.submit(counting("cancel", 2, 3));
    e.step();
    e.cancel("cancel");
    e.poll_events();
    e.submit(counting("retry", 4, 1));
    Tally t = run_out(e);
    CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Length);
    // Pages held outside the engine cannot make an idle engine wait forever.
    r->kv.create("external");
    {
        auto tx = r->kv.prepare_append("external", {1, 2, 3, 4});
        tx.commit();
    }
    e.submit(counting("blocked", 1, 1));
    e.step();
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Error && e.idle() && !e.failed());
    r->kv.release("external");
    // A capacity error inside append is request-scoped.
    r->capacity_error_once = true;
    e.submit(counting("capacity-error", 1, 1));
    e.step();
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Error && !e.failed());
    e.submit(counting("healthy", 1, 1));
    e.step();
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Length && e.idle());
}

void runner_context_limits() {
    for (const int limit : {-1, 0, 4}) {
        auto r = std::make_unique<Recorder>();
        r->limit = limit;
        CHECK(throws_as<std::invalid_argument>([&] { Engine e(std::move(r), {1, 8, 8, 5}); }));
    }
    auto oversized = std::make_unique<Recorder>();
    oversized->limit = 256;  // above the model's 128
    CHECK(throws_as<std::invalid_argument>([&] { Engine e(std::move(oversized), {1, 8, 8, 129}); }));
    for (const int context : {3, 4}) {
        auto owned = std::make_unique<Recorder>();
        Recorder* r = owned.get();
        r->limit = 4;
        Engine e(std::move(owned), {1, 8, 8, context});
        CHECK(throws_as<std::invalid_argument>([&] { e.submit(counting("too-long", context, 1)); }));
        CHECK(r->calls.empty() && r->at.empty() && e.idle() && e.poll_events().empty());
        e.submit(counting("boundary", context - 1, 1));
        CHECK(e.step() && e.idle());
        const Tally t = drain(e);
        CHECK(t.events.size() == 1 && t.events[0].token_id && t.events[0].finish_reason == FinishReason::Length);
    }
}

void chunk_positions_and_budget() {
    auto owned = std::make_unique<Recorder>();
    Recorder* r = owned.get();
    r->hit["suffix"] = 8;
    Engine e(std::move(owned), {2, 5, 3, 128});
    e.submit(counting("decoder", 1, 6));
    e.step();
    e.poll_events();
    const Request suffix = counting("suffix", 19);
    e.submit(suffix);
    std::vector<TokenId> seen;
    for (int step = 0; step < 4; ++step) {
        e.step();
        const EngineStepStats s = e.last_step_stats();
        CHECK(s.prefix_reused_tokens == (step == 0 ? 8u : 0u));
        CHECK(s.prefill_tokens == (step == 3 ? 2u : 3u) && s.decode_tokens == 1);
        for (const auto& ev : e.poll_events())
            if (ev.request_id == "suffix") {
                CHECK(step == 3 && ev.token_id && *ev.token_id == 20);
                seen.push_back(*ev.token_id);
            }
    }
    CHECK(r->restores["suffix"] == 1 && r->publishes["suffix"] == 1);
    std::size_t cursor = 8;
    for (const auto& c : r->calls) {
        if (c.id != "suffix") continue;
        CHECK(c.position == cursor && c.input.size() <= 3);
        const auto first = suffix.prompt_token_ids.begin() + static_cast<std::ptrdiff_t>(cursor);
        CHECK(std::vector<TokenId>(first, first + static_cast<std::ptrdiff_t>(c.input.size())) == c.input);
        cursor += c.input.size();
    }
    CHECK(cursor == 19);
    while (!e.idle()) {
        e.step();
        for (const auto& ev : e.poll_events())
            if (ev.request_id == "suffix") {
                CHECK(ev.token_id && *ev.token_id == 21 && ev.finish_reason == FinishReason::Length);
                seen.push_back(*ev.token_id);
            }
    }
    CHECK((seen == std::vector<TokenId>{20, 21}));
    e.step();
    CHECK(e.last_step_stats().prefill_tokens == 0 && e.last_step_stats().decode_tokens == 0);
}

void small_budget_then_cancel() {
    auto owned = std::make_unique<Recorder>();
    Recorder* r = owned.get();
    r->hit["suffix"] = 4;
    Engine e(std::move(owned), {1, 2, 5, 128});
    e.submit(counting("suffix", 13));
    e.step();
    CHECK(e.poll_events().empty() && r->calls.back().position == 4 && r->calls.back().input.size() == 2);
    CHECK(e.last_step_stats().prefix_reused_tokens == 4 && e.last_step_stats().prefill_tokens == 2);
    e.step();
    CHECK(e.poll_events().empty() && e.last_step_stats().prefill_tokens == 2);
    e.cancel("suffix");
    const Tally t = drain(e);
    CHECK(t.events.size() == 1 && !t.events[0].token_id && t.events[0].finish_reason == FinishReason::Cancelled);
    CHECK(r->publishes.empty() && r->at.empty() && r->restores["suffix"] == 1);
}

void invalid_hits_and_logits() {
    {
        auto owned = std::make_unique<Recorder>();
        Recorder* r = owned.get();
        r->hit["partial"] = 3;  // a hit may end inside a page
        Engine e(std::move(owned), {1, 4, 4, 128});
        e.submit(counting("partial", 8, 1));
        e.step();
        CHECK(e.poll_events().empty() && e.last_step_stats().prefix_reused_tokens == 3);
        CHECK(r->calls[0].position == 3 && (r->calls[0].input == std::vector<TokenId>{4, 5, 6, 7}));
        e.step();
        const Tally t = drain(e);
        CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Length);
        CHECK(r->calls[1].position == 7 && (r->calls[1].input == std::vector<TokenId>{8}));
    }
    for (const std::size_t hit : {std::size_t(8), std::size_t(100)}) {  // no prompt token left to append
        auto owned = std::make_unique<Recorder>();
        Recorder* r = owned.get();
        r->hit["bad"] = hit;
        Engine e(std::move(owned), {1, 4, 4, 128});
        e.submit(counting("bad", 8));
        e.step();
        const Tally t = drain(e);
        CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Error);
        CHECK(r->calls.empty() && r->at.empty());
    }
    auto owned = std::make_unique<Recorder>();
    Recorder* r = owned.get();
    r->nan_logits = true;
    Engine e(std::move(owned), {1, 4, 4, 128});
    e.submit(counting("nan", 3));
    e.step();
    const Tally t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Error);
    CHECK(r->publishes.empty() && r->at.empty());
}

void failure_cleanup() {
    for (const int failure : {0, 1, 2}) {
        auto owned = std::make_unique<Recorder>();
        Recorder* r = owned.get();
        r->fail_on = "broken";
        r->cleanup_failure = failure;
        Engine e(std::move(owned), {3, 8, 4, 128});
        for (const char* id : {"finished", "broken", "active", "waiting"})
            e.submit(counting(id, 1, std::string(id) == "finished" ? 1 : 2));
        CHECK(e.step());
        const Tally t = drain(e);
        CHECK(t.events.size() == 4 && e.idle() && r->clears == 1);
        CHECK(t.events[0].request_id == "finished" && t.events[0].token_id &&
              t.events[0].finish_reason == FinishReason::Length);
        std::string message = "forward failed";
        if (failure == 1) message += "; cleanup failed: stream synchronization failed";
        if (failure == 2) message += "; cleanup failed: unknown exception";
        const char* const failed[] = {"broken", "active", "waiting"};
        for (int i = 0; i < 3; ++i) {
            const GenerationEvent& ev = t.events[static_cast<std::size_t>(i + 1)];
            CHECK(ev.request_id == failed[i] && !ev.token_id && ev.finish_reason == FinishReason::Error);
            CHECK(ev.error_message == message);
        }
        // No per-sequence release or retry after the failure.
        CHECK(r->releases == 1 && r->calls.size() == 2 && r->at.size() == (failure ? 1u : 0u));
        CHECK(throws_as<std::runtime_error>([&] { e.step(); }));
        CHECK(throws_as<std::runtime_error>([&] { e.submit(counting("new", 1)); }));
        CHECK(e.poll_events().empty() && r->calls.size() == 2 && r->clears == 1);
        r->cleanup_failure = 0;
        e.shutdown();
        e.shutdown();
        CHECK(e.poll_events().empty() && r->at.empty());
    }
}

void same_step_publish_and_refill() {
    auto owned = std::make_unique<Recorder>();
    Recorder* r = owned.get();
    r->reuse_after_publish = true;
    Engine e(std::move(owned), {2, 8, 8, 128});
    e.submit(counting("seed", 5, 1));
    e.submit(counting("follower", 9, 2));
    e.submit(counting("waiting", 1, 1));
    CHECK(e.step());
    Tally t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].request_id == "seed" &&
          t.events[0].finish_reason == FinishReason::Length);
    CHECK(r->calls.size() == 2 && r->calls[0].input.size() == 5);
    CHECK(r->calls[1].id == "follower" && r->calls[1].position == 4 && r->calls[1].input.size() == 3);
    CHECK(r->restores.count("waiting") == 0);
    CHECK(e.last_step_stats().prefix_reused_tokens == 4 && e.last_step_stats().prefill_tokens == 8);
    CHECK(e.step());
    t = drain(e);
    CHECK(t.events.size() == 2 && t.events[0].request_id == "follower" && t.events[1].request_id == "waiting");
    CHECK(!t.events[0].finish_reason && t.events[1].finish_reason == FinishReason::Length);
    CHECK(r->calls[2].position == 7 && r->calls[2].input.size() == 2);
    CHECK(r->calls[3].id == "waiting" && e.last_step_stats().prefill_tokens == 3);
    CHECK(e.last_step_stats().prefix_reused_tokens == 0);
    CHECK(e.step());
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].request_id == "follower" && *t.events[0].token_id == 11);
    CHECK(t.events[0].finish_reason == FinishReason::Length && e.last_step_stats().decode_tokens == 1);
    CHECK(e.idle() && !e.step() && e.last_step_stats().decode_tokens == 0);
}

void decode_first_and_cancel() {
    auto owned = std::make_unique<Recorder>();
    Recorder* r = owned.get();
    Engine e(std::move(owned), {3, 2, 1, 128});
    e.submit(counting("a", 1, 3));
    e.submit(counting("b", 1, 3));
    e.submit(counting("prefill", 4, 1));
    e.submit(counting("cancel-waiting", 1, 1));
    e.submit(counting("next", 1, 1));
    e.step();
    CHECK(drain(e).events.size() == 2 && r->restores.count("prefill") == 0);
    e.step();
    CHECK(drain(e).events.size() == 2);
    CHECK(r->calls[2].id == "a" && r->calls[3].id == "b");
    CHECK(e.last_step_stats().decode_tokens == 2 && r->restores.count("prefill") == 0);
    e.cancel("a");
    e.cancel("cancel-waiting");
    Tally t = drain(e);
    CHECK(t.events.size() == 2 && t.events[0].finish_reason == FinishReason::Cancelled &&
          t.events[1].finish_reason == FinishReason::Cancelled);
    e.step();
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].request_id == "b" && t.events[0].finish_reason == FinishReason::Length);
    CHECK(r->calls[4].id == "b" && r->calls[5].id == "prefill");
    CHECK(r->restores.count("next") == 0);  // admitted, but the budget ran out
    e.cancel("prefill");
    e.poll_events();
    e.step();
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].request_id == "next" &&
          t.events[0].finish_reason == FinishReason::Length);
    CHECK(e.idle() && r->at.empty());
}

// ------------------------------------------------ engine_history_test.cpp
void aligned_prompt_completion() {
    const std::vector<TokenId> prompt{1, 2, 3, 4, 5, 6, 7, 8};
    for (const int cache : {0, 16})
        for (const int chunk : {2, 4, 8}) {
            auto owned = std::make_unique<KvBacked>(KvCacheConfig{4, 32, cache});
            KvBacked* r = owned.get();
            Engine e(std::move(owned), {1, 8, chunk, 128});
            e.submit(make("seed", prompt, 1));
            CHECK((run_out(e).tokens == std::vector<TokenId>{9}));
            const RunnerStats before = r->stats();
            e.submit(make("aligned", prompt, 1));
            e.step();
            const std::size_t reused = cache ? 7u : 0u;  // the full first page and 3 tokens of the second
            CHECK(e.last_step_stats().prefix_reused_tokens == reused);
            CHECK(e.last_step_stats().prefill_tokens == std::min<std::size_t>(std::size_t(chunk), prompt.size() - reused));
            CHECK(e.last_step_stats().decode_tokens == 0);
            // When the uncached suffix fits one chunk, the first step already finished it.
            CHECK(e.idle() == (std::size_t(chunk) >= prompt.size() - reused));
            CHECK((run_out(e).tokens == std::vector<TokenId>{9}));
            CHECK(e.poll_events().empty());
            const RunnerStats after = r->stats();
            CHECK(after.forward_tokens - before.forward_tokens == prompt.size() - reused);
            CHECK(after.prefix_reused_tokens - before.prefix_reused_tokens == reused);
            CHECK(r->published.back() == prompt);  // the sampled token 9 has no KV
            CHECK(after.live_sequences == 0 && after.kv_cached_blocks == (cache ? 2u : 0u));
            e.shutdown();
            CHECK(r->stats().kv_live_blocks == 0);
        }
}

void publication_history_and_boundaries() {
    auto owned = std::make_unique<KvBacked>(KvCacheConfig{4, 32, 16});
    KvBacked* r = owned.get();
    Engine e(std::move(owned), {2, 8, 2, 128});
    e.submit(make("turn1", {1, 2, 3}, 2));
    CHECK((run_out(e).tokens == std::vector<TokenId>{4, 5}));
    CHECK((r->published == std::vector<std::vector<TokenId>>{{1, 2, 3}, {1, 2, 3, 4}}));
    CHECK(r->stats().kv_cached_blocks == 2);  // the final token 5 has no KV
    e.submit(make("turn2", {1, 2, 3, 4, 5, 9}, 3));
    e.step();
    CHECK(e.last_step_stats().prefix_reused_tokens == 4 && e.last_step_stats().prefill_tokens == 2);
    Tally t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].token_id == 10);
    e.step();
    e.poll_events();
    e.step();
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].token_id == 12 && t.events[0].finish_reason == FinishReason::Length);
    CHECK((r->published.back() == std::vector<TokenId>{1, 2, 3, 4, 5, 9, 10, 11}));
    // A whole cached prompt still appends its last token for the logits.
    e.submit(make("aligned", {1, 2, 3, 4, 5, 9, 10, 11}, 1));
    e.step();
    CHECK(e.last_step_stats().prefix_reused_tokens == 7);
    t = drain(e);
    CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Length);
    e.shutdown();
    CHECK(r->stats().kv_live_blocks == 0);
}

void cancellation_eos_and_failure() {
    for (const bool eos : {false, true}) {
        auto owned = std::make_unique<KvBacked>(KvCacheConfig{4, 32, 16});
        KvBacked* r = owned.get();
        Engine e(std::move(owned), {1, 8, 8, 128});
        Request req = make("a", {1, 2, 3}, 8);
        if (eos) req.generation.eos_token_id = 5;
        e.submit(req);
        e.step();
        e.poll_events();
        e.step();
        const Tally t = drain(e);
        CHECK(t.events[0].token_id == 5);
        if (!eos) {
            e.cancel("a");
            e.poll_events();
        }
        CHECK(e.idle() && r->stats().kv_cached_blocks == 2 && r->published.back().back() == 4);
        e.submit(make("next", {1, 2, 3, 4, 5, 6}, 1));
        e.step();
        CHECK(e.last_step_stats().prefix_reused_tokens == 4);
        e.poll_events();
    }
    for (const bool nan : {false, true}) {
        auto owned = std::make_unique<KvBacked>(KvCacheConfig{4, 32, 16});
        KvBacked* r = owned.get();
        Engine e(std::move(owned), {1, 8, 8, 128});
        e.submit(make("a", {1, 2, 3}, 3));
        e.step();
        e.poll_events();
        r->fail_publish = !nan;
        r->nan_logits = nan;
        e.step();
        const Tally t = drain(e);
        CHECK(t.events.size() == 1 && t.events[0].finish_reason == FinishReason::Error && !t.events[0].token_id);
        CHECK(e.failed() && r->published.size() == 1 && r->stats().kv_live_blocks == 0);
    }
}

void fork_within_step() {
    for (const int cache : {0, 16}) {
        auto owned = std::make_unique<KvBacked>(KvCacheConfig{4, 32, cache});
        KvBacked* r = owned.get();
        Engine e(std::move(owned), {2, 8, 8, 128});
        e.submit(make("source", {1, 2, 3}, 5));
        e.step();
        e.poll_events();
        e.submit(make("fork", {1, 2, 3, 4, 50}, 1));
        e.step();
        const Tally t = drain(e);
        // The decoder fills and publishes its page before the new request
        // restores its prefix in the same step.
        CHECK(e.last_step_stats().prefix_reused_tokens == (cache ? 4u : 0u));
        CHECK(t.events.size() == 2 && t.events[0].token_id == 5 && t.events[1].token_id == 51);
        CHECK((r->kv.sequence("source").tokens == std::vector<TokenId>{1, 2, 3, 4}));
        run_out(e);
        e.shutdown();
        CHECK(r->stats().kv_live_blocks == 0);
    }
}

}  // namespace

int main() {
    capacity_admission();
    runner_context_limits();
    chunk_positions_and_budget();
    small_budget_then_cancel();
    invalid_hits_and_logits();
    failure_cleanup();
    same_step_publish_and_refill();
    decode_first_and_cancel();
    aligned_prompt_completion();
    publication_history_and_boundaries();
    cancellation_eos_and_failure();
    fork_within_step();
    std::puts("engine tests passed");
    return 0;
}
