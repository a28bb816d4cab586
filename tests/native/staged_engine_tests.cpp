// The Engine's batched path (StagedRunner) against its per-request path.
//
// PayloadRunner is a ModelRunner and StagedRunner over a real KVManager
// whose "device" is a page pool of token slots (one layer, width one). A
// forward writes its new tokens into their slots and then reads every slot
// of its history; the logits are a one-hot of a hash of what it read, so a
// stale or missing K/V slot changes the sampled token. Device order is
// modelled as a stream:
//  - append() runs its tail copy and forward at once;
//  - stage() enqueues its tail copy at once (as a device copy would be) and
//    queues the forward; run_staged() runs the queued forwards as one batch
//    in which no forward sees another's writes (they run concurrently on a
//    device): reads outside a forward's own new positions come from the
//    pool as it was when the batch started.
// Each scenario runs twice, batching on and off, and must give identical
// events and identical page tables after every step. The same-step
// publish/reuse scenarios restate the reference's
// miniprefix/tests/engine_prefill_test.cpp:267-289 (with a seed that decodes
// twice, so its forward is still queued when the follower maps its pages)
// and miniprefix/tests/engine_history_test.cpp:105-116.
#include <miniprefix/engine.h>
#include <miniprefix/kv_manager.h>

#include "staged_runner.h"

#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <sstream>
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

constexpr int kVocabulary = 128;

class PayloadRunner final : public ModelRunner, public StagedRunner {
public:
    explicit PayloadRunner(KvCacheConfig kv)
        : kv_(kv, 1, 1, 128, kVocabulary), bt_(kv.block_tokens),
          pool_(static_cast<std::size_t>(kv.max_blocks * kv.block_tokens), -1),
          writes_(static_cast<std::size_t>(kv.max_blocks), 0) {
        config_.context = 128;
        config_.vocabulary = kVocabulary;
    }
    const ModelConfig& config() const override { return config_; }
    int context_limit() const override { return 128; }
    KvAdmission reserve_request(const RequestId& id, std::size_t n) override { return kv_.reserve_request(id, n); }
    void release_reservation(const RequestId& id) noexcept override { kv_.release_reservation(id); }
    void create(const RequestId& id) override {
        kv_.create(id);
        live_.insert(id);
    }
    void fork_sequence(const RequestId& s, const RequestId& t) override {
        kv_.fork_sequence(s, t);
        forked_ = true;
    }
    std::size_t reuse_prefix(const RequestId& id, const std::vector<TokenId>& p) override { return kv_.reuse_prefix(id, p); }
    void cache_prefix(const RequestId& id) override { kv_.cache_prefix(id); }
    void clear_prefix_cache() override { kv_.clear_prefix_cache(); }
    void release(const RequestId& id) override {
        CHECK(queue_.empty());
        kv_.release(id);
        live_.erase(id);
    }
    void clear() override {
        discard_staged();
        kv_.clear();
        live_.clear();
    }
    RunnerStats stats() const override {
        RunnerStats s;
        s.update_kv_stats(kv_.stats());
        return s;
    }

    std::vector<float> append(const RequestId& id, const std::vector<TokenId>& tokens) override {
        CHECK(queue_.empty());
        auto tx = kv_.prepare_append(id, tokens);
        tx.copy_shared_tail_region([&](const KVManager::TailCopyRegion& r) { copy(r); });
        const Forward f{tx.sequence().blocks, tx.sequence().used, tokens};
        const TokenId token = run(f, pool_);
        tx.commit();
        std::vector<float> logits(kVocabulary, 0.0f);
        logits[static_cast<std::size_t>(token)] = 1.0f;
        return logits;
    }

    void stage(const RequestId& id, const std::vector<TokenId>& tokens) override {
        auto tx = kv_.prepare_append(id, tokens);
        tx.copy_shared_tail_region([&](const KVManager::TailCopyRegion& r) { copy(r); });
        const PagedSequence& s = tx.sequence();
        for (int p = s.used; p < s.used + static_cast<int>(tokens.size()); ++p)
            writes_[static_cast<std::size_t>(s.blocks[static_cast<std::size_t>(p / bt_)])] = 1;
        queue_.push_back({s.blocks, s.used, tokens});
        tx.commit();
    }
    std::vector<StagedResult> run_staged() override {
        ++passes_;
        const std::vector<int> before = pool_;  // what every forward of the batch reads
        std::vector<StagedResult> results;
        for (const Forward& f : queue_) results.push_back({run(f, before), true});
        discard_staged();
        return results;
    }
    void discard_staged() noexcept override {
        queue_.clear();
        std::fill(writes_.begin(), writes_.end(), 0);
    }
    // As the HIP runner decides it (hip_runner.cpp).
    bool stage_touches_pool(const RequestId& id, std::size_t tokens, bool publishes) const override {
        const PagedSequence& s = kv_.sequence(id);
        const std::size_t bt = static_cast<std::size_t>(bt_), used = static_cast<std::size_t>(s.used);
        const bool caches = kv_.config().prefix_cache_blocks > 0;
        if ((used + tokens + bt - 1) / bt > s.blocks.size()) return true;
        if (used % bt != 0 && (caches || forked_)) return true;
        return publishes && caches;
    }
    bool shares_staged_pages(const RequestId& id) const override {
        if (!kv_.contains(id)) return false;
        for (const int b : kv_.sequence(id).blocks)
            if (writes_[static_cast<std::size_t>(b)]) return true;
        return false;
    }

    // Every live sequence's committed table, for comparing the two runs.
    std::string tables() const {
        std::ostringstream out;
        for (const RequestId& id : live_) {
            const PagedSequence& s = kv_.sequence(id);
            out << id << "@" << s.used << ":";
            for (const int b : s.blocks) out << b << ",";
            out << ";";
        }
        return out.str();
    }

private:
    struct Forward {
        std::vector<int> blocks;
        int used;
        std::vector<TokenId> tokens;
    };
    std::size_t slot(const std::vector<int>& blocks, int position) const {
        return static_cast<std::size_t>(blocks[static_cast<std::size_t>(position / bt_)] * bt_ + position % bt_);
    }
    // The copy-on-write region in slot units (one layer, width one).
    void copy(const KVManager::TailCopyRegion& r) {
        CHECK(r.rows == 1);
        for (std::size_t i = 0; i < r.width; ++i) pool_[r.destination + i] = pool_[r.source + i];
    }
    // Writes the new tokens, reads the history (own new tokens from the
    // forward itself, the rest from `visible`), returns the sampled token.
    TokenId run(const Forward& f, const std::vector<int>& visible) {
        const int n = static_cast<int>(f.tokens.size());
        for (int i = 0; i < n; ++i) pool_[slot(f.blocks, f.used + i)] = f.tokens[static_cast<std::size_t>(i)];
        std::uint64_t h = 1469598103934665603ull;
        for (int p = 0; p < f.used + n; ++p) {
            const int v = p >= f.used ? f.tokens[static_cast<std::size_t>(p - f.used)] : visible[slot(f.blocks, p)];
            h = (h ^ static_cast<std::uint64_t>(v + 2)) * 1099511628211ull;
        }
        return static_cast<TokenId>(h % kVocabulary);
    }

    ModelConfig config_;
    KVManager kv_;
    int bt_;
    std::vector<int> pool_;
    std::vector<char> writes_;  // per block: written by a queued forward
    std::vector<Forward> queue_;
    std::set<RequestId> live_;
    bool forked_ = false;

public:
    int passes_ = 0;  // run_staged() calls
};

struct Submit {
    int at_step;
    Request request;
};

// Runs the submissions through an engine and returns a transcript of every
// step's events and page tables.
std::string transcript(KvCacheConfig kv, EngineConfig ec, const std::vector<Submit>& submits, bool batching,
                       std::vector<int>* passes = nullptr) {
    auto owned = std::make_unique<PayloadRunner>(kv);
    PayloadRunner* runner = owned.get();
    Engine engine(std::move(owned), ec);
    engine.set_batching(batching);
    std::ostringstream out;
    std::size_t next = 0;
    for (int step = 0; step < 400 && (next < submits.size() || !engine.idle()); ++step) {
        while (next < submits.size() && submits[next].at_step <= step) engine.submit(submits[next++].request);
        engine.step();
        const auto stats = engine.last_step_stats();
        out << "#" << step << " r" << stats.prefix_reused_tokens << " p" << stats.prefill_tokens << " d"
            << stats.decode_tokens << " ";
        for (const auto& e : engine.poll_events()) {
            out << e.request_id << "=" << (e.token_id ? std::to_string(*e.token_id) : "-");
            if (e.finish_reason) out << "!" << static_cast<int>(*e.finish_reason) << e.error_message;
            out << " ";
        }
        out << "| " << runner->tables() << "\n";
        CHECK(!engine.failed());
        if (passes) passes->push_back(runner->passes_);
        runner->passes_ = 0;
    }
    CHECK(engine.idle());
    return out.str();
}

Request request(const std::string& id, std::vector<TokenId> prompt, unsigned max_new,
                std::optional<TokenId> eos = std::nullopt) {
    Request r;
    r.id = id;
    r.prompt_token_ids = std::move(prompt);
    r.generation.max_new_tokens = max_new;
    r.generation.eos_token_id = eos;
    return r;
}

std::vector<TokenId> iota(int first, int count) {
    std::vector<TokenId> v;
    for (int i = 0; i < count; ++i) v.push_back(first + i);
    return v;
}

void same(KvCacheConfig kv, EngineConfig ec, const std::vector<Submit>& submits, const char* name) {
    const std::string sequential = transcript(kv, ec, submits, false);
    const std::string batched = transcript(kv, ec, submits, true);
    if (sequential != batched) {
        std::fprintf(stderr, "%s: batched run differs\n-- per request:\n%s-- batched:\n%s", name, sequential.c_str(),
                     batched.c_str());
        std::exit(1);
    }
}

// A follower maps the seed's pages (a full page and a one-token tail) in
// the step that publishes them, while the seed's forward is still queued:
// its tail copy and its forward must come after that forward.
void same_step_publish_and_reuse() {
    for (const unsigned seed_new : {1u, 2u, 3u})
        same({4, 32, 16}, {2, 8, 8, 128},
             {{0, request("seed", iota(1, 5), seed_new)}, {0, request("follower", iota(1, 9), 2)},
              {0, request("waiting", {1}, 1)}},
             "same_step_publish_and_reuse");
}

// A decoder fills and publishes a page that a new request then maps in the
// same step.
void concurrent_fork() {
    for (const int cache : {0, 16})
        same({4, 32, cache}, {2, 8, 8, 128},
             {{0, request("source", {1, 2, 3}, 5)}, {1, request("fork", {1, 2, 3, 4, 50}, 1)}}, "concurrent_fork");
}

// Many requests over shared prompt prefixes, small pools (evictions,
// waiting admissions, capacity errors), EOS, budgets and chunks.
void randomized() {
    for (unsigned seed = 1; seed <= 400; ++seed) {
        std::mt19937 rng(seed);
        auto pick = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
        const int bt = pick(2, 5);
        KvCacheConfig kv{bt, pick(12, 48), 0};
        kv.prefix_cache_blocks = pick(0, kv.max_blocks);
        EngineConfig ec{pick(1, 6), pick(1, 24), pick(1, 9), 128};
        std::vector<std::vector<TokenId>> stems;
        for (int i = 0; i < 3; ++i) {
            std::vector<TokenId> s;
            for (int j = pick(1, 12); j > 0; --j) s.push_back(pick(0, 7));
            stems.push_back(s);
        }
        std::vector<Submit> submits;
        int step = 0;
        for (int i = pick(3, 10); i > 0; --i) {
            step += pick(0, 3);
            std::vector<TokenId> prompt = stems[static_cast<std::size_t>(pick(0, 2))];
            prompt.resize(static_cast<std::size_t>(pick(1, static_cast<int>(prompt.size()))));
            for (int j = pick(0, 6); j > 0; --j) prompt.push_back(pick(0, 127));
            std::optional<TokenId> eos;
            if (pick(0, 3) == 0) eos = pick(0, 127);
            submits.push_back({step, request("r" + std::to_string(i), prompt, static_cast<unsigned>(pick(1, 8)), eos)});
        }
        same(kv, ec, submits, ("randomized seed " + std::to_string(seed)).c_str());
    }
}

// Requests that finish in a step (by length, or by an EOS that only their
// result decides) no longer run their forwards alone: the appends after them
// join the same device pass unless they take pages from the pool. Here no
// decode step crosses a page, so every decode step is one pass; the prefill
// step, whose appends each take a first page, runs a pass before each
// append that follows one that may finish.
void finishing_requests_share_a_batch() {
    const KvCacheConfig kv{16, 64, 0};
    const EngineConfig ec{8, 64, 16, 128};
    std::vector<Submit> submits;
    for (int i = 0; i < 8; ++i)
        submits.push_back({0, request("f" + std::to_string(i), iota(1 + i, 3), static_cast<unsigned>(2 + i % 3),
                                      i % 2 ? std::optional<TokenId>(5) : std::nullopt)});
    same(kv, ec, submits, "finishing_requests_share_a_batch");
    std::vector<int> passes;
    transcript(kv, ec, submits, true, &passes);
    CHECK(passes.size() >= 2);
    for (std::size_t step = 1; step < passes.size(); ++step) CHECK(passes[step] <= 1);
}

}  // namespace

int main() {
    same_step_publish_and_reuse();
    concurrent_fork();
    finishing_requests_share_a_batch();
    randomized();
    std::puts("staged engine tests passed");
    return 0;
}
