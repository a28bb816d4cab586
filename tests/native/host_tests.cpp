// Host-side MiniPrefix behaviour: paged KV pool, KV manager transactions,
// copy-on-write, prefix cache (differential against a brute-force flat
// index), scheduler and engine with a recording runner.
//
// The same source is compiled against this repository's host runtime and,
// where /root/reference exists, against the reference's own sources
// (miniprefix/src/{kv,scheduler,engine}); both builds must pass, which pins
// the restatement to the reference's observable behaviour. Known answers
// marked "ref:" restate assertions of the reference's tests.
#include <miniprefix/engine.h>
#include <miniprefix/kv_manager.h>
#include <miniprefix/scheduler.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <map>
#include <random>
#include <set>
#include <string>

using namespace miniprefix;

#define CHECK(cond)                                                                   \
    do {                                                                              \
        if (!(cond)) {                                                                \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                             \
        }                                                                             \
    } while (0)

template <class F>
bool throws(F&& f) {
    try {
        f();
    } catch (const std::exception&) {
        return true;
    }
    return false;
}
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

static void commit(KVManager& m, const RequestId& id, std::vector<TokenId> tokens) {
    auto tx = m.prepare_append(id, tokens);
    tx.copy_shared_tail([](std::size_t, std::size_t, std::size_t) {});
    tx.commit();
}

// ---------------------------------------------------------------- pool ----
static void pool_ownership() {
    KvBlockPool pool({3, 5}, 2, 4);
    PagedSequence a, b, c;
    CHECK(pool.reserved_bytes() == 5u * 3 * 2 * 4 * 8);
    pool.reserve(a, 3); a.used = 3;
    pool.reserve(b, 3); b.used = 3;
    pool.reserve(a, 7); a.used = 7;
    CHECK((a.blocks == std::vector<int>{0, 2, 3}));  // ref: LIFO, non-contiguous
    CHECK(pool.offset(a, 1, 3, 2, 4) == (2 * 2 + 1) * 3 * 4);
    CHECK(pool.live_blocks() == 4 && pool.peak_blocks() == 4);
    const auto before = a.blocks;
    CHECK(throws_as<KvCapacityError>([&] { pool.reserve(a, 13); }));
    CHECK(a.blocks == before && a.used == 7 && pool.live_blocks() == 4);
    pool.release(b);
    pool.reserve(c, 6); c.used = 6;
    CHECK((c.blocks == std::vector<int>{1, 4}));  // ref: hole reuse
    const auto original = a.blocks.size();
    pool.release(c);
    pool.reserve(a, 10);
    pool.rollback(a, original);
    CHECK(a.blocks == before && a.used == 7);
    pool.release(a);
    CHECK(pool.live_blocks() == 0 && pool.peak_blocks() == 5);
    CHECK(throws_as<std::invalid_argument>([] { KvBlockPool bad({0, 1}, 2, 4); }));
    CHECK(throws_as<std::invalid_argument>(
        [] { KvBlockPool bad({2147483647, 2147483647}, 2147483647, 2147483647); }));
    CHECK(throws_as<std::invalid_argument>([&] { pool.reserve(a, 0); a.used = 3; pool.reserve(a, 2); }));
}

// ------------------------------------------------------------- manager ----
static void reservations() {
    KVManager m({2, 3, 3}, 1, 1, 16, 100);
    CHECK(m.reserve_request("too-big", 7) == KvAdmission::Impossible);
    CHECK(m.reserve_request("a", 4) == KvAdmission::Ready);
    CHECK(m.reserve_request("b", 4) == KvAdmission::Wait);
    CHECK(m.stats().kv_live_blocks == 0);
    m.create("external");
    commit(m, "external", {1, 2});
    CHECK(throws([&] { m.prepare_append("external", {3}); }));  // unreserved growth
    m.create("a");
    commit(m, "a", {1, 2, 3, 4});
    m.cache_prefix("a");
    CHECK(throws([&] { m.prepare_append("a", {5}); }));  // beyond its reservation
    m.release("a");
    CHECK(m.reserve_request("b", 4) == KvAdmission::Ready);
    m.create("b");
    commit(m, "b", {5, 6, 7, 8});
    m.clear();
    CHECK(m.reserve_request("all", 6) == KvAdmission::Ready);
    m.release_reservation("all");
    CHECK(m.reserve_request("again", 6) == KvAdmission::Ready);
    CHECK(throws_as<std::invalid_argument>([&] { m.reserve_request("again", 1); }));
    CHECK(throws_as<std::invalid_argument>([&] { m.reserve_request("zero", 0); }));
    m.clear();
    CHECK(m.stats().kv_live_blocks == 0);
}

static void transactions() {
    KVManager m({2, 8, 2}, 2, 4, 16, 100);
    m.create("a");
    std::vector<TokenId> input{1, 2, 3};
    {
        auto tx = m.prepare_append("a", input);
        CHECK(tx.sequence().used == 0 && tx.sequence().blocks.size() == 2);
        CHECK(m.stats().forward_tokens == 0);
        CHECK(throws([&] { m.release("a"); }));
        CHECK(throws([&] { m.reset_sequence("a"); }));
        CHECK(throws([&] { m.clear(); }));
        CHECK(throws([&] { m.clear_prefix_cache(); }));
        CHECK(throws([&] { m.cache_prefix("a"); }));
        CHECK(throws([&] { m.prepare_append("a", {4}); }));
        input[0] = 99;  // the transaction owns a snapshot
        tx.commit();
        CHECK(throws([&] { tx.commit(); }));
    }
    CHECK((m.sequence("a").tokens == std::vector<TokenId>{1, 2, 3}));
    CHECK(m.sequence("a").used == 3 && m.stats().forward_tokens == 3);
    const auto blocks = m.sequence("a").blocks;
    const auto live = m.stats().kv_live_blocks;
    try {
        auto tx = m.prepare_append("a", {4, 5});
        CHECK(tx.original_blocks() == 2 && tx.sequence().blocks.size() == 3);
        throw std::runtime_error("backend failure after reservation");
    } catch (const std::runtime_error&) {
    }
    CHECK(m.sequence("a").blocks == blocks && m.stats().kv_live_blocks == live);
    CHECK(throws_as<std::invalid_argument>([&] { m.prepare_append("a", {}); }));
    CHECK(throws_as<std::invalid_argument>([&] { m.prepare_append("a", {100}); }));
    CHECK(throws_as<std::invalid_argument>([&] { m.prepare_append("a", std::vector<TokenId>(14, 1)); }));
    commit(m, "a", {4, 5});
    CHECK(m.stats().forward_tokens == 5);
    m.release("a");
    CHECK(m.stats().kv_live_blocks == 0);
    m.clear();
    CHECK(m.stats().forward_tokens == 5);  // cumulative
}

static void prefix_and_reset() {
    KVManager m({2, 8, 3}, 2, 4, 16, 100);
    m.create("source");
    commit(m, "source", {1, 2, 3, 4, 5});
    m.cache_prefix("source");
    m.release("source");
    CHECK(m.stats().kv_cache_only_blocks == 3 && m.stats().kv_live_blocks == 3);
    m.create("a");
    CHECK(m.reuse_prefix("a", {1, 2, 3, 4, 6}) == 4);
    const int first = m.sequence("a").blocks[0];
    m.create("b");
    CHECK(m.reuse_prefix("b", {1, 2, 3, 4, 7}) == 4);
    CHECK(m.sequence("b").blocks[0] == first && m.stats().kv_live_blocks == 3);
    CHECK(m.offset(m.sequence("a"), 1, 2) == (std::size_t(m.sequence("a").blocks[1]) * 2 + 1) * 2 * 4);
    m.reset_sequence("a");
    CHECK(m.sequence("a").blocks.empty() && m.sequence("a").tokens.empty());
    CHECK(m.reuse_prefix("a", {1, 2, 3, 4, 6}) == 4);
    m.clear_prefix_cache();
    CHECK(m.stats().kv_cached_blocks == 0 && m.stats().kv_live_blocks == 2);
    commit(m, "a", {6});
    CHECK(m.sequence("b").used == 4);
    m.release("a");
    m.release("b");
    CHECK(m.stats().kv_live_blocks == 0);
    CHECK(m.stats().prefix_hits == 3 && m.stats().prefix_reused_tokens == 12);
    CHECK(m.stats().forward_tokens == 6);
}

static void eviction_under_pressure() {
    {
        KVManager m({2, 3, 2}, 1, 1, 16, 100);
        m.create("source");
        commit(m, "source", {1, 2, 3, 4});
        m.cache_prefix("source");
        m.release("source");
        m.create("active");
        CHECK(m.reuse_prefix("active", {1, 2, 3, 4, 5}) == 4);
        commit(m, "active", {5});
        m.create("next");
        CHECK(throws([&] { m.prepare_append("next", {7}); }));
        CHECK(m.sequence("next").blocks.empty() && m.sequence("active").used == 5);
        CHECK(m.stats().kv_cached_blocks == 0 && m.stats().kv_live_blocks == 3);
        m.release("active");
        commit(m, "next", {7});
        CHECK(m.stats().forward_tokens == 6 && m.stats().prefix_evictions == 2);
    }
    {
        KVManager m({2, 4, 3}, 1, 1, 16, 100);
        m.create("source");
        commit(m, "source", {1, 2, 3, 4, 5, 6});
        m.cache_prefix("source");
        m.release("source");
        m.create("touch");
        CHECK(m.reuse_prefix("touch", {1, 2, 9}) == 2);
        m.release("touch");
        m.create("next");
        commit(m, "next", {7});
        commit(m, "next", {8});
        CHECK(m.stats().prefix_evictions == 0 && m.stats().kv_cached_blocks == 3);
        commit(m, "next", {9, 10});  // one more page: evict only the LRU
        CHECK(m.stats().prefix_evictions == 1 && m.stats().kv_cached_blocks == 2);
        CHECK(m.stats().kv_live_blocks == 4 && m.stats().kv_peak_blocks == 4);
        m.create("probe");
        CHECK(m.reuse_prefix("probe", {1, 2, 3, 4, 5, 6, 7}) == 2);
        CHECK(m.stats().prefix_hits == 2 && m.stats().prefix_reused_tokens == 4);
    }
    {
        KVManager m({2, 2, 2}, 1, 1, 8, 100);
        m.create("source");
        commit(m, "source", {1, 2, 3, 4});
        m.cache_prefix("source");
        m.release("source");
        m.create("next");
        CHECK(throws([&] { m.prepare_append("next", {100}); }));  // validation precedes eviction
        CHECK(m.stats().prefix_evictions == 0 && m.stats().kv_cached_blocks == 2);
        {
            auto tx = m.prepare_append("next", {5});
            CHECK(m.stats().prefix_evictions == 1 && m.stats().kv_live_blocks == 2);
        }  // rollback keeps the eviction
        CHECK(m.sequence("next").blocks.empty());
        CHECK(m.stats().kv_cached_blocks == 1 && m.stats().kv_live_blocks == 1 && m.stats().forward_tokens == 4);
        commit(m, "next", {5});
        CHECK(m.stats().prefix_evictions == 1);
    }
    for (int cache : {0, 2}) {
        KVManager m({2, 2, cache}, 1, 1, 8, 100);
        m.create("source");
        commit(m, "source", {1, 2, 3, 4});
        m.cache_prefix("source");
        m.release("source");
        m.create("next");
        bool exhausted = false;
        try {
            m.prepare_append("next", {1, 2, 3, 4, 5});
        } catch (const std::runtime_error& e) {
            exhausted = std::string(e.what()) == "paged KV block pool exhausted";  // ref: exact message
        }
        CHECK(exhausted && m.sequence("next").blocks.empty());
        CHECK(m.stats().kv_live_blocks == 0 && m.stats().prefix_evictions == std::size_t(cache));
        commit(m, "next", {1, 2, 3, 4});
        CHECK(m.stats().forward_tokens == 8);
    }
}

// ------------------------------------------------------- copy-on-write ----
static void cow_metadata_and_payload() {
    KVManager m({4, 4, 0}, 2, 3, 16, 100);
    CHECK(m.reserve_request("a", 8) == KvAdmission::Ready);
    CHECK(m.reserve_request("b", 8) == KvAdmission::Ready);
    m.create("a");
    m.create("b");
    commit(m, "a", {1, 2, 3});
    m.fork_sequence("a", "b");
    const auto original = m.sequence("b").blocks;
    CHECK(m.stats().kv_live_blocks == 1);
    CHECK(m.reserve_request("third", 1) == KvAdmission::Wait);
    for (int attempt = 0; attempt < 2; ++attempt) {
        auto tx = m.prepare_append("b", {4, 5});
        CHECK(tx.tail_copy() && tx.tail_copy()->valid_tokens == 3);
        CHECK(m.stats().kv_live_blocks == 3);
        CHECK(throws([&] { tx.commit(); }));  // payload not copied yet
        int calls = 0;
        CHECK(throws([&] {
            tx.copy_shared_tail([&](std::size_t dst, std::size_t src, std::size_t n) {
                CHECK(n == 9 && dst != src);
                if (++calls == 2) throw std::runtime_error("copy failure");
            });
        }));
        CHECK(throws([&] { tx.commit(); }));
        tx.rollback();
        CHECK(m.sequence("b").blocks == original && m.sequence("b").used == 3);
        CHECK(m.stats().kv_live_blocks == 1 && m.stats().forward_tokens == 3);
    }
    {
        auto tx = m.prepare_append("b", {4, 5});
        int regions = 0;
        tx.copy_shared_tail_region([&](const KVManager::TailCopyRegion& r) {
            CHECK(r.rows == 2 && r.pitch == 12 && r.width == 9);  // ref: region geometry
            ++regions;
        });
        CHECK(regions == 1);
        tx.commit();
    }
    CHECK(m.sequence("a").blocks == original && m.sequence("a").used == 3);
    {
        auto tx = m.prepare_append("a", {6, 7});
        CHECK(!tx.tail_copy());  // now exclusive
        tx.commit();
    }
    CHECK(m.stats().kv_live_blocks == 4);
    m.clear();
    CHECK(m.stats().kv_live_blocks == 0);
    KVManager small({4, 1, 0}, 1, 1, 8, 100);
    small.create("a");
    small.create("b");
    commit(small, "a", {1});
    CHECK(throws([&] { small.fork_sequence("a", "b"); }));
    CHECK(small.sequence("b").blocks.empty());
}

// ------------------------------------------------------------ prefix -----
// Brute-force flat index: one entry per published page keyed by the whole
// token history through that page; LRU by a logical clock; on equal match
// length the lexicographic successor side of the query wins (lower_bound
// neighbour), then the nearest key.
class FlatPrefixIndex {
    struct Entry { int block; std::uint64_t touched; };
    KvBlockPool& pool_;
    std::map<std::vector<std::int32_t>, Entry> entries_;
    std::uint64_t clock_ = 0;
public:
    std::size_t hits = 0, misses = 0, reused = 0, evictions = 0;
    explicit FlatPrefixIndex(KvBlockPool& pool) : pool_(pool) {}
    ~FlatPrefixIndex() { clear(); }
    std::size_t size() const { return entries_.size(); }
    std::size_t cache_only() const {
        std::map<int, std::size_t> leases;
        for (const auto& e : entries_) ++leases[e.second.block];
        std::size_t n = 0;
        for (const auto& l : leases) n += pool_.references(l.first) == l.second;
        return n;
    }
    void clear() {
        for (const auto& e : entries_) pool_.unref(e.second.block);
        entries_.clear();
    }
    bool evict_one() {
        if (entries_.empty()) return false;
        auto victim = entries_.begin();
        for (auto it = entries_.begin(); it != entries_.end(); ++it)
            if (it->second.touched < victim->second.touched) victim = it;
        pool_.unref(victim->second.block);
        entries_.erase(victim);
        ++evictions;
        return true;
    }
    int reuse(PagedSequence& s, const std::vector<std::int32_t>& prompt) {
        if (!pool_.config().prefix_cache_blocks) return 0;
        const std::size_t bt = std::size_t(pool_.config().block_tokens);
        const std::size_t limit = prompt.empty() ? 0 : prompt.size() - 1;
        std::vector<int> pages;
        std::size_t count = 0;
        while (count < limit) {
            const std::size_t want = std::min(bt, limit - count);
            const std::vector<std::int32_t> query(prompt.begin(), prompt.begin() + count + want);
            auto best = entries_.end();
            std::size_t matched = 0;
            for (auto it = entries_.begin(); it != entries_.end(); ++it) {
                const auto& key = it->first;
                if (key.size() <= count || key.size() > count + bt ||
                    !std::equal(key.begin(), key.begin() + count, prompt.begin()))
                    continue;
                std::size_t n = 0;
                while (n < want && count + n < key.size() && key[count + n] == prompt[count + n]) ++n;
                bool better = n > matched;
                if (n && n == matched) {
                    const bool right = !(key < query), best_right = !(best->first < query);
                    better = right != best_right ? right : (right ? key < best->first : best->first < key);
                }
                if (better) {
                    matched = n;
                    best = it;
                }
            }
            if (!matched) break;
            pages.push_back(best->second.block);
            best->second.touched = ++clock_;
            count += matched;
            if (matched != bt) break;
        }
        for (int p : pages) pool_.retain(p);
        s.blocks = pages;
        s.tokens.assign(prompt.begin(), prompt.begin() + count);
        s.used = int(count);
        if (count) {
            ++hits;
            reused += count;
        } else {
            ++misses;
        }
        return s.used;
    }
    void publish(const PagedSequence& s) {
        const std::size_t bt = std::size_t(pool_.config().block_tokens);
        const std::size_t count = std::min({s.blocks.size(), (std::size_t(s.used) + bt - 1) / bt,
                                            std::size_t(pool_.config().prefix_cache_blocks)});
        for (std::size_t i = 0; i < count; ++i) {
            std::vector<std::int32_t> key(s.tokens.begin(), s.tokens.begin() + std::min(std::size_t(s.used), (i + 1) * bt));
            auto found = entries_.find(key);
            if (found != entries_.end()) {
                found->second.touched = ++clock_;
                continue;
            }
            if (entries_.size() == std::size_t(pool_.config().prefix_cache_blocks)) evict_one();
            pool_.retain(s.blocks[i]);
            entries_.emplace(std::move(key), Entry{s.blocks[i], ++clock_});
        }
    }
};

static void grow(KvBlockPool& pool, PagedSequence& s, const std::vector<std::int32_t>& tokens) {
    pool.reserve(s, s.used + int(tokens.size()));
    s.tokens.insert(s.tokens.end(), tokens.begin(), tokens.end());
    s.used += int(tokens.size());
}

static void prefix_differential() {
    for (int capacity : {0, 1, 2, 5, 16}) {
        KvBlockPool left({2, 128, capacity}, 1, 1), right({2, 128, capacity}, 1, 1);
        ExactPrefixCache actual(left);
        FlatPrefixIndex expected(right);
        std::mt19937 random(7341 + capacity);
        for (int step = 0; step < 3000; ++step) {
            const auto action = random() % 7;
            if (action == 0) {
                CHECK(actual.evict_one() == expected.evict_one());
            } else if (action == 1) {
                actual.clear();
                expected.clear();
                CHECK(actual.index_nodes() == 0 && actual.key_token_bytes() == 0);
            } else {
                std::vector<std::int32_t> tokens;
                const int length = 1 + int(random() % 23);
                for (int i = 0; i < length; ++i) tokens.push_back(i < 4 ? int(random() % 2) : int(random() % 5));
                PagedSequence a, b;
                if (action < 4) {
                    grow(left, a, tokens);
                    grow(right, b, tokens);
                    actual.publish(a);
                    expected.publish(b);
                } else {
                    CHECK(actual.reuse(a, tokens) == expected.reuse(b, tokens));
                }
                CHECK(a.blocks == b.blocks && a.tokens == b.tokens && a.used == b.used);
                if (step % 3 == 0) CHECK(actual.evict_one() == expected.evict_one());
                for (int page = 0; page < 128; ++page) CHECK(left.references(page) == right.references(page));
                left.release(a);
                right.release(b);
            }
            CHECK(actual.size() == expected.size() && actual.hits() == expected.hits &&
                  actual.misses() == expected.misses && actual.evictions() == expected.evictions &&
                  actual.reused_tokens() == expected.reused && actual.cache_only_blocks() == expected.cache_only() &&
                  left.live_blocks() == right.live_blocks());
        }
        actual.clear();
        expected.clear();
        CHECK(left.live_blocks() == 0 && right.live_blocks() == 0 && actual.index_nodes() == 0);
    }
}

static void prefix_deep_path() {
    constexpr int depth = 8192;
    KvBlockPool pool({1, depth, depth}, 1, 1);
    ExactPrefixCache cache(pool);
    PagedSequence s;
    grow(pool, s, std::vector<std::int32_t>(depth, 1));
    cache.publish(s);
    pool.release(s);
    CHECK(cache.index_nodes() == std::size_t(depth));
    for (int i = 0; i < depth; ++i) CHECK(cache.evict_one());
    CHECK(cache.index_nodes() == 0 && pool.live_blocks() == 0);
    grow(pool, s, std::vector<std::int32_t>(depth, 2));
    cache.publish(s);
    pool.release(s);
    cache.clear();
    CHECK(cache.index_nodes() == 0 && pool.live_blocks() == 0);
}

// Lexicographic release order of clear(): observable through the free list.
static void prefix_clear_order() {
    KvBlockPool pool({2, 8, 8}, 1, 1);
    ExactPrefixCache cache(pool);
    PagedSequence x, y, z;
    grow(pool, x, {5, 5, 1});   // blocks 0, 1
    grow(pool, y, {1, 1, 9});   // blocks 2, 3
    grow(pool, z, {5, 5, 0});   // blocks 4, 5
    cache.publish(x);
    cache.publish(y);
    cache.publish(z);
    pool.release(x);
    pool.release(y);
    pool.release(z);
    // Free list now [7,6,4] (z's uncached first page went back). clear()
    // drops leases in pre-order [1,1](2) [9](3) [5,5](0) [0](5) [1](1).
    cache.clear();
    PagedSequence w;
    grow(pool, w, std::vector<std::int32_t>(16, 3));
    CHECK((w.blocks == std::vector<int>{1, 5, 0, 3, 2, 4, 6, 7}));
}

// ----------------------------------------------------------- scheduler ----
static void scheduler_policy() {
    Scheduler scheduler({4, 5, 3});
    CHECK(scheduler.admission_count(0, 8) == 4 && scheduler.admission_count(3, 8) == 1);
    CHECK(scheduler.admission_count(4, 8) == 0 && scheduler.admission_count(1, 0) == 0);
    auto plan = scheduler.plan({SchedulePhase::Prefill, SchedulePhase::Decode, SchedulePhase::Prefill,
                                SchedulePhase::Decode});
    const std::vector<std::size_t> indices = {1, 3, 0, 2}, counts = {1, 1, 3, 0};
    for (std::size_t i = 0; i < indices.size(); ++i) {
        CHECK(plan.order()[i].active_index == indices[i]);
        CHECK(plan.take_input(plan.order()[i].phase, 10) == counts[i]);
    }
    CHECK(!plan.has_budget());
    for (int size = 0; size <= 5; ++size)
        for (int mask = 0; mask < (1 << size); ++mask)
            for (int budget : {1, 2, 5, 12})
                for (int chunk : {1, 3, 8}) {
                    Scheduler s({5, budget, chunk});
                    std::vector<SchedulePhase> phases;
                    for (int i = 0; i < size; ++i)
                        phases.push_back(mask & (1 << i) ? SchedulePhase::Decode : SchedulePhase::Prefill);
                    std::vector<std::size_t> expected;
                    for (int i = 0; i < size; ++i) if (mask & (1 << i)) expected.push_back(std::size_t(i));
                    for (int i = 0; i < size; ++i) if (!(mask & (1 << i))) expected.push_back(std::size_t(i));
                    auto p = s.plan(phases);
                    int remaining = budget;
                    CHECK(p.order().size() == expected.size());
                    for (std::size_t j = 0; j < expected.size(); ++j) {
                        CHECK(p.order()[j].active_index == expected[j]);
                        CHECK(p.has_budget() == (remaining > 0));
                        if (!remaining) break;
                        const int suffix = int(expected[j]) * 2 + 1;
                        int want = 1;
                        if (phases[expected[j]] == SchedulePhase::Prefill) want = std::min({suffix, chunk, remaining});
                        CHECK(p.take_input(p.order()[j].phase, std::size_t(suffix)) == std::size_t(want));
                        remaining -= want;
                    }
                }
    CHECK(throws_as<std::invalid_argument>([] { Scheduler s({0, 1, 1}); }));
}

// -------------------------------------------------------------- engine ----
struct Call {
    RequestId id;
    std::size_t position;
    std::vector<TokenId> input;
};
class RecordingRunner final : public ModelRunner {
    ModelConfig config_;
public:
    std::map<RequestId, std::size_t> positions;
    std::vector<Call> calls;
    RequestId failing;
    int clear_calls = 0;
    RecordingRunner() {
        config_.context = 128;
        config_.vocabulary = 128;
    }
    const ModelConfig& config() const override { return config_; }
    int context_limit() const override { return 128; }
    void create(const RequestId& id) override { positions[id] = 0; }
    std::vector<float> append(const RequestId& id, const std::vector<TokenId>& tokens) override {
        calls.push_back({id, positions.at(id), tokens});
        positions[id] += tokens.size();
        if (id == failing) throw std::runtime_error("forward failed");
        std::vector<float> logits(128, 0.0f);
        logits[(tokens.back() + 1) % 128] = 1;
        return logits;
    }
    void release(const RequestId& id) override { positions.erase(id); }
    void clear() override {
        ++clear_calls;
        positions.clear();
    }
    RunnerStats stats() const override {
        RunnerStats s;
        s.kv_block_tokens = 4;
        return s;
    }
};

static void engine_order_and_events() {
    auto owned = std::make_unique<RecordingRunner>();
    RecordingRunner* runner = owned.get();
    Engine engine(std::move(owned), {2, 6, 4, 64});
    engine.submit({"a", {1, 2, 3, 4, 5, 6, 7}, {3, std::nullopt}});
    engine.submit({"b", {9}, {2, std::nullopt}});
    engine.submit({"c", {20, 21}, {1, std::nullopt}});
    CHECK(throws_as<std::invalid_argument>([&] { engine.submit({"a", {1}, {1, std::nullopt}}); }));
    std::vector<GenerationEvent> events;
    while (!engine.idle()) {
        engine.step();
        for (auto& e : engine.poll_events()) events.push_back(e);
    }
    // a: chunks of 4 then 2 (budget 6 shared with b's prompt); decode-first order.
    std::vector<std::string> trace;
    for (const auto& c : runner->calls)
        trace.push_back(c.id + ":" + std::to_string(c.position) + "+" + std::to_string(c.input.size()));
    const std::vector<std::string> expect = {"a:0+4", "b:0+1", "b:1+1", "a:4+3", "a:7+1", "c:0+2", "a:8+1"};
    CHECK(trace == expect);
    std::vector<std::string> got;
    for (const auto& e : events)
        got.push_back(e.request_id + ":" + (e.token_id ? std::to_string(*e.token_id) : "-") +
                      (e.finish_reason ? "!" : ""));
    const std::vector<std::string> expect_events = {"b:10", "b:11!", "a:8", "a:9", "c:22!", "a:10!"};
    CHECK(got == expect_events);
}

static void engine_failure_poisons() {
    auto owned = std::make_unique<RecordingRunner>();
    RecordingRunner* runner = owned.get();
    runner->failing = "b";
    Engine engine(std::move(owned), {2, 32, 16, 64});
    engine.submit({"a", {1}, {4, std::nullopt}});
    engine.submit({"b", {2}, {4, std::nullopt}});
    engine.submit({"c", {3}, {4, std::nullopt}});
    engine.step();
    const auto events = engine.poll_events();
    CHECK(engine.failed() && runner->clear_calls == 1);
    std::set<std::string> errors;
    for (const auto& e : events)
        if (e.finish_reason == FinishReason::Error) errors.insert(e.request_id);
    CHECK((errors == std::set<std::string>{"a", "b", "c"}));
    CHECK(throws([&] { engine.step(); }));
}

int main() {
    pool_ownership();
    reservations();
    transactions();
    prefix_and_reset();
    eviction_under_pressure();
    cow_metadata_and_payload();
    prefix_differential();
    prefix_deep_path();
    prefix_clear_order();
    scheduler_policy();
    engine_order_and_events();
    engine_failure_poisons();
    std::puts("host tests passed");
    return 0;
}
