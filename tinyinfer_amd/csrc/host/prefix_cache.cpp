// Exact prefix cache (reference semantics: miniprefix/src/kv/prefix_cache.cpp:8-198).
//
// Each trie node stands for one page of tokens below its parent's path; the
// final edge of a path may be shorter than a page. A node may hold one cache
// lease on the physical page that stores its tokens. Nodes with a lease sit
// in an LRU list and in their parent's ordered index of leased children,
// which answers "longest common prefix with this query page" from the two
// lexicographic neighbours of the query. Observable choices that feed the
// page allocator follow the reference exactly: eviction is strict LRU,
// clear() releases leases in lexicographic pre-order, ties on reuse prefer
// the lower_bound neighbour.
#include "miniprefix/prefix_cache.h"

#include <algorithm>
#include <iterator>
#include <map>

namespace miniprefix {
namespace {

struct Span {
    const std::int32_t* begin;
    const std::int32_t* end;
};
inline Span span_of(const std::vector<std::int32_t>& v) { return {v.data(), v.data() + v.size()}; }
inline Span span_of(const std::vector<std::int32_t>* v) { return span_of(*v); }
inline Span span_of(const Span& s) { return s; }

// Lexicographic order over token runs, usable with spans and vectors.
struct TokenOrder {
    using is_transparent = void;
    template <class A, class B>
    bool operator()(const A& a, const B& b) const {
        const Span x = span_of(a), y = span_of(b);
        return std::lexicographical_compare(x.begin, x.end, y.begin, y.end);
    }
};

}  // namespace

struct ExactPrefixCache::Trie {
    struct Node {
        Node* parent = nullptr;
        const std::vector<std::int32_t>* edge = nullptr;  // key in parent->children
        std::map<std::vector<std::int32_t>, std::unique_ptr<Node>, TokenOrder> children;
        std::map<const std::vector<std::int32_t>*, Node*, TokenOrder> leased;
        int block = -1;
        Node* older = nullptr;
        Node* newer = nullptr;
    };

    explicit Trie(std::size_t blocks) : leases(blocks, 0) {}

    Node root;
    Node* oldest = nullptr;
    Node* newest = nullptr;
    std::size_t cached = 0, nodes = 0, key_tokens = 0;
    std::vector<std::size_t> leases;  // cache leases per physical page

    void lru_remove(Node& n) noexcept {
        (n.older ? n.older->newer : oldest) = n.newer;
        (n.newer ? n.newer->older : newest) = n.older;
        n.older = n.newer = nullptr;
    }
    void lru_push(Node& n) noexcept {
        n.older = newest;
        n.newer = nullptr;
        (newest ? newest->newer : oldest) = &n;
        newest = &n;
    }
    void touch(Node& n) noexcept {
        lru_remove(n);
        lru_push(n);
    }
    // Removes empty leaves upward from n, never `keep` or the root.
    void prune(Node* n, Node* keep) noexcept {
        while (n != &root && n != keep && n->block < 0 && n->children.empty()) {
            Node* parent = n->parent;
            key_tokens -= n->edge->size();
            --nodes;
            parent->children.erase(parent->children.find(*n->edge));
            n = parent;
        }
    }
    void drop_lease(KvBlockPool& pool, Node& n, Node* keep = nullptr) noexcept {
        n.parent->leased.erase(n.edge);
        --leases[static_cast<std::size_t>(n.block)];
        lru_remove(n);
        pool.unref(n.block);
        n.block = -1;
        --cached;
        prune(&n, keep);
    }
    // Next node in lexicographic pre-order, or null.
    Node* next_preorder(Node* n) noexcept {
        if (!n->children.empty()) return n->children.begin()->second.get();
        while (n != &root) {
            Node* parent = n->parent;
            auto it = parent->children.upper_bound(*n->edge);
            if (it != parent->children.end()) return it->second.get();
            n = parent;
        }
        return nullptr;
    }
};

ExactPrefixCache::ExactPrefixCache(KvBlockPool& pool)
    : pool_(pool), trie_(std::make_unique<Trie>(static_cast<std::size_t>(pool.config().max_blocks))) {}

ExactPrefixCache::~ExactPrefixCache() { clear(); }

std::size_t ExactPrefixCache::size() const { return trie_->cached; }
std::size_t ExactPrefixCache::index_nodes() const { return trie_->nodes; }
std::size_t ExactPrefixCache::key_token_bytes() const { return trie_->key_tokens * sizeof(std::int32_t); }

std::size_t ExactPrefixCache::cache_only_blocks() const {
    std::size_t count = 0;
    for (std::size_t b = 0; b < trie_->leases.size(); ++b)
        if (trie_->leases[b] && pool_.references(static_cast<int>(b)) == trie_->leases[b]) ++count;
    return count;
}

bool ExactPrefixCache::evict_one() {
    if (!trie_->oldest) return false;
    trie_->drop_lease(pool_, *trie_->oldest);
    ++evictions_;
    return true;
}

void ExactPrefixCache::clear() noexcept {
    Trie& t = *trie_;
    Trie::Node* n = t.root.children.empty() ? nullptr : t.root.children.begin()->second.get();
    while (n) {
        Trie::Node* next = t.next_preorder(n);  // before pruning can free n
        if (n->block >= 0) t.drop_lease(pool_, *n);
        n = next;
    }
}

int ExactPrefixCache::reuse(PagedSequence& sequence, const std::vector<std::int32_t>& prompt) {
    if (sequence.used || !sequence.blocks.empty() || !sequence.tokens.empty())
        throw std::invalid_argument("prefix reuse requires an empty sequence");
    if (!pool_.config().prefix_cache_blocks) return 0;
    const std::size_t bt = static_cast<std::size_t>(pool_.config().block_tokens);
    // One prompt token always stays uncached so the append produces logits.
    const std::size_t limit = prompt.empty() ? 0 : prompt.size() - 1;
    std::vector<int> pages;
    Trie::Node* parent = &trie_->root;
    std::size_t matched_total = 0;
    while (matched_total < limit) {
        const std::size_t want = std::min(bt, limit - matched_total);
        const Span query{prompt.data() + matched_total, prompt.data() + matched_total + want};
        auto it = parent->leased.lower_bound(query);
        Trie::Node* best = nullptr;
        std::size_t best_len = 0;
        auto consider = [&](Trie::Node* candidate) {
            const auto& edge = *candidate->edge;
            std::size_t n = 0;
            while (n < want && n < edge.size() && edge[n] == query.begin[n]) ++n;
            if (n > best_len) {
                best_len = n;
                best = candidate;
            }
        };
        if (it != parent->leased.end()) consider(it->second);
        if (it != parent->leased.begin()) consider(std::prev(it)->second);
        if (!best_len) break;
        pages.push_back(best->block);
        trie_->touch(*best);
        matched_total += best_len;
        if (best_len != bt) break;  // a partial match ends the walk
        parent = best;
    }
    for (const int page : pages) pool_.retain(page);
    sequence.blocks = std::move(pages);
    sequence.tokens.assign(prompt.begin(), prompt.begin() + static_cast<std::ptrdiff_t>(matched_total));
    sequence.used = static_cast<int>(matched_total);
    if (matched_total) {
        ++hits_;
        reused_ += matched_total;
    } else {
        ++misses_;
    }
    return sequence.used;
}

void ExactPrefixCache::publish(const PagedSequence& sequence) {
    if (sequence.tokens.size() != static_cast<std::size_t>(sequence.used))
        throw std::logic_error("invalid committed KV token history");
    Trie& t = *trie_;
    const std::size_t bt = static_cast<std::size_t>(pool_.config().block_tokens);
    const std::size_t used = static_cast<std::size_t>(sequence.used);
    const std::size_t capacity = static_cast<std::size_t>(pool_.config().prefix_cache_blocks);
    const std::size_t pages = std::min({sequence.blocks.size(), (used + bt - 1) / bt, capacity});
    Trie::Node* parent = &t.root;
    for (std::size_t i = 0; i < pages; ++i) {
        const std::int32_t* first = sequence.tokens.data() + i * bt;
        const std::size_t length = std::min(bt, used - i * bt);
        const Span key{first, first + length};
        auto found = parent->children.find(key);
        if (found == parent->children.end()) {
            auto node = std::make_unique<Trie::Node>();
            found = parent->children.emplace(std::vector<std::int32_t>(first, first + length), std::move(node)).first;
            found->second->parent = parent;
            found->second->edge = &found->first;
            ++t.nodes;
            t.key_tokens += length;
        }
        Trie::Node& node = *found->second;
        if (node.block >= 0) {
            t.touch(node);
        } else {
            const int page = sequence.blocks[i];
            parent->leased.emplace(node.edge, &node);
            pool_.retain(page);
            if (t.cached == capacity) {
                t.drop_lease(pool_, *t.oldest, &node);
                ++evictions_;
            }
            ++t.leases[static_cast<std::size_t>(page)];
            node.block = page;
            t.lru_push(node);
            ++t.cached;
        }
        parent = &node;
    }
}

}  // namespace miniprefix
