// Exact prefix cache with the observable behaviour of the reference
// (miniprefix/src/kv/prefix_cache.cpp:8-198).
//
// Storage: nodes live in one vector and refer to each other by index. A
// node's children are a vector sorted by edge (lexicographic token order),
// and the children that hold a lease form a second sorted vector. Recency
// is a doubly linked list through the leased nodes, oldest first (a use
// moves a node to the newest end; nothing allocates). Publishing keeps the
// node path of the previous publication as a hint: a hinted node is taken
// when it is still the child of the expected parent with the page's tokens
// (a pruned node has no parent), so consecutive publications of one history,
// or of histories sharing a prefix, find their pages without a search.
//
// The choices that decide which physical blocks a sequence receives, and
// therefore must match the reference exactly:
//  - reuse walks from the root one page at a time; at each level the leased
//    child with the longest common prefix with the query page is one of the
//    two leased children next to the query's position in sorted order, and
//    on equal length the one at or after that position wins (:118-137); a
//    match shorter than a page ends the walk;
//  - a reuse match and a publish of an already leased page count as uses,
//    in walk order; eviction takes strictly the least recently used lease;
//  - publishing an unleased page takes its block reference before evicting
//    for room, and the page being published is never the victim (:176-192);
//  - clear() releases leases in lexicographic pre-order of the tree
//    (:104-110), which fixes the pool's free-list order afterwards.
#include "miniprefix/prefix_cache.h"

#include <algorithm>

namespace miniprefix {
namespace {

using Edge = std::vector<std::int32_t>;

bool run_less(const std::int32_t* a, std::size_t na, const std::int32_t* b, std::size_t nb) {
    return std::lexicographical_compare(a, a + na, b, b + nb);
}

std::size_t common_prefix(const Edge& edge, const std::int32_t* query, std::size_t n) {
    const std::size_t limit = std::min(edge.size(), n);
    std::size_t i = 0;
    while (i < limit && edge[i] == query[i]) ++i;
    return i;
}

}  // namespace

class ExactPrefixCache::Tree {
public:
    static constexpr int kRoot = 0;
    static constexpr int kNone = -1;

private:
    struct Node {
        int parent = kNone;
        Edge edge;
        std::vector<int> children;  // sorted by edge
        std::vector<int> leased;    // the children holding a lease, sorted by edge
        int block = kNone;
        int older = kNone, newer = kNone;  // recency list of leased nodes
    };

    Node& at(int id) { return nodes_[static_cast<std::size_t>(id)]; }
    const Node& at(int id) const { return nodes_[static_cast<std::size_t>(id)]; }

    // First entry of a sorted list whose edge is not less than the run.
    template <class List>
    auto first_not_less(List& list, const std::int32_t* run, std::size_t n) const {
        return std::partition_point(list.begin(), list.end(), [&](int id) {
            const Edge& e = at(id).edge;
            return run_less(e.data(), e.size(), run, n);
        });
    }

public:

    explicit Tree(std::size_t blocks) : nodes_(1), leases_per_block_(blocks, 0) {}

    std::size_t leases() const { return leases_; }
    std::size_t live_nodes() const { return live_nodes_; }
    std::size_t key_tokens() const { return key_tokens_; }
    bool leased(int id) const { return at(id).block != kNone; }
    int block_of(int id) const { return at(id).block; }

    std::size_t cache_only_blocks(const KvBlockPool& pool) const {
        std::size_t count = 0;
        for (std::size_t b = 0; b < leases_per_block_.size(); ++b) {
            const std::size_t leases = leases_per_block_[b];
            if (leases && pool.references(static_cast<int>(b)) == leases) ++count;
        }
        return count;
    }

    // The child of `parent` whose edge is exactly the run, or kNone.
    int child(int parent, const std::int32_t* run, std::size_t n) const {
        const std::vector<int>& list = at(parent).children;
        const auto it = first_not_less(list, run, n);
        if (it == list.end()) return kNone;
        const Edge& e = at(*it).edge;
        return e.size() == n && std::equal(e.begin(), e.end(), run) ? *it : kNone;
    }

    int add_child(int parent, const std::int32_t* run, std::size_t n) {
        // Room for clear()'s traversal stack, which must not allocate.
        if (stack_.capacity() < live_nodes_ + 1) stack_.reserve(2 * (live_nodes_ + 1));
        int id;
        if (!free_.empty()) {
            id = free_.back();
            free_.pop_back();
        } else {
            id = static_cast<int>(nodes_.size());
            nodes_.emplace_back();
            free_.reserve(nodes_.size());  // prune() pushes slots back without allocating
        }
        Node& node = at(id);
        node.parent = parent;
        node.edge.assign(run, run + n);
        std::vector<int>& list = at(parent).children;
        list.insert(first_not_less(list, run, n), id);
        ++live_nodes_;
        key_tokens_ += n;
        return id;
    }

    // The leased child of `parent` sharing the longest prefix with the
    // query run, and that length (0: none).
    std::pair<int, std::size_t> best_leased_child(int parent, const std::int32_t* query, std::size_t n) const {
        const std::vector<int>& list = at(parent).leased;
        const auto it = first_not_less(list, query, n);
        int best = kNone;
        std::size_t length = 0;
        if (it != list.end()) {
            best = *it;
            length = common_prefix(at(best).edge, query, n);
        }
        if (it != list.begin()) {
            const int before = *std::prev(it);
            const std::size_t l = common_prefix(at(before).edge, query, n);
            if (l > length) {
                best = before;
                length = l;
            }
        }
        return {best, length};
    }

    // `id` when it is the child of `parent` whose edge is the run.
    bool is_child(int id, int parent, const std::int32_t* run, std::size_t n) const {
        if (id < 0 || static_cast<std::size_t>(id) >= nodes_.size()) return false;
        const Node& node = at(id);
        return node.parent == parent && node.edge.size() == n && std::equal(node.edge.begin(), node.edge.end(), run);
    }

    void lease(int id, int block) {
        Node& node = at(id);
        std::vector<int>& list = at(node.parent).leased;
        list.insert(first_not_less(list, node.edge.data(), node.edge.size()), id);
        node.block = block;
        link_newest(id);
        ++leases_per_block_[static_cast<std::size_t>(block)];
        ++leases_;
    }

    void touch(int id) {
        if (newest_ == id) return;
        unlink(id);
        link_newest(id);
    }

    std::vector<int>& hint() { return hint_; }

    // Drops the lease of `id` (one block reference) and removes the
    // unleased leaves this leaves behind, never `keep`.
    void unlease(KvBlockPool& pool, int id, int keep = kNone) noexcept {
        Node& node = at(id);
        std::vector<int>& list = at(node.parent).leased;
        list.erase(first_not_less(list, node.edge.data(), node.edge.size()));
        unlink(id);
        const int block = node.block;
        node.block = kNone;
        --leases_per_block_[static_cast<std::size_t>(block)];
        --leases_;
        pool.unref(block);
        prune(id, keep);
    }

    void evict_oldest(KvBlockPool& pool, int keep = kNone) noexcept { unlease(pool, oldest_, keep); }

    // Removes `id` and then its ancestors while they are unleased leaves.
    void prune(int id, int keep = kNone) noexcept {
        while (id != kRoot && id != keep && at(id).block == kNone && at(id).children.empty()) {
            Node& node = at(id);
            const int parent = node.parent;
            std::vector<int>& siblings = at(parent).children;
            siblings.erase(first_not_less(siblings, node.edge.data(), node.edge.size()));
            key_tokens_ -= node.edge.size();
            --live_nodes_;
            node.parent = kNone;
            node.edge.clear();
            free_.push_back(id);  // capacity: at most one slot per node ever made
            id = parent;
        }
    }

    // Releases every lease in lexicographic pre-order (depth first, children
    // in edge order), with a stack whose capacity add_child keeps ready.
    void clear(KvBlockPool& pool) noexcept {
        stack_.clear();
        const std::vector<int>& top = at(kRoot).children;
        stack_.insert(stack_.end(), top.rbegin(), top.rend());
        while (!stack_.empty()) {
            const int id = stack_.back();
            stack_.pop_back();
            const std::vector<int>& kids = at(id).children;
            stack_.insert(stack_.end(), kids.rbegin(), kids.rend());
            // Pruning below only removes this node or nodes already visited.
            if (leased(id)) unlease(pool, id);
        }
    }

private:
    void link_newest(int id) {
        Node& node = at(id);
        node.older = newest_;
        node.newer = kNone;
        if (newest_ != kNone) at(newest_).newer = id;
        else oldest_ = id;
        newest_ = id;
    }
    void unlink(int id) {
        Node& node = at(id);
        if (node.older != kNone) at(node.older).newer = node.newer;
        else oldest_ = node.newer;
        if (node.newer != kNone) at(node.newer).older = node.older;
        else newest_ = node.older;
        node.older = node.newer = kNone;
    }

    std::vector<Node> nodes_;  // nodes_[kRoot] is the empty root
    std::vector<int> free_;
    std::vector<int> stack_;
    std::vector<int> hint_;  // node path of the previous publication
    int oldest_ = kNone, newest_ = kNone;  // recency list ends
    std::vector<std::size_t> leases_per_block_;
    std::size_t leases_ = 0, live_nodes_ = 0, key_tokens_ = 0;
};

ExactPrefixCache::ExactPrefixCache(KvBlockPool& pool)
    : pool_(pool), tree_(std::make_unique<Tree>(static_cast<std::size_t>(pool.config().max_blocks))) {}

ExactPrefixCache::~ExactPrefixCache() { clear(); }

std::size_t ExactPrefixCache::size() const { return tree_->leases(); }
std::size_t ExactPrefixCache::index_nodes() const { return tree_->live_nodes(); }
std::size_t ExactPrefixCache::key_token_bytes() const { return tree_->key_tokens() * sizeof(std::int32_t); }
std::size_t ExactPrefixCache::cache_only_blocks() const { return tree_->cache_only_blocks(pool_); }

void ExactPrefixCache::clear() noexcept { tree_->clear(pool_); }

bool ExactPrefixCache::evict_one() {
    if (!tree_->leases()) return false;
    tree_->evict_oldest(pool_);
    ++evictions_;
    return true;
}

int ExactPrefixCache::reuse(PagedSequence& sequence, const std::vector<std::int32_t>& prompt) {
    if (sequence.used || !sequence.blocks.empty() || !sequence.tokens.empty())
        throw std::invalid_argument("prefix reuse requires an empty sequence");
    if (!pool_.config().prefix_cache_blocks) return 0;
    const std::size_t page = static_cast<std::size_t>(pool_.config().block_tokens);
    // The last prompt token is never taken from the cache: appending it
    // produces the logits of the next token.
    const std::size_t limit = prompt.empty() ? 0 : prompt.size() - 1;
    std::vector<int> blocks;
    std::size_t covered = 0;
    int parent = Tree::kRoot;
    while (covered < limit) {
        const std::size_t want = std::min(page, limit - covered);
        const auto match = tree_->best_leased_child(parent, prompt.data() + covered, want);
        if (!match.second) break;
        blocks.push_back(tree_->block_of(match.first));
        tree_->touch(match.first);
        covered += match.second;
        if (match.second < page) break;  // a partial page ends the path
        parent = match.first;
    }
    for (const int b : blocks) pool_.retain(b);
    sequence.blocks = std::move(blocks);
    sequence.tokens.assign(prompt.begin(), prompt.begin() + static_cast<std::ptrdiff_t>(covered));
    sequence.used = static_cast<int>(covered);
    if (covered) {
        ++hits_;
        reused_ += covered;
    } else {
        ++misses_;
    }
    return sequence.used;
}

void ExactPrefixCache::publish(const PagedSequence& sequence) {
    if (sequence.tokens.size() != static_cast<std::size_t>(sequence.used))
        throw std::logic_error("invalid committed KV token history");
    const std::size_t page = static_cast<std::size_t>(pool_.config().block_tokens);
    const std::size_t used = static_cast<std::size_t>(sequence.used);
    const std::size_t capacity = static_cast<std::size_t>(pool_.config().prefix_cache_blocks);
    const std::size_t pages = std::min({sequence.blocks.size(), (used + page - 1) / page, capacity});
    int parent = Tree::kRoot;
    std::vector<int>& hint = tree_->hint();
    if (hint.capacity() < pages) hint.reserve(pages);
    for (std::size_t i = 0; i < pages; ++i) {
        const std::int32_t* run = sequence.tokens.data() + i * page;
        const std::size_t length = std::min(page, used - i * page);
        int node = i < hint.size() && tree_->is_child(hint[i], parent, run, length) ? hint[i]
                                                                                    : tree_->child(parent, run, length);
        if (node == Tree::kNone) node = tree_->add_child(parent, run, length);
        if (tree_->leased(node)) {
            tree_->touch(node);
        } else {
            const int block = sequence.blocks[i];
            try {
                pool_.retain(block);  // before any eviction can release the same block
            } catch (...) {
                tree_->prune(node);
                throw;
            }
            if (tree_->leases() == capacity) {
                tree_->evict_oldest(pool_, node);
                ++evictions_;
            }
            tree_->lease(node, block);
        }
        if (i < hint.size()) hint[i] = node;
        else hint.push_back(node);
        parent = node;
    }
    hint.resize(pages);
}

}  // namespace miniprefix
