// Exact prefix cache over token pages (reference interface:
// miniprefix/include/miniprefix/prefix_cache.h:9-34).
//
// A cached history is a path of pages from an empty root; each node stands
// for one page of tokens below its parent's path, and only the last page of
// a path may be shorter than a page. A node may hold one cache lease on the
// physical block that stores its tokens. Nodes without a lease survive only
// as ancestors of nodes that still have one.
#pragma once
#include "paged_kv.h"
#include <memory>

namespace miniprefix {

class ExactPrefixCache {
public:
    explicit ExactPrefixCache(KvBlockPool& pool);
    ExactPrefixCache(const ExactPrefixCache&) = delete;
    ExactPrefixCache& operator=(const ExactPrefixCache&) = delete;
    ~ExactPrefixCache();
    // Cache leases held.
    std::size_t size() const;
    // Nodes of the page tree (leased or not), and the tokens their edges hold.
    std::size_t index_nodes() const;
    std::size_t key_token_bytes() const;
    std::size_t hits() const { return hits_; }
    std::size_t misses() const { return misses_; }
    std::size_t reused_tokens() const { return reused_; }
    std::size_t evictions() const { return evictions_; }
    // Blocks whose only references are cache leases.
    std::size_t cache_only_blocks() const;
    void clear() noexcept;
    // Maps the longest cached prefix of prompt[0, size-1) into an empty
    // sequence (retaining its blocks) and returns the tokens it covers.
    int reuse(PagedSequence& sequence, const std::vector<std::int32_t>& prompt);
    // Leases every page of the committed history (up to the capacity).
    void publish(const PagedSequence& sequence);
    // Drops the least recently used cache lease; false when there is none.
    bool evict_one();

private:
    class Tree;
    KvBlockPool& pool_;
    std::unique_ptr<Tree> tree_;
    std::size_t hits_ = 0, misses_ = 0, reused_ = 0, evictions_ = 0;
};

}  // namespace miniprefix
