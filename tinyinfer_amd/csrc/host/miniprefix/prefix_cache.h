// Exact token-page trie with variable-length final edges, an LRU of cache
// leases and per-node lexicographic indexes of leased children (reference:
// miniprefix/include/miniprefix/prefix_cache.h:9-34).
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
    std::size_t size() const;
    std::size_t index_nodes() const;
    std::size_t key_token_bytes() const;
    std::size_t hits() const { return hits_; }
    std::size_t misses() const { return misses_; }
    std::size_t reused_tokens() const { return reused_; }
    std::size_t evictions() const { return evictions_; }
    std::size_t cache_only_blocks() const;
    void clear() noexcept;
    // Maps the longest cached prefix of prompt[0, size-1) into an empty sequence.
    int reuse(PagedSequence& sequence, const std::vector<std::int32_t>& prompt);
    void publish(const PagedSequence& sequence);
    // Drops the least recently used cache lease; false when there is none.
    bool evict_one();

private:
    struct Trie;
    KvBlockPool& pool_;
    std::unique_ptr<Trie> trie_;
    std::size_t hits_ = 0, misses_ = 0, reused_ = 0, evictions_ = 0;
};

}  // namespace miniprefix
