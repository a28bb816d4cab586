// Paged KV ownership (reference: miniprefix/include/miniprefix/paged_kv.h:8-51).
// Storage of one pool is [physical block][layer][slot][kv width]. The block
// pool hands out pages from a LIFO free list initialised so block 0 comes
// first, counts references, and reserves atomically.
#pragma once
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <vector>

namespace miniprefix {

class KvCapacityError : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

enum class KvAdmission { Ready, Wait, Impossible };

struct KvCacheConfig {
    int block_tokens = 16;
    int max_blocks = 128;
    int prefix_cache_blocks = 0;
};

// Complete pages are immutable; a shared partial tail is copied before writes.
struct PagedSequence {
    int used = 0;
    std::vector<int> blocks;
    std::vector<std::int32_t> tokens;
};

class KvBlockPool {
public:
    KvBlockPool(KvCacheConfig config, int layers, int width);
    const KvCacheConfig& config() const { return config_; }
    std::size_t block_elements() const { return block_elements_; }
    std::size_t block_bytes() const { return block_elements_ * sizeof(float) * 2; }
    std::size_t reserved_bytes() const { return block_bytes() * static_cast<std::size_t>(config_.max_blocks); }
    std::size_t live_blocks() const { return live_; }
    std::size_t peak_blocks() const { return peak_; }
    std::size_t free_blocks() const { return free_.size(); }
    std::size_t references(int block) const { return refs_.at(static_cast<std::size_t>(block)); }
    int allocate();
    void retain(int block);
    void unref(int block) noexcept;
    // Grows `sequence` to cover `end` tokens; all-or-nothing.
    void reserve(PagedSequence& sequence, int end);
    void rollback(PagedSequence& sequence, std::size_t original_blocks) noexcept;
    void release(PagedSequence& sequence) noexcept;
    std::size_t offset(const PagedSequence& sequence, int layer, int token, int layers, int width) const;

private:
    void take(int block);
    KvCacheConfig config_;
    std::size_t block_elements_ = 0, live_ = 0, peak_ = 0;
    std::vector<int> free_;
    std::vector<std::size_t> refs_;
};

}  // namespace miniprefix
