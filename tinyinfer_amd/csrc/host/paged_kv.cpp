// Physical page pool (reference semantics: miniprefix/src/kv/paged_kv.cpp:7-56).
#include "miniprefix/paged_kv.h"

#include <algorithm>
#include <limits>

namespace miniprefix {

KvBlockPool::KvBlockPool(KvCacheConfig config, int layers, int width) : config_(config) {
    if (config.block_tokens < 1 || config.max_blocks < 1 || layers < 1 || width < 1 ||
        config.prefix_cache_blocks < 0 || config.prefix_cache_blocks > config.max_blocks)
        throw std::invalid_argument("invalid paged KV configuration");
    // Both pools together must stay addressable in bytes.
    const std::size_t limit = std::numeric_limits<std::size_t>::max() / sizeof(float) / 2;
    std::size_t total = static_cast<std::size_t>(layers);
    for (const int factor : {config.block_tokens, width, config.max_blocks}) {
        if (total > limit / static_cast<std::size_t>(factor)) throw std::invalid_argument("paged KV size overflow");
        total *= static_cast<std::size_t>(factor);
    }
    block_elements_ = total / static_cast<std::size_t>(config.max_blocks);
    refs_.assign(static_cast<std::size_t>(config.max_blocks), 0);
    // LIFO: the back of the list is handed out first, so block 0 goes first.
    free_.resize(static_cast<std::size_t>(config.max_blocks));
    for (int i = 0; i < config.max_blocks; ++i) free_[static_cast<std::size_t>(i)] = config.max_blocks - 1 - i;
}

void KvBlockPool::take(int block) {
    refs_[static_cast<std::size_t>(block)] = 1;
    ++live_;
}

int KvBlockPool::allocate() {
    if (free_.empty()) throw KvCapacityError("paged KV block pool exhausted");
    const int block = free_.back();
    free_.pop_back();
    take(block);
    peak_ = std::max(peak_, live_);
    return block;
}

void KvBlockPool::retain(int block) { ++refs_.at(static_cast<std::size_t>(block)); }

void KvBlockPool::unref(int block) noexcept {
    auto& count = refs_[static_cast<std::size_t>(block)];
    if (--count == 0) {
        free_.push_back(block);
        --live_;
    }
}

void KvBlockPool::reserve(PagedSequence& sequence, int end) {
    if (end < sequence.used) throw std::invalid_argument("paged KV cannot truncate through reserve");
    const std::size_t bt = static_cast<std::size_t>(config_.block_tokens);
    const std::size_t needed = (static_cast<std::size_t>(end) + bt - 1) / bt;
    if (needed <= sequence.blocks.size()) return;
    const std::size_t extra = needed - sequence.blocks.size();
    if (extra > free_.size()) throw KvCapacityError("paged KV block pool exhausted");
    sequence.blocks.reserve(needed);
    for (std::size_t i = 0; i < extra; ++i) {
        const int block = free_.back();
        free_.pop_back();
        sequence.blocks.push_back(block);
        take(block);
    }
    peak_ = std::max(peak_, live_);
}

void KvBlockPool::rollback(PagedSequence& sequence, std::size_t original_blocks) noexcept {
    while (sequence.blocks.size() > original_blocks) {
        unref(sequence.blocks.back());
        sequence.blocks.pop_back();
    }
}

void KvBlockPool::release(PagedSequence& sequence) noexcept {
    rollback(sequence, 0);
    sequence.used = 0;
    sequence.tokens.clear();
}

std::size_t KvBlockPool::offset(const PagedSequence& sequence, int layer, int token, int layers, int width) const {
    const std::size_t bt = static_cast<std::size_t>(config_.block_tokens);
    const std::size_t page = static_cast<std::size_t>(token) / bt, slot = static_cast<std::size_t>(token) % bt;
    const std::size_t block = static_cast<std::size_t>(sequence.blocks.at(page));
    return ((block * static_cast<std::size_t>(layers) + static_cast<std::size_t>(layer)) * bt + slot) *
           static_cast<std::size_t>(width);
}

}  // namespace miniprefix
