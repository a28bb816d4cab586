// KV manager (reference semantics: miniprefix/src/kv/kv_manager.cpp:4-209).
// Reservations are a logical ledger of worst-case pages; an append reserves
// pages (evicting cache leases LRU-first while short), swaps a shared partial
// tail for a fresh page to copy into, and only commits tokens on success.
#include "miniprefix/kv_manager.h"

#include <algorithm>

namespace miniprefix {

KVManager::KVManager(KvCacheConfig config, int layers, int width, int context, int vocabulary)
    : layers_(layers), width_(width), context_(context), vocabulary_(vocabulary), pool_(config, layers, width),
      prefix_(pool_) {
    if (context < 1 || vocabulary < 1) throw std::invalid_argument("invalid KV manager context/vocabulary");
}

KVManager::~KVManager() {
    for (auto& entry : sequences_) pool_.release(entry.second.sequence);
    prefix_.clear();
}

std::size_t KVManager::max_sequence_blocks() const {
    const std::size_t bt = static_cast<std::size_t>(config().block_tokens);
    return (static_cast<std::size_t>(context_) + bt - 1) / bt;
}

void KVManager::require_idle() const {
    if (append_active_) throw std::logic_error("KV append transaction is active");
}

KVManager::State& KVManager::idle_state(const RequestId& id) {
    require_idle();
    State& state = sequences_.at(id);
    if (state.appending) throw std::logic_error("sequence has an active KV append");
    return state;
}

void KVManager::validate_tokens(const std::vector<TokenId>& tokens) const {
    for (const TokenId t : tokens)
        if (t < 0 || t >= vocabulary_) throw std::invalid_argument("invalid token");
}

std::size_t KVManager::committed_blocks() const {
    std::size_t total = 0;
    for (const auto& r : reservations_) total += r.second;
    for (const auto& s : sequences_)
        if (!reservations_.count(s.first)) total += s.second.sequence.blocks.size();
    return total;
}

KvAdmission KVManager::reserve_request(const RequestId& id, std::size_t max_tokens) {
    require_idle();
    if (contains(id) || reservations_.count(id)) throw std::invalid_argument("duplicate KV reservation");
    if (!max_tokens || max_tokens > static_cast<std::size_t>(context_))
        throw std::invalid_argument("invalid KV reservation context");
    const std::size_t pages = 1 + (max_tokens - 1) / static_cast<std::size_t>(config().block_tokens);
    const std::size_t total = static_cast<std::size_t>(config().max_blocks);
    if (pages > total) return KvAdmission::Impossible;
    const std::size_t committed = committed_blocks();
    if (committed > total || pages > total - committed) return KvAdmission::Wait;
    reservations_.emplace(id, pages);
    return KvAdmission::Ready;
}

void KVManager::create(const RequestId& id) {
    require_idle();
    if (!sequences_.emplace(id, State{}).second) throw std::invalid_argument("sequence already exists");
}

void KVManager::fork_sequence(const RequestId& source, const RequestId& target) {
    require_idle();
    const PagedSequence& original = sequences_.at(source).sequence;
    PagedSequence& destination = idle_state(target).sequence;
    if (source == target || destination.used || !destination.blocks.empty() || !destination.tokens.empty())
        throw std::invalid_argument("fork requires a distinct empty target");
    const auto reservation = reservations_.find(target);
    if (reservation != reservations_.end()) {
        if (original.blocks.size() > reservation->second) throw KvCapacityError("fork exceeds KV reservation");
    } else {
        const std::size_t used = committed_blocks(), total = static_cast<std::size_t>(config().max_blocks);
        if (used > total || original.blocks.size() > total - used)
            throw KvCapacityError("fork exceeds unreserved KV capacity");
    }
    PagedSequence copy = original;  // host metadata first, then the page leases
    for (const int block : copy.blocks) pool_.retain(block);
    destination = std::move(copy);
}

std::size_t KVManager::reuse_prefix(const RequestId& id, const std::vector<TokenId>& prompt) {
    if (prompt.empty() || prompt.size() > static_cast<std::size_t>(context_))
        throw std::invalid_argument("invalid prefix context");
    for (const TokenId t : prompt)
        if (t < 0 || t >= vocabulary_) throw std::invalid_argument("invalid prefix token");
    PagedSequence& sequence = idle_state(id).sequence;
    ++costs_.lookup_calls;
    CostTimer timer(cost_timing_, costs_.lookup_ns);
    const std::size_t count = static_cast<std::size_t>(prefix_.reuse(sequence, prompt));
    const auto reservation = reservations_.find(id);
    if (reservation != reservations_.end() && sequence.blocks.size() > reservation->second) {
        pool_.release(sequence);
        throw KvCapacityError("request exceeds KV reservation");
    }
    if (!reservations_.empty() && committed_blocks() > static_cast<std::size_t>(config().max_blocks)) {
        pool_.release(sequence);
        throw KvCapacityError("KV capacity reserved by active requests");
    }
    return count;
}

void KVManager::cache_prefix(const RequestId& id) {
    PagedSequence& sequence = idle_state(id).sequence;
    ++costs_.publish_calls;
    CostTimer timer(cost_timing_, costs_.publish_ns);
    prefix_.publish(sequence);
}

void KVManager::clear_prefix_cache() {
    require_idle();
    // Cache-only pages may still be read by an in-flight append.
    for (const auto& s : sequences_)
        if (s.second.appending) throw std::logic_error("cannot clear prefix cache during KV append");
    prefix_.clear();
}

void KVManager::reserve_pages(const RequestId& id, PagedSequence& sequence, int end, bool& cow) {
    const std::size_t bt = static_cast<std::size_t>(config().block_tokens);
    const std::size_t count = (static_cast<std::size_t>(end) + bt - 1) / bt;
    const std::size_t required = count > sequence.blocks.size() ? count - sequence.blocks.size() : 0;
    if (!reservations_.empty()) {
        const auto found = reservations_.find(id);
        if (found != reservations_.end()) {
            if (count > found->second) throw KvCapacityError("request exceeds KV reservation");
        } else {
            const std::size_t committed = committed_blocks(), total = static_cast<std::size_t>(config().max_blocks);
            if (committed > total || required > total - committed)
                throw KvCapacityError("KV capacity reserved by active requests");
        }
    }
    // Evicting drops a cache lease, not necessarily a page; re-check after
    // each victim. If the tail was shared only with the cache and that lease
    // goes, it becomes exclusive and needs no copy.
    while (pool_.free_blocks() < required + static_cast<std::size_t>(cow) && prefix_.evict_one())
        if (cow && pool_.references(sequence.blocks.back()) == 1) cow = false;
    if (cow && pool_.free_blocks() < required + 1) throw KvCapacityError("paged KV block pool exhausted");
    pool_.reserve(sequence, end);
}

KVManager::Append::Append(KVManager& owner, const RequestId& id, const std::vector<TokenId>& tokens)
    : owner_(&owner), state_(&owner.idle_state(id)), tokens_(tokens),
      original_blocks_(state_->sequence.blocks.size()) {
    PagedSequence& sequence = state_->sequence;
    if (tokens.empty() || tokens.size() > static_cast<std::size_t>(owner.context_ - sequence.used))
        throw std::invalid_argument("context overflow/empty input");
    owner.validate_tokens(tokens);
    // Room for commit() to append without throwing, grown geometrically so
    // that a decode step does not copy the whole history.
    const std::size_t need = static_cast<std::size_t>(sequence.used) + tokens.size();
    if (need > sequence.tokens.capacity()) sequence.tokens.reserve(std::max(need, 2 * sequence.tokens.capacity()));
    const int valid = sequence.used % owner.config().block_tokens;
    bool cow = valid && owner.pool_.references(sequence.blocks.back()) > 1;
    owner.reserve_pages(id, sequence, sequence.used + static_cast<int>(tokens.size()), cow);
    if (cow) {
        // reserve_pages left room for the replacement after the new pages.
        const int shared = sequence.blocks[original_blocks_ - 1];
        const int fresh = owner.pool_.allocate();
        copy_ = TailCopy{shared, fresh, valid};
        sequence.blocks[original_blocks_ - 1] = fresh;
    }
    state_->appending = true;
    owner.append_active_ = true;
}

KVManager::Append::~Append() { rollback(); }

const PagedSequence& KVManager::Append::sequence() const {
    if (!owner_) throw std::logic_error("KV append already finished");
    return state_->sequence;
}

void KVManager::Append::copy_shared_tail(const std::function<void(std::size_t, std::size_t, std::size_t)>& copier) {
    copy_shared_tail_region([&](const TailCopyRegion& r) {
        for (std::size_t row = 0; row < r.rows; ++row)
            copier(r.destination + row * r.pitch, r.source + row * r.pitch, r.width);
    });
}

void KVManager::Append::copy_shared_tail_region(const std::function<void(const TailCopyRegion&)>& copier) {
    if (!owner_) throw std::logic_error("KV append already finished");
    if (!copy_) return;
    copied_ = false;
    const std::size_t pitch = static_cast<std::size_t>(owner_->config().block_tokens) *
                              static_cast<std::size_t>(owner_->width_);
    const std::size_t rows = static_cast<std::size_t>(owner_->layers_);
    copier({static_cast<std::size_t>(copy_->destination) * rows * pitch,
            static_cast<std::size_t>(copy_->source) * rows * pitch, pitch,
            static_cast<std::size_t>(copy_->valid_tokens) * static_cast<std::size_t>(owner_->width_), rows});
    copied_ = true;
}

void KVManager::Append::commit() {
    if (!owner_) throw std::logic_error("KV append already finished");
    if (copy_ && !copied_) throw std::logic_error("shared tail payload was not copied");
    PagedSequence& sequence = state_->sequence;
    sequence.tokens.insert(sequence.tokens.end(), tokens_.begin(), tokens_.end());
    sequence.used += static_cast<int>(tokens_.size());
    owner_->forward_tokens_ += tokens_.size();
    if (copy_) owner_->pool_.unref(copy_->source);
    state_->appending = false;
    owner_->append_active_ = false;
    owner_ = nullptr;
}

void KVManager::Append::rollback() noexcept {
    if (!owner_) return;
    owner_->pool_.rollback(state_->sequence, original_blocks_);
    if (copy_) {
        state_->sequence.blocks[original_blocks_ - 1] = copy_->source;
        owner_->pool_.unref(copy_->destination);
    }
    state_->appending = false;
    owner_->append_active_ = false;
    owner_ = nullptr;
}

void KVManager::reset_sequence(const RequestId& id) { pool_.release(idle_state(id).sequence); }

void KVManager::release(const RequestId& id) {
    require_idle();
    auto it = sequences_.find(id);
    if (it == sequences_.end()) throw std::invalid_argument("unknown sequence");
    if (it->second.appending) throw std::logic_error("cannot release sequence during KV append");
    pool_.release(it->second.sequence);
    sequences_.erase(it);
    reservations_.erase(id);
}

void KVManager::clear() {
    require_idle();
    for (const auto& s : sequences_)
        if (s.second.appending) throw std::logic_error("cannot clear sequences during KV append");
    for (auto& s : sequences_) pool_.release(s.second.sequence);  // id order
    sequences_.clear();
    prefix_.clear();
    reservations_.clear();
}

KvStats KVManager::stats() const {
    KvStats r;
    r.live_sequences = sequences_.size();
    r.forward_tokens = forward_tokens_;
    r.kv_block_tokens = static_cast<std::size_t>(config().block_tokens);
    r.kv_total_blocks = static_cast<std::size_t>(config().max_blocks);
    r.kv_live_blocks = pool_.live_blocks();
    r.kv_peak_blocks = pool_.peak_blocks();
    r.kv_reserved_bytes = pool_.reserved_bytes();
    r.live_kv_bytes = pool_.live_blocks() * pool_.block_bytes();
    r.peak_kv_bytes = pool_.peak_blocks() * pool_.block_bytes();
    r.prefix_cache_capacity = static_cast<std::size_t>(config().prefix_cache_blocks);
    r.kv_cached_blocks = prefix_.size();
    r.kv_cache_only_blocks = prefix_.cache_only_blocks();
    r.prefix_hits = prefix_.hits();
    r.prefix_misses = prefix_.misses();
    r.prefix_reused_tokens = prefix_.reused_tokens();
    r.prefix_evictions = prefix_.evictions();
    return r;
}

}  // namespace miniprefix
