// KV manager with the observable behaviour of the reference
// (miniprefix/src/kv/kv_manager.cpp:4-209): the same admission answers,
// errors and messages, and the same sequence of pool operations, so page
// tables and copy-on-write outcomes are identical.
//
// Design: one ordered map of entries per request id, each holding the id's
// reservation and/or its sequence. The pages held against the pool's
// capacity (all reservations plus the blocks of sequences without one) are
// kept as two running sums updated wherever a count changes, so admission
// and every append check capacity in O(1) instead of walking all requests.
#include "miniprefix/kv_manager.h"

#include <algorithm>

namespace miniprefix {

KVManager::KVManager(KvCacheConfig config, int layers, int width, int context, int vocabulary)
    : layers_(layers), width_(width), context_(context), vocabulary_(vocabulary), pool_(config, layers, width),
      prefix_(pool_) {
    if (context < 1 || vocabulary < 1) throw std::invalid_argument("invalid KV manager context/vocabulary");
}

KVManager::~KVManager() {
    for (auto& item : entries_)
        if (item.second.live) pool_.release(item.second.sequence);
    prefix_.clear();
}

std::size_t KVManager::pages_for(std::size_t tokens) const {
    const std::size_t page = static_cast<std::size_t>(config().block_tokens);
    return (tokens + page - 1) / page;
}

std::size_t KVManager::max_sequence_blocks() const { return pages_for(static_cast<std::size_t>(context_)); }

bool KVManager::contains(const RequestId& id) const {
    const auto it = entries_.find(id);
    return it != entries_.end() && it->second.live;
}

const KVManager::Entry& KVManager::live_entry(const RequestId& id) const {
    const auto it = entries_.find(id);
    if (it == entries_.end() || !it->second.live) throw std::out_of_range("unknown KV sequence");
    return it->second;
}

const PagedSequence& KVManager::sequence(const RequestId& id) const { return live_entry(id).sequence; }

void KVManager::require_no_append() const {
    if (append_open_) throw std::logic_error("KV append transaction is active");
}

KVManager::Entry& KVManager::idle_sequence(const RequestId& id) {
    require_no_append();
    Entry& entry = const_cast<Entry&>(live_entry(id));
    if (entry.appending) throw std::logic_error("sequence has an active KV append");
    return entry;
}

void KVManager::check_tokens(const std::vector<TokenId>& tokens, const char* message) const {
    for (const TokenId t : tokens)
        if (t < 0 || t >= vocabulary_) throw std::invalid_argument(message);
}

void KVManager::recount(const Entry& entry, std::size_t before) noexcept {
    if (!entry.live || entry.reservation) return;
    unreserved_blocks_ += entry.sequence.blocks.size();  // modular: the sum ends exact
    unreserved_blocks_ -= before;
}

KvAdmission KVManager::reserve_request(const RequestId& id, std::size_t max_tokens) {
    require_no_append();
    if (entries_.count(id)) throw std::invalid_argument("duplicate KV reservation");  // live or reserved
    if (!max_tokens || max_tokens > static_cast<std::size_t>(context_))
        throw std::invalid_argument("invalid KV reservation context");
    const std::size_t pages = pages_for(max_tokens);
    const std::size_t capacity = static_cast<std::size_t>(config().max_blocks);
    if (pages > capacity) return KvAdmission::Impossible;
    const std::size_t held = committed_pages();
    if (held > capacity || pages > capacity - held) return KvAdmission::Wait;
    entries_[id].reservation = pages;
    ++reservations_;
    reserved_pages_ += pages;
    return KvAdmission::Ready;
}

void KVManager::release_reservation(const RequestId& id) noexcept {
    const auto it = entries_.find(id);
    if (it == entries_.end() || !it->second.reservation) return;
    Entry& entry = it->second;
    reserved_pages_ -= *entry.reservation;
    --reservations_;
    entry.reservation.reset();
    if (entry.live) unreserved_blocks_ += entry.sequence.blocks.size();
    else entries_.erase(it);
}

void KVManager::create(const RequestId& id) {
    require_no_append();
    Entry& entry = entries_[id];
    if (entry.live) throw std::invalid_argument("sequence already exists");
    entry.live = true;
}

void KVManager::fork_sequence(const RequestId& source, const RequestId& target) {
    require_no_append();
    const Entry& from = live_entry(source);
    Entry& to = idle_sequence(target);
    PagedSequence& dst = to.sequence;
    if (source == target || dst.used || !dst.blocks.empty() || !dst.tokens.empty())
        throw std::invalid_argument("fork requires a distinct empty target");
    const std::size_t pages = from.sequence.blocks.size();
    if (to.reservation) {
        if (pages > *to.reservation) throw KvCapacityError("fork exceeds KV reservation");
    } else {
        const std::size_t held = committed_pages(), capacity = static_cast<std::size_t>(config().max_blocks);
        if (held > capacity || pages > capacity - held) throw KvCapacityError("fork exceeds unreserved KV capacity");
    }
    PagedSequence copy = from.sequence;  // any allocation failure precedes the new references
    for (const int block : copy.blocks) pool_.retain(block);
    dst = std::move(copy);
    recount(to, 0);
}

std::size_t KVManager::reuse_prefix(const RequestId& id, const std::vector<TokenId>& prompt) {
    if (prompt.empty() || prompt.size() > static_cast<std::size_t>(context_))
        throw std::invalid_argument("invalid prefix context");
    check_tokens(prompt, "invalid prefix token");
    Entry& entry = idle_sequence(id);
    ++costs_.lookup_calls;
    CostTimer timer(cost_timing_, costs_.lookup_ns);
    const std::size_t before = entry.sequence.blocks.size();
    const std::size_t reused = static_cast<std::size_t>(prefix_.reuse(entry.sequence, prompt));
    recount(entry, before);
    const char* refusal = nullptr;
    if (entry.reservation && entry.sequence.blocks.size() > *entry.reservation)
        refusal = "request exceeds KV reservation";
    else if (reservations_ && committed_pages() > static_cast<std::size_t>(config().max_blocks))
        refusal = "KV capacity reserved by active requests";
    if (refusal) {
        const std::size_t mapped = entry.sequence.blocks.size();
        pool_.release(entry.sequence);
        recount(entry, mapped);
        throw KvCapacityError(refusal);
    }
    return reused;
}

void KVManager::cache_prefix(const RequestId& id) {
    Entry& entry = idle_sequence(id);
    ++costs_.publish_calls;
    CostTimer timer(cost_timing_, costs_.publish_ns);
    prefix_.publish(entry.sequence);
}

void KVManager::clear_prefix_cache() {
    // Even a cache-only page may still be read by an open append's forward.
    require_no_append();
    prefix_.clear();
}

// Capacity for growing `entry` to `end` tokens: the reservation (or, for an
// unreserved sequence, the capacity nobody has reserved) must cover the new
// pages; cache leases are then dropped oldest first until the pool can hand
// out the new pages plus, when `cow`, a page to copy the shared tail into.
// A dropped lease may have been the tail's only other holder, in which case
// the tail is written in place and needs no copy.
void KVManager::make_room(Entry& entry, int end, bool& cow) {
    PagedSequence& s = entry.sequence;
    const std::size_t target = pages_for(static_cast<std::size_t>(end));
    const std::size_t fresh = target > s.blocks.size() ? target - s.blocks.size() : 0;
    if (reservations_) {
        if (entry.reservation) {
            if (target > *entry.reservation) throw KvCapacityError("request exceeds KV reservation");
        } else {
            const std::size_t held = committed_pages(), capacity = static_cast<std::size_t>(config().max_blocks);
            if (held > capacity || fresh > capacity - held)
                throw KvCapacityError("KV capacity reserved by active requests");
        }
    }
    while (pool_.free_blocks() < fresh + (cow ? 1 : 0) && prefix_.evict_one())
        if (cow && pool_.references(s.blocks.back()) == 1) cow = false;
    if (cow && pool_.free_blocks() < fresh + 1) throw KvCapacityError("paged KV block pool exhausted");
    pool_.reserve(s, end);
}

KVManager::Append::Append(KVManager& owner, const RequestId& id, const std::vector<TokenId>& tokens)
    : manager_(&owner), entry_(&owner.idle_sequence(id)), input_(tokens),
      blocks_before_(entry_->sequence.blocks.size()) {
    PagedSequence& s = entry_->sequence;
    if (tokens.empty() || tokens.size() > static_cast<std::size_t>(owner.context_ - s.used))
        throw std::invalid_argument("context overflow/empty input");
    owner.check_tokens(tokens, "invalid token");
    // Token capacity for commit() (which must not throw), grown geometrically
    // so that decode steps do not copy the whole history each time.
    const std::size_t need = static_cast<std::size_t>(s.used) + tokens.size();
    if (need > s.tokens.capacity()) s.tokens.reserve(std::max(need, 2 * s.tokens.capacity()));
    const int valid = s.used % owner.config().block_tokens;
    bool cow = valid != 0 && owner.pool_.references(s.blocks.back()) > 1;
    owner.make_room(*entry_, s.used + static_cast<int>(tokens.size()), cow);
    owner.recount(*entry_, blocks_before_);
    if (cow) {
        // make_room kept a free page for the copy target.
        const int shared = s.blocks[blocks_before_ - 1];
        const int fresh = owner.pool_.allocate();
        cow_ = TailCopy{shared, fresh, valid};
        s.blocks[blocks_before_ - 1] = fresh;
    }
    entry_->appending = true;
    owner.append_open_ = true;
}

KVManager::Append::~Append() { rollback(); }

const PagedSequence& KVManager::Append::sequence() const {
    if (!manager_) throw std::logic_error("KV append already finished");
    return entry_->sequence;
}

void KVManager::Append::copy_shared_tail(const std::function<void(std::size_t, std::size_t, std::size_t)>& copier) {
    copy_shared_tail_region([&](const TailCopyRegion& r) {
        for (std::size_t layer = 0; layer < r.rows; ++layer)
            copier(r.destination + layer * r.pitch, r.source + layer * r.pitch, r.width);
    });
}

void KVManager::Append::copy_shared_tail_region(const std::function<void(const TailCopyRegion&)>& copier) {
    if (!manager_) throw std::logic_error("KV append already finished");
    if (!cow_) return;
    cow_done_ = false;
    const std::size_t width = static_cast<std::size_t>(manager_->width_);
    const std::size_t span = static_cast<std::size_t>(manager_->config().block_tokens) * width;  // page x layer
    const std::size_t layers = static_cast<std::size_t>(manager_->layers_);
    const std::size_t block = span * layers;
    copier({static_cast<std::size_t>(cow_->destination) * block, static_cast<std::size_t>(cow_->source) * block, span,
            static_cast<std::size_t>(cow_->valid_tokens) * width, layers});
    cow_done_ = true;
}

void KVManager::Append::commit() {
    if (!manager_) throw std::logic_error("KV append already finished");
    if (cow_ && !cow_done_) throw std::logic_error("shared tail payload was not copied");
    PagedSequence& s = entry_->sequence;
    s.tokens.insert(s.tokens.end(), input_.begin(), input_.end());
    s.used += static_cast<int>(input_.size());
    manager_->forward_tokens_ += input_.size();
    if (cow_) manager_->pool_.unref(cow_->source);  // the sequence now holds the copy
    entry_->appending = false;
    manager_->append_open_ = false;
    manager_ = nullptr;
}

void KVManager::Append::rollback() noexcept {
    if (!manager_) return;
    KVManager& m = *manager_;
    PagedSequence& s = entry_->sequence;
    const std::size_t grown = s.blocks.size();
    m.pool_.rollback(s, blocks_before_);  // new pages first, newest first
    if (cow_) {
        s.blocks[blocks_before_ - 1] = cow_->source;
        m.pool_.unref(cow_->destination);
    }
    m.recount(*entry_, grown);
    entry_->appending = false;
    m.append_open_ = false;
    manager_ = nullptr;
}

void KVManager::reset_sequence(const RequestId& id) {
    Entry& entry = idle_sequence(id);
    const std::size_t before = entry.sequence.blocks.size();
    pool_.release(entry.sequence);
    recount(entry, before);
}

void KVManager::release(const RequestId& id) {
    require_no_append();
    const auto it = entries_.find(id);
    if (it == entries_.end() || !it->second.live) throw std::invalid_argument("unknown sequence");
    Entry& entry = it->second;
    if (entry.appending) throw std::logic_error("cannot release sequence during KV append");
    if (entry.reservation) {
        reserved_pages_ -= *entry.reservation;
        --reservations_;
    } else {
        unreserved_blocks_ -= entry.sequence.blocks.size();
    }
    pool_.release(entry.sequence);
    entries_.erase(it);
}

void KVManager::clear() {
    require_no_append();
    for (auto& item : entries_)
        if (item.second.live) pool_.release(item.second.sequence);
    entries_.clear();
    reservations_ = reserved_pages_ = unreserved_blocks_ = 0;
    prefix_.clear();
}

KvStats KVManager::stats() const {
    KvStats r;
    for (const auto& item : entries_) r.live_sequences += item.second.live ? 1 : 0;
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
