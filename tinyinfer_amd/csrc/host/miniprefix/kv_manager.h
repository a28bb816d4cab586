// Sequence metadata, page references, prefix leases, reservations and the
// single open append transaction (reference interface:
// miniprefix/include/miniprefix/kv_manager.h:10-96). Payload, device tables
// and completion stay in the backend. Single-threaded.
#pragma once
#include "cost_stats.h"
#include "prefix_cache.h"
#include "request.h"
#include <functional>
#include <map>
#include <optional>

namespace miniprefix {

struct KvStats {
    std::size_t live_sequences = 0, live_kv_bytes = 0, peak_kv_bytes = 0, forward_tokens = 0;
    std::size_t kv_block_tokens = 0, kv_total_blocks = 0, kv_live_blocks = 0, kv_peak_blocks = 0;
    std::size_t kv_reserved_bytes = 0;
    std::size_t prefix_cache_capacity = 0, kv_cached_blocks = 0, kv_cache_only_blocks = 0;
    std::size_t prefix_hits = 0, prefix_misses = 0, prefix_reused_tokens = 0, prefix_evictions = 0;
};

class KVManager {
    // Everything known about one request id: its page reservation and/or
    // its sequence.
    struct Entry {
        std::optional<std::size_t> reservation;  // worst-case pages
        bool live = false;                       // a sequence exists
        bool appending = false;
        PagedSequence sequence;
    };

public:
    struct TailCopy {
        int source, destination, valid_tokens;
    };
    // Float-element offsets, pitch and width in ONE pool (K or V); rows are layers.
    struct TailCopyRegion {
        std::size_t destination, source, pitch, width, rows;
    };
    // One append: pages reserved and a shared partial tail swapped for a copy
    // target at construction; commit publishes the tokens; destruction or
    // rollback restores the original pages. The backend must finish device
    // work touching these pages before commit or rollback.
    class Append {
        friend class KVManager;
        Append(KVManager& owner, const RequestId& id, const std::vector<TokenId>& tokens);

    public:
        Append(const Append&) = delete;
        Append& operator=(const Append&) = delete;
        Append(Append&&) = delete;
        Append& operator=(Append&&) = delete;
        ~Append();
        const PagedSequence& sequence() const;
        std::size_t original_blocks() const { return blocks_before_; }
        const std::optional<TailCopy>& tail_copy() const { return cow_; }
        // One call per layer row; the copier copies BOTH K and V.
        void copy_shared_tail(const std::function<void(std::size_t, std::size_t, std::size_t)>& copier);
        // One call for the strided region; the copier copies BOTH K and V.
        void copy_shared_tail_region(const std::function<void(const TailCopyRegion&)>& copier);
        void commit();
        void rollback() noexcept;

    private:
        KVManager* manager_;  // null once finished
        Entry* entry_;
        std::vector<TokenId> input_;
        std::size_t blocks_before_;
        std::optional<TailCopy> cow_;
        bool cow_done_ = false;
    };

    KVManager(KvCacheConfig config, int layers, int width, int context, int vocabulary);
    KVManager(const KVManager&) = delete;
    KVManager& operator=(const KVManager&) = delete;
    ~KVManager();
    const KvCacheConfig& config() const { return pool_.config(); }
    int context_limit() const { return context_; }
    std::size_t reserved_bytes() const { return pool_.reserved_bytes(); }
    std::size_t max_sequence_blocks() const;
    bool contains(const RequestId& id) const;
    const PagedSequence& sequence(const RequestId& id) const;
    std::size_t offset(const PagedSequence& sequence, int layer, int token) const {
        return pool_.offset(sequence, layer, token, layers_, width_);
    }
    KvAdmission reserve_request(const RequestId& id, std::size_t max_tokens);
    void release_reservation(const RequestId& id) noexcept;
    void create(const RequestId& id);
    void fork_sequence(const RequestId& source, const RequestId& target);
    std::size_t reuse_prefix(const RequestId& id, const std::vector<TokenId>& prompt);
    void cache_prefix(const RequestId& id);
    void clear_prefix_cache();
    Append prepare_append(const RequestId& id, const std::vector<TokenId>& tokens) {
        return Append(*this, id, tokens);
    }
    void reset_sequence(const RequestId& id);
    void release(const RequestId& id);
    void clear();
    KvStats stats() const;
    void set_cost_timing(bool enabled) { cost_timing_ = enabled; }
    CostStats cost_stats() const { return costs_; }

private:
    void require_no_append() const;
    const Entry& live_entry(const RequestId& id) const;
    Entry& idle_sequence(const RequestId& id);
    void check_tokens(const std::vector<TokenId>& tokens, const char* message) const;
    std::size_t pages_for(std::size_t tokens) const;
    // Pages held against the pool's capacity: every reservation plus the
    // blocks of sequences without one. Kept as two running sums.
    std::size_t committed_pages() const { return reserved_pages_ + unreserved_blocks_; }
    // Updates the running sum after `entry`'s block count changed from `before`.
    void recount(const Entry& entry, std::size_t before) noexcept;
    void make_room(Entry& entry, int end, bool& cow);

    int layers_, width_, context_, vocabulary_;
    KvBlockPool pool_;
    ExactPrefixCache prefix_;
    std::map<RequestId, Entry> entries_;  // by id: clear() releases in id order
    std::size_t reservations_ = 0, reserved_pages_ = 0, unreserved_blocks_ = 0;
    std::size_t forward_tokens_ = 0;
    bool append_open_ = false;
    bool cost_timing_ = false;
    CostStats costs_;
};

}  // namespace miniprefix
