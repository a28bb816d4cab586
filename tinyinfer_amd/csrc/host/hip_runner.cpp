// HipRunner: the ModelRunner over the device backend's C ABI (include/mp_hip.h).
// It owns one KVManager, as the reference's CudaRunner does
// (miniprefix/src/backend/cuda/llama_runner.cu:51-186), and keeps its
// transaction discipline: prepare, copy the shared tail, upload new table
// entries, forward, synchronize, check, then commit -- or roll back and mark
// the device table dirty.
//
// It also implements StagedRunner (staged_runner.h): stage() commits the
// transaction and queues the forward; run_staged() computes the queued
// forwards in one device pass.
//
// The file builds against this repository's headers and, unchanged, against
// the reference's (miniprefix/include/miniprefix/model.h, with weights held
// as tinyinfer::Tensor): it uses only the reference's ModelRunner, KVManager
// and ModelWeights interfaces, reads tensors through numel() and data<float>(),
// and brings its own extension header.
#include "miniprefix/model.h"

#include "mp_hip.h"
#include "staged_runner.h"

#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace miniprefix {
namespace {

class HipRunner final : public ModelRunner, public StagedRunner {
public:
    HipRunner(std::shared_ptr<ModelWeights> weights, int context, KvCacheConfig kv, int arithmetic)
        : weights_(std::move(weights)),
          kv_(kv, config().layers, config().kv_width(), context, config().vocabulary) {
        if (context < 1 || context > config().context) throw std::invalid_argument("invalid runner context");
        const ModelConfig& c = config();
        const mp_model_desc m{c.layers, c.hidden, c.intermediate, c.heads, c.kv_heads, c.vocabulary, context,
                              c.rms_epsilon, c.rope_theta, c.tied ? 1 : 0, arithmetic};
        table_entries_ = static_cast<int>(kv_.max_sequence_blocks());
        const mp_kv_desc d{kv.block_tokens, kv.max_blocks, kMaxSequences, table_entries_};
        const int status = mp_hip_create(&m, &d, &device_);
        if (status) throw std::runtime_error("create HIP backend: status " + std::to_string(status));
        try {
            upload_weights();
        } catch (...) {
            mp_hip_destroy(device_);
            throw;
        }
        for (int s = kMaxSequences - 1; s >= 0; --s) free_slots_.push_back(s);
        staged_writes_.assign(static_cast<std::size_t>(kv.max_blocks), 0);
    }
    ~HipRunner() override {
        if (device_) mp_hip_destroy(device_);
    }

    const ModelConfig& config() const override { return weights_->config; }
    int context_limit() const override { return kv_.context_limit(); }
    KvAdmission reserve_request(const RequestId& id, std::size_t tokens) override { return kv_.reserve_request(id, tokens); }
    void release_reservation(const RequestId& id) noexcept override { kv_.release_reservation(id); }
    CostStats cost_stats() const override {
        CostStats r = kv_.cost_stats();
        r.cow_pages = costs_.cow_pages;
        r.cow_bytes = costs_.cow_bytes;
        r.cow_copy_ns = costs_.cow_copy_ns;
        r.cow_timed_copies = costs_.cow_timed_copies;
        return r;
    }
    void set_cost_timing(bool enabled) override {
        cost_timing_ = enabled;
        kv_.set_cost_timing(enabled);
    }

    void create(const RequestId& id) override {
        if (kv_.contains(id)) throw std::invalid_argument("sequence already exists");
        if (free_slots_.empty()) throw std::runtime_error("HIP block table arena exhausted");
        kv_.create(id);
        kept_.erase(id);
        tables_[id] = Table{free_slots_.back(), false};
        free_slots_.pop_back();
    }
    void fork_sequence(const RequestId& source, const RequestId& target) override {
        sync("fork completion");
        kv_.fork_sequence(source, target);
        forked_ = true;
        tables_.at(target).dirty = true;  // written whole by the next append
    }
    std::size_t reuse_prefix(const RequestId& id, const std::vector<TokenId>& prompt) override {
        const std::size_t used = kv_.reuse_prefix(id, prompt);
        if (used) {
            try {
                // Queued; the next forward applies the entries before any kernel reads them.
                write_table(tables_.at(id).slot, 0, kv_.sequence(id));
            } catch (...) {
                kv_.reset_sequence(id);
                throw;
            }
        }
        return used;
    }
    void cache_prefix(const RequestId& id) override { kv_.cache_prefix(id); }
    void clear_prefix_cache() override {
        sync("clear prefix completion");
        kv_.clear_prefix_cache();
    }

    std::vector<float> append(const RequestId& id, const std::vector<TokenId>& tokens) override {
        if (!staged_.empty()) throw std::logic_error("append while forwards are staged");
        auto tx = kv_.prepare_append(id, tokens);
        Table& table = tables_.at(id);
        const int used = tx.sequence().used;
        std::vector<float> logits(static_cast<std::size_t>(config().vocabulary));
        try {
            copy_tail(tx);
            write_new_entries(tx, table);
            const mp_seq_step step{table.slot, used, static_cast<std::int32_t>(tokens.size())};
            std::int32_t argmax = 0, nonfinite = 0;
            const int status = mp_hip_forward(device_, &step, 1, tokens.data(), logits.data(), &argmax, &nonfinite);
            if (status == MP_NONFINITE) throw std::runtime_error("nonfinite HIP logits");
            check(status, "model forward");
        } catch (...) {
            mp_hip_sync(device_);
            table.dirty = true;
            tx.rollback();
            throw;
        }
        tx.commit();
        table.dirty = false;
        if (keep_logits_) kept_[id] = logits;
        return logits;
    }

    void stage(const RequestId& id, const std::vector<TokenId>& tokens) override {
        auto tx = kv_.prepare_append(id, tokens);
        Table& table = tables_.at(id);
        const PagedSequence& s = tx.sequence();
        const int used = s.used;
        try {
            if (tx.tail_copy() && staged_writes_[static_cast<std::size_t>(tx.tail_copy()->source)])
                throw std::logic_error("copy-on-write source holds tokens of a queued forward");
            copy_tail(tx);
            write_new_entries(tx, table);
        } catch (...) {
            mp_hip_sync(device_);
            table.dirty = true;
            tx.rollback();
            throw;
        }
        // The pages this forward writes: those of positions used..used+n-1.
        const int bt = kv_.config().block_tokens;
        const int last = (used + static_cast<int>(tokens.size()) - 1) / bt;
        for (int p = used / bt; p <= last; ++p) {
            const int block = s.blocks[static_cast<std::size_t>(p)];
            if (!staged_writes_[static_cast<std::size_t>(block)]) {
                staged_writes_[static_cast<std::size_t>(block)] = 1;
                written_.push_back(block);
            }
        }
        tx.commit();
        table.dirty = false;
        staged_.push_back({table.slot, used, static_cast<std::int32_t>(tokens.size())});
        staged_ids_.push_back(id);
        staged_tokens_.insert(staged_tokens_.end(), tokens.begin(), tokens.end());
    }
    std::vector<StagedResult> run_staged() override {
        std::vector<StagedResult> results(staged_.size());
        if (staged_.empty()) return results;
        std::vector<std::int32_t> argmax(staged_.size()), nonfinite(staged_.size());
        // Logits travel to the host only when they are kept (keep_logits).
        const std::size_t vocab = static_cast<std::size_t>(config().vocabulary);
        std::vector<float> logits(keep_logits_ ? staged_.size() * vocab : 0);
        const std::vector<RequestId> ids = staged_ids_;
        const int status = mp_hip_forward(device_, staged_.data(), static_cast<std::int32_t>(staged_.size()),
                                          staged_tokens_.data(), keep_logits_ ? logits.data() : nullptr,
                                          argmax.data(), nonfinite.data());
        discard_staged();
        if (status != MP_OK && status != MP_NONFINITE) check(status, "model forward");
        for (std::size_t i = 0; i < results.size(); ++i) results[i] = {argmax[i], nonfinite[i] == 0};
        if (keep_logits_)
            for (std::size_t i = 0; i < ids.size(); ++i)
                kept_[ids[i]].assign(logits.begin() + static_cast<std::ptrdiff_t>(i * vocab),
                                     logits.begin() + static_cast<std::ptrdiff_t>((i + 1) * vocab));
        return results;
    }
    void discard_staged() noexcept override {
        staged_.clear();
        staged_ids_.clear();
        staged_tokens_.clear();
        for (const int block : written_) staged_writes_[static_cast<std::size_t>(block)] = 0;
        written_.clear();
    }
    // New pages, or (conservatively) a tail page that a prefix cache or a
    // fork may share and a copy-on-write would replace; or a publication
    // into a prefix cache.
    bool stage_touches_pool(const RequestId& id, std::size_t tokens, bool publishes) const override {
        const PagedSequence& s = kv_.sequence(id);
        const std::size_t bt = static_cast<std::size_t>(kv_.config().block_tokens);
        const std::size_t used = static_cast<std::size_t>(s.used);
        const bool caches = kv_.config().prefix_cache_blocks > 0;
        if ((used + tokens + bt - 1) / bt > s.blocks.size()) return true;
        if (used % bt != 0 && (caches || forked_)) return true;
        return publishes && caches;
    }
    bool shares_staged_pages(const RequestId& id) const override {
        if (written_.empty() || !kv_.contains(id)) return false;
        for (const int block : kv_.sequence(id).blocks)
            if (staged_writes_[static_cast<std::size_t>(block)]) return true;
        return false;
    }

    void release(const RequestId& id) override {
        sync("release completion");
        kv_.release(id);
        free_table(id);
    }
    void clear() override {
        sync("clear completion");
        discard_staged();
        kv_.clear();
        for (auto& t : tables_) free_slots_.push_back(t.second.slot);
        tables_.clear();
        kept_.clear();
    }
    RunnerStats stats() const override {
        RunnerStats r;
        mp_hip_counters c{};
        mp_hip_stats(device_, &c);
        r.device_weight_bytes = c.device_weight_bytes;
        r.weight_uploaded_bytes = c.weight_uploaded_bytes;
        r.token_uploaded_bytes = c.token_uploaded_bytes;
        r.kv_uploaded_bytes = c.kv_uploaded_bytes;
        r.logits_downloaded_bytes = c.logits_downloaded_bytes;
        r.device_allocations = c.device_allocations;
        r.device_workspace_bytes = c.device_workspace_bytes;
        r.block_table_uploaded_bytes = c.block_table_uploaded_bytes;
        r.update_kv_stats(kv_.stats());
        r.block_table_device_bytes = tables_.size() * static_cast<std::size_t>(table_entries_) * sizeof(std::int32_t);
        return r;
    }

    // Committed page table of a sequence (tests compare it with the reference's).
    const PagedSequence& sequence(const RequestId& id) const { return kv_.sequence(id); }
    mp_hip* device() { return device_; }

    // Logit keeping (no counterpart in the reference, whose append returns
    // the logits to its caller): while enabled, every forward's last-row
    // logits of each sequence, append or batched, are kept on the host until
    // the next forward of that sequence (also after its release, which the
    // Engine performs in the step that emits its last token; until the id is
    // created again or the runner cleared), so a caller of the batched
    // Engine (which downloads only the argmax otherwise) can read them.
    void keep_logits(bool enabled) {
        keep_logits_ = enabled;
        if (!enabled) kept_.clear();
    }
    const std::vector<float>* kept_logits(const RequestId& id) const {
        const auto it = kept_.find(id);
        return it == kept_.end() ? nullptr : &it->second;
    }

private:
    static constexpr int kMaxSequences = 1024;
    struct Table {
        int slot;
        bool dirty;
    };

    void check(int status, const char* what) {
        if (status) throw std::runtime_error(std::string(what) + ": " + mp_hip_last_error(device_));
    }
    void sync(const char* what) { check(mp_hip_sync(device_), what); }

    void upload_weights() {
        const ModelConfig& c = config();
        auto put = [&](int layer, int slot, const std::string& name) {
            const auto& t = weights_->get(name);
            check(mp_hip_upload_tensor(device_, layer, slot, t.template data<float>(), t.numel()), "upload weights");
        };
        put(-1, MP_TENSOR_EMBEDDING, "model.embed_tokens.weight");
        put(-1, MP_TENSOR_FINAL_NORM, "model.norm.weight");
        if (!c.tied) put(-1, MP_TENSOR_LM_HEAD, "lm_head.weight");
        static const char* const kSlots[] = {"input_layernorm", "self_attn.q_proj", "self_attn.k_proj",
                                             "self_attn.v_proj", "self_attn.o_proj", "post_attention_layernorm",
                                             "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"};
        for (int l = 0; l < c.layers; ++l)
            for (int j = 0; j < 9; ++j)
                put(l, j, "model.layers." + std::to_string(l) + "." + kSlots[j] + ".weight");
    }

    void write_table(int slot, std::size_t first, const PagedSequence& s) {
        if (s.blocks.size() <= first) return;
        check(mp_hip_table_write(device_, slot, static_cast<std::int32_t>(first), s.blocks.data() + first,
                                 static_cast<std::int32_t>(s.blocks.size() - first)),
              "upload block table entries");
    }

    // New entries only; after a COW swap the swapped entry too; all when dirty.
    void write_new_entries(const KVManager::Append& tx, const Table& table) {
        const std::size_t original = tx.original_blocks();
        const std::size_t first = table.dirty ? 0 : (tx.tail_copy() ? original - 1 : original);
        write_table(table.slot, first, tx.sequence());
    }

    void copy_tail(KVManager::Append& tx) {
        if (tx.tail_copy()) ++costs_.cow_pages;
        tx.copy_shared_tail_region([&](const KVManager::TailCopyRegion& r) {
            const mp_tail_region region{r.destination, r.source, r.pitch, r.width, r.rows};
            if (cost_timing_) {
                std::uint64_t ns = 0;
                check(mp_hip_copy_tail_timed(device_, &region, &ns), "COW copy");
                costs_.cow_copy_ns += ns;
                ++costs_.cow_timed_copies;
            } else {
                check(mp_hip_copy_tail(device_, &region), "COW copy");
            }
            costs_.cow_bytes += 2 * r.width * r.rows * sizeof(float);
        });
    }

    void free_table(const RequestId& id) {
        auto it = tables_.find(id);
        if (it == tables_.end()) return;
        free_slots_.push_back(it->second.slot);
        tables_.erase(it);
    }

    std::shared_ptr<ModelWeights> weights_;
    KVManager kv_;
    mp_hip* device_ = nullptr;
    int table_entries_ = 0;
    std::map<RequestId, Table> tables_;
    std::vector<int> free_slots_;
    std::vector<mp_seq_step> staged_;
    std::vector<RequestId> staged_ids_;
    std::vector<TokenId> staged_tokens_;
    std::vector<char> staged_writes_;  // per block: written by a queued forward
    std::vector<int> written_;         // the blocks marked in staged_writes_
    CostStats costs_;
    bool cost_timing_ = false;
    bool keep_logits_ = false;
    bool forked_ = false;  // a fork_sequence() made shared tails possible
    std::map<RequestId, std::vector<float>> kept_;
};

}  // namespace

std::unique_ptr<ModelRunner> make_hip_runner(std::shared_ptr<ModelWeights> weights, int context, KvCacheConfig kv) {
    return std::make_unique<HipRunner>(std::move(weights), context, kv, MP_ARITHMETIC_EXACT);
}

// The same runner with a chosen arithmetic (MP_ARITHMETIC_EXACT or
// MP_ARITHMETIC_FAST, include/mp_hip.h).
std::unique_ptr<ModelRunner> make_hip_runner(std::shared_ptr<ModelWeights> weights, int context, KvCacheConfig kv,
                                             int arithmetic) {
    return std::make_unique<HipRunner>(std::move(weights), context, kv, arithmetic);
}

// Page table of a sequence for runners built by make_hip_runner.
bool hip_runner_sequence(const ModelRunner& runner, const RequestId& id, const PagedSequence** out) {
    const auto* hip = dynamic_cast<const HipRunner*>(&runner);
    if (!hip) return false;
    *out = &hip->sequence(id);
    return true;
}

// Logit keeping of runners built by make_hip_runner (HipRunner::keep_logits).
bool hip_runner_keep_logits(ModelRunner& runner, bool enabled) {
    auto* hip = dynamic_cast<HipRunner*>(&runner);
    if (!hip) return false;
    hip->keep_logits(enabled);
    return true;
}
bool hip_runner_kept_logits(const ModelRunner& runner, const RequestId& id, const std::vector<float>** out) {
    const auto* hip = dynamic_cast<const HipRunner*>(&runner);
    if (!hip) return false;
    *out = hip->kept_logits(id);
    return true;
}

// Device context of a runner built by make_hip_runner.
void* hip_runner_device(ModelRunner& runner) {
    auto* hip = dynamic_cast<HipRunner*>(&runner);
    return hip ? hip->device() : nullptr;
}

}  // namespace miniprefix
