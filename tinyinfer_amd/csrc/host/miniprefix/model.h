// Model description, weights and the runner interface (reference:
// miniprefix/include/miniprefix/model.h:9-62). ModelRunner is the drop-in
// boundary: unchanged names, signatures and defaults.
#pragma once
#include "kv_manager.h"
#include "request.h"
#include <map>
#include <memory>
#include <string>
#include <type_traits>

namespace miniprefix {

struct ModelConfig {
    int layers = 0, hidden = 0, intermediate = 0, heads = 0, kv_heads = 0, vocabulary = 0, context = 0, eos = 0;
    float rms_epsilon = 0, rope_theta = 0;
    bool tied = true;
    int head_dimension() const { return hidden / heads; }
    int kv_width() const { return kv_heads * head_dimension(); }
    void validate() const;
};

// Row-major FP32 host tensor. Its element accessors have the names and
// meaning of tinyinfer::Tensor's (include/tinyinfer/core/tensor.h:46-53), so
// code that reads weights through them builds against either weight type.
struct HostTensor {
    std::vector<std::int64_t> shape;
    std::vector<float> values;
    std::size_t numel() const { return values.size(); }
    template <class T>
    const T* data() const {
        static_assert(std::is_same<T, float>::value, "FP32 tensor");
        return values.data();
    }
    template <class T>
    T* data() {
        static_assert(std::is_same<T, float>::value, "FP32 tensor");
        return values.data();
    }
};

struct ModelWeights {
    ModelConfig config;
    std::map<std::string, HostTensor> tensors;
    // MPFX0001 checkpoint (reference loader miniprefix/src/model/model.cpp:20-56).
    static std::shared_ptr<ModelWeights> load(const std::string& path);
    // Random-init model: every projection and the embedding N(0, stddev^2)
    // from the SplitMix64/Box-Muller streams of synthetic.h, norms 1.0.
    static std::shared_ptr<ModelWeights> synthetic(const ModelConfig& config, std::uint64_t seed, double stddev);
    const HostTensor& get(const std::string& name) const { return tensors.at(name); }
};

struct RunnerStats {
    std::size_t live_sequences = 0, live_kv_bytes = 0, peak_kv_bytes = 0, forward_tokens = 0;
    std::size_t device_weight_bytes = 0, weight_uploaded_bytes = 0, token_uploaded_bytes = 0;
    std::size_t kv_uploaded_bytes = 0, logits_downloaded_bytes = 0, device_allocations = 0;
    std::size_t device_workspace_bytes = 0;
    std::size_t kv_block_tokens = 0, kv_total_blocks = 0, kv_live_blocks = 0, kv_peak_blocks = 0;
    std::size_t kv_reserved_bytes = 0, block_table_uploaded_bytes = 0, block_table_device_bytes = 0;
    std::size_t prefix_cache_capacity = 0, kv_cached_blocks = 0, kv_cache_only_blocks = 0;
    std::size_t prefix_hits = 0, prefix_misses = 0, prefix_reused_tokens = 0, prefix_evictions = 0;
    void update_kv_stats(const KvStats& stats);
};

class ModelRunner {
public:
    virtual ~ModelRunner() = default;
    virtual const ModelConfig& config() const = 0;
    virtual int context_limit() const = 0;
    virtual KvAdmission reserve_request(const RequestId&, std::size_t) { return KvAdmission::Ready; }
    virtual void release_reservation(const RequestId&) noexcept {}
    virtual void create(const RequestId&) = 0;
    virtual void fork_sequence(const RequestId&, const RequestId&) { throw std::logic_error("fork unsupported"); }
    virtual std::size_t reuse_prefix(const RequestId&, const std::vector<TokenId>&) { return 0; }
    virtual void cache_prefix(const RequestId&) {}
    virtual void clear_prefix_cache() {}
    virtual std::vector<float> append(const RequestId&, const std::vector<TokenId>&) = 0;
    virtual void release(const RequestId&) = 0;
    virtual void clear() = 0;
    virtual RunnerStats stats() const = 0;
    virtual CostStats cost_stats() const { return {}; }
    virtual void set_cost_timing(bool) {}
};

// Device backend over the C ABI of include/mp_hip.h: exact arithmetic (logits
// bit-identical to the reference CPU path), or the arithmetic chosen by
// `arithmetic` (MP_ARITHMETIC_EXACT or MP_ARITHMETIC_FAST).
std::unique_ptr<ModelRunner> make_hip_runner(std::shared_ptr<ModelWeights>, int context, KvCacheConfig kv = {});
std::unique_ptr<ModelRunner> make_hip_runner(std::shared_ptr<ModelWeights>, int context, KvCacheConfig kv,
                                             int arithmetic);

}  // namespace miniprefix
