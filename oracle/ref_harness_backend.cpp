// TEST INFRASTRUCTURE ONLY. Glue that builds the C entry points of
// include/miniprefix_c.h against the reference's own MiniPrefix sources
// (compiled from /root/reference by oracle/ref.mk into oracle/_ref/).
//
// Runner kinds:
//   0: the reference CpuRunner (make_cpu_runner), unmodified;
//   1: a runner pairing the reference's KVManager with the oracle forward
//      (mp_oracle.c, bit-identical to CpuRunner's arithmetic), which exposes
//      page tables so tests can compare them with the HIP runner's.
#include "harness_backend.h"

#include <cstring>

extern "C" {
#include "mp_oracle.h"
}

namespace mpx {
namespace {

using namespace miniprefix;

const char* const kSlots[] = {"input_layernorm", "self_attn.q_proj", "self_attn.k_proj",
                              "self_attn.v_proj", "self_attn.o_proj", "post_attention_layernorm",
                              "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"};

mpo_config oracle_config(const ModelConfig& c) {
    return mpo_config{c.layers, c.hidden, c.intermediate, c.heads, c.kv_heads, c.vocabulary,
                      c.context, c.eos, c.rms_epsilon, c.rope_theta, c.tied ? 1 : 0};
}

class OracleKvRunner final : public ModelRunner {
public:
    OracleKvRunner(std::shared_ptr<ModelWeights> w, int context, KvCacheConfig kv)
        : weights_(std::move(w)), kv_(kv, config().layers, config().kv_width(), context, config().vocabulary) {
        if (context < 1 || context > config().context) throw std::invalid_argument("invalid runner context");
        const ModelConfig& c = config();
        std::vector<const float*> layers;
        for (int l = 0; l < c.layers; ++l)
            for (const char* slot : kSlots)
                layers.push_back(weights_->get("model.layers." + std::to_string(l) + "." + slot + ".weight").data<float>());
        const mpo_config oc = oracle_config(c);
        model_ = mpo_model_from_tensors(&oc, weights_->get("model.embed_tokens.weight").data<float>(),
                                        weights_->get("model.norm.weight").data<float>(), layers.data(),
                                        c.tied ? nullptr : weights_->get("lm_head.weight").data<float>());
        if (!model_) throw std::invalid_argument("invalid oracle model");
        keys_.assign(kv_.reserved_bytes() / sizeof(float) / 2, 0.0f);
        values_.assign(keys_.size(), 0.0f);
    }
    ~OracleKvRunner() override { mpo_model_free(model_); }
    const ModelConfig& config() const override { return weights_->config; }
    int context_limit() const override { return kv_.context_limit(); }
    KvAdmission reserve_request(const RequestId& id, std::size_t t) override { return kv_.reserve_request(id, t); }
    void release_reservation(const RequestId& id) noexcept override { kv_.release_reservation(id); }
    void create(const RequestId& id) override { kv_.create(id); }
    void fork_sequence(const RequestId& s, const RequestId& t) override { kv_.fork_sequence(s, t); }
    std::size_t reuse_prefix(const RequestId& id, const std::vector<TokenId>& p) override { return kv_.reuse_prefix(id, p); }
    void cache_prefix(const RequestId& id) override { kv_.cache_prefix(id); }
    void clear_prefix_cache() override { kv_.clear_prefix_cache(); }
    CostStats cost_stats() const override {
        CostStats r = kv_.cost_stats();
        r.cow_pages = cow_pages_;
        r.cow_bytes = cow_bytes_;
        return r;
    }
    void set_cost_timing(bool e) override { kv_.set_cost_timing(e); }
    std::vector<float> append(const RequestId& id, const std::vector<TokenId>& tokens) override {
        auto tx = kv_.prepare_append(id, tokens);
        const PagedSequence& s = tx.sequence();
        if (tx.tail_copy()) ++cow_pages_;
        tx.copy_shared_tail([&](std::size_t dst, std::size_t src, std::size_t n) {
            std::copy_n(keys_.data() + src, n, keys_.data() + dst);
            std::copy_n(values_.data() + src, n, values_.data() + dst);
            cow_bytes_ += 2 * n * sizeof(float);
        });
        std::vector<float> logits(static_cast<std::size_t>(config().vocabulary));
        const int status = mpo_append(model_, keys_.data(), values_.data(), kv_.config().block_tokens,
                                      s.blocks.data(), static_cast<int>(s.blocks.size()), s.used, tokens.data(),
                                      static_cast<int>(tokens.size()), logits.data());
        if (status == -2) throw std::runtime_error("nonfinite logits");
        if (status) throw std::invalid_argument("invalid oracle append");
        tx.commit();
        return logits;
    }
    void release(const RequestId& id) override { kv_.release(id); }
    void clear() override { kv_.clear(); }
    RunnerStats stats() const override {
        RunnerStats r;
        r.update_kv_stats(kv_.stats());
        return r;
    }
    const PagedSequence& sequence(const RequestId& id) const { return kv_.sequence(id); }

private:
    std::shared_ptr<ModelWeights> weights_;
    KVManager kv_;
    mpo_model* model_ = nullptr;
    std::vector<float> keys_, values_;
    std::uint64_t cow_pages_ = 0, cow_bytes_ = 0;
};

}  // namespace

std::shared_ptr<ModelWeights> synthetic_weights(const ModelConfig& c, std::uint64_t seed, double stddev) {
    c.validate();
    auto w = std::make_shared<ModelWeights>();
    w->config = c;
    auto add = [&](const std::string& name, tinyinfer::Shape shape, std::uint64_t stream, bool ones) {
        tinyinfer::Tensor t(shape);
        if (ones)
            for (std::size_t i = 0; i < t.numel(); ++i) t.data<float>()[i] = 1.0f;
        else
            mpo_fill_normal(t.data<float>(), t.numel(), seed, stream, stddev);
        w->tensors.emplace(name, std::move(t));
    };
    const std::int64_t h = c.hidden, kv = c.kv_width(), i = c.intermediate, v = c.vocabulary;
    add("model.embed_tokens.weight", {v, h}, 0, false);
    add("model.norm.weight", {h}, 1, true);
    for (int l = 0; l < c.layers; ++l) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        const tinyinfer::Shape shapes[] = {{h}, {h, h}, {h, kv}, {h, kv}, {h, h}, {h}, {h, i}, {h, i}, {i, h}};
        for (int j = 0; j < 9; ++j)
            add(p + kSlots[j] + ".weight", shapes[j], 2ull + 9ull * static_cast<std::uint64_t>(l) + static_cast<std::uint64_t>(j),
                j == 0 || j == 5);
    }
    if (!c.tied) add("lm_head.weight", {h, v}, 2ull + 9ull * static_cast<std::uint64_t>(c.layers), false);
    return w;
}

std::shared_ptr<ModelWeights> load_weights(const std::string& path) { return ModelWeights::load(path); }

bool weights_tensor(const ModelWeights& w, const std::string& name, const float** data, std::size_t* count) {
    const auto it = w.tensors.find(name);
    if (it == w.tensors.end()) return false;
    *data = it->second.data<float>();
    *count = it->second.numel();
    return true;
}

bool weights_set(ModelWeights& w, const std::string& name, const float* data, std::size_t count) {
    const auto it = w.tensors.find(name);
    if (it == w.tensors.end() || it->second.numel() != count) return false;
    std::memcpy(it->second.data<float>(), data, count * sizeof(float));
    return true;
}

std::unique_ptr<ModelRunner> make_runner(int kind, std::shared_ptr<ModelWeights> w, int context, KvCacheConfig kv) {
    if (kind == 0) return make_cpu_runner(std::move(w), context, kv);
    if (kind == 1) return std::make_unique<OracleKvRunner>(std::move(w), context, kv);
    throw std::invalid_argument("unknown runner kind");
}

void set_batching(Engine&, bool) { throw std::logic_error("the reference Engine steps one request at a time"); }

bool sequence_of(const ModelRunner& runner, const std::string& id, std::vector<int>* blocks, int* used) {
    const auto* r = dynamic_cast<const OracleKvRunner*>(&runner);
    if (!r) return false;
    *blocks = r->sequence(id).blocks;
    *used = r->sequence(id).used;
    return true;
}

void* device_of(ModelRunner&) { return nullptr; }

bool keep_logits(ModelRunner&, bool) { return false; }

bool kept_logits(const ModelRunner&, const std::string&, const std::vector<float>**) { return false; }

}  // namespace mpx
