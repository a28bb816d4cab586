// Model configuration, weights and stats mapping (reference semantics:
// miniprefix/src/model/model.cpp:9-65).
#include "miniprefix/model.h"
#include "synthetic.h"

#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>

namespace miniprefix {

void ModelConfig::validate() const {
    if (layers < 1 || layers > 128 || hidden < 2 || hidden > 8192 || intermediate < 1 || intermediate > 65536 ||
        heads < 1 || kv_heads < 1 || hidden % heads || heads % kv_heads || (hidden / heads) % 2 ||
        hidden / heads > 256 || vocabulary < 2 || vocabulary > 262144 || context < 1 || context > 131072 ||
        eos < 0 || eos >= vocabulary || !std::isfinite(rms_epsilon) || rms_epsilon <= 0 ||
        !std::isfinite(rope_theta) || rope_theta <= 1)
        throw std::invalid_argument("unsupported/invalid Llama configuration");
}

namespace {

// Expected tensors and [in,out] shapes (model.cpp:28-38 of the reference).
std::map<std::string, std::vector<std::int64_t>> expected_shapes(const ModelConfig& c) {
    std::map<std::string, std::vector<std::int64_t>> shapes{{"model.embed_tokens.weight", {c.vocabulary, c.hidden}},
                                                            {"model.norm.weight", {c.hidden}}};
    if (!c.tied) shapes["lm_head.weight"] = {c.hidden, c.vocabulary};
    for (int l = 0; l < c.layers; ++l) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        shapes[p + "input_layernorm.weight"] = {c.hidden};
        shapes[p + "post_attention_layernorm.weight"] = {c.hidden};
        shapes[p + "self_attn.q_proj.weight"] = {c.hidden, c.hidden};
        shapes[p + "self_attn.k_proj.weight"] = {c.hidden, c.kv_width()};
        shapes[p + "self_attn.v_proj.weight"] = {c.hidden, c.kv_width()};
        shapes[p + "self_attn.o_proj.weight"] = {c.hidden, c.hidden};
        shapes[p + "mlp.gate_proj.weight"] = {c.hidden, c.intermediate};
        shapes[p + "mlp.up_proj.weight"] = {c.hidden, c.intermediate};
        shapes[p + "mlp.down_proj.weight"] = {c.intermediate, c.hidden};
    }
    return shapes;
}

template <class T>
T read_value(std::ifstream& file) {
    T value{};
    if (!file.read(reinterpret_cast<char*>(&value), sizeof(T))) throw std::runtime_error("truncated model");
    return value;
}

}  // namespace

// MPFX0001: magic, 8 int32 config fields, eps and theta as float32, a uint32
// tied flag, a uint32 tensor count, then per tensor: uint32 name length,
// name, uint32 rank, int32 dims, uint64 byte count, FP32 data. Little endian.
std::shared_ptr<ModelWeights> ModelWeights::load(const std::string& path) {
    std::ifstream file(path, std::ios::binary);
    if (!file) throw std::runtime_error("cannot open model: " + path);
    char magic[8];
    if (!file.read(magic, 8) || std::memcmp(magic, "MPFX0001", 8)) throw std::runtime_error("invalid model format");
    auto model = std::make_shared<ModelWeights>();
    ModelConfig& c = model->config;
    for (int* field : {&c.layers, &c.hidden, &c.intermediate, &c.heads, &c.kv_heads, &c.vocabulary, &c.context, &c.eos})
        *field = read_value<std::int32_t>(file);
    c.rms_epsilon = read_value<float>(file);
    c.rope_theta = read_value<float>(file);
    const auto tied = read_value<std::uint32_t>(file);
    if (tied > 1) throw std::runtime_error("invalid tied flag");
    c.tied = tied != 0;
    c.validate();
    const auto shapes = expected_shapes(c);
    const auto count = read_value<std::uint32_t>(file);
    if (count != shapes.size()) throw std::runtime_error("model tensor count mismatch");
    const auto file_bytes = std::filesystem::file_size(path);
    for (std::uint32_t i = 0; i < count; ++i) {
        const auto length = read_value<std::uint32_t>(file);
        if (length < 1 || length > 256) throw std::runtime_error("invalid tensor name");
        std::string name(length, '\0');
        if (!file.read(name.data(), length)) throw std::runtime_error("truncated name");
        const auto found = shapes.find(name);
        if (found == shapes.end() || model->tensors.count(name)) throw std::runtime_error("unknown/duplicate tensor: " + name);
        const auto rank = read_value<std::uint32_t>(file);
        if (rank != found->second.size()) throw std::runtime_error("tensor rank mismatch");
        HostTensor tensor;
        std::uint64_t elements = 1;
        for (std::uint32_t d = 0; d < rank; ++d) {
            const auto dim = read_value<std::int32_t>(file);
            if (dim != found->second[d]) throw std::runtime_error("tensor shape mismatch: " + name);
            tensor.shape.push_back(dim);
            elements *= static_cast<std::uint64_t>(dim);
        }
        const auto bytes = read_value<std::uint64_t>(file);
        const auto offset = static_cast<std::uint64_t>(file.tellg());
        if (bytes != elements * sizeof(float) || offset > file_bytes || bytes > file_bytes - offset)
            throw std::runtime_error("invalid tensor bytes");
        tensor.values.resize(elements);
        if (!file.read(reinterpret_cast<char*>(tensor.values.data()), static_cast<std::streamsize>(bytes)))
            throw std::runtime_error("truncated tensor");
        for (const float v : tensor.values)
            if (!std::isfinite(v)) throw std::runtime_error("nonfinite weights");
        model->tensors.emplace(name, std::move(tensor));
    }
    if (file.peek() != std::char_traits<char>::eof()) throw std::runtime_error("trailing model data");
    return model;
}

std::shared_ptr<ModelWeights> ModelWeights::synthetic(const ModelConfig& c, std::uint64_t seed, double stddev) {
    c.validate();
    auto model = std::make_shared<ModelWeights>();
    model->config = c;
    static const char* const kSlots[] = {"input_layernorm", "self_attn.q_proj", "self_attn.k_proj",
                                         "self_attn.v_proj", "self_attn.o_proj", "post_attention_layernorm",
                                         "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"};
    const auto shapes = expected_shapes(c);
    auto make = [&](const std::string& name, std::uint64_t stream, bool ones) {
        HostTensor t;
        t.shape = shapes.at(name);
        std::size_t n = 1;
        for (const auto d : t.shape) n *= static_cast<std::size_t>(d);
        t.values.resize(n);
        if (ones) std::fill(t.values.begin(), t.values.end(), 1.0f);
        else synthetic::normal(t.values.data(), n, seed, stream, stddev);
        model->tensors.emplace(name, std::move(t));
    };
    // Stream ids: embedding 0, final norm 1, layer l slot j -> 2 + 9l + j,
    // untied head 2 + 9*layers.
    make("model.embed_tokens.weight", 0, false);
    make("model.norm.weight", 1, true);
    for (int l = 0; l < c.layers; ++l)
        for (int j = 0; j < 9; ++j)
            make("model.layers." + std::to_string(l) + "." + kSlots[j] + ".weight",
                 2ull + 9ull * static_cast<std::uint64_t>(l) + static_cast<std::uint64_t>(j), j == 0 || j == 5);
    if (!c.tied) make("lm_head.weight", 2ull + 9ull * static_cast<std::uint64_t>(c.layers), false);
    return model;
}

void RunnerStats::update_kv_stats(const KvStats& s) {
    live_sequences = s.live_sequences;
    live_kv_bytes = s.live_kv_bytes;
    peak_kv_bytes = s.peak_kv_bytes;
    forward_tokens = s.forward_tokens;
    kv_block_tokens = s.kv_block_tokens;
    kv_total_blocks = s.kv_total_blocks;
    kv_live_blocks = s.kv_live_blocks;
    kv_peak_blocks = s.kv_peak_blocks;
    kv_reserved_bytes = s.kv_reserved_bytes;
    prefix_cache_capacity = s.prefix_cache_capacity;
    kv_cached_blocks = s.kv_cached_blocks;
    kv_cache_only_blocks = s.kv_cache_only_blocks;
    prefix_hits = s.prefix_hits;
    prefix_misses = s.prefix_misses;
    prefix_reused_tokens = s.prefix_reused_tokens;
    prefix_evictions = s.prefix_evictions;
}

}  // namespace miniprefix
