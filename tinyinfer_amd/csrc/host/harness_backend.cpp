// Weights and runners of this library for the C entry points.
#include "harness_backend.h"

#include "mp_hip.h"

#include <cstring>

namespace miniprefix {
bool hip_runner_sequence(const ModelRunner& runner, const RequestId& id, const PagedSequence** out);
void* hip_runner_device(ModelRunner& runner);
bool hip_runner_keep_logits(ModelRunner& runner, bool enabled);
bool hip_runner_kept_logits(const ModelRunner& runner, const RequestId& id, const std::vector<float>** out);
}

namespace mpx {

std::shared_ptr<miniprefix::ModelWeights> synthetic_weights(const miniprefix::ModelConfig& config, std::uint64_t seed,
                                                            double stddev) {
    return miniprefix::ModelWeights::synthetic(config, seed, stddev);
}

std::shared_ptr<miniprefix::ModelWeights> load_weights(const std::string& path) {
    return miniprefix::ModelWeights::load(path);
}

bool weights_tensor(const miniprefix::ModelWeights& weights, const std::string& name, const float** data,
                    std::size_t* count) {
    const auto it = weights.tensors.find(name);
    if (it == weights.tensors.end()) return false;
    *data = it->second.values.data();
    *count = it->second.values.size();
    return true;
}

bool weights_set(miniprefix::ModelWeights& weights, const std::string& name, const float* data, std::size_t count) {
    const auto it = weights.tensors.find(name);
    if (it == weights.tensors.end() || it->second.values.size() != count) return false;
    std::memcpy(it->second.values.data(), data, count * sizeof(float));
    return true;
}

// Kind 0: the HIP runner in the exact arithmetic (logits bit-identical to the
// reference CPU path); kind 2: the HIP runner in the fast arithmetic.
std::unique_ptr<miniprefix::ModelRunner> make_runner(int kind, std::shared_ptr<miniprefix::ModelWeights> weights,
                                                     int context, miniprefix::KvCacheConfig kv) {
    if (kind == 0) return miniprefix::make_hip_runner(std::move(weights), context, kv);
    if (kind == 2) return miniprefix::make_hip_runner(std::move(weights), context, kv, MP_ARITHMETIC_FAST);
    throw std::invalid_argument("unknown runner kind");
}

void set_batching(miniprefix::Engine& engine, bool enabled) { engine.set_batching(enabled); }

bool sequence_of(const miniprefix::ModelRunner& runner, const std::string& id, std::vector<int>* blocks, int* used) {
    const miniprefix::PagedSequence* s = nullptr;
    if (!miniprefix::hip_runner_sequence(runner, id, &s)) return false;
    *blocks = s->blocks;
    *used = s->used;
    return true;
}

void* device_of(miniprefix::ModelRunner& runner) { return miniprefix::hip_runner_device(runner); }

bool keep_logits(miniprefix::ModelRunner& runner, bool enabled) {
    return miniprefix::hip_runner_keep_logits(runner, enabled);
}

bool kept_logits(const miniprefix::ModelRunner& runner, const std::string& id, const std::vector<float>** out) {
    return miniprefix::hip_runner_kept_logits(runner, id, out);
}

}  // namespace mpx
