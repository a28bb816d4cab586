// The few operations of the C entry points (include/miniprefix_c.h) that
// depend on how a build represents weights and which runners it offers.
#pragma once
#include <miniprefix/engine.h>
#include <miniprefix/model.h>

#include <memory>
#include <string>
#include <vector>

namespace mpx {

std::shared_ptr<miniprefix::ModelWeights> synthetic_weights(const miniprefix::ModelConfig& config, std::uint64_t seed,
                                                            double stddev);
std::shared_ptr<miniprefix::ModelWeights> load_weights(const std::string& path);
bool weights_tensor(const miniprefix::ModelWeights& weights, const std::string& name, const float** data,
                    std::size_t* count);
bool weights_set(miniprefix::ModelWeights& weights, const std::string& name, const float* data, std::size_t count);
std::unique_ptr<miniprefix::ModelRunner> make_runner(int kind, std::shared_ptr<miniprefix::ModelWeights> weights,
                                                     int context, miniprefix::KvCacheConfig kv);
// Switches the engine between batched and per-request stepping.
void set_batching(miniprefix::Engine& engine, bool enabled);
// Committed page table of a sequence, when the runner exposes it.
bool sequence_of(const miniprefix::ModelRunner& runner, const std::string& id, std::vector<int>* blocks, int* used);
// The runner's device context, or nullptr.
void* device_of(miniprefix::ModelRunner& runner);
// Logit keeping (HipRunner::keep_logits); false when the runner lacks it.
bool keep_logits(miniprefix::ModelRunner& runner, bool enabled);
// The kept logits of sequence `id` (*out null if none); false when the
// runner lacks logit keeping.
bool kept_logits(const miniprefix::ModelRunner& runner, const std::string& id, const std::vector<float>** out);

}  // namespace mpx
