// C entry points of the host runtime (include/miniprefix_c.h). Exceptions
// become status codes; their messages stay readable through mpx_last_error().
#include "miniprefix_c.h"

#include "harness_backend.h"
#include <miniprefix/engine.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>

using namespace miniprefix;

namespace {

thread_local std::string g_error;

template <class F>
int guarded(F&& f) {
    try {
        f();
        g_error.clear();
        return MPX_OK;
    } catch (const KvCapacityError& e) {
        g_error = e.what();
        return MPX_KV_CAPACITY;
    } catch (const std::invalid_argument& e) {
        g_error = e.what();
        return MPX_INVALID_ARGUMENT;
    } catch (const std::logic_error& e) {
        g_error = e.what();
        return dynamic_cast<const std::out_of_range*>(&e) ? MPX_OTHER : MPX_LOGIC_ERROR;
    } catch (const std::runtime_error& e) {
        g_error = e.what();
        return MPX_RUNTIME_ERROR;
    } catch (const std::exception& e) {
        g_error = e.what();
        return MPX_OTHER;
    } catch (...) {
        g_error = "unknown exception";
        return MPX_OTHER;
    }
}

struct Weights {
    std::shared_ptr<ModelWeights> model;
};
// A runner handle stays valid after mpx_engine_create: ownership of the
// runner moves into the engine and the handle becomes a borrowed view that
// the engine frees.
struct Runner {
    std::unique_ptr<ModelRunner> owned;
    ModelRunner* runner;
    bool borrowed = false;
};
struct EngineBox {
    std::unique_ptr<Engine> engine;
    Runner* view;
    // Events taken from the engine but not yet delivered (the caller's
    // buffer was too short); the next poll of this engine returns them first.
    std::vector<GenerationEvent> pending;
    ~EngineBox() { delete view; }
};

ModelConfig to_config(const mpx_config& c) {
    ModelConfig m;
    m.layers = c.layers;
    m.hidden = c.hidden;
    m.intermediate = c.intermediate;
    m.heads = c.heads;
    m.kv_heads = c.kv_heads;
    m.vocabulary = c.vocabulary;
    m.context = c.context;
    m.eos = c.eos;
    m.rms_epsilon = c.rms_epsilon;
    m.rope_theta = c.rope_theta;
    m.tied = c.tied != 0;
    return m;
}

ModelRunner& runner_of(void* r) {
    if (!r) throw std::invalid_argument("null runner");
    return *static_cast<Runner*>(r)->runner;
}
const ModelRunner& runner_of(const void* r) {
    if (!r) throw std::invalid_argument("null runner");
    return *static_cast<const Runner*>(r)->runner;
}

void json_string(std::string& out, const std::string& s) {
    out += '"';
    for (const char ch : s) {
        if (ch == '"' || ch == '\\') {
            out += '\\';
            out += ch;
        } else if (static_cast<unsigned char>(ch) < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", ch);
            out += buf;
        } else {
            out += ch;
        }
    }
    out += '"';
}

const char* finish_name(FinishReason r) {
    switch (r) {
    case FinishReason::Eos: return "eos";
    case FinishReason::Length: return "length";
    case FinishReason::Cancelled: return "cancelled";
    case FinishReason::Error: return "error";
    }
    return "error";
}

}  // namespace

extern "C" {

const char* mpx_last_error(void) { return g_error.c_str(); }

void* mpx_weights_synthetic(const mpx_config* config, uint64_t seed, double stddev) {
    Weights* out = nullptr;
    if (guarded([&] {
            if (!config) throw std::invalid_argument("null config");
            out = new Weights{mpx::synthetic_weights(to_config(*config), seed, stddev)};
        }))
        return nullptr;
    return out;
}

void* mpx_weights_load(const char* path) {
    Weights* out = nullptr;
    if (guarded([&] { out = new Weights{mpx::load_weights(path ? path : "")}; })) return nullptr;
    return out;
}

int mpx_weights_config(const void* weights, mpx_config* out) {
    return guarded([&] {
        if (!weights || !out) throw std::invalid_argument("null argument");
        const ModelConfig& c = static_cast<const Weights*>(weights)->model->config;
        *out = mpx_config{c.layers, c.hidden, c.intermediate, c.heads, c.kv_heads, c.vocabulary, c.context, c.eos,
                          c.rms_epsilon, c.rope_theta, c.tied ? 1 : 0};
    });
}

int mpx_weights_tensor(const void* weights, const char* name, const float** data, size_t* count) {
    return guarded([&] {
        if (!weights || !name || !data || !count) throw std::invalid_argument("null argument");
        if (!mpx::weights_tensor(*static_cast<const Weights*>(weights)->model, name, data, count))
            throw std::invalid_argument(std::string("unknown tensor: ") + name);
    });
}

int mpx_weights_set(void* weights, const char* name, const float* data, size_t count) {
    return guarded([&] {
        if (!weights || !name || !data) throw std::invalid_argument("null argument");
        if (!mpx::weights_set(*static_cast<Weights*>(weights)->model, name, data, count))
            throw std::invalid_argument(std::string("unknown tensor or size: ") + name);
    });
}

void mpx_weights_free(void* weights) { delete static_cast<Weights*>(weights); }

void* mpx_runner_create(void* weights, int32_t kind, int32_t context, int32_t block_tokens, int32_t max_blocks,
                        int32_t prefix_cache_blocks) {
    Runner* out = nullptr;
    if (guarded([&] {
            if (!weights) throw std::invalid_argument("null weights");
            KvCacheConfig kv;
            kv.block_tokens = block_tokens;
            kv.max_blocks = max_blocks;
            kv.prefix_cache_blocks = prefix_cache_blocks;
            auto made = mpx::make_runner(kind, static_cast<Weights*>(weights)->model, context, kv);
            ModelRunner* raw = made.get();
            out = new Runner{std::move(made), raw};
        }))
        return nullptr;
    return out;
}

void mpx_runner_free(void* runner) {
    Runner* r = static_cast<Runner*>(runner);
    if (r && !r->borrowed) delete r;
}

int mpx_runner_reserve(void* runner, const char* id, size_t tokens, int32_t* admission) {
    return guarded([&] {
        const KvAdmission a = runner_of(runner).reserve_request(id, tokens);
        if (admission) *admission = a == KvAdmission::Ready ? 0 : a == KvAdmission::Wait ? 1 : 2;
    });
}

int mpx_runner_release_reservation(void* runner, const char* id) {
    return guarded([&] { runner_of(runner).release_reservation(id); });
}

int mpx_runner_create_sequence(void* runner, const char* id) {
    return guarded([&] { runner_of(runner).create(id); });
}

int mpx_runner_fork(void* runner, const char* source, const char* target) {
    return guarded([&] { runner_of(runner).fork_sequence(source, target); });
}

int mpx_runner_reuse_prefix(void* runner, const char* id, const int32_t* prompt, int32_t count, size_t* reused) {
    return guarded([&] {
        const std::vector<TokenId> p(prompt, prompt + (count > 0 ? count : 0));
        const std::size_t r = runner_of(runner).reuse_prefix(id, p);
        if (reused) *reused = r;
    });
}

int mpx_runner_cache_prefix(void* runner, const char* id) {
    return guarded([&] { runner_of(runner).cache_prefix(id); });
}

int mpx_runner_clear_prefix_cache(void* runner) {
    return guarded([&] { runner_of(runner).clear_prefix_cache(); });
}

int mpx_runner_append(void* runner, const char* id, const int32_t* tokens, int32_t count, float* logits) {
    return guarded([&] {
        const std::vector<TokenId> t(tokens, tokens + (count > 0 ? count : 0));
        const std::vector<float> out = runner_of(runner).append(id, t);
        if (logits) std::memcpy(logits, out.data(), out.size() * sizeof(float));
    });
}

int mpx_runner_release(void* runner, const char* id) {
    return guarded([&] { runner_of(runner).release(id); });
}

int mpx_runner_clear(void* runner) {
    return guarded([&] { runner_of(runner).clear(); });
}

int mpx_runner_stats(const void* runner, uint64_t* out) {
    return guarded([&] {
        const RunnerStats s = runner_of(runner).stats();
        const std::size_t fields[] = {s.live_sequences, s.live_kv_bytes, s.peak_kv_bytes, s.forward_tokens,
                                      s.device_weight_bytes, s.weight_uploaded_bytes, s.token_uploaded_bytes,
                                      s.kv_uploaded_bytes, s.logits_downloaded_bytes, s.device_allocations,
                                      s.device_workspace_bytes, s.kv_block_tokens, s.kv_total_blocks,
                                      s.kv_live_blocks, s.kv_peak_blocks, s.kv_reserved_bytes,
                                      s.block_table_uploaded_bytes, s.block_table_device_bytes,
                                      s.prefix_cache_capacity, s.kv_cached_blocks, s.kv_cache_only_blocks,
                                      s.prefix_hits, s.prefix_misses, s.prefix_reused_tokens, s.prefix_evictions};
        for (std::size_t i = 0; i < 25; ++i) out[i] = fields[i];
    });
}

int mpx_runner_cost_stats(const void* runner, uint64_t* out) {
    return guarded([&] {
        const CostStats c = runner_of(runner).cost_stats();
        const std::uint64_t fields[] = {c.lookup_calls, c.lookup_ns, c.publish_calls, c.publish_ns,
                                        c.cow_pages, c.cow_bytes, c.cow_copy_ns, c.cow_timed_copies};
        for (std::size_t i = 0; i < 8; ++i) out[i] = fields[i];
    });
}

int mpx_runner_set_cost_timing(void* runner, int32_t enabled) {
    return guarded([&] { runner_of(runner).set_cost_timing(enabled != 0); });
}

int mpx_runner_sequence(const void* runner, const char* id, int32_t* blocks, int32_t capacity, int32_t* count,
                        int32_t* used) {
    return guarded([&] {
        std::vector<int> b;
        int u = 0;
        if (!mpx::sequence_of(runner_of(runner), id, &b, &u))
            throw std::logic_error("runner does not expose page tables");
        if (count) *count = static_cast<int32_t>(b.size());
        if (used) *used = u;
        for (std::size_t i = 0; i < b.size() && static_cast<int32_t>(i) < capacity; ++i) blocks[i] = b[i];
    });
}

int mpx_runner_keep_logits(void* runner, int32_t enabled) {
    return guarded([&] {
        if (!mpx::keep_logits(runner_of(runner), enabled != 0))
            throw std::logic_error("runner does not keep logits");
    });
}

int mpx_runner_kept_logits(const void* runner, const char* id, float* logits, size_t capacity, size_t* count) {
    return guarded([&] {
        const std::vector<float>* kept = nullptr;
        if (!mpx::kept_logits(runner_of(runner), id, &kept)) throw std::logic_error("runner does not keep logits");
        if (!kept) throw std::out_of_range("no kept logits for this sequence");
        if (count) *count = kept->size();
        if (logits) std::memcpy(logits, kept->data(), std::min(capacity, kept->size()) * sizeof(float));
    });
}

void* mpx_runner_device(void* runner) {
    void* out = nullptr;
    if (guarded([&] { out = mpx::device_of(runner_of(runner)); })) return nullptr;
    return out;
}

void* mpx_engine_create(void* runner, int32_t max_batch_size, int32_t token_budget, int32_t prefill_chunk,
                        int32_t context) {
    EngineBox* out = nullptr;
    if (guarded([&] {
            if (!runner) throw std::invalid_argument("null runner");
            Runner* r = static_cast<Runner*>(runner);
            if (r->borrowed || !r->owned) throw std::invalid_argument("runner already owned by an engine");
            EngineConfig config{max_batch_size, token_budget, prefill_chunk, context};
            auto engine = std::make_unique<Engine>(std::move(r->owned), config);
            r->borrowed = true;
            out = new EngineBox{std::move(engine), r};
        }))
        return nullptr;
    return out;
}

void mpx_engine_free(void* engine) { delete static_cast<EngineBox*>(engine); }

int mpx_engine_set_batching(void* engine, int32_t enabled) {
    return guarded([&] { mpx::set_batching(*static_cast<EngineBox*>(engine)->engine, enabled != 0); });
}

int mpx_engine_submit(void* engine, const char* id, const int32_t* prompt, int32_t count, uint32_t max_new_tokens,
                      int32_t eos_token_id) {
    return guarded([&] {
        Request r;
        r.id = id ? id : "";
        r.prompt_token_ids.assign(prompt, prompt + (count > 0 ? count : 0));
        r.generation.max_new_tokens = max_new_tokens;
        if (eos_token_id >= 0) r.generation.eos_token_id = eos_token_id;
        static_cast<EngineBox*>(engine)->engine->submit(std::move(r));
    });
}

int mpx_engine_step(void* engine, int32_t* progressed) {
    return guarded([&] {
        const bool p = static_cast<EngineBox*>(engine)->engine->step();
        if (progressed) *progressed = p ? 1 : 0;
    });
}

int mpx_engine_poll(void* engine, char* buffer, size_t capacity, size_t* needed) {
    return guarded([&] {
        EngineBox& box = *static_cast<EngineBox*>(engine);
        std::vector<GenerationEvent>& pending = box.pending;
        auto fresh = box.engine->poll_events();
        pending.insert(pending.end(), fresh.begin(), fresh.end());
        std::string json = "[";
        for (std::size_t i = 0; i < pending.size(); ++i) {
            const GenerationEvent& e = pending[i];
            if (i) json += ',';
            json += "{\"id\":";
            json_string(json, e.request_id);
            json += ",\"token\":";
            json += e.token_id ? std::to_string(*e.token_id) : "null";
            json += ",\"finish\":";
            if (e.finish_reason) json_string(json, finish_name(*e.finish_reason));
            else json += "null";
            json += ",\"error\":";
            json_string(json, e.error_message);
            json += '}';
        }
        json += ']';
        if (needed) *needed = json.size();
        if (buffer && json.size() < capacity) {
            std::memcpy(buffer, json.c_str(), json.size() + 1);
            pending.clear();
        }
    });
}

int mpx_engine_cancel(void* engine, const char* id) {
    return guarded([&] { static_cast<EngineBox*>(engine)->engine->cancel(id); });
}

int mpx_engine_shutdown(void* engine) {
    return guarded([&] { static_cast<EngineBox*>(engine)->engine->shutdown(); });
}

int mpx_engine_state(const void* engine, int32_t* idle, int32_t* failed) {
    return guarded([&] {
        const Engine& e = *static_cast<const EngineBox*>(engine)->engine;
        if (idle) *idle = e.idle() ? 1 : 0;
        if (failed) *failed = e.failed() ? 1 : 0;
    });
}

int mpx_engine_step_stats(const void* engine, uint64_t* out) {
    return guarded([&] {
        const EngineStepStats& s = static_cast<const EngineBox*>(engine)->engine->last_step_stats();
        out[0] = s.prefix_reused_tokens;
        out[1] = s.prefill_tokens;
        out[2] = s.decode_tokens;
    });
}

void* mpx_engine_runner(void* engine) { return engine ? static_cast<EngineBox*>(engine)->view : nullptr; }

}  // extern "C"
