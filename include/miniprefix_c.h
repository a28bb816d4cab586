/*
 * miniprefix_c.h -- C entry points of the MiniPrefix host runtime (Engine,
 * ModelRunner, weights) for bindings such as ctypes. It is the in-process
 * counterpart of the reference's worker protocol
 * (miniprefix/apps/protocol/command.cpp, session.cpp): the same Engine
 * operations (submit/step/poll/cancel/shutdown, engine.h:12-36) and
 * ModelRunner operations (model.h:35-58), with C types.
 *
 * Every int-returning function returns 0 or a negative status mirroring the
 * C++ exception the reference throws; mpx_last_error() holds its message
 * (per thread).
 */
#ifndef MINIPREFIX_C_H
#define MINIPREFIX_C_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MPX_OK = 0,
    MPX_INVALID_ARGUMENT = -1, /* std::invalid_argument */
    MPX_RUNTIME_ERROR = -2,    /* std::runtime_error (device failure, non-finite logits) */
    MPX_KV_CAPACITY = -5,      /* miniprefix::KvCapacityError */
    MPX_LOGIC_ERROR = -6,      /* std::logic_error */
    MPX_OTHER = -7             /* std::out_of_range (unknown id) and anything else */
};

typedef struct mpx_config {
    int32_t layers, hidden, intermediate, heads, kv_heads, vocabulary, context, eos;
    float rms_epsilon, rope_theta;
    int32_t tied;
} mpx_config;

const char* mpx_last_error(void);

/* Weights (ModelWeights). Synthetic weights follow the SplitMix64 /
 * Box-Muller specification of synthetic.h. */
void* mpx_weights_synthetic(const mpx_config* config, uint64_t seed, double stddev);
void* mpx_weights_load(const char* path);
int mpx_weights_config(const void* weights, mpx_config* out);
int mpx_weights_tensor(const void* weights, const char* name, const float** data, size_t* count);
int mpx_weights_set(void* weights, const char* name, const float* data, size_t count);
void mpx_weights_free(void* weights);

/* ModelRunner. kind 0 is the library's device runner in the exact arithmetic
 * (logits bit-identical to the reference CPU path), kind 2 the same runner in
 * the fast arithmetic (MP_ARITHMETIC_FAST of mp_hip.h). */
void* mpx_runner_create(void* weights, int32_t kind, int32_t context, int32_t block_tokens, int32_t max_blocks,
                        int32_t prefix_cache_blocks);
void mpx_runner_free(void* runner);
int mpx_runner_reserve(void* runner, const char* id, size_t tokens, int32_t* admission);
int mpx_runner_release_reservation(void* runner, const char* id);
int mpx_runner_create_sequence(void* runner, const char* id);
int mpx_runner_fork(void* runner, const char* source, const char* target);
int mpx_runner_reuse_prefix(void* runner, const char* id, const int32_t* prompt, int32_t count, size_t* reused);
int mpx_runner_cache_prefix(void* runner, const char* id);
int mpx_runner_clear_prefix_cache(void* runner);
/* logits: vocabulary floats, may be NULL. */
int mpx_runner_append(void* runner, const char* id, const int32_t* tokens, int32_t count, float* logits);
int mpx_runner_release(void* runner, const char* id);
int mpx_runner_clear(void* runner);
/* 25 fields in RunnerStats order (model.h:23-34). */
int mpx_runner_stats(const void* runner, uint64_t* out);
/* 8 fields in CostStats order (cost_stats.h:6-9). */
int mpx_runner_cost_stats(const void* runner, uint64_t* out);
int mpx_runner_set_cost_timing(void* runner, int32_t enabled);
/* Committed page table; MPX_LOGIC_ERROR if the runner does not expose it. */
int mpx_runner_sequence(const void* runner, const char* id, int32_t* blocks, int32_t capacity, int32_t* count,
                        int32_t* used);
/* Logit keeping, no counterpart in the reference (whose append returns the
 * logits to its caller; the batched Engine step of this library downloads
 * only the greedy argmax): while enabled, the last-row logits of every
 * sequence a forward computes, per-request append or batched step, are kept
 * on the host until that sequence's next forward, its next creation (a
 * released sequence keeps them: the Engine releases a request in the step
 * that emits its last token) or a clear.
 * MPX_LOGIC_ERROR for a runner without it. mpx_runner_kept_logits copies up
 * to `capacity` floats of sequence `id`'s kept logits into `logits` (may be
 * NULL) and their count into `count`; MPX_OTHER when none are kept. */
int mpx_runner_keep_logits(void* runner, int32_t enabled);
int mpx_runner_kept_logits(const void* runner, const char* id, float* logits, size_t capacity, size_t* count);
/* The runner's device context (an mp_hip*, include/mp_hip.h), or NULL for a
 * runner without one; for instrumentation such as mp_hip_set_timing. */
void* mpx_runner_device(void* runner);

/* Engine; takes ownership of the runner. The runner handle stays usable as
 * a borrowed view (mpx_runner_free ignores it) until mpx_engine_free. */
void* mpx_engine_create(void* runner, int32_t max_batch_size, int32_t token_budget, int32_t prefill_chunk,
                        int32_t context);
void mpx_engine_free(void* engine);
int mpx_engine_set_batching(void* engine, int32_t enabled);
int mpx_engine_submit(void* engine, const char* id, const int32_t* prompt, int32_t count, uint32_t max_new_tokens,
                      int32_t eos_token_id /* < 0: none */);
int mpx_engine_step(void* engine, int32_t* progressed);
/* Events as a JSON array of {"id","token","finish","error"} objects; `needed`
 * receives the byte length (without the NUL). Events are consumed only when
 * they fit in `capacity`. */
int mpx_engine_poll(void* engine, char* buffer, size_t capacity, size_t* needed);
int mpx_engine_cancel(void* engine, const char* id);
int mpx_engine_shutdown(void* engine);
int mpx_engine_state(const void* engine, int32_t* idle, int32_t* failed);
/* prefix_reused_tokens, prefill_tokens, decode_tokens of the last step. */
int mpx_engine_step_stats(const void* engine, uint64_t* out);
/* The engine's runner handle (borrowed). */
void* mpx_engine_runner(void* engine);

#ifdef __cplusplus
}
#endif
#endif
