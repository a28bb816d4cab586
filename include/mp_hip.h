/*
 * mp_hip.h -- C ABI of the MI355X (gfx950) device backend for MiniPrefix's
 * FP32 generation path.
 *
 * The reference keeps its device forward inside CudaRunner
 * (miniprefix/src/backend/cuda/llama_runner.cu:51-186); the host side
 * (Engine, Scheduler, KVManager, ExactPrefixCache) talks to it only through
 * the ModelRunner virtual interface (miniprefix/include/miniprefix/model.h:35-58).
 * This header is the thin layer below a ModelRunner: weights resident in HBM,
 * paged K/V pools, device block tables, the copy-on-write tail copy and the
 * chunk forward. It has no C++, torch or HIP types in its signatures.
 *
 * Conventions:
 *  - every function returns 0 on success or a negative MP_* status; the
 *    message of the last failure on a context is mp_hip_last_error();
 *  - host pointers are borrowed for the duration of the call only;
 *  - every call that takes a context is synchronous (device work is complete
 *    when it returns) unless documented otherwise, matching the reference's
 *    synchronous append (llama_runner.cu:170);
 *  - a context is single-threaded, like the reference's KVManager
 *    (miniprefix/include/miniprefix/kv_manager.h:18-19).
 *
 * Arithmetic: in the exact mode every kernel reproduces the reference CPU
 * path's floating-point evaluation order (sequential-k projections with
 * separate multiply and add, sequential RMSNorm and softmax sums, two-pass
 * softmax, glibc-compatible expf, host-computed RoPE angles), so logits are
 * bit-identical to miniprefix/src/backend/cpu/llama_runner.cpp:60-104; the
 * fast mode trades that for matrix cores (MP_ARITHMETIC_FAST below).
 */
#ifndef MP_HIP_H
#define MP_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MP_OK = 0,
    MP_INVALID_ARGUMENT = -1, /* std::invalid_argument in the reference */
    MP_DEVICE_ERROR = -2,     /* runtime_error("what: "+error string), resources.cpp:6-8 */
    MP_OUT_OF_MEMORY = -3,
    MP_NONFINITE = -4         /* runtime_error("nonfinite ... logits"), llama_runner.cu:173 */
};

/* Arithmetic of a context (mp_model_desc.arithmetic):
 * - MP_ARITHMETIC_EXACT: every sum in the reference CPU path's order
 *   (sequential k, separate multiply and add, two-pass softmax): logits
 *   bit-identical to miniprefix/src/backend/cpu/llama_runner.cpp:60-104;
 * - MP_ARITHMETIC_FAST: projections and the LM head on FP32 matrix cores,
 *   decode attention split over the context (flash-decoding) and prefill
 *   attention on the matrix cores (flash attention), in their own summation
 *   order: logits within 1e-3 relative and decode attention within 1e-4
 *   absolute of the reference, greedy tokens checked against it. The
 *   attention paths need 16-token pages, 64-wide heads and at most 4 query
 *   heads per KV head (else they run the exact kernels). Needs hidden,
 *   intermediate, q+2*kv width and vocabulary multiples of 16, else the
 *   context computes exactly. */
enum { MP_ARITHMETIC_EXACT = 0, MP_ARITHMETIC_FAST = 1 };

/* Model shape; same fields and limits as ModelConfig (model.h:9-16,
 * model.cpp:9-15), plus the arithmetic mode (no counterpart in the reference). */
typedef struct mp_model_desc {
    int32_t layers, hidden, intermediate, heads, kv_heads, vocabulary, context;
    float rms_epsilon, rope_theta;
    int32_t tied;
    int32_t arithmetic;
} mp_model_desc;

/* Paged KV geometry (KvCacheConfig, paged_kv.h:13-17) plus the device block
 * table arena: max_sequences tables of max_sequence_blocks int32 entries
 * (KVManager::max_sequence_blocks, kv_manager.cpp:16-18). */
typedef struct mp_kv_desc {
    int32_t block_tokens, max_blocks, max_sequences, max_sequence_blocks;
} mp_kv_desc;

/* Strided tail region in float elements of ONE pool (K or V); rows are
 * layers (KVManager::TailCopyRegion, kv_manager.h:40-41). */
typedef struct mp_tail_region {
    uint64_t destination, source, pitch, width, rows;
} mp_tail_region;

/* One sequence's slice of a forward call: `count` new tokens starting at
 * committed position `used`, block table in arena slot `table_slot`. */
typedef struct mp_seq_step {
    int32_t table_slot, used, count;
} mp_seq_step;

typedef struct mp_hip_counters {
    uint64_t device_weight_bytes, weight_uploaded_bytes, token_uploaded_bytes;
    uint64_t kv_uploaded_bytes, logits_downloaded_bytes, device_allocations;
    uint64_t device_workspace_bytes, block_table_uploaded_bytes, block_table_device_bytes;
    uint64_t kv_pool_bytes, forward_calls, forward_rows, cow_copies, cow_bytes;
} mp_hip_counters;

typedef struct mp_hip mp_hip;

/* Replaces the CudaRunner constructor's device half (llama_runner.cu:78-87):
 * selects the current device, creates one stream, allocates the K and V pools
 * (max_blocks*layers*block_tokens*kv_width floats each, zeroed), the table
 * arena and the RoPE table for `context` positions. Weights follow with
 * mp_hip_upload_tensor. */
int mp_hip_create(const mp_model_desc* model, const mp_kv_desc* kv, mp_hip** out);
/* Synchronizes and frees everything (CudaRunner::~CudaRunner, :88). */
int mp_hip_destroy(mp_hip* h);
/* Message of the last failure on `h`; for h = NULL, of the last failed
 * context-free call (the stand-alone attention entry points) on this thread. */
const char* mp_hip_last_error(const mp_hip* h);

/* Tensor slots, canonical per-layer order. layer = -1 for the model-level
 * tensors. Data is FP32 in the reference's stored layout: projections
 * [in,out] row-major (model.cpp:33-37), embedding [vocab,hidden], norms
 * [hidden], untied head [hidden,vocab]. Replaces upload_parameter (:72-76). */
enum {
    MP_TENSOR_INPUT_NORM = 0, MP_TENSOR_Q, MP_TENSOR_K, MP_TENSOR_V, MP_TENSOR_O,
    MP_TENSOR_POST_NORM, MP_TENSOR_GATE, MP_TENSOR_UP, MP_TENSOR_DOWN,
    MP_TENSOR_EMBEDDING = 100, MP_TENSOR_FINAL_NORM = 101, MP_TENSOR_LM_HEAD = 102
};
int mp_hip_upload_tensor(mp_hip* h, int32_t layer, int32_t slot, const float* data, size_t count);
/* Reports whether every tensor the model needs has been uploaded. */
int mp_hip_ready(const mp_hip* h, int32_t* ready);

/* Writes table entries [first, first+count) of arena slot `slot`
 * (block-table H2D, llama_runner.cu:110-117,139-143). */
int mp_hip_table_write(mp_hip* h, int32_t slot, int32_t first, const int32_t* blocks, int32_t count);

/* Copy-on-write of a shared partial tail: copies the region in BOTH the K
 * and the V pool with one kernel (llama_runner.cu:130-137). The region must
 * be one KVManager forms: pitch = block_tokens*kv_width, rows = layers,
 * width = valid tokens * kv_width, source and destination page bases.
 * Inside a page the pools use the device order, and the copy moves the
 * valid tokens' K and V in that order (the same bytes the reference's 2-D
 * copy moves, counted the same way in the COW statistics). Other regions
 * are MP_INVALID_ARGUMENT. Queued: the copies queued since the last
 * forward run as one launch at the start of the next forward (or at
 * mp_hip_sync), before any kernel touches the pools; a copy that would read
 * or write a page a queued copy writes (or write a page one reads) first
 * flushes the queue, so the result is that of the calls in order. */
int mp_hip_copy_tail(mp_hip* h, const mp_tail_region* region);

/* Same copy, timed with device events around it (the reference's opt-in
 * COW timing, llama_runner.cu:129-138,171-172): flushes the queue first
 * (untimed), then launches and times this copy alone. Synchronous. */
int mp_hip_copy_tail_timed(mp_hip* h, const mp_tail_region* region, uint64_t* nanoseconds);

/* Chunk forward of `nseq` sequences (CpuRunner::append's device half,
 * llama_runner.cpp:70-102): embeds `tokens` (sum of counts, sequence-major),
 * runs every layer writing K/V at positions used..used+count-1 through each
 * sequence's table, and produces for each sequence the logits of its LAST
 * token. `logits` (nseq*vocab floats) may be NULL; `argmax` (nseq) receives
 * the first index of the maximum logit (std::max_element, engine.cpp:99);
 * `nonfinite` (nseq, may be NULL) receives 1 for a sequence with any
 * non-finite logit. Returns MP_NONFINITE if any produced logit is not
 * finite (llama_runner.cu:173); outputs are still written. Synchronous. */
int mp_hip_forward(mp_hip* h, const mp_seq_step* steps, int32_t nseq, const int32_t* tokens,
                   float* logits, int32_t* argmax, int32_t* nonfinite);

/* Stand-alone paged GQA decode attention on caller-owned DEVICE buffers
 * (the attention of llama_runner.cpp:85-93 for one query row of length
 * `length`). q: [heads*dim]; pools: [blocks][layers][block_tokens][kv_heads*dim];
 * table: device int32 page table; out: [heads*dim]. `stream` is a
 * hipStream_t or NULL for the null stream. Asynchronous. */
int mp_hip_paged_attention_decode(const float* q, const float* keys, const float* values,
                                  const int32_t* table, int32_t length, int32_t layer,
                                  int32_t layers, int32_t block_tokens, int32_t heads,
                                  int32_t kv_heads, int32_t dim, float* out, void* stream);

/* The decode attention of the fast arithmetic (MP_ARITHMETIC_FAST): the
 * kernels a fast-mode forward runs for its one-token rows, on caller-owned
 * DEVICE buffers, for `rows` query rows at once (the attention of
 * llama_runner.cpp:85-93 in the flash-decoding order: splits of
 * 16-256 tokens, each with a running maximum, denominator and weighted sum,
 * combined at the end; within 1e-4 absolute of the reference on its scale of
 * inputs). q: [rows][heads*dim]; out: [rows][heads*dim]; row r attends
 * lengths[r] tokens (host array) through its page table at
 * tables + r*table_stride (device int32). The pools hold the forward's
 * device page order (mp_hip_kv_pools; layout.h: per (block, layer) KV head
 * major, K as [d/4][slot][4], V as [slot/4][d][4]), not the reference's
 * [slot][kv_width]. Needs block_tokens 16, dim 64 and at most 4 query heads
 * per KV head, else MP_INVALID_ARGUMENT (message:
 * mp_hip_last_error(NULL)). Allocates its work lists and partials per call
 * and is synchronous on `stream` (NULL: the null stream). */
int mp_hip_paged_attention_decode_fast(const float* q, const float* keys, const float* values,
                                       const int32_t* tables, int32_t table_stride, const int32_t* lengths,
                                       int32_t rows, int32_t layer, int32_t layers, int32_t block_tokens,
                                       int32_t heads, int32_t kv_heads, int32_t dim, float* out, void* stream);

/* The same attention as mp_hip_paged_attention_decode with no allocation of
 * any kind: no counterpart in the reference; for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * allocation). The scores of a long row go to a 1 MiB device array of the
 * library (one per GPU, held until the process ends) instead of a per-call
 * hipMalloc; a row must satisfy heads * round_up(length, 16) <= 262144, or
 * the call returns MP_INVALID_ARGUMENT (message: mp_hip_last_error(NULL)).
 * Calls that overlap on one GPU share the array and race. Asynchronous on
 * `stream`. */
int mp_hip_paged_attention_decode_noalloc(const float* q, const float* keys, const float* values,
                                          const int32_t* table, int32_t length, int32_t layer,
                                          int32_t layers, int32_t block_tokens, int32_t heads,
                                          int32_t kv_heads, int32_t dim, float* out, void* stream);

/* Applies queued table entries and copies, then waits for all work on the
 * context's stream (StreamBlas::synchronize). */
int mp_hip_sync(mp_hip* h);
int mp_hip_stats(const mp_hip* h, mp_hip_counters* out);

/* Device pointers of the K and V pools (for tests and profiling); their
 * contents include queued copies after mp_hip_sync. */
int mp_hip_kv_pools(const mp_hip* h, float** keys, float** values, size_t* elements);

/* The context's stream (hipStream_t), e.g. for recording events around calls. */
void* mp_hip_stream(const mp_hip* h);

/* Kernel timing of forward calls with HIP events on the context's stream
 * (instrumentation; no counterpart in the reference). `classes` is a mask of
 * MP_TIME_* bits; each enabled class brackets its launches with events and
 * accumulates their elapsed time when the forward call completes. Setting
 * the mask resets the totals. One ATTENTION launch is one layer's attention
 * (score, softmax and value kernels); one PROJECTION launch is one GEMM
 * (QKV, O, gate/up or down); one HEAD launch is final norm, LM head and
 * argmax of a call. Attention events ride on the kernel dispatches; the
 * others are stream markers between kernels. With MP_TIME_SAMPLED only one
 * layer per forward call is timed (layer = call count modulo layers), which
 * keeps the instrumentation's own cost out of a throughput measurement. */
enum { MP_TIME_ATTENTION = 1, MP_TIME_PROJECTION = 2, MP_TIME_HEAD = 4, MP_TIME_SAMPLED = 8 };
typedef struct mp_hip_timing_totals {
    uint64_t attention_ns, attention_launches;
    uint64_t projection_ns, projection_launches;
    uint64_t head_ns, head_launches;
} mp_hip_timing_totals;
int mp_hip_set_timing(mp_hip* h, uint32_t classes);
int mp_hip_kernel_times(const mp_hip* h, mp_hip_timing_totals* out);

/* Graph replay of fast-arithmetic decode steps (no counterpart in the
 * reference, which launches every kernel of every step): a decode step
 * (every sequence one token) of up to 16 sequences and of a shape seen in
 * the previous call -- the same number of sequences, logits wanted or not,
 * rows longer and shorter than 256 tokens present or not -- is captured
 * once as a HIP graph of its launches and replayed at later steps of that
 * shape, with the step's metadata uploaded before the replay; results are
 * bit-identical to direct launches. On by default; off while kernel timing
 * (mp_hip_set_timing) is on. mp_hip_set_graphs(h, 0) switches it off (and retires the graphs);
 * mp_hip_graphs_captured reports how many graphs the context holds. */
int mp_hip_set_graphs(mp_hip* h, int32_t enabled);
int mp_hip_graphs_captured(const mp_hip* h, int32_t* count);

#ifdef __cplusplus
}
#endif
#endif
