// C ABI of the MI355X device backend (include/mp_hip.h).
//
// One context owns: the resident weights, every projection stored transposed
// ([out][in]; Q|K|V concatenated per layer into one [q+2kv][hidden] matrix;
// the tied LM head is the embedding itself, which already is [vocab][hidden]),
// the K and V page pools, the block-table arena, the RoPE cos/sin table, a
// grow-only workspace (activations in the row-tile quad layout of layout.h)
// and one stream. It corresponds to
// the device half of CudaRunner (miniprefix/src/backend/cuda/llama_runner.cu:51-186)
// and its resources (resources.cpp:13-45).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/mp_hip.h"
#include "kernels.h"
#include "layout.h"

namespace {

using mphip::Epilogue;

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace

struct mp_hip {
    mp_model_desc model{};
    mp_kv_desc kv{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::string error;
    mp_hip_counters stats{};
    // weights
    float* embedding = nullptr;      // [vocab, hidden]
    float* head = nullptr;           // [vocab, hidden]: the embedding when tied
    float* final_norm = nullptr;     // [hidden]
    std::vector<float*> input_norm, post_norm, qkv, o, gate, up, down;
    // Fast arithmetic: the projections also row-major [out][in] (q|k|v in
    // natural column order) for the GEMV of decode steps of up to four
    // sequences (fast_gemv.hip), where the shape allows.
    bool gemv = false;
    std::vector<float*> qkv_rows, o_rows, gate_rows, up_rows, down_rows;
    std::vector<unsigned char> uploaded;  // per (layer, slot) + model tensors
    // paged KV
    float* keys = nullptr;
    float* values = nullptr;
    size_t pool_elements = 0;
    int32_t* tables = nullptr;
    // RoPE
    float* cos_table = nullptr;
    float* sin_table = nullptr;
    // workspace (grow-only, sized in rows)
    int workspace_rows = 0;
    int workspace_seqs = 0;
    float *x = nullptr, *xn = nullptr, *qkv_out = nullptr, *ctx = nullptr, *ffn = nullptr;
    float *last = nullptr, *logits = nullptr, *scratch = nullptr;
    size_t scratch_floats = 0;
    // Fast arithmetic (MP_ARITHMETIC_FAST with shapes that allow it): row
    // sums of squares of the residual stream in 16-column partials
    // [hidden/16][workspace rows] for the RMSNorm of the next projection, and
    // the decode attention's split partials (grow-only).
    bool fast = false;
    float* ssq = nullptr;
    int32_t* row_block = nullptr;  // [workspace rows]: page of each row's position (decode)
    float* row_rope = nullptr;     // [workspace rows][head dim]: cos | sin at each row's position
    float* fast_partials = nullptr;
    size_t fast_partial_floats = 0;
    float* best_value = nullptr;  // LM-head partials [seqs][groups]
    int32_t* best_index = nullptr;
    int32_t* best_bad = nullptr;
    float* staging = nullptr;  // weight upload staging (grow-only)
    size_t staging_floats = 0;
    int32_t* meta = nullptr;  // tokens | row_seq | row_pos | seq_slot | seq_last_row | blocks | items
    size_t meta_capacity = 0;   // int32 entries
    int32_t* results = nullptr;  // argmax[seqs] | nonfinite[seqs] | device error word
    // Block-table entries written since the last flush (table index ->
    // block id): applied on the device at the start of the next forward
    // (or sync), uploaded with that call's metadata.
    std::unordered_map<int32_t, int32_t> pending_tables;
    // Host copy of the whole table arena (every entry written so far), from
    // which the forward puts short rows' page ids into their work items.
    std::vector<int32_t> host_tables;
    // Copies-on-write queued since the last flush, in call order; launched
    // as one kernel at the start of the next forward (or sync), before any
    // kernel reads or writes the pools. No queued copy touches a page
    // another queued copy writes (a conflicting copy flushes the queue).
    std::vector<mphip::TailCopy> pending_copies;
    // Pinned host staging of the metadata upload and of the results, reused
    // across calls; `staged` marks the last upload out of the meta staging.
    int32_t* host_meta = nullptr;
    size_t host_meta_capacity = 0;  // int32 entries
    int32_t* host_results = nullptr;
    size_t host_results_capacity = 0;
    hipEvent_t staged = nullptr;
    hipEvent_t done = nullptr;  // end of a forward call's queued work
    std::vector<void*> allocations;
    // Decode steps replayed from captured graphs (mp_hip_set_graphs): one
    // graph per shape (sequences, logits wanted, split and short rows
    // present); `generation` changes whenever a buffer the captured launches
    // use moves, which retires every graph. A shape is captured at its second
    // step in a row.
    struct GraphKey {
        int nseq = -1;
        bool logits = false, splits = false, shorts = false;
        uint64_t generation = 0;
        bool operator==(const GraphKey& o) const {
            return nseq == o.nseq && logits == o.logits && splits == o.splits && shorts == o.shorts &&
                   generation == o.generation;
        }
    };
    struct Graph {
        GraphKey key;
        hipGraphExec_t exec = nullptr;
    };
    bool graphs_enabled = true;
    uint64_t generation = 0;
    GraphKey last_key;
    std::vector<Graph> graphs;
    // kernel timing (mp_hip_set_timing): event pairs of one forward call
    uint32_t timing = 0;
    std::vector<hipEvent_t> events;
    std::vector<uint32_t> spans;  // class of event pair i
    mp_hip_timing_totals times{};
};

namespace {

int fail(mp_hip* h, int status, const std::string& message) {
    if (h) h->error = message;
    return status;
}

int check(mp_hip* h, hipError_t e, const char* what) {
    if (e == hipSuccess) return MP_OK;
    return fail(h, e == hipErrorOutOfMemory ? MP_OUT_OF_MEMORY : MP_DEVICE_ERROR,
                std::string(what) + ": " + hipGetErrorString(e));
}

// Waits for the context's stream (internal: buffers about to be replaced).
int stream_sync(mp_hip* h) { return check(h, hipStreamSynchronize(h->stream), "model completion"); }

// Waits for the work queued on the stream so far by polling an event: the
// forward's result download is what the next step waits on, and a polling
// wait returns as soon as it lands, where a blocking wait adds the wake-up.
int stream_wait_polling(mp_hip* h, const char* what) {
    hipError_t e = hipEventRecord(h->done, h->stream);
    while (e == hipSuccess) {
        e = hipEventQuery(h->done);
        if (e == hipErrorNotReady) e = hipSuccess;
        else break;
    }
    return check(h, e, what);
}

int device_alloc(mp_hip* h, void** out, size_t bytes, const char* what) {
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes ? bytes : 4);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return check(h, e, what);
    }
    h->allocations.push_back(p);
    ++h->stats.device_allocations;
    *out = p;
    return MP_OK;
}

void device_free(mp_hip* h, void* p) {
    if (!p) return;
    for (auto& a : h->allocations)
        if (a == p) {
            a = nullptr;
            break;
        }
    (void)hipFree(p);
}

// Decode steps of up to this many sequences replay graphs: at B=1 a step ran
// 0.895 vs 0.920 ms (graph vs direct launches), at B=64 1.81 vs 1.78 ms
// (the capacity-sized attention grids cost more than the launches save).
constexpr int kGraphMaxSequences = 16;

// Retires every captured graph (the buffers they launch on are about to
// move, or graphs were switched off); nothing may be in flight.
void retire_graphs(mp_hip* h) {
    for (auto& g : h->graphs)
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
    h->graphs.clear();
    ++h->generation;
}

int kv_width(const mp_model_desc& m) { return m.kv_heads * (m.hidden / m.heads); }
int qkv_width(const mp_model_desc& m) { return m.hidden + 2 * kv_width(m); }

bool valid_model(const mp_model_desc& c) {
    // ModelConfig::validate (miniprefix/src/model/model.cpp:9-15), minus eos.
    return !(c.layers < 1 || c.layers > 128 || c.hidden < 2 || c.hidden > 8192 ||
             c.intermediate < 1 || c.intermediate > 65536 || c.heads < 1 || c.kv_heads < 1 ||
             c.hidden % c.heads || c.heads % c.kv_heads || (c.hidden / c.heads) % 2 ||
             c.hidden / c.heads > 256 || c.vocabulary < 2 || c.vocabulary > 262144 ||
             c.context < 1 || c.context > 131072 || !std::isfinite(c.rms_epsilon) ||
             c.rms_epsilon <= 0 || !std::isfinite(c.rope_theta) || c.rope_theta <= 1);
}

size_t tensor_elements(const mp_model_desc& c, int layer, int slot) {
    const size_t hd = c.hidden, kv = kv_width(c), in = c.intermediate;
    if (layer < 0) {
        if (slot == MP_TENSOR_EMBEDDING) return (size_t)c.vocabulary * hd;
        if (slot == MP_TENSOR_FINAL_NORM) return hd;
        if (slot == MP_TENSOR_LM_HEAD) return c.tied ? 0 : hd * c.vocabulary;
        return 0;
    }
    switch (slot) {
    case MP_TENSOR_INPUT_NORM: case MP_TENSOR_POST_NORM: return hd;
    case MP_TENSOR_Q: case MP_TENSOR_O: return hd * hd;
    case MP_TENSOR_K: case MP_TENSOR_V: return hd * kv;
    case MP_TENSOR_GATE: case MP_TENSOR_UP: case MP_TENSOR_DOWN: return hd * in;
    default: return 0;
    }
}

int uploaded_index(const mp_model_desc& c, int layer, int slot) {
    if (layer >= 0) return layer * 9 + slot;
    return c.layers * 9 + (slot - MP_TENSOR_EMBEDDING);
}

// RoPE angles exactly as llama_runner.cpp:19-20 evaluates them (float pow,
// cos, sin of the host C library), for positions 0..context-1.
void rope_tables(const mp_model_desc& c, std::vector<float>& cs, std::vector<float>& sn) {
    const int dim = c.hidden / c.heads, half = dim / 2;
    cs.resize((size_t)c.context * half);
    sn.resize(cs.size());
    for (int p = 0; p < c.context; ++p)
        for (int d = 0; d < half; ++d) {
            const float angle = float(p) / std::pow(c.rope_theta, float(2 * d) / float(dim));
            cs[(size_t)p * half + d] = std::cos(angle);
            sn[(size_t)p * half + d] = std::sin(angle);
        }
}

// The fast decode and prefill attention kernels serve the rows: fast
// arithmetic, 16-token pages, 64-wide heads, at most 4 query heads per KV
// head (else the exact kernels run).
bool fast_attention_rows(const mp_hip* h) {
    const mp_model_desc& c = h->model;
    return h->fast && h->kv.block_tokens == 16 && c.hidden / c.heads == 64 && c.heads / c.kv_heads <= 4;
}

int score_stride(int max_length) { return (max_length + 15) & ~15; }
int score_chunks(int max_length) { return (max_length + 255) / 256; }
// Score rows and per-256-token chunk maxima of every (row, head).
size_t attention_scratch_floats(const mp_model_desc& c, int rows, int max_length) {
    return (size_t)rows * c.heads * ((size_t)score_stride(max_length) + score_chunks(max_length));
}

// Split partials of the fast decode attention for `seqs` sequences: per
// (sequence, KV head) the most splits a row within the context limit has,
// each G x 64 outputs + (maximum, denominator).
size_t fast_partial_floats(const mp_hip* h, int seqs) {
    const mp_model_desc& c = h->model;
    return (size_t)seqs * c.kv_heads * mphip::fast_attention_max_splits(c.context) * (c.heads / c.kv_heads) *
           (64 + 2);
}

// Grow-only workspace. Sized so that a decode never allocates once the
// workspace has grown to its batch: the exact attention's score rows of a
// call of up to 256 rows are sized for the context limit (a longer call's
// for its longest row), the fast attention's split partials for the
// context limit and the workspace's sequences.
int ensure_workspace(mp_hip* h, int rows, int seqs, int max_length) {
    const mp_model_desc& c = h->model;
    const bool exact_rows = !fast_attention_rows(h);
    const size_t need_scratch =
        exact_rows ? attention_scratch_floats(c, rows, rows <= 256 ? std::max(max_length, c.context) : max_length) : 0;
    if (rows <= h->workspace_rows && seqs <= h->workspace_seqs && need_scratch <= h->scratch_floats)
        return MP_OK;
    int status = stream_sync(h);
    if (status) return status;
    retire_graphs(h);
    // Whole row tiles, so every quad-layout tile a kernel touches exists.
    const int R = ((rows > h->workspace_rows ? rows : h->workspace_rows) + 63) / 64 * 64;
    const int S = ((seqs > h->workspace_seqs ? seqs : h->workspace_seqs) + 63) / 64 * 64;
    for (void* p : {(void*)h->x, (void*)h->xn, (void*)h->qkv_out, (void*)h->ctx, (void*)h->ffn,
                    (void*)h->last, (void*)h->logits, (void*)h->results,
                    (void*)h->best_value, (void*)h->best_index, (void*)h->best_bad, (void*)h->ssq,
                    (void*)h->row_block, (void*)h->row_rope, (void*)h->fast_partials})
        device_free(h, p);
    h->x = h->xn = h->qkv_out = h->ctx = h->ffn = h->last = h->logits = h->best_value = h->ssq = nullptr;
    h->results = h->best_index = h->best_bad = h->row_block = nullptr;
    h->row_rope = h->fast_partials = nullptr;
    h->workspace_rows = h->workspace_seqs = 0;
    const size_t hd = c.hidden;
    const size_t groups = h->fast ? std::max<size_t>(mphip::head_groups(c.vocabulary), c.vocabulary / 16)
                                  : mphip::head_groups(c.vocabulary);
    struct Item { void** p; size_t bytes; };
    const Item items[] = {
        {(void**)&h->x, sizeof(float) * R * hd},
        {(void**)&h->xn, sizeof(float) * R * hd},
        {(void**)&h->qkv_out, sizeof(float) * R * (size_t)qkv_width(c)},
        {(void**)&h->ctx, sizeof(float) * R * hd},
        {(void**)&h->ffn, sizeof(float) * R * (size_t)c.intermediate},
        {(void**)&h->last, sizeof(float) * S * hd},
        {(void**)&h->logits, sizeof(float) * S * (size_t)c.vocabulary},
        {(void**)&h->results, sizeof(int32_t) * (2 * (size_t)S + 4)},
        {(void**)&h->best_value, sizeof(float) * S * groups},
        {(void**)&h->best_index, sizeof(int32_t) * S * groups},
        {(void**)&h->best_bad, sizeof(int32_t) * S * groups},
        {(void**)&h->ssq, h->fast ? sizeof(float) * R * (hd / 16) : 0},
        {(void**)&h->row_block, h->fast ? sizeof(int32_t) * R : 0},
        {(void**)&h->row_rope, h->fast ? sizeof(float) * R * (size_t)(hd / c.heads) : 0},
        {(void**)&h->fast_partials, fast_attention_rows(h) ? sizeof(float) * fast_partial_floats(h, S) : 0},
    };
    size_t total = 0;
    for (const auto& it : items) {
        if ((status = device_alloc(h, it.p, it.bytes, "allocate workspace"))) return status;
        total += it.bytes;
    }
    // Padding rows of the activation tiles are read (never stored) by the
    // projections: start them finite.
    for (void* p : {(void*)h->x, (void*)h->xn, (void*)h->qkv_out, (void*)h->ctx, (void*)h->ffn, (void*)h->last})
        if ((status = check(h, hipMemsetAsync(p, 0, p == h->last ? sizeof(float) * S * hd
                                                   : p == h->qkv_out ? sizeof(float) * R * (size_t)qkv_width(c)
                                                   : p == h->ffn ? sizeof(float) * R * (size_t)c.intermediate
                                                                 : sizeof(float) * R * hd, h->stream),
                            "clear workspace")))
            return status;
    if (need_scratch > h->scratch_floats) {
        device_free(h, h->scratch);
        h->scratch = nullptr;
        h->scratch_floats = 0;
        if ((status = device_alloc(h, (void**)&h->scratch, sizeof(float) * need_scratch,
                                   "allocate attention scratch")))
            return status;
        h->scratch_floats = need_scratch;
    }
    h->workspace_rows = R;
    h->workspace_seqs = S;
    h->fast_partial_floats = fast_attention_rows(h) ? fast_partial_floats(h, S) : 0;
    h->stats.device_workspace_bytes = total + sizeof(float) * h->scratch_floats;
    return MP_OK;
}

// Grow-only pinned host buffer of `entries` int32 (contents not kept).
int ensure_pinned(mp_hip* h, int32_t** buffer, size_t* capacity, size_t entries, const char* what) {
    if (entries <= *capacity) return MP_OK;
    int status = stream_sync(h);
    if (status) return status;
    if (*buffer) (void)hipHostFree(*buffer);
    *buffer = nullptr;
    *capacity = 0;
    const size_t cap = entries + entries / 2;
    if ((status = check(h, hipHostMalloc((void**)buffer, sizeof(int32_t) * cap, hipHostMallocDefault), what)))
        return status;
    *capacity = cap;
    return MP_OK;
}

// Grow-only per-call metadata (int32 entries), device and pinned host.
int ensure_call_buffers(mp_hip* h, size_t meta_entries) {
    int status = MP_OK;
    // The previous upload out of the host staging must have been read.
    if (h->staged && (status = check(h, hipEventSynchronize(h->staged), "metadata upload"))) return status;
    if ((status = ensure_pinned(h, &h->host_meta, &h->host_meta_capacity, meta_entries, "allocate pinned metadata")))
        return status;
    if (meta_entries > h->meta_capacity) {
        if ((status = stream_sync(h))) return status;
        retire_graphs(h);
        device_free(h, h->meta);
        h->meta = nullptr;
        h->meta_capacity = 0;
        const size_t cap = meta_entries + meta_entries / 2;
        if ((status = device_alloc(h, (void**)&h->meta, sizeof(int32_t) * cap, "allocate call metadata"))) return status;
        h->meta_capacity = cap;
    }
    return status;
}

// Appends the pending block-table entries to `dst` as (index, block) pairs
// and clears them; returns the number of pairs.
size_t take_pending_tables(mp_hip* h, int32_t* dst) {
    size_t n = 0;
    for (const auto& kv : h->pending_tables) {
        dst[2 * n] = kv.first;
        dst[2 * n + 1] = kv.second;
        ++n;
    }
    h->pending_tables.clear();
    return n;
}

// Appends the queued copies-on-write to `dst` (three int32 each) and clears
// them; returns the number of copies.
size_t take_pending_copies(mp_hip* h, int32_t* dst) {
    const size_t n = h->pending_copies.size();
    if (n) std::memcpy(dst, h->pending_copies.data(), sizeof(mphip::TailCopy) * n);
    h->pending_copies.clear();
    return n;
}

// Launches `count` copies from the device metadata at `at`.
int launch_copies(mp_hip* h, const int32_t* at, size_t count) {
    const mp_model_desc& c = h->model;
    return check(h, mphip::launch_copy_tails(h->stream, h->keys, h->values,
                                             reinterpret_cast<const mphip::TailCopy*>(at), (int)count, c.layers,
                                             h->kv.block_tokens, c.kv_heads, c.hidden / c.heads),
                 "COW copy");
}

// Uploads and applies the queued block-table entries and copies-on-write on
// the context's stream.
int flush_pending(mp_hip* h) {
    static_assert(sizeof(mphip::TailCopy) == 3 * sizeof(int32_t), "copies travel as three int32");
    if (h->pending_tables.empty() && h->pending_copies.empty()) return MP_OK;
    const size_t n = h->pending_tables.size(), copies = h->pending_copies.size();
    int status = ensure_call_buffers(h, 2 * n + 3 * copies);
    if (status) return status;
    take_pending_tables(h, h->host_meta);
    take_pending_copies(h, h->host_meta + 2 * n);
    status = check(h, hipMemcpyAsync(h->meta, h->host_meta, sizeof(int32_t) * (2 * n + 3 * copies),
                                      hipMemcpyHostToDevice, h->stream), "upload block table entries");
    if (!status) status = check(h, hipEventRecord(h->staged, h->stream), "metadata upload event");
    if (!status && n)
        status = check(h, mphip::launch_table_update(h->stream, h->tables, reinterpret_cast<const int2*>(h->meta),
                                                     (int)n), "apply block table entries");
    if (!status && copies) status = launch_copies(h, h->meta + 2 * n, copies);
    return status;
}

}  // namespace

namespace mphip {
namespace {
thread_local std::string g_free_error = "no error";
}  // namespace
void set_free_error(const std::string& message) { g_free_error = message; }
}  // namespace mphip

extern "C" {

int mp_hip_create(const mp_model_desc* model, const mp_kv_desc* kv, mp_hip** out) {
    if (!model || !kv || !out) return MP_INVALID_ARGUMENT;
    *out = nullptr;
    mp_hip* h = new (std::nothrow) mp_hip();
    if (!h) return MP_OUT_OF_MEMORY;
    h->model = *model;
    h->kv = *kv;
    const mp_model_desc& c = h->model;
    if (c.arithmetic != MP_ARITHMETIC_EXACT && c.arithmetic != MP_ARITHMETIC_FAST) {
        delete h;
        return MP_INVALID_ARGUMENT;
    }
    h->fast = c.arithmetic == MP_ARITHMETIC_FAST && c.hidden % 16 == 0 && c.intermediate % 16 == 0 &&
              kv_width(c) % 16 == 0 && c.vocabulary % 16 == 0;
    // Pages are streamed as float4 runs of tokens: the device path needs a
    // page size that is a multiple of 4 tokens, head_dim a multiple of 4 and
    // at most 64 (one output lane per d) and at most 8 query heads per KV
    // head; the quad activation layout needs hidden and intermediate
    // multiples of 4.
    if (!valid_model(c) || (c.hidden / c.heads) % 4 || c.hidden / c.heads > 64 || c.hidden % 4 ||
        c.intermediate % 4 || c.heads / c.kv_heads > 8 ||
        kv->block_tokens < 4 || kv->block_tokens % 4 ||
        kv->block_tokens * (c.hidden / c.heads) > 8192 || kv->max_blocks < 1 ||
        kv->max_sequences < 1 || kv->max_sequence_blocks < 1 || kv->max_sequence_blocks > 2048 ||
        // page offsets are 32-bit float4 indices in the decode attention
        (uint64_t)kv->max_blocks * (uint64_t)c.layers * (uint64_t)kv->block_tokens *
                (uint64_t)(c.kv_heads * (c.hidden / c.heads)) / 4 > 0xFFFFFFFFull) {
        delete h;
        return MP_INVALID_ARGUMENT;
    }
    int status = check(h, hipGetDevice(&h->device), "get device");
    if (!status) status = check(h, hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking), "create model stream");
    if (!status) status = check(h, hipEventCreateWithFlags(&h->staged, hipEventDisableTiming), "create upload event");
    if (!status) status = check(h, hipEventCreateWithFlags(&h->done, hipEventDisableTiming), "create completion event");
    const size_t hd = c.hidden;
    h->input_norm.assign(c.layers, nullptr);
    h->post_norm.assign(c.layers, nullptr);
    h->qkv.assign(c.layers, nullptr);
    h->o.assign(c.layers, nullptr);
    h->gate.assign(c.layers, nullptr);
    h->up.assign(c.layers, nullptr);
    h->down.assign(c.layers, nullptr);
    h->uploaded.assign((size_t)c.layers * 9 + 3, 0);
    if (c.tied) h->uploaded[(size_t)c.layers * 9 + 2] = 1;
    auto alloc_weights = [&](float** p, size_t elements) {
        if (status) return;
        status = device_alloc(h, (void**)p, elements * sizeof(float), "allocate weights");
        if (!status) h->stats.device_weight_bytes += elements * sizeof(float);
    };
    alloc_weights(&h->embedding, (size_t)c.vocabulary * hd);
    if (c.tied) h->head = h->embedding;
    else alloc_weights(&h->head, (size_t)c.vocabulary * hd);
    alloc_weights(&h->final_norm, hd);
    h->gemv = h->fast && kv->block_tokens == 16 && c.heads / c.kv_heads <= 4 &&
              mphip::gemv_fits(c.hidden, c.intermediate, c.heads, c.kv_heads);
    for (auto* v : {&h->qkv_rows, &h->o_rows, &h->gate_rows, &h->up_rows, &h->down_rows})
        v->assign(h->gemv ? c.layers : 0, nullptr);
    for (int l = 0; l < c.layers; ++l) {
        alloc_weights(&h->input_norm[l], hd);
        alloc_weights(&h->post_norm[l], hd);
        alloc_weights(&h->qkv[l], hd * qkv_width(c));
        alloc_weights(&h->o[l], hd * hd);
        alloc_weights(&h->gate[l], hd * c.intermediate);
        alloc_weights(&h->up[l], hd * c.intermediate);
        alloc_weights(&h->down[l], hd * c.intermediate);
        if (h->gemv) {
            alloc_weights(&h->qkv_rows[l], hd * qkv_width(c));
            alloc_weights(&h->o_rows[l], hd * hd);
            alloc_weights(&h->gate_rows[l], hd * c.intermediate);
            alloc_weights(&h->up_rows[l], hd * c.intermediate);
            alloc_weights(&h->down_rows[l], hd * c.intermediate);
        }
    }
    // Pools: [block][layer][slot][kv_width] (miniprefix/src/kv/paged_kv.cpp:53-56).
    h->pool_elements = (size_t)kv->max_blocks * c.layers * kv->block_tokens * kv_width(c);
    if (!status) status = device_alloc(h, (void**)&h->keys, h->pool_elements * sizeof(float), "allocate keys");
    if (!status) status = device_alloc(h, (void**)&h->values, h->pool_elements * sizeof(float), "allocate values");
    if (!status) status = check(h, hipMemsetAsync(h->keys, 0, h->pool_elements * sizeof(float), h->stream), "clear keys");
    if (!status) status = check(h, hipMemsetAsync(h->values, 0, h->pool_elements * sizeof(float), h->stream), "clear values");
    h->stats.kv_pool_bytes = 2 * h->pool_elements * sizeof(float);
    const size_t table_bytes = sizeof(int32_t) * (size_t)kv->max_sequences * kv->max_sequence_blocks;
    if (!status) status = device_alloc(h, (void**)&h->tables, table_bytes, "allocate block tables");
    if (!status) status = check(h, hipMemsetAsync(h->tables, 0, table_bytes, h->stream), "clear block tables");
    h->stats.block_table_device_bytes = table_bytes;
    h->host_tables.assign((size_t)kv->max_sequences * kv->max_sequence_blocks, 0);
    if (!status) {
        std::vector<float> cs, sn;
        rope_tables(c, cs, sn);
        status = device_alloc(h, (void**)&h->cos_table, cs.size() * sizeof(float), "allocate rope table");
        if (!status) status = device_alloc(h, (void**)&h->sin_table, sn.size() * sizeof(float), "allocate rope table");
        if (!status) status = check(h, hipMemcpyAsync(h->cos_table, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice, h->stream), "upload rope table");
        if (!status) status = check(h, hipMemcpyAsync(h->sin_table, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice, h->stream), "upload rope table");
        if (!status) status = check(h, hipStreamSynchronize(h->stream), "rope table completion");
    }
    if (status) {
        const int s = status;
        std::fprintf(stderr, "mp_hip_create: %s\n", h->error.c_str());
        mp_hip_destroy(h);
        return s;
    }
    *out = h;
    return MP_OK;
}

int mp_hip_destroy(mp_hip* h) {
    if (!h) return MP_OK;
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    retire_graphs(h);
    for (hipEvent_t ev : h->events) (void)hipEventDestroy(ev);
    if (h->staged) (void)hipEventDestroy(h->staged);
    if (h->done) (void)hipEventDestroy(h->done);
    if (h->host_meta) (void)hipHostFree(h->host_meta);
    if (h->host_results) (void)hipHostFree(h->host_results);
    for (void* p : h->allocations)
        if (p) (void)hipFree(p);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
    return MP_OK;
}

const char* mp_hip_last_error(const mp_hip* h) { return h ? h->error.c_str() : mphip::g_free_error.c_str(); }

int mp_hip_upload_tensor(mp_hip* h, int32_t layer, int32_t slot, const float* data, size_t count) {
    if (!h || !data) return fail(h, MP_INVALID_ARGUMENT, "null tensor");
    const mp_model_desc& c = h->model;
    if (layer < -1 || layer >= c.layers) return fail(h, MP_INVALID_ARGUMENT, "invalid tensor layer");
    if ((layer >= 0 && (slot < 0 || slot > MP_TENSOR_DOWN)) ||
        (layer < 0 && (slot < MP_TENSOR_EMBEDDING || slot > MP_TENSOR_LM_HEAD)))
        return fail(h, MP_INVALID_ARGUMENT, "invalid tensor slot");
    const size_t expected = tensor_elements(c, layer, slot);
    if (!expected || count != expected) return fail(h, MP_INVALID_ARGUMENT, "tensor shape mismatch");
    // Non-finite weights are accepted, as the reference runners accept them
    // (cow_test.cpp:135): they surface as non-finite logits of the forwards
    // that read them (MP_NONFINITE), which the runner rolls back.
    const size_t bytes = count * sizeof(float);
    const int hd = c.hidden, kvw = kv_width(c), in = c.intermediate;
    hipError_t e = hipSuccess;
    const hipMemcpyKind h2d = hipMemcpyHostToDevice;
    // Projections arrive [in][out] (model.cpp:33-37). The exact arithmetic
    // stores them [out][in], the fast one in the matrix-core fragment order
    // of layout.h (the embedding too, which arrives [vocab][hidden] =
    // [out][in]), through a staging buffer; norms are stored as given.
    auto staged = [&]() -> hipError_t {
        if (h->staging_floats < count) {
            device_free(h, h->staging);
            h->staging = nullptr;
            h->staging_floats = 0;
            if (device_alloc(h, (void**)&h->staging, bytes, "allocate upload staging")) return hipErrorOutOfMemory;
            h->staging_floats = count;
        }
        return hipMemcpyAsync(h->staging, data, bytes, h2d, h->stream);
    };
    // Fast mode with 64-wide heads: q and k pair-permuted for the RoPE
    // projection (fast_rope_column).
    const bool rope = h->fast && c.hidden / c.heads == 64 && (slot == MP_TENSOR_Q || slot == MP_TENSOR_K);
    // `rows_dst`: the row-major copy of the GEMV path (fast mode), or null.
    auto transposed = [&](float* dst, int rows, int cols, float* rows_dst = nullptr) -> hipError_t {
        hipError_t r = staged();
        if (r != hipSuccess) return r;
        r = h->fast ? mphip::launch_to_fragments(h->stream, h->staging, dst, cols, rows, true, layer >= 0 && rope)
                    : mphip::launch_transpose(h->stream, h->staging, dst, rows, cols, rows);
        if (r == hipSuccess && rows_dst) r = mphip::launch_transpose(h->stream, h->staging, rows_dst, rows, cols, rows);
        return r;
    };
    auto row_copy = [&](const std::vector<float*>& v, size_t offset) -> float* {
        return h->gemv ? v[layer] + offset : nullptr;
    };
    if (layer < 0) {
        if (slot == MP_TENSOR_EMBEDDING) {
            if (!h->fast) {
                e = hipMemcpyAsync(h->embedding, data, bytes, h2d, h->stream);
            } else {
                e = staged();
                if (e == hipSuccess)
                    e = mphip::launch_to_fragments(h->stream, h->staging, h->embedding, c.vocabulary, hd, false);
            }
        } else if (slot == MP_TENSOR_FINAL_NORM) {
            e = hipMemcpyAsync(h->final_norm, data, bytes, h2d, h->stream);
        } else {
            e = transposed(h->head, hd, c.vocabulary);
        }
    } else {
        float* qkv = h->qkv[layer];
        switch (slot) {
        case MP_TENSOR_INPUT_NORM: e = hipMemcpyAsync(h->input_norm[layer], data, bytes, h2d, h->stream); break;
        case MP_TENSOR_POST_NORM: e = hipMemcpyAsync(h->post_norm[layer], data, bytes, h2d, h->stream); break;
        case MP_TENSOR_Q: e = transposed(qkv, hd, hd, row_copy(h->qkv_rows, 0)); break;
        case MP_TENSOR_K: e = transposed(qkv + (size_t)hd * hd, hd, kvw, row_copy(h->qkv_rows, (size_t)hd * hd)); break;
        case MP_TENSOR_V:
            e = transposed(qkv + (size_t)(hd + kvw) * hd, hd, kvw, row_copy(h->qkv_rows, (size_t)(hd + kvw) * hd));
            break;
        case MP_TENSOR_O: e = transposed(h->o[layer], hd, hd, row_copy(h->o_rows, 0)); break;
        case MP_TENSOR_GATE: e = transposed(h->gate[layer], hd, in, row_copy(h->gate_rows, 0)); break;
        case MP_TENSOR_UP: e = transposed(h->up[layer], hd, in, row_copy(h->up_rows, 0)); break;
        case MP_TENSOR_DOWN: e = transposed(h->down[layer], in, hd, row_copy(h->down_rows, 0)); break;
        }
    }
    int status = check(h, e, "upload weights");
    if (!status) status = check(h, hipStreamSynchronize(h->stream), "weight upload completion");
    if (status) return status;
    h->uploaded[uploaded_index(c, layer, slot)] = 1;
    h->stats.weight_uploaded_bytes += bytes;
    int32_t ready = 0;
    mp_hip_ready(h, &ready);
    if (ready && h->staging) {
        device_free(h, h->staging);
        h->staging = nullptr;
        h->staging_floats = 0;
    }
    return MP_OK;
}

int mp_hip_ready(const mp_hip* h, int32_t* ready) {
    if (!h || !ready) return MP_INVALID_ARGUMENT;
    *ready = 1;
    for (unsigned char u : h->uploaded)
        if (!u) *ready = 0;
    return MP_OK;
}

int mp_hip_table_write(mp_hip* h, int32_t slot, int32_t first, const int32_t* blocks, int32_t count) {
    if (!h) return MP_INVALID_ARGUMENT;
    if (slot < 0 || slot >= h->kv.max_sequences || first < 0 || count < 0 ||
        (int64_t)first + count > h->kv.max_sequence_blocks || (count && !blocks))
        return fail(h, MP_INVALID_ARGUMENT, "invalid block table write");
    for (int32_t i = 0; i < count; ++i)
        if (blocks[i] < 0 || blocks[i] >= h->kv.max_blocks)
            return fail(h, MP_INVALID_ARGUMENT, "block id out of range");
    if (!count) return MP_OK;
    // Queued; the next forward (or sync) uploads the entries with its own
    // metadata and applies them before any kernel reads a table.
    const int32_t base = slot * h->kv.max_sequence_blocks + first;
    for (int32_t i = 0; i < count; ++i) {
        h->pending_tables[base + i] = blocks[i];
        h->host_tables[(size_t)base + i] = blocks[i];
    }
    h->stats.block_table_uploaded_bytes += sizeof(int32_t) * count;
    return MP_OK;
}

int mp_hip_copy_tail(mp_hip* h, const mp_tail_region* r) {
    if (!h || !r) return MP_INVALID_ARGUMENT;
    if (!r->rows || !r->width) return MP_OK;
    // Only the regions KVManager forms (kv_manager.cpp:160-169): one page of
    // every layer, pitch = one page-layer span, width = valid tokens x
    // kv_width, page-aligned source and destination. The pools keep the
    // reference's page bases but their own order inside a page, so the copy
    // moves the valid slots in that order (launch_copy_tails).
    const mp_model_desc& c = h->model;
    const uint64_t kvw = (uint64_t)kv_width(c);
    const uint64_t page = (uint64_t)h->kv.block_tokens * kvw;
    const uint64_t block = page * (uint64_t)c.layers;
    if (r->pitch != page || r->rows != (uint64_t)c.layers || r->width % kvw || r->width > page ||
        r->destination % block || r->source % block || r->destination / block >= (uint64_t)h->kv.max_blocks ||
        r->source / block >= (uint64_t)h->kv.max_blocks)
        return fail(h, MP_INVALID_ARGUMENT, "tail copy region is not a page region of the pools");
    const mphip::TailCopy copy{(int32_t)(r->destination / block), (int32_t)(r->source / block),
                               (int32_t)(r->width / kvw)};
    // Queued copies run side by side; one that reads or writes a page a
    // queued copy writes, or writes a page a queued copy reads, waits for
    // them (the queue is flushed first).
    for (const mphip::TailCopy& q : h->pending_copies)
        if (q.destination == copy.source || q.destination == copy.destination || q.source == copy.destination) {
            const int status = flush_pending(h);
            if (status) return status;
            break;
        }
    h->pending_copies.push_back(copy);
    ++h->stats.cow_copies;
    h->stats.cow_bytes += 2 * r->width * r->rows * sizeof(float);
    return MP_OK;
}

int mp_hip_copy_tail_timed(mp_hip* h, const mp_tail_region* region, uint64_t* nanoseconds) {
    if (!h || !nanoseconds) return MP_INVALID_ARGUMENT;
    // Earlier queued work goes first, outside the timed span.
    int status = flush_pending(h);
    if (status) return status;
    hipEvent_t begin = nullptr, end = nullptr;
    status = check(h, hipEventCreate(&begin), "COW event begin");
    if (!status) status = check(h, hipEventCreate(&end), "COW event end");
    if (!status) status = mp_hip_copy_tail(h, region);
    if (!status) status = check(h, hipEventRecord(begin, h->stream), "COW timing begin");
    if (!status) status = flush_pending(h);
    if (!status) status = check(h, hipEventRecord(end, h->stream), "COW timing end");
    if (!status) status = check(h, hipEventSynchronize(end), "COW completion");
    float ms = 0.0f;
    if (!status) status = check(h, hipEventElapsedTime(&ms, begin, end), "COW elapsed");
    if (!status) *nanoseconds = (uint64_t)(ms * 1e6);
    if (begin) (void)hipEventDestroy(begin);
    if (end) (void)hipEventDestroy(end);
    return status;
}

int mp_hip_forward(mp_hip* h, const mp_seq_step* steps, int32_t nseq, const int32_t* tokens,
                   float* logits, int32_t* argmax, int32_t* nonfinite) {
    if (!h || !steps || nseq < 1 || !tokens || !argmax)
        return fail(h, MP_INVALID_ARGUMENT, "invalid forward arguments");
    const mp_model_desc& c = h->model;
    int32_t ready = 0;
    mp_hip_ready(h, &ready);
    if (!ready) return fail(h, MP_INVALID_ARGUMENT, "weights not uploaded");
    int64_t rows = 0;
    int max_length = 1;
    for (int s = 0; s < nseq; ++s) {
        const mp_seq_step& st = steps[s];
        if (st.table_slot < 0 || st.table_slot >= h->kv.max_sequences || st.count < 1 ||
            st.used < 0 || (int64_t)st.used + st.count > c.context ||
            ((int64_t)st.used + st.count + h->kv.block_tokens - 1) / h->kv.block_tokens >
                h->kv.max_sequence_blocks)
            return fail(h, MP_INVALID_ARGUMENT, "invalid sequence step");
        rows += st.count;
        if (st.used + st.count > max_length) max_length = st.used + st.count;
    }
    if (rows > (1 << 20)) return fail(h, MP_INVALID_ARGUMENT, "too many rows");
    const int R = (int)rows;
    for (int i = 0; i < R; ++i)
        if (tokens[i] < 0 || tokens[i] >= c.vocabulary) return fail(h, MP_INVALID_ARGUMENT, "invalid token");
    int status = ensure_workspace(h, R, nseq, max_length);
    if (status) return status;
    // Row metadata: tokens | row_seq | row_pos | seq_slot | seq_last_row |
    // attention row blocks (first row, rows) by decreasing attended length |
    // scores work items (block, chunk).
    const int block_rows = mphip::attention_row_block(c.heads, c.kv_heads, c.hidden / c.heads);
    // Fast mode (16-token pages, 64-wide heads, at most 4 query heads per KV
    // head): every one-token sequence takes the decode attention kernels,
    // also in a step that prefills others, so a decoding row's result does
    // not depend on the rest of the batch; the prefill rows take the
    // matrix-core prefill kernel (fast_prefill.hip). The row-block kernels
    // serve the exact mode.
    const int group_ = c.heads / c.kv_heads;
    const bool fast_rows = fast_attention_rows(h);
    struct Block { int first, rows, length; };
    std::vector<Block> blocks;
    bool decode = true;
    for (int s = 0; s < nseq; ++s)
        if (steps[s].count != 1) decode = false;
    for (int s = 0, first = 0; s < nseq; first += steps[s].count, ++s) {
        if (fast_rows) continue;
        for (int i = 0; i < steps[s].count; i += block_rows) {
            const int rows_b = std::min(block_rows, steps[s].count - i);
            blocks.push_back({first + i, rows_b, steps[s].used + i + rows_b});
        }
    }
    std::stable_sort(blocks.begin(), blocks.end(), [](const Block& a, const Block& b) { return a.length > b.length; });
    size_t items = 0;
    for (const Block& b : blocks) items += (size_t)(b.length + 255) / 256;
    const size_t nblocks = blocks.size();
    const size_t table_pairs = h->pending_tables.size();
    const size_t copies = h->pending_copies.size();
    // Fast-mode decode attention of the one-token sequences: work items
    // (row, KV head, first token, tokens | split << 16) over each row's
    // splits (fast_attention_split); rows of up to 256 tokens as (row, KV
    // head, tokens) items of the one-work-group kernel; the rows the merge
    // kernel combines. The split depends on nothing but the row.
    const bool fast_decode = fast_rows && decode;  // q|k|v with the RoPE epilogue
    size_t fast_items = 0, fast_short = 0, fast_merge = 0, fast_pre = 0;
    int max_splits = 0;
    if (fast_rows)
        for (int q = 0; q < nseq; ++q) {
            if (steps[q].count != 1) {
                fast_pre += (size_t)(steps[q].count + 15) / 16 * c.kv_heads;  // 16-row blocks x KV heads
                continue;
            }
            const int length = steps[q].used + 1, split = mphip::fast_attention_split(length);
            const int splits = (length + split - 1) / split;
            if (mphip::fast_attention_short(length)) {
                fast_short += (size_t)c.kv_heads;
                continue;
            }
            fast_items += (size_t)c.kv_heads * splits;
            ++fast_merge;
            max_splits = std::max(max_splits, splits);
        }
    const bool fast_any = fast_items + fast_short + fast_pre > 0;
    // Metadata (int32): tokens | row_seq | row_pos | seq_slot | seq_last_row |
    // blocks | items, then (16-byte aligned) the fast attention's lists at
    // offsets that depend only on the rows and sequences -- counts [4] |
    // merged rows (room for every sequence) | short items (room for every
    // sequence and KV head) | split items -- then the prefill items, the
    // block-table entries and the copies. A decode step's launches thus
    // read the same addresses at every step of the same shape.
    auto align4 = [](size_t n) { return (n + 3) / 4 * 4; };
    const size_t base_entries = 3 * (size_t)R + 2 * (size_t)nseq + 2 * nblocks + 2 * items;
    const size_t fast_at = align4(base_entries);
    const size_t merge_at = fast_at + 4;
    const size_t short_at = merge_at + 4 * (size_t)nseq;
    const size_t items_at = short_at + (size_t)mphip::kShortItemInts * nseq * c.kv_heads;
    const size_t pre_at = fast_rows ? align4(items_at + 4 * fast_items) : fast_at;
    const size_t tables_at = pre_at + 4 * fast_pre;
    const size_t copies_at = tables_at + 2 * table_pairs;
    const size_t entries = copies_at + 3 * copies;
    // The metadata buffers are sized for any call of this many rows and
    // sequences within the context limit (and its table entries and
    // copies), so a decode does not grow them; the split items' capacity is
    // every split of every sequence at the context limit.
    const int split_stride = mphip::fast_attention_max_splits(c.context);
    const size_t items_capacity = (size_t)nseq * c.kv_heads * split_stride;
    const size_t chunks_limit = (size_t)score_chunks(c.context);
    const size_t bound = 3 * (size_t)R + 2 * (size_t)nseq + 2 * (size_t)R * (1 + chunks_limit) + 16 +
                         2 * table_pairs + 3 * copies +
                         (fast_rows ? 4 + 4 * (size_t)nseq + (size_t)mphip::kShortItemInts * nseq * c.kv_heads +
                                          4 * items_capacity +
                                          4 * ((size_t)R / 16 + (size_t)nseq) * c.kv_heads
                                    : 0);
    if ((status = ensure_call_buffers(h, std::max(entries, bound)))) return status;
    if (fast_any && (max_splits > split_stride || (size_t)nseq > (size_t)h->workspace_seqs || fast_items > items_capacity))
        return fail(h, MP_DEVICE_ERROR, "attention partials smaller than the call");
    int32_t* const m0 = h->host_meta;
    int32_t* m_tokens = m0;
    int32_t* m_seq = m_tokens + R;
    int32_t* m_pos = m_seq + R;
    int32_t* m_slot = m_pos + R;
    int32_t* m_last = m_slot + nseq;
    int32_t* m_blocks = m_last + nseq;
    int32_t* m_items = m_blocks + 2 * nblocks;
    int32_t* m_tables = m0 + tables_at;
    int32_t* m_copies = m0 + copies_at;
    take_pending_tables(h, m_tables);
    take_pending_copies(h, m_copies);
    int r = 0;
    for (int s = 0; s < nseq; ++s) {
        for (int i = 0; i < steps[s].count; ++i, ++r) {
            m_tokens[r] = tokens[r];
            m_seq[r] = s;
            m_pos[r] = steps[s].used + i;
        }
        m_slot[s] = steps[s].table_slot;
        m_last[s] = r - 1;
    }
    size_t it = 0;
    for (size_t b = 0; b < nblocks; ++b) {
        m_blocks[2 * b] = blocks[b].first;
        m_blocks[2 * b + 1] = blocks[b].rows;
        for (int ch = 0; ch < (blocks[b].length + 255) / 256; ++ch, ++it) {
            m_items[2 * it] = (int32_t)b;
            m_items[2 * it + 1] = ch;
        }
    }
    int32_t* const m_fast = m0 + items_at;
    if (fast_rows) {
        int32_t* const m_counts = m0 + fast_at;
        m_counts[0] = (int32_t)fast_items;
        m_counts[1] = (int32_t)fast_short;
        m_counts[2] = (int32_t)fast_merge;
        m_counts[3] = 0;
    }
    if (fast_any) {
        // A one-token sequence q's row is m_last[q]. Whole splits first, then
        // each row's shorter last split (attention per layer: config 4 15.8-16.1
        // vs 17.2 us in row order, config 5B 80.1 vs 82.4, config 3 within
        // noise); a split's KV heads side by side, so that the waves of one
        // work-group read the adjacent pages of one (block, layer) together
        // (config 3 30.65-30.87 vs 30.86-30.96 us, config 5B 81.7-81.8 vs
        // 82.2-82.6 with each KV head's splits in a run).
        size_t f = 0;
        for (int pass = 0; pass < 2; ++pass)
            for (int q = 0; q < nseq; ++q) {
                const int length = steps[q].used + 1, split = mphip::fast_attention_split(length);
                const int splits = (length + split - 1) / split;
                if (steps[q].count != 1 || mphip::fast_attention_short(length)) continue;
                for (int sp = 0; sp < splits; ++sp)
                    for (int kvh = 0; kvh < c.kv_heads; ++kvh) {
                        const int n = std::min(split, length - sp * split);
                        if ((n == split) != (pass == 0)) continue;
                        m_fast[4 * f] = m_last[q];
                        m_fast[4 * f + 1] = steps[q].table_slot * c.kv_heads + kvh;
                        m_fast[4 * f + 2] = q;
                        m_fast[4 * f + 3] = mphip::fast_attention_item_w(n, sp, split);
                        ++f;
                    }
            }
        int32_t* const m_short = m0 + short_at;
        int32_t* const m_merge = m0 + merge_at;
        size_t r = 0, mr = 0;
        for (int q = 0; q < nseq; ++q) {
            if (steps[q].count != 1) continue;
            if (!mphip::fast_attention_short(steps[q].used + 1)) {
                const int length = steps[q].used + 1, split = mphip::fast_attention_split(length);
                m_merge[4 * mr] = m_last[q];
                m_merge[4 * mr + 1] = q;
                m_merge[4 * mr + 2] = (length + split - 1) / split;
                m_merge[4 * mr + 3] = 0;
                ++mr;
                continue;
            }
            const int length = steps[q].used + 1, pages = (length + 15) / 16;
            const int32_t* row_table = h->host_tables.data() + (size_t)steps[q].table_slot * h->kv.max_sequence_blocks;
            for (int kvh = 0; kvh < c.kv_heads; ++kvh, ++r) {
                int32_t* item = m_short + (size_t)mphip::kShortItemInts * r;
                item[0] = m_last[q];
                item[1] = steps[q].table_slot * c.kv_heads + kvh;
                item[2] = length;
                item[3] = 0;
                for (int k = 0; k < mphip::kShortItemInts - 4; ++k) item[4 + k] = row_table[std::min(k, pages - 1)];
            }
        }
        // Prefill: (first row, slot * kv_heads + KV head, position, rows) per
        // 16-row block of each prefilling sequence and KV head.
        int32_t* const m_pre = m0 + pre_at;
        size_t pr = 0;
        for (int q = 0; q < nseq; ++q) {
            if (steps[q].count == 1) continue;
            const int first = m_last[q] - steps[q].count + 1;
            for (int b = 0; b < steps[q].count; b += 16)
                for (int kvh = 0; kvh < c.kv_heads; ++kvh, ++pr) {
                    m_pre[4 * pr] = first + b;
                    m_pre[4 * pr + 1] = steps[q].table_slot * c.kv_heads + kvh;
                    m_pre[4 * pr + 2] = steps[q].used + b;
                    m_pre[4 * pr + 3] = std::min(16, steps[q].count - b);
                }
        }
    }
    status = check(h, hipMemcpyAsync(h->meta, m0, sizeof(int32_t) * entries, hipMemcpyHostToDevice, h->stream),
                   "upload input tokens");
    if (!status) status = check(h, hipEventRecord(h->staged, h->stream), "metadata upload event");
    if (!status && table_pairs)
        status = check(h, mphip::launch_table_update(h->stream, h->tables,
                                                     reinterpret_cast<const int2*>(h->meta + tables_at),
                                                     (int)table_pairs), "apply block table entries");
    if (!status && copies) status = launch_copies(h, h->meta + copies_at, copies);
    if (status) return status;
    h->stats.token_uploaded_bytes += sizeof(int32_t) * R;
    mphip::RowMeta meta{h->meta, h->meta + R, h->meta + 2 * (size_t)R, h->meta + 3 * (size_t)R,
                        h->meta + 3 * (size_t)R + nseq};
    const int dim = c.hidden / c.heads, kvw = kv_width(c), qw = qkv_width(c);
    mphip::PagedKv kv{h->keys, h->values, h->tables, h->kv.max_sequence_blocks,
                      c.layers, h->kv.block_tokens, kvw};
    mphip::AttentionWork work{};
    work.blocks = reinterpret_cast<const int2*>(m_blocks - m0 + h->meta);
    work.items = reinterpret_cast<const int2*>(m_items - m0 + h->meta);
    work.blocks_count = (int)nblocks;
    work.items_count = (int)items;
    work.scores = h->scratch;
    work.stride = score_stride(max_length);
    work.chunks = score_chunks(max_length);
    work.chunk_max = h->scratch + (size_t)R * c.heads * work.stride;
    int32_t* const device_error = h->results + 2 * (size_t)nseq;
    work.error = device_error;
    hipStream_t s = h->stream;
    // Launches of an enabled timing class are bracketed by a pair of events
    // from the pool that mp_hip_set_timing sized for one forward call:
    // recorded by the kernel dispatches themselves for attention, as stream
    // markers around the launch otherwise.
    h->spans.clear();
    const bool sampled = (h->timing & MP_TIME_SAMPLED) != 0;
    const int sample_layer = (int)(h->stats.forward_calls % (uint64_t)c.layers);
    int layer_now = -1;  // the layer being launched, -1 outside the layers
    auto timing_on = [&](uint32_t cls) {
        return (h->timing & cls) && (!sampled || layer_now == sample_layer);
    };
    auto timed = [&](uint32_t cls, auto&& launch) -> hipError_t {
        if (!timing_on(cls)) return launch();
        const size_t pair = 2 * h->spans.size();
        hipError_t r = hipEventRecord(h->events[pair], s);
        if (r == hipSuccess) r = launch();
        if (r == hipSuccess) r = hipEventRecord(h->events[pair + 1], s);
        h->spans.push_back(cls);
        return r;
    };
    auto attention_events = [&]() {
        mphip::LaunchEvents ev;
        if (timing_on(MP_TIME_ATTENTION)) {
            const size_t pair = 2 * h->spans.size();
            ev.start = h->events[pair];
            ev.stop = h->events[pair + 1];
            h->spans.push_back(MP_TIME_ATTENTION);
        }
        return ev;
    };
    const uint32_t P = MP_TIME_PROJECTION;
    auto gemm = [&](mphip::Epilogue epi, const float* x, int rows, int inner, const float* w, const float* w2,
                    int columns, float* out) {
        mphip::GemmArgs a{};
        a.x = x;
        a.w = w;
        a.w2 = w2;
        a.out = out;
        a.rows = rows;
        a.inner = inner;
        a.columns = columns;
        return mphip::launch_gemm(s, epi, a);
    };
    const int hd = c.hidden, in = c.intermediate;
    const float eps = c.rms_epsilon;
    // RMSNorm of the residual stream h->x followed by a projection: one
    // launch where the shape allows, else rms_kernel into h->xn and the GEMM.
    auto normed_gemm = [&](mphip::Epilogue epi, const float* norm, int rows, int inner, const float* w,
                           const float* w2, int columns, float* out) {
        mphip::GemmArgs a{};
        a.x = h->x;
        a.w = w;
        a.w2 = w2;
        a.out = out;
        a.rows = rows;
        a.inner = inner;
        a.columns = columns;
        a.norm = norm;
        a.eps = eps;
        if (mphip::gemm_normed_fits(epi, a)) return mphip::launch_gemm_normed(s, epi, a);
        hipError_t r = mphip::launch_rms(s, h->x, nullptr, norm, h->xn, rows, inner, eps);
        if (r == hipSuccess) r = gemm(epi, h->xn, rows, inner, w, w2, columns, out);
        return r;
    };
    // The fast decode's q|k|v projection takes each row's page and rotation
    // from per-row arrays that the embedding kernel fills.
    mphip::RowRope row_rope{meta, h->tables, h->kv.max_sequence_blocks, h->kv.block_tokens, dim / 2,
                            h->cos_table, h->sin_table, h->row_block, h->row_rope};
    auto launch_embedding = [&]() {
        return mphip::launch_embed(s, h->embedding, meta.tokens, h->x, R, hd, device_error,
                                   fast_decode ? &row_rope : nullptr, h->fast);
    };
    // The fast arithmetic's launches from the embedding to the argmax; with
    // graph_grids the attention grids are sized by the lists' capacities, for
    // a capture that later steps of the same shape replay.
    bool graph_grids = false;
    // A decode step of up to four sequences runs its projections as GEMV
    // (fast_gemv.hip) over the row-major weights; RMSNorm is then computed
    // inside the q|k|v and gate/up projections, and the sums of squares the
    // LM head's folded norm reads are taken after the last layer.
    const bool gemv_rows = h->gemv && fast_decode && nseq <= mphip::kGemvRows;
    auto gemv = [&](mphip::Epilogue epi, const float* x, int inner, const float* w, const float* w2, int columns,
                    float* out, const float* norm, int layer) {
        mphip::GemvArgs a{};
        a.rows = R;
        a.x = x;
        a.w = w;
        a.w2 = w2;
        a.out = out;
        a.norm = norm;
        a.eps = eps;
        a.inner = inner;
        a.columns = columns;
        a.heads = c.heads;
        a.layer = layer;
        a.kv = kv;
        a.meta = meta;
        a.row_block = h->row_block;
        a.row_rope = h->row_rope;
        return mphip::launch_gemv(s, epi, a);
    };
    auto launch_fast_forward = [&]() -> hipError_t {
        hipError_t e = launch_embedding();
        // Matrix-core projections; RMSNorm folded into the next projection
        // through per-16-column sums of squares of the residual stream.
        const int ssq_stride = h->workspace_rows, parts = hd / 16;
        int rope_columns = 0;
        auto fast = [&](mphip::Epilogue epi, const float* x, int inner, const float* w, const float* w2, int columns,
                        float* out, const float* norm) {
            mphip::FastGemmArgs a{};
            a.rope_columns = rope_columns;
            a.x = x;
            a.w = w;
            a.w2 = w2;
            a.out = out;
            a.rows = R;
            a.inner = inner;
            a.columns = columns;
            a.norm = norm;
            a.eps = eps;
            a.ssq_in = h->ssq;
            a.ssq_out = h->ssq;
            a.ssq_parts = parts;
            a.ssq_stride = ssq_stride;
            return mphip::launch_fast_gemm(s, epi, a);
        };
        mphip::FastAttentionWork fw{};
        fw.counts = graph_grids ? h->meta + fast_at : nullptr;
        fw.items = h->meta + items_at;
        fw.items_count = (int)fast_items;
        fw.items_capacity = (int)items_capacity;
        fw.short_items = h->meta + short_at;
        fw.short_count = (int)fast_short;
        fw.short_capacity = nseq * c.kv_heads;
        fw.merge_rows = h->meta + merge_at;
        fw.merge_count = (int)fast_merge;
        fw.merge_capacity = nseq;
        fw.capacity_grids = graph_grids;
        fw.max_splits = max_splits;
        fw.split_stride = split_stride;
        fw.partial_out = h->fast_partials;
        fw.partial_ml = h->fast_partials + (size_t)h->workspace_seqs * c.kv_heads * split_stride * group_ * 64;
        fw.kv_heads = c.kv_heads;
        auto set_prefetch = [&](int l) {
            // This layer's remaining projections, then the next layer's q|k|v.
            // Not for the GEMV projections, whose many wavefronts keep their
            // own loads in flight: at B=1 the prefetch-only work-groups cost
            // the attention more than they saved (1,346 vs 1,400 tok/s).
            const bool g = gemv_rows;
            const float* ranges[] = {h->o[l], h->gate[l], h->up[l], h->down[l],
                                     l + 1 < c.layers ? h->qkv[l + 1] : nullptr};
            const uint64_t bytes[] = {sizeof(float) * hd * hd, sizeof(float) * hd * in, sizeof(float) * hd * in,
                                      sizeof(float) * hd * in,
                                      l + 1 < c.layers ? sizeof(float) * hd * (uint64_t)qw : 0};
            for (int r = 0; r < mphip::FastAttentionWork::kPrefetchRanges; ++r) {
                fw.prefetch[r] = r < 5 && !g ? ranges[r] : nullptr;
                fw.prefetch_bytes[r] = r < 5 && !g && ranges[r] ? bytes[r] : 0;
            }
        };
        if (e == hipSuccess && !gemv_rows) e = mphip::launch_fast_ssq(s, h->x, R, hd, h->ssq, ssq_stride);
        for (int l = 0; l < c.layers && e == hipSuccess; ++l) {
            layer_now = l;
            if (gemv_rows) {
                e = timed(P, [&] { return gemv(mphip::kRope, h->x, hd, h->qkv_rows[l], nullptr, qw, h->qkv_out, h->input_norm[l], l); });
            } else if (fast_decode) {
                // q|k|v with RoPE and the KV append in the epilogue.
                e = timed(P, [&] {
                    mphip::FastGemmArgs a{};
                    a.x = h->x;
                    a.w = h->qkv[l];
                    a.out = h->qkv_out;
                    a.rows = R;
                    a.inner = hd;
                    a.columns = qw;
                    a.norm = h->input_norm[l];
                    a.eps = eps;
                    a.ssq_in = h->ssq;
                    a.ssq_parts = parts;
                    a.ssq_stride = ssq_stride;
                    a.meta = meta;
                    a.kv = kv;
                    a.layer = l;
                    a.heads = c.heads;
                    a.row_block = h->row_block;
                    a.row_rope = h->row_rope;
                    return mphip::launch_fast_gemm(s, mphip::kRope, a);
                });
            } else {
                // q and k come out of the pair-permuted weights in natural order.
                rope_columns = dim == 64 ? hd + kvw : 0;
                e = timed(P, [&] { return fast(mphip::kStore, h->x, hd, h->qkv[l], nullptr, qw, h->qkv_out, h->input_norm[l]); });
                rope_columns = 0;
            }
            if (e == hipSuccess) {
                if (fast_decode) {
                    set_prefetch(l);
                    e = timed(MP_TIME_ATTENTION, [&] {
                        return mphip::launch_fast_attention(s, h->qkv_out, qw, R, c.heads, c.kv_heads, meta, kv, l,
                                                            h->ctx, hd, fw);
                    });
                } else if (fast_rows) {
                    // RoPE and the K/V append of every row, then the prefill
                    // rows; the one-token rows after them.
                    e = mphip::launch_rope_append(s, h->qkv_out, qw, R, c.heads, c.kv_heads, dim, h->cos_table,
                                                  h->sin_table, meta, kv, l);
                    if (e == hipSuccess)
                        e = mphip::launch_fast_prefill(s, h->qkv_out, qw, c.heads, c.kv_heads, kv, l,
                                                       h->meta + pre_at, (int)fast_pre, h->ctx, hd);
                    if (e == hipSuccess && fast_items + fast_short > 0)
                        e = mphip::launch_fast_attention(s, h->qkv_out, qw, R, c.heads, c.kv_heads, meta, kv, l,
                                                         h->ctx, hd, fw);
                } else {
                    e = mphip::launch_attention(s, h->qkv_out, qw, R, c.heads, c.kv_heads, dim, meta, kv, l, h->ctx, hd,
                                                work, decode, mphip::RopeTables{h->cos_table, h->sin_table},
                                                attention_events());
                }
            }
            if (gemv_rows) {
                if (e == hipSuccess) e = timed(P, [&] { return gemv(mphip::kResidual, h->ctx, hd, h->o_rows[l], nullptr, hd, h->x, nullptr, l); });
                if (e == hipSuccess)
                    e = timed(P, [&] { return gemv(mphip::kSwiglu, h->x, hd, h->gate_rows[l], h->up_rows[l], in, h->ffn, h->post_norm[l], l); });
                if (e == hipSuccess) e = timed(P, [&] { return gemv(mphip::kResidual, h->ffn, in, h->down_rows[l], nullptr, hd, h->x, nullptr, l); });
                continue;
            }
            if (e == hipSuccess) e = timed(P, [&] { return fast(mphip::kResidual, h->ctx, hd, h->o[l], nullptr, hd, h->x, nullptr); });
            if (e == hipSuccess)
                e = timed(P, [&] { return fast(mphip::kSwiglu, h->x, hd, h->gate[l], h->up[l], in, h->ffn, h->post_norm[l]); });
            if (e == hipSuccess) e = timed(P, [&] { return fast(mphip::kResidual, h->ffn, in, h->down[l], nullptr, hd, h->x, nullptr); });
        }
        // The LM head's folded norm reads per-16-column sums of squares, which
        // the GEMV projections do not write.
        if (e == hipSuccess && gemv_rows) e = mphip::launch_fast_ssq(s, h->x, R, hd, h->ssq, ssq_stride);
        layer_now = sampled ? -2 : -1;
        if (e == hipSuccess) e = timed(MP_TIME_HEAD, [&] {
            mphip::FastGemmArgs a{};
            a.x = h->x;
            a.w = h->head;
            a.rows = nseq;
            a.inner = hd;
            a.columns = c.vocabulary;
            a.norm = h->final_norm;
            a.eps = eps;
            a.ssq_in = h->ssq;
            a.ssq_parts = parts;
            a.ssq_stride = ssq_stride;
            a.row_map = decode ? nullptr : meta.seq_last_row;  // decode: row s is sequence s's last
            a.logits = logits ? h->logits : nullptr;
            a.best_value = h->best_value;
            a.best_index = h->best_index;
            a.bad = h->best_bad;
            a.groups = c.vocabulary / mphip::fast_head_group_columns(c.vocabulary);
            hipError_t r = mphip::launch_fast_gemm(s, mphip::kHead, a);
            mphip::GemmArgs g{};
            g.rows = nseq;
            g.best_value = h->best_value;
            g.best_index = h->best_index;
            g.bad = h->best_bad;
            g.groups = a.groups;
            if (r == hipSuccess) r = mphip::launch_head_argmax(s, g, h->results, h->results + nseq);
            return r;
        });
        return e;
    };
    hipError_t e = hipSuccess;
    if (!h->fast) {
        e = launch_embedding();
    } else if (!(fast_decode && h->timing == 0 && h->graphs_enabled && nseq <= kGraphMaxSequences)) {
        e = launch_fast_forward();
    } else {
        // Decode steps of one shape replay one captured graph of the launches
        // (the metadata they read is uploaded above, at fixed offsets, and
        // the lists' counts are read on the device); a shape is captured at
        // its second step in a row.
        mp_hip::GraphKey key;
        key.nseq = nseq;
        key.logits = logits != nullptr;
        key.splits = fast_items > 0;
        key.shorts = fast_short > 0;
        key.generation = h->generation;
        hipGraphExec_t exec = nullptr;
        for (const auto& g : h->graphs)
            if (g.key == key) exec = g.exec;
        if (!exec && key == h->last_key) {
            hipGraph_t graph = nullptr;
            graph_grids = true;
            e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
            if (e == hipSuccess) {
                const hipError_t launched = launch_fast_forward();
                const hipError_t ended = hipStreamEndCapture(s, &graph);
                e = launched != hipSuccess ? launched : ended;
            }
            if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            if (graph) (void)hipGraphDestroy(graph);
            graph_grids = false;
            if (e == hipSuccess) {
                if (h->graphs.size() >= 8) {
                    (void)hipGraphExecDestroy(h->graphs.front().exec);
                    h->graphs.erase(h->graphs.begin());
                }
                h->graphs.push_back({key, exec});
            } else {
                // Capture refused: this context stays on direct launches.
                (void)hipGetLastError();
                exec = nullptr;
                h->graphs_enabled = false;
                e = hipSuccess;
            }
        }
        h->last_key = key;
        e = exec ? hipGraphLaunch(exec, s) : launch_fast_forward();
    }
    for (int l = 0; !h->fast && l < c.layers && e == hipSuccess; ++l) {
        layer_now = l;
        e = timed(P, [&] { return normed_gemm(mphip::kStore, h->input_norm[l], R, hd, h->qkv[l], nullptr, qw, h->qkv_out); });
        if (e == hipSuccess)
            e = mphip::launch_attention(s, h->qkv_out, qw, R, c.heads, c.kv_heads, dim, meta, kv, l, h->ctx, hd, work,
                                        decode, mphip::RopeTables{h->cos_table, h->sin_table}, attention_events());
        if (e == hipSuccess) e = timed(P, [&] { return gemm(mphip::kResidual, h->ctx, R, hd, h->o[l], nullptr, hd, h->x); });
        if (e == hipSuccess)
            e = timed(P, [&] { return normed_gemm(mphip::kSwiglu, h->post_norm[l], R, hd, h->gate[l], h->up[l], in, h->ffn); });
        if (e == hipSuccess) e = timed(P, [&] { return gemm(mphip::kResidual, h->ffn, R, in, h->down[l], nullptr, hd, h->x); });
    }
    if (!h->fast) layer_now = sampled ? -2 : -1;  // a sampled call times no head
    if (!h->fast && e == hipSuccess) e = timed(MP_TIME_HEAD, [&] {
        // Final norm of each sequence's last row, then the LM head with the
        // greedy argmax folded into its epilogue (logits are written only
        // when the caller asks for them).
        hipError_t r = mphip::launch_rms(s, h->x, meta.seq_last_row, h->final_norm, h->last, nseq, hd, eps);
        mphip::GemmArgs a{};
        a.x = h->last;
        a.w = h->head;
        a.out = logits ? h->logits : nullptr;
        a.rows = nseq;
        a.inner = hd;
        a.columns = c.vocabulary;
        a.best_value = h->best_value;
        a.best_index = h->best_index;
        a.bad = h->best_bad;
        a.groups = mphip::head_groups(c.vocabulary);
        if (r == hipSuccess) r = mphip::launch_gemm(s, mphip::kHead, a);
        if (r == hipSuccess) r = mphip::launch_head_argmax(s, a, h->results, h->results + nseq);
        return r;
    });
    if ((status = check(h, e, "model kernel launch"))) return status;
    if ((status = ensure_pinned(h, &h->host_results, &h->host_results_capacity, 2 * (size_t)nseq + 1,
                                "allocate pinned results")))
        return status;
    int32_t* const results = h->host_results;
    status = check(h, hipMemcpyAsync(results, h->results, sizeof(int32_t) * (2 * nseq + 1), hipMemcpyDeviceToHost, s),
                   "download argmax");
    if (!status && logits) {
        status = check(h, hipMemcpyAsync(logits, h->logits, sizeof(float) * (size_t)nseq * c.vocabulary, hipMemcpyDeviceToHost, s), "download logits");
        if (!status) h->stats.logits_downloaded_bytes += sizeof(float) * (size_t)nseq * c.vocabulary;
    }
    if (!status) status = stream_wait_polling(h, "model completion");
    if (status) return status;
    for (size_t i = 0; i < h->spans.size(); ++i) {
        float ms = 0.0f;
        if ((status = check(h, hipEventElapsedTime(&ms, h->events[2 * i], h->events[2 * i + 1]), "kernel timing")))
            return status;
        const uint64_t ns = (uint64_t)((double)ms * 1e6);
        mp_hip_timing_totals& t = h->times;
        if (h->spans[i] == MP_TIME_ATTENTION) t.attention_ns += ns, ++t.attention_launches;
        if (h->spans[i] == MP_TIME_PROJECTION) t.projection_ns += ns, ++t.projection_launches;
        if (h->spans[i] == MP_TIME_HEAD) t.head_ns += ns, ++t.head_launches;
    }
    if (results[2 * (size_t)nseq])
        return fail(h, MP_DEVICE_ERROR, "attention kernel gave up a bounded wait; results discarded");
    std::memcpy(argmax, results, sizeof(int32_t) * nseq);
    if (nonfinite) std::memcpy(nonfinite, results + nseq, sizeof(int32_t) * nseq);
    ++h->stats.forward_calls;
    h->stats.forward_rows += R;
    for (int i = 0; i < nseq; ++i)
        if (results[(size_t)nseq + i]) return fail(h, MP_NONFINITE, "nonfinite HIP logits");
    return MP_OK;
}

int mp_hip_paged_attention_decode(const float* q, const float* keys, const float* values,
                                  const int32_t* table, int32_t length, int32_t layer,
                                  int32_t layers, int32_t block_tokens, int32_t heads,
                                  int32_t kv_heads, int32_t dim, float* out, void* stream) {
    if (!q || !keys || !values || !table || !out || length < 1 || layer < 0 || layer >= layers ||
        block_tokens < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads || dim < 4 || dim % 4 ||
        dim > 256 || heads / kv_heads > 8) {
        mphip::set_free_error("invalid paged attention arguments");
        return MP_INVALID_ARGUMENT;
    }
    const int group = heads / kv_heads;
    float* scratch = nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if ((size_t)group * (size_t)((length + 15) & ~15) > (size_t)mphip::kAttentionLdsScores) {
        // Long rows keep their scores in global memory; synchronous so the
        // temporary can be released before returning.
        const size_t floats = (size_t)kv_heads * group * (size_t)((length + 15) & ~15);
        if (hipMalloc(&scratch, floats * sizeof(float)) != hipSuccess) return MP_OUT_OF_MEMORY;
    }
    hipError_t e = mphip::launch_attention_single(s, q, keys, values, table, length, layer, layers,
                                                  block_tokens, heads, kv_heads, dim, out, scratch);
    if (scratch) {
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        (void)hipFree(scratch);
    }
    return e == hipSuccess ? MP_OK : MP_DEVICE_ERROR;
}

int mp_hip_paged_attention_decode_fast(const float* q, const float* keys, const float* values,
                                       const int32_t* tables, int32_t table_stride, const int32_t* lengths,
                                       int32_t rows, int32_t layer, int32_t layers, int32_t block_tokens,
                                       int32_t heads, int32_t kv_heads, int32_t dim, float* out, void* stream) {
    if (!q || !keys || !values || !tables || !lengths || !out || rows < 1 || table_stride < 1 || layer < 0 ||
        layer >= layers || block_tokens != 16 || dim != 64 || heads < 1 || kv_heads < 1 || heads % kv_heads ||
        heads / kv_heads > 4) {
        mphip::set_free_error("invalid fast paged attention arguments (pages of 16 tokens, head dim 64 and at "
                              "most 4 query heads per KV head)");
        return MP_INVALID_ARGUMENT;
    }
    const int group = heads / kv_heads;
    // Work lists as the forward builds them for one-token rows (row r is
    // sequence r): rows of up to 256 tokens in one work-group each, longer
    // rows as splits (whole splits first) merged afterwards.
    std::vector<int32_t> split_items, short_items, merge_rows, positions(rows);
    int max_splits = 0, longest = 1;
    // The short rows' page ids go into their items: a host copy of their
    // table rows.
    std::vector<int32_t> host_table;
    for (int r = 0; r < rows; ++r) {
        const int length = lengths[r];
        if (length < 1 || (length + 15) / 16 > table_stride) {
            mphip::set_free_error("invalid fast paged attention row length");
            return MP_INVALID_ARGUMENT;
        }
        positions[r] = length - 1;
        longest = std::max(longest, length);
        if (mphip::fast_attention_short(length)) {
            const int pages = (length + 15) / 16;
            host_table.resize(pages);
            if (hipMemcpy(host_table.data(), tables + (size_t)r * table_stride, sizeof(int32_t) * pages,
                          hipMemcpyDeviceToHost) != hipSuccess) {
                mphip::set_free_error("fast paged attention: reading a page table");
                return MP_DEVICE_ERROR;
            }
            for (int kvh = 0; kvh < kv_heads; ++kvh) {
                short_items.insert(short_items.end(), {r, r * kv_heads + kvh, length, 0});
                for (int k = 0; k < mphip::kShortItemInts - 4; ++k)
                    short_items.push_back(host_table[std::min(k, pages - 1)]);
            }
            continue;
        }
        const int split = mphip::fast_attention_split(length), splits = (length + split - 1) / split;
        max_splits = std::max(max_splits, splits);
        merge_rows.insert(merge_rows.end(), {r, r, splits, 0});
    }
    for (int pass = 0; pass < 2; ++pass)
        for (int r = 0; r < rows; ++r) {
            const int length = lengths[r];
            if (mphip::fast_attention_short(length)) continue;
            const int split = mphip::fast_attention_split(length), splits = (length + split - 1) / split;
            for (int kvh = 0; kvh < kv_heads; ++kvh)
                for (int sp = 0; sp < splits; ++sp) {
                    const int n = std::min(split, length - sp * split);
                    if ((n == split) != (pass == 0)) continue;
                    split_items.insert(split_items.end(),
                                       {r, r * kv_heads + kvh, r, mphip::fast_attention_item_w(n, sp, split)});
                }
        }
    // One device buffer: the counts and int32 lists (16-byte aligned), then
    // the partials.
    const std::vector<int32_t> counts = {(int32_t)(split_items.size() / 4),
                                         (int32_t)(short_items.size() / mphip::kShortItemInts),
                                         (int32_t)(merge_rows.size() / 4), 0};
    const size_t ints = counts.size() + split_items.size() + short_items.size() + merge_rows.size() + positions.size();
    const size_t int_bytes = (ints * sizeof(int32_t) + 255) / 256 * 256;
    const size_t partial_floats = (size_t)rows * kv_heads * max_splits * group * (64 + 2);
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* buffer = nullptr;
    hipError_t e = hipMalloc(&buffer, int_bytes + partial_floats * sizeof(float));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        mphip::set_free_error(std::string("allocate fast attention work: ") + hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? MP_OUT_OF_MEMORY : MP_DEVICE_ERROR;
    }
    std::vector<int32_t> host;
    host.reserve(ints);
    for (const std::vector<int32_t>* part : {&counts, (const std::vector<int32_t>*)&split_items,
                                             (const std::vector<int32_t>*)&short_items,
                                             (const std::vector<int32_t>*)&merge_rows,
                                             (const std::vector<int32_t>*)&positions})
        host.insert(host.end(), part->begin(), part->end());
    int32_t* const dev = reinterpret_cast<int32_t*>(buffer);
    e = hipMemcpyAsync(dev, host.data(), ints * sizeof(int32_t), hipMemcpyHostToDevice, s);
    mphip::FastAttentionWork w{};
    w.items = dev + counts.size();
    w.items_count = w.items_capacity = counts[0];
    w.short_items = w.items + split_items.size();
    w.short_count = w.short_capacity = counts[1];
    w.merge_rows = w.short_items + short_items.size();
    w.merge_count = w.merge_capacity = counts[2];
    w.max_splits = max_splits;
    w.split_stride = max_splits;
    w.partial_out = reinterpret_cast<float*>(buffer + int_bytes);
    w.partial_ml = w.partial_out + (size_t)rows * kv_heads * max_splits * group * 64;
    w.kv_heads = kv_heads;
    mphip::RowMeta meta{};
    meta.row_pos = w.merge_rows + merge_rows.size();
    const mphip::PagedKv kv{const_cast<float*>(keys), const_cast<float*>(values), tables, table_stride, layers,
                            block_tokens, kv_heads * dim};
    if (e == hipSuccess)
        e = mphip::launch_fast_attention(s, q, heads * dim, rows, heads, kv_heads, meta, kv, layer, out, heads * dim,
                                         w, true);
    // Synchronous, so that the work lists can be released before returning.
    const hipError_t done = hipStreamSynchronize(s);
    if (e == hipSuccess) e = done;
    (void)hipFree(buffer);
    if (e != hipSuccess) {
        mphip::set_free_error(std::string("fast paged attention: ") + hipGetErrorString(e));
        return MP_DEVICE_ERROR;
    }
    return MP_OK;
}

int mp_hip_sync(mp_hip* h) {
    if (!h) return MP_INVALID_ARGUMENT;
    const int status = flush_pending(h);
    if (status) return status;
    return check(h, hipStreamSynchronize(h->stream), "model completion");
}

int mp_hip_stats(const mp_hip* h, mp_hip_counters* out) {
    if (!h || !out) return MP_INVALID_ARGUMENT;
    *out = h->stats;
    return MP_OK;
}

int mp_hip_kv_pools(const mp_hip* h, float** keys, float** values, size_t* elements) {
    if (!h) return MP_INVALID_ARGUMENT;
    if (keys) *keys = h->keys;
    if (values) *values = h->values;
    if (elements) *elements = h->pool_elements;
    return MP_OK;
}

void* mp_hip_stream(const mp_hip* h) { return h ? (void*)h->stream : nullptr; }

int mp_hip_set_timing(mp_hip* h, uint32_t classes) {
    if (!h || (classes & ~15u)) return fail(h, MP_INVALID_ARGUMENT, "invalid timing classes");
    int status = mp_hip_sync(h);
    if (status) return status;
    // One pair per GEMM and attention of every layer plus the head.
    const size_t need = 2 * (5 * (size_t)h->model.layers + 1);
    while (h->events.size() < need) {
        hipEvent_t ev = nullptr;
        if ((status = check(h, hipEventCreateWithFlags(&ev, hipEventDisableSystemFence), "create timing event")))
            return status;
        h->events.push_back(ev);
    }
    h->timing = classes;
    h->times = mp_hip_timing_totals{};
    return MP_OK;
}

int mp_hip_set_graphs(mp_hip* h, int32_t enabled) {
    if (!h) return MP_INVALID_ARGUMENT;
    int status = mp_hip_sync(h);
    if (status) return status;
    retire_graphs(h);
    h->graphs_enabled = enabled != 0;
    h->last_key = mp_hip::GraphKey{};
    return MP_OK;
}

int mp_hip_graphs_captured(const mp_hip* h, int32_t* count) {
    if (!h || !count) return MP_INVALID_ARGUMENT;
    *count = (int32_t)h->graphs.size();
    return MP_OK;
}

int mp_hip_kernel_times(const mp_hip* h, mp_hip_timing_totals* out) {
    if (!h || !out) return MP_INVALID_ARGUMENT;
    *out = h->times;
    return MP_OK;
}

}  // extern "C"
