/*
 * MiniPrefix CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference CPU generation path
 * (miniprefix/src/backend/cpu/llama_runner.cpp:10-104 with the projection
 * arithmetic of src/backend/cpu/matmul_kernel.cpp:101-109,289-354 and the
 * residual add of src/ops/basic_ops.cpp:93-106), op for op and in the same
 * floating-point order, so that its outputs are bit-identical to the reference
 * built with its default (SSE2, no FMA) flags.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only to check results against it. The product path
 * never does.
 *
 * Build: `make -C oracle` (gcc -ffp-contract=off; libm supplies expf, powf,
 * cosf and sinf exactly as the reference's std::exp/pow/cos/sin on float).
 */
#ifndef MP_ORACLE_H
#define MP_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic synthetic data (same specification as the product's
 *      generator; see mpo_stream_init) ---------------------------------- */
uint64_t mpo_splitmix64_next(uint64_t* state);
/* state = seed ^ (stream+1)*0xD1B54A32D192ED03 */
uint64_t mpo_stream_init(uint64_t seed, uint64_t stream);
/* N(0, stddev^2) by Box-Muller in double, pairs (r cos, r sin). */
void mpo_fill_normal(float* dst, size_t count, uint64_t seed, uint64_t stream, double stddev);
/* Uniform ids in [0, vocabulary): splitmix64 output modulo vocabulary. */
void mpo_fill_tokens(int32_t* dst, size_t count, uint64_t seed, uint64_t stream, int32_t vocabulary);
/* Fisher-Yates permutation of 0..count-1 driven by splitmix64 modulo (i+1). */
void mpo_permutation(int32_t* dst, int32_t count, uint64_t seed, uint64_t stream);

/* ---- model ----------------------------------------------------------- */
typedef struct mpo_config {
    int layers, hidden, intermediate, heads, kv_heads, vocabulary, context, eos;
    float rms_epsilon, rope_theta;
    int tied;
} mpo_config;

/* Per-layer tensor slots in canonical order; stored [in,out] row-major like
 * the reference's ModelWeights (miniprefix/src/model/model.cpp:28-38). */
enum {
    MPO_INPUT_NORM = 0, MPO_Q, MPO_K, MPO_V, MPO_O, MPO_POST_NORM, MPO_GATE, MPO_UP, MPO_DOWN,
    MPO_LAYER_TENSORS
};

typedef struct mpo_model mpo_model;

/* Synthetic random-init model: every projection and the embedding drawn from
 * N(0, stddev^2); all RMSNorm weights 1.0. Tensor stream ids: embedding 0,
 * final norm 1, layer l slot j -> 2 + 9*l + j, untied head 2 + 9*layers. */
mpo_model* mpo_model_synthetic(const mpo_config* config, uint64_t seed, double stddev);
/* Model over caller-owned weights (copied). `layer_tensors` holds layers*9
 * pointers in canonical slot order; `lm_head` is [hidden, vocab] or NULL if tied. */
mpo_model* mpo_model_from_tensors(const mpo_config* config, const float* embedding,
                                  const float* final_norm, const float* const* layer_tensors,
                                  const float* lm_head);
void mpo_model_free(mpo_model* model);
const mpo_config* mpo_model_config(const mpo_model* model);
/* Borrowed pointer to a tensor: slot -1 embedding, -2 final norm, -3 untied head. */
const float* mpo_model_tensor(const mpo_model* model, int layer, int slot);

/* One append of `count` tokens to a paged sequence whose committed length is
 * `used` (reference CpuRunner::append, llama_runner.cpp:60-104). `blocks` is
 * the sequence's page table after reservation; the pools are laid out
 * [block][layer][slot][kv_width] (miniprefix/src/kv/paged_kv.cpp:53-56).
 * Writes K/V for positions used..used+count-1 and the last row's logits.
 * Returns 0, or -1 for invalid input, -2 for non-finite logits. */
int mpo_append(const mpo_model* model, float* keys, float* values, int block_tokens,
               const int32_t* blocks, int block_count, int used,
               const int32_t* tokens, int count, float* logits);

/* ---- single ops, for kernel-level parity ------------------------------ */
void mpo_rms(const float* x, const float* weight, float* out, int rows, int width, float eps);
/* out[rows, columns] = x[rows, inner] * w[inner, columns], sequential k. */
void mpo_linear(const float* x, const float* w, float* out, int rows, int inner, int columns);
/* Tied head: out[rows, vocabulary] = x * embedding^T, sequential k. */
void mpo_linear_transposed(const float* x, const float* embedding, float* out,
                           int rows, int inner, int vocabulary);
void mpo_rope(float* x, int rows, int heads, int dim, int start, float theta);
/* The angle table the reference evaluates inline: cos/sin of
 * float(pos)/powf(theta, float(2d)/float(dim)), [positions][dim/2] each. */
void mpo_rope_table(float* cos_out, float* sin_out, int positions, int dim, float theta);
void mpo_swiglu(float* gate, const float* up, size_t count);
void mpo_add(float* x, const float* y, size_t count);
float mpo_expf(float x);

/* Causal GQA attention of `rows` query rows whose first row sits at position
 * `start`, against one layer of the paged pools (llama_runner.cpp:85-93).
 * q is [rows, heads, dim]; out is [rows, heads*dim]. */
void mpo_attention(const float* q, const float* keys, const float* values,
                   const int32_t* blocks, int start, int rows, int layer, int layers,
                   int block_tokens, int heads, int kv_heads, int dim, float* out);

#ifdef __cplusplus
}
#endif
#endif
