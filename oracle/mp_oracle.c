/*
 * MiniPrefix CPU oracle -- TEST INFRASTRUCTURE ONLY (see mp_oracle.h).
 *
 * Every floating-point expression below keeps the reference's evaluation
 * order and its separate multiply/add roundings; the file is compiled with
 * -ffp-contract=off so no FMA is formed.
 */
#include "mp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- data -- */
uint64_t mpo_splitmix64_next(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t mpo_stream_init(uint64_t seed, uint64_t stream) {
    return seed ^ ((stream + 1ull) * 0xD1B54A32D192ED03ull);
}

void mpo_fill_normal(float* dst, size_t count, uint64_t seed, uint64_t stream, double stddev) {
    uint64_t state = mpo_stream_init(seed, stream);
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < count) {
        const uint64_t a = mpo_splitmix64_next(&state), b = mpo_splitmix64_next(&state);
        const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53; /* (0, 1] */
        const double u2 = (double)(b >> 11) * 0x1.0p-53;       /* [0, 1) */
        const double r = sqrt(-2.0 * log(u1)), theta = two_pi * u2;
        dst[i++] = (float)(stddev * (r * cos(theta)));
        if (i < count) dst[i++] = (float)(stddev * (r * sin(theta)));
    }
}

void mpo_fill_tokens(int32_t* dst, size_t count, uint64_t seed, uint64_t stream, int32_t vocabulary) {
    uint64_t state = mpo_stream_init(seed, stream);
    for (size_t i = 0; i < count; ++i)
        dst[i] = (int32_t)(mpo_splitmix64_next(&state) % (uint64_t)vocabulary);
}

void mpo_permutation(int32_t* dst, int32_t count, uint64_t seed, uint64_t stream) {
    uint64_t state = mpo_stream_init(seed, stream);
    for (int32_t i = 0; i < count; ++i) dst[i] = i;
    for (int32_t i = count - 1; i > 0; --i) {
        const int32_t j = (int32_t)(mpo_splitmix64_next(&state) % (uint64_t)(i + 1));
        const int32_t t = dst[i];
        dst[i] = dst[j];
        dst[j] = t;
    }
}

/* ------------------------------------------------------------------ ops -- */
/* llama_runner.cpp:10-16: sequential sum of squares, 1/sqrt(mean+eps),
 * then (x*scale)*w. */
void mpo_rms(const float* x, const float* weight, float* out, int rows, int width, float eps) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * width;
        float sum = 0;
        for (int d = 0; d < width; ++d) {
            const float v = xr[d];
            sum += v * v;
        }
        const float scale = 1 / sqrtf(sum / (float)width + eps);
        for (int d = 0; d < width; ++d) out[(size_t)r * width + d] = xr[d] * scale * weight[d];
    }
}

/* matmul_kernel.cpp:289-354 with the SSE2 micro-kernel (:101-109): the
 * output starts at 0 and each column accumulates x[k]*w[k][c] for
 * k = 0..inner-1 in order, multiply and add rounded separately. Columns are
 * tiled here only for cache reuse; no column's summation order changes. */
void mpo_linear(const float* x, const float* w, float* out, int rows, int inner, int columns) {
    const int tile = 256;
    memset(out, 0, sizeof(float) * (size_t)rows * (size_t)columns);
    for (int c0 = 0; c0 < columns; c0 += tile) {
        const int c1 = c0 + tile < columns ? c0 + tile : columns;
        for (int k = 0; k < inner; ++k) {
            const float* wk = w + (size_t)k * columns;
            for (int r = 0; r < rows; ++r) {
                const float xk = x[(size_t)r * inner + k];
                float* o = out + (size_t)r * columns;
                for (int c = c0; c < c1; ++c) o[c] = o[c] + xk * wk[c];
            }
        }
    }
}

/* The tied head packs embedding^T (PackedMatMulRhs(E, true),
 * matmul_kernel.cpp:172-189) and runs the same sequential-k product. */
void mpo_linear_transposed(const float* x, const float* embedding, float* out,
                           int rows, int inner, int vocabulary) {
    float* packed = (float*)malloc(sizeof(float) * (size_t)inner * (size_t)vocabulary);
    for (int k = 0; k < inner; ++k)
        for (int v = 0; v < vocabulary; ++v)
            packed[(size_t)k * vocabulary + v] = embedding[(size_t)v * inner + k];
    mpo_linear(x, packed, out, rows, inner, vocabulary);
    free(packed);
}

/* llama_runner.cpp:17-22: split-half rotation, pairs (d, d+dim/2). */
void mpo_rope(float* x, int rows, int heads, int dim, int start, float theta) {
    for (int row = 0; row < rows; ++row)
        for (int h = 0; h < heads; ++h)
            for (int d = 0; d < dim / 2; ++d) {
                const float angle = (float)(start + row) / powf(theta, (float)(2 * d) / (float)dim);
                const float cs = cosf(angle), sn = sinf(angle);
                const size_t i = ((size_t)row * heads + h) * dim + d, j = i + dim / 2;
                const float a = x[i], b = x[j];
                x[i] = a * cs - b * sn;
                x[j] = b * cs + a * sn;
            }
}

void mpo_rope_table(float* cos_out, float* sin_out, int positions, int dim, float theta) {
    for (int p = 0; p < positions; ++p)
        for (int d = 0; d < dim / 2; ++d) {
            const float angle = (float)p / powf(theta, (float)(2 * d) / (float)dim);
            cos_out[(size_t)p * (dim / 2) + d] = cosf(angle);
            sin_out[(size_t)p * (dim / 2) + d] = sinf(angle);
        }
}

/* llama_runner.cpp:97: g = (g/(1+exp(-g)))*u. */
void mpo_swiglu(float* gate, const float* up, size_t count) {
    for (size_t i = 0; i < count; ++i) {
        const float a = gate[i];
        gate[i] = (a / (1 + expf(-a))) * up[i];
    }
}

/* basic_ops.cpp:93-106 (elementwise float add). */
void mpo_add(float* x, const float* y, size_t count) {
    for (size_t i = 0; i < count; ++i) x[i] = x[i] + y[i];
}

float mpo_expf(float x) { return expf(x); }

static size_t pool_offset(const int32_t* blocks, int layer, int token, int layers,
                          int block_tokens, int width) {
    return (((size_t)blocks[token / block_tokens] * (size_t)layers + (size_t)layer) *
                (size_t)block_tokens + (size_t)(token % block_tokens)) * (size_t)width;
}

/* llama_runner.cpp:85-93: two-pass softmax per (row, head), scores divided
 * by sqrt(dim), p = score/denominator inside the PV sum. */
void mpo_attention(const float* q, const float* keys, const float* values,
                   const int32_t* blocks, int start, int rows, int layer, int layers,
                   int block_tokens, int heads, int kv_heads, int dim, float* out) {
    const int kv_width = kv_heads * dim, group = heads / kv_heads;
    const int total = start + rows;
    size_t* offsets = (size_t*)malloc(sizeof(size_t) * (size_t)total);
    float* scores = (float*)malloc(sizeof(float) * (size_t)total);
    for (int t = 0; t < total; ++t)
        offsets[t] = pool_offset(blocks, layer, t, layers, block_tokens, kv_width);
    const float root = sqrtf((float)dim);
    for (int row = 0; row < rows; ++row)
        for (int h = 0; h < heads; ++h) {
            const int length = start + row + 1, kh = h / group;
            const float* qh = q + ((size_t)row * heads + h) * dim;
            float maximum = -INFINITY;
            for (int t = 0; t < length; ++t) {
                const float* k = keys + offsets[t] + (size_t)kh * dim;
                float score = 0;
                for (int d = 0; d < dim; ++d) score += qh[d] * k[d];
                scores[t] = score / root;
                maximum = maximum < scores[t] ? scores[t] : maximum; /* std::max */
            }
            float denominator = 0;
            for (int t = 0; t < length; ++t) {
                scores[t] = expf(scores[t] - maximum);
                denominator += scores[t];
            }
            for (int d = 0; d < dim; ++d) {
                float sum = 0;
                for (int t = 0; t < length; ++t)
                    sum += (scores[t] / denominator) * values[offsets[t] + (size_t)kh * dim + d];
                out[((size_t)row * heads + h) * dim + d] = sum;
            }
        }
    free(scores);
    free(offsets);
}

/* --------------------------------------------------------------- model -- */
struct mpo_model {
    mpo_config config;
    float* embedding;
    float* final_norm;
    float* lm_head; /* [hidden, vocabulary] packed: untied head, or tied E^T */
    float** layers; /* layers * MPO_LAYER_TENSORS */
    int tied_packed;
};

static size_t slot_elements(const mpo_config* c, int slot) {
    const size_t h = (size_t)c->hidden, kv = (size_t)(c->hidden / c->heads) * (size_t)c->kv_heads,
                 i = (size_t)c->intermediate;
    switch (slot) {
    case MPO_INPUT_NORM: case MPO_POST_NORM: return h;
    case MPO_Q: case MPO_O: return h * h;
    case MPO_K: case MPO_V: return h * kv;
    case MPO_GATE: case MPO_UP: case MPO_DOWN: return h * i;
    default: return 0;
    }
}

static int valid_config(const mpo_config* c) {
    return c->layers >= 1 && c->hidden >= 2 && c->heads >= 1 && c->kv_heads >= 1 &&
           c->hidden % c->heads == 0 && c->heads % c->kv_heads == 0 &&
           (c->hidden / c->heads) % 2 == 0 && c->vocabulary >= 2 && c->intermediate >= 1 &&
           c->context >= 1;
}

static mpo_model* model_alloc(const mpo_config* c) {
    if (!valid_config(c)) return NULL;
    mpo_model* m = (mpo_model*)calloc(1, sizeof(mpo_model));
    m->config = *c;
    m->embedding = (float*)malloc(sizeof(float) * (size_t)c->vocabulary * (size_t)c->hidden);
    m->final_norm = (float*)malloc(sizeof(float) * (size_t)c->hidden);
    m->lm_head = (float*)malloc(sizeof(float) * (size_t)c->vocabulary * (size_t)c->hidden);
    m->layers = (float**)calloc((size_t)c->layers * MPO_LAYER_TENSORS, sizeof(float*));
    for (int l = 0; l < c->layers; ++l)
        for (int s = 0; s < MPO_LAYER_TENSORS; ++s)
            m->layers[l * MPO_LAYER_TENSORS + s] = (float*)malloc(sizeof(float) * slot_elements(c, s));
    return m;
}

static void pack_tied_head(mpo_model* m) {
    const mpo_config* c = &m->config;
    for (int k = 0; k < c->hidden; ++k)
        for (int v = 0; v < c->vocabulary; ++v)
            m->lm_head[(size_t)k * c->vocabulary + v] = m->embedding[(size_t)v * c->hidden + k];
}

mpo_model* mpo_model_synthetic(const mpo_config* c, uint64_t seed, double stddev) {
    mpo_model* m = model_alloc(c);
    if (!m) return NULL;
    mpo_fill_normal(m->embedding, (size_t)c->vocabulary * c->hidden, seed, 0, stddev);
    for (int d = 0; d < c->hidden; ++d) m->final_norm[d] = 1.0f;
    for (int l = 0; l < c->layers; ++l)
        for (int s = 0; s < MPO_LAYER_TENSORS; ++s) {
            float* t = m->layers[l * MPO_LAYER_TENSORS + s];
            const size_t n = slot_elements(c, s);
            if (s == MPO_INPUT_NORM || s == MPO_POST_NORM)
                for (size_t i = 0; i < n; ++i) t[i] = 1.0f;
            else
                mpo_fill_normal(t, n, seed, 2ull + 9ull * (uint64_t)l + (uint64_t)s, stddev);
        }
    if (c->tied) pack_tied_head(m);
    else mpo_fill_normal(m->lm_head, (size_t)c->vocabulary * c->hidden, seed,
                         2ull + 9ull * (uint64_t)c->layers, stddev);
    return m;
}

mpo_model* mpo_model_from_tensors(const mpo_config* c, const float* embedding,
                                  const float* final_norm, const float* const* layer_tensors,
                                  const float* lm_head) {
    mpo_model* m = model_alloc(c);
    if (!m) return NULL;
    memcpy(m->embedding, embedding, sizeof(float) * (size_t)c->vocabulary * c->hidden);
    memcpy(m->final_norm, final_norm, sizeof(float) * (size_t)c->hidden);
    for (int l = 0; l < c->layers; ++l)
        for (int s = 0; s < MPO_LAYER_TENSORS; ++s)
            memcpy(m->layers[l * MPO_LAYER_TENSORS + s], layer_tensors[l * MPO_LAYER_TENSORS + s],
                   sizeof(float) * slot_elements(c, s));
    if (c->tied || !lm_head) pack_tied_head(m);
    else memcpy(m->lm_head, lm_head, sizeof(float) * (size_t)c->vocabulary * c->hidden);
    return m;
}

void mpo_model_free(mpo_model* m) {
    if (!m) return;
    for (int l = 0; l < m->config.layers; ++l)
        for (int s = 0; s < MPO_LAYER_TENSORS; ++s) free(m->layers[l * MPO_LAYER_TENSORS + s]);
    free(m->layers);
    free(m->embedding);
    free(m->final_norm);
    free(m->lm_head);
    free(m);
}

const mpo_config* mpo_model_config(const mpo_model* m) { return &m->config; }

const float* mpo_model_tensor(const mpo_model* m, int layer, int slot) {
    if (slot == -1) return m->embedding;
    if (slot == -2) return m->final_norm;
    if (slot == -3) return m->config.tied ? NULL : m->lm_head;
    if (layer < 0 || layer >= m->config.layers || slot < 0 || slot >= MPO_LAYER_TENSORS) return NULL;
    return m->layers[layer * MPO_LAYER_TENSORS + slot];
}

/* llama_runner.cpp:60-104 (after the KV transaction and COW copy, which the
 * caller performs on the pools before this call). */
int mpo_append(const mpo_model* m, float* keys, float* values, int block_tokens,
               const int32_t* blocks, int block_count, int used,
               const int32_t* tokens, int n, float* logits) {
    const mpo_config* c = &m->config;
    const int dim = c->hidden / c->heads, kv = c->kv_heads * dim, H = c->hidden, I = c->intermediate;
    if (n < 1 || used < 0 || block_tokens < 1 || used + n > c->context ||
        (used + n + block_tokens - 1) / block_tokens > block_count)
        return -1;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= c->vocabulary) return -1;
    float* x = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* normalized = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* q = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* k = (float*)malloc(sizeof(float) * (size_t)n * kv);
    float* v = (float*)malloc(sizeof(float) * (size_t)n * kv);
    float* context = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* projection = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* gate = (float*)malloc(sizeof(float) * (size_t)n * I);
    float* up = (float*)malloc(sizeof(float) * (size_t)n * I);
    for (int row = 0; row < n; ++row)
        memcpy(x + (size_t)row * H, m->embedding + (size_t)tokens[row] * H, sizeof(float) * H);
    for (int l = 0; l < c->layers; ++l) {
        float* const* w = m->layers + (size_t)l * MPO_LAYER_TENSORS;
        mpo_rms(x, w[MPO_INPUT_NORM], normalized, n, H, c->rms_epsilon);
        mpo_linear(normalized, w[MPO_Q], q, n, H, H);
        mpo_linear(normalized, w[MPO_K], k, n, H, kv);
        mpo_linear(normalized, w[MPO_V], v, n, H, kv);
        mpo_rope(q, n, c->heads, dim, used, c->rope_theta);
        mpo_rope(k, n, c->kv_heads, dim, used, c->rope_theta);
        for (int row = 0; row < n; ++row) {
            const size_t off = pool_offset(blocks, l, used + row, c->layers, block_tokens, kv);
            memcpy(keys + off, k + (size_t)row * kv, sizeof(float) * kv);
            memcpy(values + off, v + (size_t)row * kv, sizeof(float) * kv);
        }
        mpo_attention(q, keys, values, blocks, used, n, l, c->layers, block_tokens, c->heads,
                      c->kv_heads, dim, context);
        mpo_linear(context, w[MPO_O], projection, n, H, H);
        mpo_add(x, projection, (size_t)n * H);
        mpo_rms(x, w[MPO_POST_NORM], normalized, n, H, c->rms_epsilon);
        mpo_linear(normalized, w[MPO_GATE], gate, n, H, I);
        mpo_linear(normalized, w[MPO_UP], up, n, H, I);
        mpo_swiglu(gate, up, (size_t)n * I);
        mpo_linear(gate, w[MPO_DOWN], projection, n, I, H);
        mpo_add(x, projection, (size_t)n * H);
    }
    mpo_rms(x + (size_t)(n - 1) * H, m->final_norm, normalized, 1, H, c->rms_epsilon);
    mpo_linear(normalized, m->lm_head, logits, 1, H, c->vocabulary);
    int status = 0;
    for (int i = 0; i < c->vocabulary; ++i)
        if (!isfinite(logits[i])) status = -2;
    free(x); free(normalized); free(q); free(k); free(v);
    free(context); free(projection); free(gate); free(up);
    return status;
}
