/*
 * ORACLE — test infrastructure only.
 *
 * Scalar CPU restatement of StarLight's reference kernels
 * (the files under crates/backends/backend-cpu/src/reference/). Only tests/, the smoke
 * check and the CPU-baseline leg of bench.py load this library, and only to
 * check or time against it; the product (starlight_amd/) never links or calls it.
 *
 * Contract kept from the reference (backend-cpu/README.md:55-67):
 *   - f32 data, row-major, no strides;
 *   - lengths and shapes are validated before the first write;
 *   - fixed accumulation order, no FMA (build with -ffp-contract=off),
 *     no fast-math; transcendental calls go to the platform libm exactly where
 *     the Rust code calls f32::exp / f64::powf / f64::sin / f64::cos.
 *
 * Every function returns SLR_OK or an error kind and, on error, stores a
 * static reason string in *why (mirrors KernelError, reference/mod.rs:44-61).
 *
 * The quantization helpers at the end have no counterpart in the reference
 * (sl-precision is absent from it); they restate the convention this project
 * adopts and are pinned by closed-form tests, not by reference vectors.
 *
 * Threads: the reference is single-threaded, and so is this library by
 * default (the CPU-baseline timing runs it that way). slr_set_threads(n)
 * lets the tests spread the independent outputs of matmul, attention,
 * swiglu and rms_norm_matmul over n OpenMP threads; every output element is
 * still computed by one thread in the reference's order, so the results are
 * bit-identical for any n.
 */
#include <math.h>
#include <stdlib.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

enum {
    SLR_OK = 0,
    SLR_LENGTH_MISMATCH = 1,
    SLR_SHAPE_OVERFLOW = 2,
    SLR_INVALID_SHAPE = 3,
    SLR_UNSUPPORTED = 4,
};

static int g_threads = 1;

/* Number of OpenMP threads the parallel loops use (1: sequential). */
void slr_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int slr_get_threads(void) { return g_threads; }

static const char *const MSG_LENGTH = "kernel received a slice of the wrong length";
static const char *const MSG_OVERFLOW = "tensor shape product overflows usize";

/* shape_len (reference/mod.rs:82-89): checked product of dimensions. */
static int shape_len(const size_t *dims, size_t count, size_t *out, const char **why) {
    size_t product = 1;
    for (size_t i = 0; i < count; ++i) {
        if (dims[i] != 0 && product > SIZE_MAX / dims[i]) {
            *why = MSG_OVERFLOW;
            return SLR_SHAPE_OVERFLOW;
        }
        product *= dims[i];
    }
    *out = product;
    return SLR_OK;
}

#define SHAPE(dst, ...)                                                               \
    do {                                                                              \
        const size_t dims_[] = {__VA_ARGS__};                                         \
        int rc_ = shape_len(dims_, sizeof(dims_) / sizeof(dims_[0]), &(dst), why);   \
        if (rc_ != SLR_OK) return rc_;                                                \
    } while (0)

/* expect_len (reference/mod.rs:91-97). */
#define EXPECT(actual, expected)                 \
    do {                                         \
        if ((size_t)(actual) != (size_t)(expected)) { \
            *why = MSG_LENGTH;                   \
            return SLR_LENGTH_MISMATCH;          \
        }                                        \
    } while (0)

#define INVALID(reason)          \
    do {                         \
        *why = (reason);         \
        return SLR_INVALID_SHAPE; \
    } while (0)

/* dot (reference/mod.rs:104-110): sequential sum of products, left to right. */
static float dot(const float *left, const float *right, size_t n) {
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float product = left[i] * right[i];
        sum = sum + product;
    }
    return sum;
}

/* matmul_nt (reference/matmul.rs:29-59): out[b,m,n] = dot(a[b,m,:], b[b,n,:]). */
int slr_matmul_nt(const float *a, size_t a_len, const float *b, size_t b_len, float *out,
                  size_t out_len, size_t batch, size_t m, size_t k, size_t n, const char **why) {
    size_t la, lb, lo;
    SHAPE(la, batch, m, k);
    SHAPE(lb, batch, n, k);
    SHAPE(lo, batch, m, n);
    EXPECT(a_len, la);
    EXPECT(b_len, lb);
    EXPECT(out_len, lo);
    for (size_t bi = 0; bi < batch; ++bi) {
        const float *ab = a + bi * m * k;
        const float *bb = b + bi * n * k;
        float *ob = out + bi * m * n;
#pragma omp parallel for collapse(2) schedule(static) num_threads(g_threads) if (g_threads > 1 && m * n > 64)
        for (size_t row = 0; row < m; ++row)
            for (size_t col = 0; col < n; ++col)
                ob[row * n + col] = dot(ab + row * k, bb + col * k, k);
    }
    return SLR_OK;
}

/* matmul_nn (reference/matmul.rs:77-110): b is [batch, k, n]. */
int slr_matmul_nn(const float *a, size_t a_len, const float *b, size_t b_len, float *out,
                  size_t out_len, size_t batch, size_t m, size_t k, size_t n, const char **why) {
    size_t la, lb, lo;
    SHAPE(la, batch, m, k);
    SHAPE(lb, batch, k, n);
    SHAPE(lo, batch, m, n);
    EXPECT(a_len, la);
    EXPECT(b_len, lb);
    EXPECT(out_len, lo);
    for (size_t bi = 0; bi < batch; ++bi) {
        const float *ab = a + bi * m * k;
        const float *bb = b + bi * k * n;
        float *ob = out + bi * m * n;
#pragma omp parallel for collapse(2) schedule(static) num_threads(g_threads) if (g_threads > 1 && m * n > 64)
        for (size_t row = 0; row < m; ++row) {
            for (size_t col = 0; col < n; ++col) {
                float sum = 0.0f;
                for (size_t d = 0; d < k; ++d) {
                    float product = ab[row * k + d] * bb[d * n + col];
                    sum = sum + product;
                }
                ob[row * n + col] = sum;
            }
        }
    }
    return SLR_OK;
}

/* One stable softmax over row[0..count) in place (reference/softmax.rs:29-38). */
static void softmax_row(float *row, size_t count) {
    float maximum = -INFINITY;
    for (size_t i = 0; i < count; ++i) maximum = fmaxf(maximum, row[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < count; ++i) {
        row[i] = expf(row[i] - maximum);
        sum = sum + row[i];
    }
    float inverse = 1.0f / sum;
    for (size_t i = 0; i < count; ++i) row[i] = row[i] * inverse;
}

/* softmax (reference/softmax.rs:19-42), in place over [rows, cols]. */
int slr_softmax(float *x, size_t x_len, size_t rows, size_t cols, const char **why) {
    if (rows == 0 || cols == 0) INVALID("softmax requires nonzero rows and cols");
    size_t len;
    SHAPE(len, rows, cols);
    EXPECT(x_len, len);
    for (size_t r = 0; r < rows; ++r) softmax_row(x + r * cols, cols);
    return SLR_OK;
}

/* softmax_causal (reference/softmax.rs:61-114). */
int slr_softmax_causal(float *x, size_t x_len, size_t rows, size_t cols, size_t seq,
                       size_t past_len, const char **why) {
    if (rows == 0 || cols == 0) INVALID("softmax_causal requires nonzero rows and cols");
    if (seq == 0) INVALID("softmax_causal requires a nonzero seq");
    if (past_len > SIZE_MAX - seq) {
        *why = MSG_OVERFLOW;
        return SLR_SHAPE_OVERFLOW;
    }
    if (cols != past_len + seq) INVALID("softmax_causal requires cols == past_len + seq");
    if (rows % seq != 0) INVALID("softmax_causal requires rows to be a multiple of seq");
    size_t len;
    SHAPE(len, rows, cols);
    EXPECT(x_len, len);
    for (size_t r = 0; r < rows; ++r) {
        size_t last_visible = past_len + r % seq;
        float *row = x + r * cols;
        softmax_row(row, last_visible + 1);
        for (size_t c = last_visible + 1; c < cols; ++c) row[c] = 0.0f;
    }
    return SLR_OK;
}

/* rms_norm (reference/norm.rs:27-60): out = (x * inv) * w, inv computed once. */
int slr_rms_norm(const float *x, size_t x_len, const float *weight, size_t w_len, float *out,
                 size_t out_len, size_t rows, size_t hidden, float eps, const char **why) {
    if (hidden == 0) INVALID("rms_norm requires a nonzero hidden size");
    size_t len;
    SHAPE(len, rows, hidden);
    EXPECT(x_len, len);
    EXPECT(w_len, hidden);
    EXPECT(out_len, len);
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * hidden;
        float *orow = out + r * hidden;
        float ss = 0.0f;
        for (size_t i = 0; i < hidden; ++i) {
            float sq = xr[i] * xr[i];
            ss = ss + sq;
        }
        float mean_square = ss / (float)hidden;
        float inverse_rms = 1.0f / sqrtf(mean_square + eps);
        for (size_t i = 0; i < hidden; ++i) {
            float scaled = xr[i] * inverse_rms;
            orow[i] = scaled * weight[i];
        }
    }
    return SLR_OK;
}

/* validate_rope (reference/rope.rs:9-24). */
static int validate_rope(size_t x_len, size_t pos_len, size_t batch, size_t heads, size_t seq,
                         size_t head_dim, const char **why) {
    if (head_dim == 0 || head_dim % 2 != 0) INVALID("head_dim must be a positive even number");
    size_t lx, lp;
    SHAPE(lx, batch, heads, seq, head_dim);
    EXPECT(x_len, lx);
    SHAPE(lp, batch, seq);
    EXPECT(pos_len, lp);
    return SLR_OK;
}

/* rope_angle (reference/rope.rs:32-35): position / theta^(2*pair/head_dim) in f64. */
static double rope_angle(double position, size_t pair, size_t head_dim, double theta) {
    double exponent = 2.0 * (double)pair / (double)head_dim;
    return position / pow(theta, exponent);
}

/* Shared body of rope_neox (rope.rs:55-99) and rope_gptj (rope.rs:108-141);
 * `interleaved` selects the (2i, 2i+1) pairing of GPT-J. */
static int rope_apply(float *x, size_t x_len, const uint32_t *positions, size_t pos_len,
                      size_t batch, size_t heads, size_t seq, size_t head_dim, float theta_f32,
                      int interleaved, const char **why) {
    int rc = validate_rope(x_len, pos_len, batch, heads, seq, head_dim, why);
    if (rc != SLR_OK) return rc;
    size_t half = head_dim / 2;
    double theta = (double)theta_f32;
    for (size_t b = 0; b < batch; ++b) {
        for (size_t t = 0; t < seq; ++t) {
            double position = (double)positions[b * seq + t];
            for (size_t pair = 0; pair < half; ++pair) {
                double angle = rope_angle(position, pair, head_dim, theta);
                float sine = (float)sin(angle);
                float cosine = (float)cos(angle);
                size_t i0 = interleaved ? 2 * pair : pair;
                size_t i1 = interleaved ? 2 * pair + 1 : pair + half;
                for (size_t h = 0; h < heads; ++h) {
                    float *base = x + ((b * heads + h) * seq + t) * head_dim;
                    float first = base[i0];
                    float second = base[i1];
                    float fc = first * cosine, ss = second * sine;
                    float fs = first * sine, sc = second * cosine;
                    base[i0] = fc - ss;
                    base[i1] = fs + sc;
                }
            }
        }
    }
    return SLR_OK;
}

int slr_rope_neox(float *x, size_t x_len, const uint32_t *positions, size_t pos_len, size_t batch,
                  size_t heads, size_t seq, size_t head_dim, float theta, const char **why) {
    return rope_apply(x, x_len, positions, pos_len, batch, heads, seq, head_dim, theta, 0, why);
}

int slr_rope_gptj(float *x, size_t x_len, const uint32_t *positions, size_t pos_len, size_t batch,
                  size_t heads, size_t seq, size_t head_dim, float theta, const char **why) {
    return rope_apply(x, x_len, positions, pos_len, batch, heads, seq, head_dim, theta, 1, why);
}

/* silu_scalar (reference/elementwise.rs:10-12): x * (1 / (1 + exp(-x))). */
static float silu_scalar(float value) {
    float denom = 1.0f + expf(-value);
    return value * (1.0f / denom);
}

/* silu (elementwise.rs:20-25), in place. */
int slr_silu(float *x, size_t len, const char **why) {
    (void)why;
    for (size_t i = 0; i < len; ++i) x[i] = silu_scalar(x[i]);
    return SLR_OK;
}

/* mul (elementwise.rs:35-43). */
int slr_mul(const float *a, size_t a_len, const float *b, size_t b_len, float *out, size_t out_len,
            size_t len, const char **why) {
    EXPECT(a_len, len);
    EXPECT(b_len, len);
    EXPECT(out_len, len);
    for (size_t i = 0; i < len; ++i) out[i] = a[i] * b[i];
    return SLR_OK;
}

/* add (elementwise.rs:53-61). */
int slr_add(const float *a, size_t a_len, const float *b, size_t b_len, float *out, size_t out_len,
            size_t len, const char **why) {
    EXPECT(a_len, len);
    EXPECT(b_len, len);
    EXPECT(out_len, len);
    for (size_t i = 0; i < len; ++i) out[i] = a[i] + b[i];
    return SLR_OK;
}

/* scale (elementwise.rs:69-74), in place. */
int slr_scale(float *x, size_t len, float factor, const char **why) {
    (void)why;
    for (size_t i = 0; i < len; ++i) x[i] = x[i] * factor;
    return SLR_OK;
}

/* gather (reference/layout.rs:25-52): every id is checked before any write. */
int slr_gather(const float *table, size_t table_len, const uint32_t *ids, size_t ids_len, float *out,
               size_t out_len, size_t vocab, size_t hidden, size_t rows, const char **why) {
    size_t lt, lo;
    SHAPE(lt, vocab, hidden);
    EXPECT(table_len, lt);
    EXPECT(ids_len, rows);
    SHAPE(lo, rows, hidden);
    EXPECT(out_len, lo);
    for (size_t r = 0; r < rows; ++r)
        if ((size_t)ids[r] >= vocab) INVALID("id out of range");
    for (size_t r = 0; r < rows; ++r)
        memcpy(out + r * hidden, table + (size_t)ids[r] * hidden, hidden * sizeof(float));
    return SLR_OK;
}

/* last_token (reference/layout.rs:71-94): copies position seq_len-1 of every batch row. */
int slr_last_token(const float *input, size_t in_len, float *out, size_t out_len, size_t batch,
                   size_t seq, size_t hidden, size_t seq_len, const char **why) {
    if (seq_len < 1 || seq_len > seq) INVALID("last_token requires 1 <= seq_len <= seq");
    size_t li, lo;
    SHAPE(li, batch, seq, hidden);
    EXPECT(in_len, li);
    SHAPE(lo, batch, hidden);
    EXPECT(out_len, lo);
    for (size_t b = 0; b < batch; ++b)
        memcpy(out + b * hidden, input + (b * seq + seq_len - 1) * hidden, hidden * sizeof(float));
    return SLR_OK;
}

/* split_heads (layout.rs:107-136) when `split`, merge_heads (layout.rs:144-166) otherwise. */
static int heads_permute(const float *input, size_t in_len, float *out, size_t out_len, size_t batch,
                         size_t seq, size_t heads, size_t head_dim, int split, const char **why) {
    size_t total;
    SHAPE(total, batch, seq, heads, head_dim);
    EXPECT(in_len, total);
    EXPECT(out_len, total);
    for (size_t b = 0; b < batch; ++b)
        for (size_t t = 0; t < seq; ++t)
            for (size_t h = 0; h < heads; ++h) {
                size_t token_major = ((b * seq + t) * heads + h) * head_dim;
                size_t head_major = ((b * heads + h) * seq + t) * head_dim;
                if (split)
                    memcpy(out + head_major, input + token_major, head_dim * sizeof(float));
                else
                    memcpy(out + token_major, input + head_major, head_dim * sizeof(float));
            }
    return SLR_OK;
}

int slr_split_heads(const float *input, size_t in_len, float *out, size_t out_len, size_t batch,
                    size_t seq, size_t heads, size_t head_dim, const char **why) {
    return heads_permute(input, in_len, out, out_len, batch, seq, heads, head_dim, 1, why);
}

int slr_merge_heads(const float *input, size_t in_len, float *out, size_t out_len, size_t batch,
                    size_t seq, size_t heads, size_t head_dim, const char **why) {
    return heads_permute(input, in_len, out, out_len, batch, seq, heads, head_dim, 0, why);
}

/* kv_append (reference/attention.rs:33-83).
 * cache[batch, layers, 2, max_seq, kv_heads, head_dim]; k/v [batch, kv_heads, seq, head_dim]. */
int slr_kv_append(const float *k, size_t k_len, const float *v, size_t v_len, float *cache,
                  size_t cache_len, size_t batch, size_t layers, size_t layer, size_t kv_heads,
                  size_t head_dim, size_t max_seq, size_t past_len, size_t seq, const char **why) {
    size_t kv_len, c_len;
    SHAPE(kv_len, batch, kv_heads, seq, head_dim);
    SHAPE(c_len, batch, layers, 2, max_seq, kv_heads, head_dim);
    EXPECT(k_len, kv_len);
    EXPECT(v_len, kv_len);
    EXPECT(cache_len, c_len);
    if (layer >= layers) INVALID("layer out of range");
    if (past_len > SIZE_MAX - seq) {
        *why = MSG_OVERFLOW;
        return SLR_SHAPE_OVERFLOW;
    }
    if (past_len + seq > max_seq) INVALID("past_len + seq exceeds max_seq");
    size_t time_stride = kv_heads * head_dim;
    size_t parity_stride = max_seq * time_stride;
    size_t layer_stride = 2 * parity_stride;
    size_t batch_stride = layers * layer_stride;
    for (size_t b = 0; b < batch; ++b)
        for (size_t h = 0; h < kv_heads; ++h)
            for (size_t t = 0; t < seq; ++t) {
                size_t src = ((b * kv_heads + h) * seq + t) * head_dim;
                size_t dst = b * batch_stride + layer * layer_stride + (past_len + t) * time_stride +
                             h * head_dim;
                memcpy(cache + dst, k + src, head_dim * sizeof(float));
                memcpy(cache + dst + parity_stride, v + src, head_dim * sizeof(float));
            }
    return SLR_OK;
}

/* causal_attention (reference/attention.rs:129-219): kv_append, then for every
 * (b, h, t) three passes over keys 0..=past_len+t — max, denominator, weighted
 * value sum — recomputing the score in each pass exactly as the reference does. */
int slr_causal_attention(const float *q, size_t q_len, const float *k_new, size_t k_len,
                         const float *v_new, size_t v_len, float *cache, size_t cache_len, float *out,
                         size_t out_len, size_t batch, size_t layers, size_t layer, size_t heads,
                         size_t kv_heads, size_t seq, size_t past_len, size_t head_dim,
                         size_t max_seq, float scale, const char **why) {
    if (kv_heads == 0) INVALID("kv_heads must be nonzero");
    if (heads == 0) INVALID("heads must be nonzero");
    if (heads % kv_heads != 0) INVALID("heads must be a multiple of kv_heads");
    size_t ql;
    SHAPE(ql, batch, heads, seq, head_dim);
    EXPECT(q_len, ql);
    EXPECT(out_len, ql);
    int rc = slr_kv_append(k_new, k_len, v_new, v_len, cache, cache_len, batch, layers, layer,
                           kv_heads, head_dim, max_seq, past_len, seq, why);
    if (rc != SLR_OK) return rc;

    size_t group = heads / kv_heads;
    size_t time_stride = kv_heads * head_dim;
    size_t parity_stride = max_seq * time_stride;
    size_t layer_stride = 2 * parity_stride;
    size_t batch_stride = layers * layer_stride;
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(g_threads) if (g_threads > 1 && batch * heads > 1)
    for (size_t b = 0; b < batch; ++b)
        for (size_t h = 0; h < heads; ++h) {
            size_t kv_head = h / group;
            for (size_t t = 0; t < seq; ++t) {
                size_t key_count = past_len + t + 1;
                const float *query = q + ((b * heads + h) * seq + t) * head_dim;
                const float *keys = cache + b * batch_stride + layer * layer_stride + kv_head * head_dim;
                const float *values = keys + parity_stride;
                float maximum = -INFINITY;
                for (size_t j = 0; j < key_count; ++j) {
                    float score = dot(query, keys + j * time_stride, head_dim) * scale;
                    if (score > maximum) maximum = score;
                }
                float denominator = 0.0f;
                for (size_t j = 0; j < key_count; ++j) {
                    float score = dot(query, keys + j * time_stride, head_dim) * scale;
                    denominator = denominator + expf(score - maximum);
                }
                float inverse = 1.0f / denominator;
                float *orow = out + ((b * heads + h) * seq + t) * head_dim;
                for (size_t d = 0; d < head_dim; ++d) orow[d] = 0.0f;
                for (size_t j = 0; j < key_count; ++j) {
                    float score = dot(query, keys + j * time_stride, head_dim) * scale;
                    float probability = expf(score - maximum) * inverse;
                    const float *vrow = values + j * time_stride;
                    for (size_t d = 0; d < head_dim; ++d) {
                        float term = probability * vrow[d];
                        orow[d] = orow[d] + term;
                    }
                }
            }
        }
    return SLR_OK;
}

/* Decode attention over a paged KV cache (no reference counterpart: gaps
 * G-17/G-18, ARCH-0008:123-124). For each batch row b with L = seq_lens[b]
 * cached positions: kv_append of the row's new K/V at position L, then the
 * reference's causal_attention for its one query per head over positions
 * 0..L (attention.rs:129-219: max, denominator and weighted-sum passes with
 * the score recomputed each time), reading position j from slot j % page_size
 * of page block_table[b * pages_per_seq + j / page_size]. The pool is
 * [layers][num_pages][2][page_size][kv_heads][head_dim]. */
int slr_paged_attention_decode(const float *q, const float *k_new, const float *v_new, float *pool,
                               size_t pool_len, const uint32_t *block_table, const uint32_t *seq_lens, float *out,
                               size_t batch, size_t layers, size_t layer, size_t num_pages, size_t page_size,
                               size_t pages_per_seq, size_t heads, size_t kv_heads, size_t head_dim, float scale,
                               const char **why) {
    if (kv_heads == 0) INVALID("kv_heads must be nonzero");
    if (heads == 0) INVALID("heads must be nonzero");
    if (heads % kv_heads != 0) INVALID("heads must be a multiple of kv_heads");
    if (page_size == 0) INVALID("page_size must be nonzero");
    if (layer >= layers) INVALID("layer is out of range");
    size_t want;
    SHAPE(want, layers, num_pages, 2, page_size, kv_heads, head_dim);
    EXPECT(pool_len, want);
    size_t time_stride = kv_heads * head_dim;
    size_t parity_stride = page_size * time_stride;
    size_t page_stride = 2 * parity_stride;
    float *layer_base = pool + layer * num_pages * page_stride;
    for (size_t b = 0; b < batch; ++b) {
        size_t L = seq_lens[b];
        if (L / page_size >= pages_per_seq) INVALID("paged KV length exceeds the row's block table");
        for (size_t pi = 0; pi <= L / page_size; ++pi)
            if (block_table[b * pages_per_seq + pi] >= num_pages) INVALID("page id out of range");
    }
    for (size_t b = 0; b < batch; ++b) {
        uint32_t wpage = block_table[b * pages_per_seq + seq_lens[b] / page_size];
        for (size_t o = 0; o < batch; ++o) {
            if (o == b) continue;
            for (size_t pi = 0; pi <= seq_lens[o] / page_size; ++pi)
                if (block_table[o * pages_per_seq + pi] == wpage) INVALID("a row appends into a page another row reads");
        }
    }
    /* kv_append of every row first, as the reference appends before attending */
    for (size_t b = 0; b < batch; ++b) {
        size_t L = seq_lens[b];
        float *row = layer_base + block_table[b * pages_per_seq + L / page_size] * page_stride +
                     (L % page_size) * time_stride;
        for (size_t h = 0; h < kv_heads; ++h) {
            memcpy(row + h * head_dim, k_new + (b * kv_heads + h) * head_dim, head_dim * sizeof(float));
            memcpy(row + parity_stride + h * head_dim, v_new + (b * kv_heads + h) * head_dim,
                   head_dim * sizeof(float));
        }
    }
    size_t group = heads / kv_heads;
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(g_threads) if (g_threads > 1 && batch * heads > 1)
    for (size_t b = 0; b < batch; ++b)
        for (size_t h = 0; h < heads; ++h) {
            size_t kv_head = h / group;
            size_t key_count = seq_lens[b] + 1;
            const uint32_t *table = block_table + b * pages_per_seq;
            const float *query = q + (b * heads + h) * head_dim;
#define PAGED_KEY(j) (layer_base + table[(j) / page_size] * page_stride + ((j) % page_size) * time_stride + \
                      kv_head * head_dim)
            float maximum = -INFINITY;
            for (size_t j = 0; j < key_count; ++j) {
                float score = dot(query, PAGED_KEY(j), head_dim) * scale;
                if (score > maximum) maximum = score;
            }
            float denominator = 0.0f;
            for (size_t j = 0; j < key_count; ++j) {
                float score = dot(query, PAGED_KEY(j), head_dim) * scale;
                denominator = denominator + expf(score - maximum);
            }
            float inverse = 1.0f / denominator;
            float *orow = out + (b * heads + h) * head_dim;
            for (size_t d = 0; d < head_dim; ++d) orow[d] = 0.0f;
            for (size_t j = 0; j < key_count; ++j) {
                float score = dot(query, PAGED_KEY(j), head_dim) * scale;
                float probability = expf(score - maximum) * inverse;
                const float *vrow = PAGED_KEY(j) + parity_stride;
                for (size_t d = 0; d < head_dim; ++d) {
                    float term = probability * vrow[d];
                    orow[d] = orow[d] + term;
                }
            }
#undef PAGED_KEY
        }
    return SLR_OK;
}

/* swiglu (reference/swiglu.rs:40-84): per row, per intermediate index i,
 * g = silu(dot(x, Wg[i])), u = dot(x, Wu[i]), out[r, j] += (g*u) * Wd[j, i]. */
int slr_swiglu(const float *x, size_t x_len, const float *w_gate, size_t g_len, const float *w_up,
               size_t u_len, const float *w_down, size_t d_len, float *out, size_t out_len, size_t rows,
               size_t hidden, size_t inter, const char **why) {
    if (hidden == 0) INVALID("swiglu requires a nonzero hidden size");
    if (inter == 0) INVALID("swiglu requires a nonzero inter size");
    size_t lt, lw, ld;
    SHAPE(lt, rows, hidden);
    EXPECT(x_len, lt);
    SHAPE(lw, inter, hidden);
    EXPECT(g_len, lw);
    EXPECT(u_len, lw);
    SHAPE(ld, hidden, inter);
    EXPECT(d_len, ld);
    EXPECT(out_len, lt);
    /* The reference runs i outer, j inner; out[r, j] sees the same sequence
     * of additions (i ascending) with j outer, which lets the threaded
     * version give each thread whole output elements. */
    float *weights = (float *)malloc((inter ? inter : 1) * sizeof(float));
    if (weights == NULL) INVALID("swiglu could not allocate its row buffer");
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * hidden;
        float *orow = out + r * hidden;
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
        for (size_t i = 0; i < inter; ++i) {
            float gate = silu_scalar(dot(xr, w_gate + i * hidden, hidden));
            float up = dot(xr, w_up + i * hidden, hidden);
            weights[i] = gate * up;
        }
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
        for (size_t j = 0; j < hidden; ++j) {
            float acc = 0.0f;
            for (size_t i = 0; i < inter; ++i) {
                float term = weights[i] * w_down[j * inter + i];
                acc = acc + term;
            }
            orow[j] = acc;
        }
    }
    free(weights);
    return SLR_OK;
}

/* rms_norm_matmul (reference/fused.rs:41-90):
 * out[r, c] = sum_i ((x[i] * inv) * weight[i]) * w[c, i], left to right. */
int slr_rms_norm_matmul(const float *x, size_t x_len, const float *weight, size_t wt_len,
                        const float *w, size_t w_len, float *out, size_t out_len, size_t rows,
                        size_t hidden, size_t out_features, float eps, const char **why) {
    if (hidden == 0) INVALID("rms_norm_matmul requires a nonzero hidden size");
    if (out_features == 0) INVALID("rms_norm_matmul requires a nonzero out_features");
    size_t lx, lo, lw;
    SHAPE(lx, rows, hidden);
    SHAPE(lo, rows, out_features);
    EXPECT(x_len, lx);
    EXPECT(wt_len, hidden);
    SHAPE(lw, out_features, hidden);
    EXPECT(w_len, lw);
    EXPECT(out_len, lo);
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * hidden;
        float ss = 0.0f;
        for (size_t i = 0; i < hidden; ++i) {
            float sq = xr[i] * xr[i];
            ss = ss + sq;
        }
        float mean_square = ss / (float)hidden;
        float inverse_rms = 1.0f / sqrtf(mean_square + eps);
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
        for (size_t c = 0; c < out_features; ++c) {
            const float *wr = w + c * hidden;
            float sum = 0.0f;
            for (size_t i = 0; i < hidden; ++i) {
                float t0 = xr[i] * inverse_rms;
                float t1 = t0 * weight[i];
                float t2 = t1 * wr[i];
                sum = sum + t2;
            }
            out[r * out_features + c] = sum;
        }
    }
    return SLR_OK;
}

/* ------------------------------------------------------------------------- */
/* Test-support LCG (reference/mod.rs:118-148): PCG multiplier/increment,    */
/* output = state >> 33, uniform = low + (high - low) * (f32)(u / u32::MAX). */
/* ------------------------------------------------------------------------- */

uint32_t slr_lcg_next_u32(uint64_t *state) {
    *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
    return (uint32_t)(*state >> 33);
}

void slr_lcg_fill(uint64_t *state, float *values, size_t n, float low, float high) {
    for (size_t i = 0; i < n; ++i) {
        double unit = (double)slr_lcg_next_u32(state) / 4294967295.0;
        float unit32 = (float)unit;
        float span = high - low;
        float scaled = span * unit32;
        values[i] = low + scaled;
    }
}

/* Lcg::below (reference/mod.rs:142-146). */
size_t slr_lcg_below(uint64_t *state, size_t upper) {
    return (size_t)slr_lcg_next_u32(state) % upper;
}

/* ------------------------------------------------------------------------- */
/* Group-wise symmetric quantization (no reference code exists; the layout   */
/* is this project's convention and is parity-unpinned against sl-precision). */
/*   scale[n, g] = max|w[n, g*G .. g*G+G)| / qmax   (qmax 7 for INT4, 127 INT8) */
/*   q = clamp(round_half_away(w / scale), -qmax, qmax); scale 0 -> q 0       */
/*   INT8: one int8 per element, row-major.                                  */
/*   INT4: two's-complement nibbles, element k of a row in byte k/2,         */
/*         even k in the low nibble, rows padded to whole bytes.             */
/*   dequant: w' = (float)q * scale (one f32 multiply).                      */
/* ------------------------------------------------------------------------- */

static int8_t round_half_away(float v) {
    float t = truncf(v);
    float frac = v - t; /* exact for |v| < 2^23 */
    if (frac >= 0.5f) t += 1.0f;
    else if (frac <= -0.5f) t -= 1.0f;
    return (int8_t)t;
}

int slr_quantize_groupwise(const float *w, size_t n, size_t k, size_t group, int bits,
                           uint8_t *payload, float *scales, const char **why) {
    if (group == 0 || k % group != 0) INVALID("k must be a positive multiple of group_size");
    if (bits != 4 && bits != 8) {
        *why = "quantization format must be INT4 or INT8";
        return SLR_UNSUPPORTED;
    }
    int qmax = bits == 4 ? 7 : 127;
    size_t groups = k / group;
    size_t row_bytes = bits == 4 ? (k + 1) / 2 : k;
    memset(payload, 0, n * row_bytes);
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && n > 1)
    for (size_t r = 0; r < n; ++r) {
        for (size_t g = 0; g < groups; ++g) {
            const float *src = w + r * k + g * group;
            float amax = 0.0f;
            for (size_t i = 0; i < group; ++i) amax = fmaxf(amax, fabsf(src[i]));
            float s = amax / (float)qmax;
            scales[r * groups + g] = s;
            for (size_t i = 0; i < group; ++i) {
                int q = 0;
                if (s != 0.0f) {
                    q = round_half_away(src[i] / s);
                    if (q > qmax) q = qmax;
                    if (q < -qmax) q = -qmax;
                }
                size_t col = g * group + i;
                if (bits == 8) {
                    payload[r * row_bytes + col] = (uint8_t)(int8_t)q;
                } else {
                    uint8_t nib = (uint8_t)q & 0x0F;
                    payload[r * row_bytes + col / 2] |= (uint8_t)(col % 2 ? nib << 4 : nib);
                }
            }
        }
    }
    return SLR_OK;
}

/* Unpacks the integer codes to int8 (bit-exact check of the packing). */
int slr_unpack_codes(const uint8_t *payload, size_t n, size_t k, int bits, int8_t *codes,
                     const char **why) {
    if (bits != 4 && bits != 8) {
        *why = "quantization format must be INT4 or INT8";
        return SLR_UNSUPPORTED;
    }
    size_t row_bytes = bits == 4 ? (k + 1) / 2 : k;
    for (size_t r = 0; r < n; ++r)
        for (size_t c = 0; c < k; ++c) {
            if (bits == 8) {
                codes[r * k + c] = (int8_t)payload[r * row_bytes + c];
            } else {
                uint8_t byte = payload[r * row_bytes + c / 2];
                int nib = c % 2 ? byte >> 4 : byte & 0x0F;
                codes[r * k + c] = (int8_t)(nib >= 8 ? nib - 16 : nib);
            }
        }
    return SLR_OK;
}

/* dequant(q, s): w' = (float)q * scale[n, k / group]. */
int slr_dequantize_groupwise(const uint8_t *payload, const float *scales, size_t n, size_t k,
                             size_t group, int bits, float *out, const char **why) {
    if (group == 0 || k % group != 0) INVALID("k must be a positive multiple of group_size");
    if (bits != 4 && bits != 8) {
        *why = "quantization format must be INT4 or INT8";
        return SLR_UNSUPPORTED;
    }
    size_t groups = k / group;
    size_t row_bytes = bits == 4 ? (k + 1) / 2 : k;
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && n > 1)
    for (size_t r = 0; r < n; ++r)
        for (size_t c = 0; c < k; ++c) {
            int q;
            if (bits == 8) {
                q = (int8_t)payload[r * row_bytes + c];
            } else {
                uint8_t byte = payload[r * row_bytes + c / 2];
                int nib = c % 2 ? byte >> 4 : byte & 0x0F;
                q = nib >= 8 ? nib - 16 : nib;
            }
            out[r * k + c] = (float)q * scales[r * groups + c / group];
        }
    return SLR_OK;
}
