/*
 * mimir_oracle.c -- CPU restatement of Mimir's fused elementwise / row-reduction
 * layer path.  TEST INFRASTRUCTURE ONLY (the checker for the HIP kernels and the
 * "port" CPU baseline); never part of the product library.
 *
 * Each function restates the reference's scalar algorithm in plain C with the
 * same float32 intermediates and the same glibc libm calls.  Citations are to
 * brit45/mimir-framework.  Single-threaded, like the reference ops.
 */
#include "mimir_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_EINVAL 1

/* LayerOps.hpp:264-319.  The reference's two sums carry `#pragma omp simd
 * reduction(+:...)` (:290, :297), which lets the compiler split them into
 * vector-lane partial sums; they are taken here in index order.  The two agree
 * within the path's tolerance at the row widths the tests pin against
 * oracle/_ref (tests/test_oracle_vs_reference.py, up to 3000 per group); over
 * whole-vector rows of millions of floats neither is near the float64 value
 * (2^25 normal floats: the reference 1e-2 off, index order 0.2), and the HIP
 * path is held to the reference's compiled output and to the float64 value
 * instead. */
int oracle_layernorm(const float* x, int64_t N, int64_t in_features,
                     const float* gamma, const float* beta, float eps, float* y) {
    /* LayerOps.hpp:276-280: normalized = in_features > 0 ? in_features : N,
     * throw unless normalized > 0 and N % normalized == 0. */
    const int64_t n = in_features > 0 ? in_features : N;
    if (n <= 0 || N < 0 || (N % n) != 0) return ORACLE_EINVAL;
    /* The reference only adds the bias inside `if (weights)` (:310-313): a bias
     * without a scale is not expressible there. */
    if (beta && !gamma) return ORACLE_EINVAL;
    const int64_t groups = N / n;
    for (int64_t g = 0; g < groups; ++g) {
        const float* xr = x + g * n;
        float* yr = y + g * n;
        float mean = 0.0f; /* :291-295 */
        for (int64_t i = 0; i < n; ++i) mean += xr[i];
        mean /= (float)n;
        float var = 0.0f; /* :297-303, two-pass variance */
        for (int64_t i = 0; i < n; ++i) {
            const float d = xr[i] - mean;
            var += d * d;
        }
        var /= (float)n;
        const float inv_std = 1.0f / sqrtf(var + eps); /* :305 */
        for (int64_t i = 0; i < n; ++i) {           /* :307-315 */
            float v = (xr[i] - mean) * inv_std;
            if (gamma) {
                v *= gamma[i];
                if (beta) v += beta[i];
            }
            yr[i] = v;
        }
    }
    return ORACLE_OK;
}

/* LayerOpsExt.hpp:345-378 (one group over the whole input). */
int oracle_rmsnorm_whole(const float* x, int64_t N, const float* w, int64_t w_len,
                         float eps, float* y) {
    if (N < 0 || w_len < 0) return ORACLE_EINVAL;
    float rms_sq = 0.0f; /* :357-361 */
    for (int64_t i = 0; i < N; ++i) rms_sq += x[i] * x[i];
    rms_sq /= (float)N;
    const float rms = sqrtf(rms_sq + eps);
    const int64_t wn = w ? w_len : 0; /* :364-366 */
    for (int64_t i = 0; i < N; ++i) { /* :368-375 */
        float v = x[i] / rms;
        if (wn && i < wn) v *= w[i];
        y[i] = v;
    }
    return ORACLE_OK;
}

/* Layers.hpp:1003-1021 (per-row twin). */
int oracle_rmsnorm_rows(const float* x, int64_t rows, int64_t cols,
                        const float* gamma, float eps, float* y) {
    if (rows < 0 || cols <= 0) return ORACLE_EINVAL;
    for (int64_t g = 0; g < rows; ++g) {
        const float* xr = x + g * cols;
        float* yr = y + g * cols;
        float rms = 0.0f; /* :1009-1013 */
        for (int64_t i = 0; i < cols; ++i) {
            const float v = xr[i];
            rms += v * v;
        }
        rms = sqrtf(rms / (float)cols + eps); /* :1014 */
        for (int64_t i = 0; i < cols; ++i) {   /* :1016-1019 */
            float v = xr[i] / rms;
            if (gamma) v *= gamma[i];
            yr[i] = v;
        }
    }
    return ORACLE_OK;
}

int oracle_add_rmsnorm(const float* x, const float* residual, int64_t rows,
                       int64_t cols, const float* gamma, float eps,
                       float* residual_out, float* y) {
    if (rows < 0 || cols <= 0) return ORACLE_EINVAL;
    const int64_t n = rows * cols;
    /* add_forward equal-size branch, LayerOps.hpp:154-169: one rounding per element */
    for (int64_t i = 0; i < n; ++i) residual_out[i] = x[i] + residual[i];
    return oracle_rmsnorm_rows(residual_out, rows, cols, gamma, eps, y);
}

/* LayerOps.hpp:142-199 */
int oracle_add(const float* a, int64_t na, const float* b, int64_t nb, float* y) {
    if (na <= 0 || nb <= 0) return ORACLE_EINVAL; /* :150-152 */
    if (na == nb) {                                /* :154-169 */
        for (int64_t i = 0; i < na; ++i) y[i] = a[i] + b[i];
        return ORACLE_OK;
    }
    const float* big = a;
    const float* small = b;
    int64_t big_n = na, small_n = nb;
    if (nb > na) { /* :172-177 */
        big = b; small = a; big_n = nb; small_n = na;
    }
    if (small_n == 1) { /* :181-188 */
        const float s = small[0];
        for (int64_t i = 0; i < big_n; ++i) y[i] = big[i] + s;
        return ORACLE_OK;
    }
    if (big_n % small_n != 0) return ORACLE_EINVAL; /* :190-192 */
    for (int64_t i = 0; i < big_n; ++i) y[i] = big[i] + small[i % small_n]; /* :194-197 */
    return ORACLE_OK;
}

/* LayerOps.hpp:205-230 */
int oracle_mul(const float* a, int64_t na, const float* b, int64_t nb, float* y) {
    if (na != nb || na < 0) return ORACLE_EINVAL; /* :209-211 */
    for (int64_t i = 0; i < na; ++i) y[i] = a[i] * b[i];
    return ORACLE_OK;
}

/* std::max(m, v) returns m unless m < v (so a NaN already held in m stays). */
static inline float ref_max(float m, float v) { return (m < v) ? v : m; }

int oracle_softmax_rows(const float* x, int64_t rows, int64_t cols, int mode, float* y) {
    if (rows < 0 || cols <= 0) return ORACLE_EINVAL;
    if (mode != ORACLE_SOFTMAX_DIV_EPS && mode != ORACLE_SOFTMAX_MUL_INV &&
        mode != ORACLE_SOFTMAX_LOG)
        return ORACLE_EINVAL;
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        float* yr = y + r * cols;
        float m = xr[0]; /* LayerOps.hpp:957-960 / std::max_element at :331 */
        for (int64_t j = 1; j < cols; ++j) m = ref_max(m, xr[j]);
        float sum = 0.0f; /* :963-967 / :334-339 */
        for (int64_t j = 0; j < cols; ++j) {
            const float e = expf(xr[j] - m);
            yr[j] = e;
            sum += e;
        }
        if (mode == ORACLE_SOFTMAX_DIV_EPS) { /* :970-972 */
            for (int64_t j = 0; j < cols; ++j) yr[j] /= (sum + 1e-9f);
        } else if (mode == ORACLE_SOFTMAX_MUL_INV) { /* :342, :355-358 */
            const float inv_sum = 1.0f / sum;
            for (int64_t j = 0; j < cols; ++j) yr[j] *= inv_sum;
        } else { /* LogSoftmax, :345-353 */
            const float log_denom = logf(sum);
            for (int64_t j = 0; j < cols; ++j) yr[j] = (xr[j] - m) - log_denom;
        }
    }
    return ORACLE_OK;
}

/* LayerOps.hpp:556-568 */
static inline float gelu1(float x) {
    const float k = sqrtf(2.0f / 3.14159265359f);
    const float cdf = 0.5f * (1.0f + tanhf(k * (x + 0.044715f * x * x * x)));
    return x * cdf;
}

/* LayerOps.hpp:570-581 */
static inline float silu1(float x) {
    const float sigmoid = 1.0f / (1.0f + expf(-x));
    return x * sigmoid;
}

void oracle_gelu(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = gelu1(x[i]);
}

void oracle_silu(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = silu1(x[i]);
}

void oracle_silu_mul(const float* gate, const float* up, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = silu1(gate[i]) * up[i];
}

void oracle_gelu_mul(const float* gate, const float* up, int64_t n, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = gelu1(gate[i]) * up[i];
}

/* Shared body of the two inline gathers (Model.cpp:1176-1203, 5307-5330). */
static int embed_check(int64_t n_ids, int64_t table_len, int32_t* vocab, int32_t* dim) {
    if (n_ids < 0) return ORACLE_EINVAL;
    if (*vocab < 1) *vocab = 1; /* Model.cpp:1176-1177: std::max(1, ...) */
    if (*dim < 1) *dim = 1;
    if (table_len < (int64_t)(*vocab) * (int64_t)(*dim)) return ORACLE_EINVAL; /* :1181-1182 */
    return ORACLE_OK;
}

static void embed_row(int32_t id, int64_t t, const float* table, int32_t vocab,
                      int32_t dim, int32_t pad, float* y) {
    float* out = y + t * (int64_t)dim;
    memset(out, 0, (size_t)dim * sizeof(float)); /* out.assign(outN, 0.0f), :1190 */
    if (pad >= 0 && id == pad) return;           /* :1196 */
    if (id < 0 || id >= vocab) return;           /* :1197, silent */
    const float* w = table + (int64_t)id * (int64_t)dim;
    for (int32_t d = 0; d < dim; ++d) out[d] = w[d]; /* :1200-1202 */
}

int oracle_embedding_i32(const int32_t* ids, int64_t n_ids, const float* table,
                         int64_t table_len, int32_t vocab, int32_t dim,
                         int32_t padding_idx, float* y) {
    if (embed_check(n_ids, table_len, &vocab, &dim)) return ORACLE_EINVAL;
    for (int64_t t = 0; t < n_ids; ++t) embed_row(ids[t], t, table, vocab, dim, padding_idx, y);
    return ORACLE_OK;
}

int oracle_embedding_f32(const float* ids, int64_t n_ids, const float* table,
                         int64_t table_len, int32_t vocab, int32_t dim,
                         int32_t padding_idx, float* y) {
    if (embed_check(n_ids, table_len, &vocab, &dim)) return ORACLE_EINVAL;
    for (int64_t t = 0; t < n_ids; ++t) {
        /* Model.cpp:5321: static_cast<int>(std::llround(static_cast<double>(x[t]))) */
        const int32_t id = (int32_t)llround((double)ids[t]);
        embed_row(id, t, table, vocab, dim, padding_idx, y);
    }
    return ORACLE_OK;
}

int oracle_rope_table(int64_t rows, int64_t head_dim, double theta,
                      float* cos_tab, float* sin_tab) {
    if (rows < 0 || head_dim <= 0 || (head_dim & 1) || !(theta > 0.0)) return ORACLE_EINVAL;
    const int64_t half = head_dim / 2;
    for (int64_t p = 0; p < rows; ++p) {
        for (int64_t i = 0; i < half; ++i) {
            const double inv_freq = 1.0 / pow(theta, (double)(2 * i) / (double)head_dim);
            const double a = (double)p * inv_freq;
            cos_tab[p * half + i] = (float)cos(a);
            sin_tab[p * half + i] = (float)sin(a);
        }
    }
    return ORACLE_OK;
}

int oracle_rope(const float* x, float* y, int64_t B, int64_t S, int64_t H,
                int64_t D, int64_t pos_offset, const float* cos_tab,
                const float* sin_tab, int64_t table_rows) {
    if (B < 0 || S < 0 || H < 0 || D <= 0 || (D & 1) || pos_offset < 0) return ORACLE_EINVAL;
    if (S > 0 && pos_offset + S > table_rows) return ORACLE_EINVAL;
    const int64_t half = D / 2;
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t s = 0; s < S; ++s) {
            const float* c = cos_tab + (pos_offset + s) * half;
            const float* sn = sin_tab + (pos_offset + s) * half;
            for (int64_t h = 0; h < H; ++h) {
                const int64_t base = ((b * S + s) * H + h) * D;
                for (int64_t i = 0; i < half; ++i) {
                    const float x0 = x[base + i];
                    const float x1 = x[base + half + i];
                    y[base + i] = x0 * c[i] - x1 * sn[i];
                    y[base + half + i] = x1 * c[i] + x0 * sn[i];
                }
            }
        }
    }
    return ORACLE_OK;
}

/* ------------------------------------------------------------------------
 * Backward of the same ops: the branches of Model::backwardPass
 * (Model.cpp:7305-9153) for the path's layer types.
 * ------------------------------------------------------------------------ */

/* accumulate_grad, Model.cpp:7329-7341: dst += src (dst already holds a
 * gradient; the "dst empty -> copy" case is a plain copy). */
void oracle_accumulate(float* dst, const float* src, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] += src[i];
}

/* LayerNorm branch, Model.cpp:7719-7821. */
int oracle_layernorm_bwd(const float* x, const float* dy, int64_t N, int64_t in_features,
                         const float* gamma, int has_bias, float eps, float* dx,
                         float* grad_params) {
    const int64_t feat = in_features > 0 ? in_features : N; /* :7730 */
    if (feat <= 0 || N <= 0 || (N % feat) != 0) return ORACLE_EINVAL; /* :7732-7737 */
    const int64_t tokens = N / feat;
    const int affine = gamma != NULL;
    float* dgamma = NULL;
    float* dbeta = NULL;
    if (affine) { /* :7757-7758, zero-initialised, added to grad_weights at :7809-7819 */
        dgamma = (float*)calloc((size_t)feat, sizeof(float));
        dbeta = (float*)calloc((size_t)feat, sizeof(float));
        if (!dgamma || !dbeta) {
            free(dgamma);
            free(dbeta);
            return ORACLE_EINVAL;
        }
    }
    for (int64_t t = 0; t < tokens; ++t) {
        const float* xr = x + t * feat;
        const float* g = dy + t * feat;
        float* d = dx + t * feat;
        float mean = 0.0f; /* :7765-7768 */
        for (int64_t i = 0; i < feat; ++i) mean += xr[i];
        mean /= (float)feat;
        float var = 0.0f; /* :7770-7776 */
        for (int64_t i = 0; i < feat; ++i) {
            const float dd = xr[i] - mean;
            var += dd * dd;
        }
        var /= (float)feat;
        const float inv_std = 1.0f / sqrtf(var + eps); /* :7777 */
        float sum_dxhat = 0.0f, sum_dxhat_xhat = 0.0f;
        for (int64_t i = 0; i < feat; ++i) { /* :7783-7797 */
            const float xhat = (xr[i] - mean) * inv_std;
            const float gm = gamma ? gamma[i] : 1.0f;
            const float dxhat = g[i] * gm;
            if (affine) {
                dgamma[i] += g[i] * xhat;
                if (has_bias) dbeta[i] += g[i];
            }
            sum_dxhat += dxhat;
            sum_dxhat_xhat += dxhat * xhat;
        }
        const float invF = 1.0f / (float)feat; /* :7799-7805 */
        for (int64_t i = 0; i < feat; ++i) {
            const float xhat = (xr[i] - mean) * inv_std;
            const float gm = gamma ? gamma[i] : 1.0f;
            const float dxhat = g[i] * gm;
            d[i] = inv_std * invF * ((float)feat * dxhat - sum_dxhat - xhat * sum_dxhat_xhat);
        }
    }
    if (affine && grad_params) { /* :7809-7819 */
        for (int64_t i = 0; i < feat; ++i) grad_params[i] += dgamma[i];
        if (has_bias)
            for (int64_t i = 0; i < feat; ++i) grad_params[feat + i] += dbeta[i];
    }
    free(dgamma);
    free(dbeta);
    return ORACLE_OK;
}

/* GELU branch, Model.cpp:9026-9051 (tanh approximation). */
void oracle_gelu_bwd(const float* x, const float* dy, int64_t n, float* dx) {
    for (int64_t i = 0; i < n; ++i) {
        const float xv = x[i];
        const float c = 0.044715f;
        const float s = sqrtf(2.0f / 3.14159265359f);
        const float u = s * (xv + c * xv * xv * xv);
        const float t = tanhf(u);
        const float sech2 = 1.0f - t * t;
        const float du_dx = s * (1.0f + 3.0f * c * xv * xv);
        const float dgelu = 0.5f * (1.0f + t) + 0.5f * xv * sech2 * du_dx;
        dx[i] = dy[i] * dgelu;
    }
}

/* SiLU branch, Model.cpp:7993-8032. */
void oracle_silu_bwd(const float* x, const float* dy, int64_t n, float* dx) {
    for (int64_t i = 0; i < n; ++i) {
        const float xv = x[i];
        const float s = 1.0f / (1.0f + expf(-xv));
        const float ds = s * (1.0f - s);
        const float dy_dx = s + xv * ds;
        dx[i] = dy[i] * dy_dx;
    }
}

/* Multiply branch, Model.cpp:7647-7665: da = dy*b, db = dy*a. */
void oracle_mul_bwd(const float* a, const float* b, const float* dy, int64_t n, float* da,
                    float* db) {
    for (int64_t i = 0; i < n; ++i) {
        da[i] = dy[i] * b[i];
        db[i] = dy[i] * a[i];
    }
}

/* Add branch, Model.cpp:7541-7601: the gradient of the broadcast (smaller)
 * operand, a sum over the big operand's gradient (scalar: all of it; repeat:
 * per position j over the tiles).  The big operand's gradient is dy itself. */
int oracle_add_bwd_small(const float* dy, int64_t n_big, int64_t n_small, float* d_small) {
    if (n_small <= 0 || n_big <= 0) return ORACLE_EINVAL;
    if (n_small == 1) { /* :7581-7585 */
        float sum = 0.0f;
        for (int64_t i = 0; i < n_big; ++i) sum += dy[i];
        d_small[0] = sum;
        return ORACLE_OK;
    }
    if (n_big % n_small != 0) return ORACLE_EINVAL; /* :7595-7599 */
    for (int64_t j = 0; j < n_small; ++j) d_small[j] = 0.0f; /* :7586-7594 */
    for (int64_t t = 0; t < n_big / n_small; ++t)
        for (int64_t j = 0; j < n_small; ++j) d_small[j] += dy[t * n_small + j];
    return ORACLE_OK;
}

/* Embedding branch, Model.cpp:7429-7461: grad_table[id*dim + d] +=
 * dy[t*dim + d] in token order; padding and out-of-range ids are skipped. */
static int embed_bwd_check(int64_t n_ids, int64_t table_len, int32_t* vocab, int32_t* dim) {
    if (n_ids < 0) return ORACLE_EINVAL;
    if (*vocab < 1) *vocab = 1; /* :7434-7435 */
    if (*dim < 1) *dim = 1;
    if (table_len < (int64_t)(*vocab) * (int64_t)(*dim)) return ORACLE_EINVAL; /* :7443-7447 */
    return ORACLE_OK;
}

static void embed_bwd_row(int32_t id, int64_t t, const float* dy, float* grad_table,
                          int32_t vocab, int32_t dim, int32_t pad) {
    if (pad >= 0 && id == pad) return; /* :7454 */
    if (id < 0 || id >= vocab) return; /* :7455 */
    float* gw = grad_table + (int64_t)id * dim;
    const float* g = dy + t * (int64_t)dim;
    for (int32_t d = 0; d < dim; ++d) gw[d] += g[d]; /* :7456-7460 */
}

int oracle_embedding_bwd_i32(const int32_t* ids, int64_t n_ids, const float* dy,
                             float* grad_table, int64_t table_len, int32_t vocab, int32_t dim,
                             int32_t padding_idx) {
    if (embed_bwd_check(n_ids, table_len, &vocab, &dim)) return ORACLE_EINVAL;
    for (int64_t t = 0; t < n_ids; ++t) embed_bwd_row(ids[t], t, dy, grad_table, vocab, dim, padding_idx);
    return ORACLE_OK;
}

int oracle_embedding_bwd_f32(const float* ids, int64_t n_ids, const float* dy, float* grad_table,
                             int64_t table_len, int32_t vocab, int32_t dim, int32_t padding_idx) {
    if (embed_bwd_check(n_ids, table_len, &vocab, &dim)) return ORACLE_EINVAL;
    for (int64_t t = 0; t < n_ids; ++t) {
        const int32_t id = (int32_t)llround((double)ids[t]); /* :7453 */
        embed_bwd_row(id, t, dy, grad_table, vocab, dim, padding_idx);
    }
    return ORACLE_OK;
}

/* The attention core of LayerOps::self_attention_forward, LayerOps.hpp:1045-1089
 * (between the QKV projection and the output projection; the same core is
 * cross_attention_forward's, :1163-1209, with kv_len keys) for `batch`
 * independent sequences.  Query i of sequence b reads its Q row at
 * (b*q_len + i)*ld_q and writes its output row at (b*q_len + i)*ld_out; key j
 * reads K and V rows at (b*kv_len + j)*ld_kv.  Head h owns columns
 * [h*head_dim, (h+1)*head_dim).  Per head and query i:
 *   s_j = (sum_k Q[i][k] K[j][k]) * scale      (k in index order, :1059-1065)
 *   masked (causal, j > i): s_j = -1e9, not taken into the max (:1054-1057)
 *   max starts at -1e30 (:1052); e_j = expf(s_j - max); sum in j order (:1069-1075)
 *   p_j = e_j * (1 / (sum + 1e-9f)) (:1076-1079)
 *   out[i][k] = sum_j p_j V[j][k], j in index order (:1081-1088).
 * The reference as compiled (g++ -O3 -mfma; C++ keeps GCC's default
 * -ffp-contract=fast) fuses the weighted-sum step acc += p*V into one fused
 * multiply-add and keeps the score dot product as a multiply then an add;
 * fmaf in the PV loop restates that, and the two agree bit for bit on the
 * tests' shapes (tests/test_oracle_attention.py). */
int oracle_attention(const float* q, int64_t ld_q, const float* k, const float* v, int64_t ld_kv,
                     float* out, int64_t ld_out, int64_t batch, int64_t q_len, int64_t kv_len,
                     int64_t heads, int64_t head_dim, float scale, int causal) {
    const int64_t width = heads * head_dim;
    if (batch < 0 || q_len < 0 || kv_len < 0 || heads <= 0 || head_dim <= 0 || ld_q < width ||
        ld_kv < width || ld_out < width)
        return ORACLE_EINVAL;
    if (batch == 0 || q_len == 0) return ORACLE_OK;
    float* row = (float*)malloc((size_t)(kv_len > 0 ? kv_len : 1) * sizeof(float));
    if (!row) return ORACLE_EINVAL;
    for (int64_t b = 0; b < batch; ++b) {
        const float* qb = q + b * q_len * ld_q;
        const float* kb = k + b * kv_len * ld_kv;
        const float* vb = v + b * kv_len * ld_kv;
        float* ob = out + b * q_len * ld_out;
        for (int64_t h = 0; h < heads; ++h) {
            const int64_t off = h * head_dim;
            for (int64_t i = 0; i < q_len; ++i) {
                const float* qi = qb + i * ld_q + off;
                float max_val = -1e30f;
                for (int64_t j = 0; j < kv_len; ++j) {
                    if (causal && j > i) {
                        row[j] = -1e9f;
                        continue;
                    }
                    const float* kj = kb + j * ld_kv + off;
                    float dot = 0.0f;
                    for (int64_t d = 0; d < head_dim; ++d) dot += qi[d] * kj[d];
                    const float s = dot * scale;
                    row[j] = s;
                    if (s > max_val) max_val = s;
                }
                float sum = 0.0f;
                for (int64_t j = 0; j < kv_len; ++j) {
                    const float e = expf(row[j] - max_val);
                    row[j] = e;
                    sum += e;
                }
                const float inv_sum = 1.0f / (sum + 1e-9f);
                for (int64_t j = 0; j < kv_len; ++j) row[j] *= inv_sum;
                float* oi = ob + i * ld_out + off;
                for (int64_t d = 0; d < head_dim; ++d) {
                    float acc = 0.0f;
                    for (int64_t j = 0; j < kv_len; ++j) acc = fmaf(row[j], vb[j * ld_kv + off + d], acc);
                    oi[d] = acc;
                }
            }
        }
    }
    free(row);
    return ORACLE_OK;
}

/* The per-head core of backward_self_attention (Model.cpp:6892-7028) and
 * backward_cross_attention (:7122-7246), over `batch` sequences laid out as
 * for oracle_attention; dout is the gradient of the attended heads (the
 * reference's dAtt).  Per head, in the reference's loop order:
 *   P[i][j]: s = (sum_k q_ik k_jk) * scale, masked (causal, j > i) -1e9;
 *            max from -1e30 over every j; e = expf(s - max), sum in j order;
 *            p = e * (1 / (sum + 1e-9f))                       (:6892-6920)
 *   dv[j][k] = 0 + sum_i P[i][j] dout[i][k]  (i in order)       (:6967-6977)
 *   dP[i][j] = sum_k dout[i][k] v[j][k]                         (:6979-6989)
 *   dot_i = sum_j dP[i][j] P[i][j] (softmax_row_dot, :6841-6845)
 *   dS[i][j] = masked ? 0 : (dP[i][j] - dot_i) * P[i][j]        (:6991-7005)
 *   dq[i][k] = 0 + (sum_j dS[i][j] k[j][k]) * scale              (:7007-7016)
 *   dk[j][k] = 0 + (sum_i dS[i][j] q[i][k]) * scale              (:7018-7028)
 * dq rows stride ld_dq, dk / dv rows stride ld_dkv.
 * The reference's runtime as compiled (g++ -O2 -mfma, C++'s default
 * -ffp-contract=fast) fuses every one of these multiply-accumulate loops --
 * the score dot as well, unlike the -O3 build of LayerOps' forward -- into
 * fused multiply-adds; fmaf restates that.  Of the 64 fused / unfused
 * combinations only this one matches Model::backwardPass bit for bit
 * (tests/test_oracle_attention_bwd.py). */
int oracle_attention_bwd(const float* q, int64_t ld_q, const float* k, const float* v, int64_t ld_kv,
                         const float* dout, int64_t ld_dout, float* dq, int64_t ld_dq, float* dk, float* dv,
                         int64_t ld_dkv, int64_t batch, int64_t q_len, int64_t kv_len, int64_t heads,
                         int64_t head_dim, float scale, int causal) {
    const int64_t width = heads * head_dim;
    if (batch < 0 || q_len < 0 || kv_len < 0 || heads <= 0 || head_dim <= 0 || ld_q < width ||
        ld_kv < width || ld_dout < width || ld_dq < width || ld_dkv < width)
        return ORACLE_EINVAL;
    if (batch == 0 || q_len == 0) return ORACLE_OK;
    const size_t tt = (size_t)q_len * (size_t)(kv_len > 0 ? kv_len : 1);
    float* P = (float*)malloc(tt * sizeof(float));
    float* dP = (float*)malloc(tt * sizeof(float));
    float* dS = (float*)malloc(tt * sizeof(float));
    if (!P || !dP || !dS) {
        free(P);
        free(dP);
        free(dS);
        return ORACLE_EINVAL;
    }
    for (int64_t b = 0; b < batch; ++b) {
        const float* qb = q + b * q_len * ld_q;
        const float* kb = k + b * kv_len * ld_kv;
        const float* vb = v + b * kv_len * ld_kv;
        const float* ob = dout + b * q_len * ld_dout;
        float* dqb = dq + b * q_len * ld_dq;
        float* dkb = dk + b * kv_len * ld_dkv;
        float* dvb = dv + b * kv_len * ld_dkv;
        for (int64_t h = 0; h < heads; ++h) {
            const int64_t off = h * head_dim;
            for (int64_t i = 0; i < q_len; ++i) {
                float* pr = P + i * kv_len;
                float maxv = -1e30f;
                for (int64_t j = 0; j < kv_len; ++j) {
                    float s = -1e9f;
                    if (!(causal && j > i)) {
                        float dot = 0.0f;
                        for (int64_t d = 0; d < head_dim; ++d)
                            dot = fmaf(qb[i * ld_q + off + d], kb[j * ld_kv + off + d], dot);
                        s = dot * scale;
                    }
                    pr[j] = s;
                    if (s > maxv) maxv = s;
                }
                float sum = 0.0f;
                for (int64_t j = 0; j < kv_len; ++j) {
                    const float e = expf(pr[j] - maxv);
                    pr[j] = e;
                    sum += e;
                }
                const float inv = 1.0f / (sum + 1e-9f);
                for (int64_t j = 0; j < kv_len; ++j) pr[j] *= inv;
            }
            for (int64_t j = 0; j < kv_len; ++j)
                for (int64_t d = 0; d < head_dim; ++d) {
                    float sum = 0.0f;
                    for (int64_t i = 0; i < q_len; ++i)
                        sum = fmaf(P[i * kv_len + j], ob[i * ld_dout + off + d], sum);
                    dvb[j * ld_dkv + off + d] = 0.0f + sum;
                }
            for (int64_t i = 0; i < q_len; ++i)
                for (int64_t j = 0; j < kv_len; ++j) {
                    float sum = 0.0f;
                    for (int64_t d = 0; d < head_dim; ++d)
                        sum = fmaf(ob[i * ld_dout + off + d], vb[j * ld_kv + off + d], sum);
                    dP[i * kv_len + j] = sum;
                }
            for (int64_t i = 0; i < q_len; ++i) {
                const float* pr = P + i * kv_len;
                const float* dpr = dP + i * kv_len;
                float dot = 0.0f;
                for (int64_t j = 0; j < kv_len; ++j) dot = fmaf(dpr[j], pr[j], dot);
                for (int64_t j = 0; j < kv_len; ++j)
                    dS[i * kv_len + j] = (causal && j > i) ? 0.0f : (dpr[j] - dot) * pr[j];
            }
            for (int64_t i = 0; i < q_len; ++i)
                for (int64_t d = 0; d < head_dim; ++d) {
                    float sum = 0.0f;
                    for (int64_t j = 0; j < kv_len; ++j)
                        sum = fmaf(dS[i * kv_len + j], kb[j * ld_kv + off + d], sum);
                    dqb[i * ld_dq + off + d] = 0.0f + sum * scale;
                }
            for (int64_t j = 0; j < kv_len; ++j)
                for (int64_t d = 0; d < head_dim; ++d) {
                    float sum = 0.0f;
                    for (int64_t i = 0; i < q_len; ++i)
                        sum = fmaf(dS[i * kv_len + j], qb[i * ld_q + off + d], sum);
                    dkb[j * ld_dkv + off + d] = 0.0f + sum * scale;
                }
        }
    }
    free(P);
    free(dP);
    free(dS);
    return ORACLE_OK;
}
