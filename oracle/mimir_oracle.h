/*
 * mimir_oracle.h -- CPU restatement of Mimir's fused elementwise / row-reduction
 * layer path.  TEST INFRASTRUCTURE ONLY: this library is the checker that the
 * HIP kernels are compared against (tests/, __graft_entry__.smoke(), and the
 * cpu_baseline leg of bench.py).  It is never linked into, loaded by or called
 * from the product library (libmimir_hip.so).
 *
 * Every function follows the reference's scalar algorithm step by step
 * (same operation order, same float32 intermediates, glibc libm for exp/tanh/
 * sqrt), single-threaded like the reference (none of these reference ops uses
 * an `omp parallel` region).  Reference citations are relative to
 * brit45/mimir-framework's tree.
 *
 * Status codes: 0 = ok, 1 = invalid argument (the cases where the reference
 * throws std::runtime_error).
 *
 * Pinning (how each function is checked, see tests/):
 *   oracle_layernorm        reference KAT + compiled reference + closed form
 *   oracle_rmsnorm_*        reference KAT + compiled reference + closed form
 *   oracle_add / _mul       reference KATs + compiled reference (bit-exact)
 *   oracle_softmax_*        reference KAT + compiled reference + invariants
 *   oracle_gelu / _silu     reference KATs + compiled reference + float64 form
 *   oracle_embedding_*      reference KATs + brute-force gather (bit-exact)
 *   oracle_rope*            no reference implementation exists; pinned by the
 *                           float64 closed form of rotary embedding (Su et al.
 *                           2021, "RoFormer") and its invariants.
 *   oracle_*_bwd            the reference's own Model::backwardPass, compiled
 *                           in place (oracle/_ref), on graphs of these layers;
 *                           float64 derivatives of the forward closed forms;
 *                           brute-force scatter-add for the embedding.
 *   oracle_attention        the reference's LayerOps::self_attention_forward,
 *                           compiled in place, with one-hot inputs and an
 *                           identity output projection (bit-exact); float64
 *                           softmax attention; closed-form special cases.
 */
#ifndef MIMIR_ORACLE_H
#define MIMIR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* LayerOps::layernorm_forward, LayerOps.hpp:264-319.
 * n = group size (layer.in_features, or N when in_features <= 0).
 * gamma may be NULL (affine == false); beta may be NULL (use_bias == false). */
int oracle_layernorm(const float* x, int64_t N, int64_t in_features,
                     const float* gamma, const float* beta, float eps, float* y);

/* LayerOpsExt::rms_norm_forward, LayerOpsExt.hpp:345-378: ONE group over all
 * N elements; the weight multiplies element i only when i < w_len. */
int oracle_rmsnorm_whole(const float* x, int64_t N, const float* w, int64_t w_len,
                         float eps, float* y);

/* Normalization::rms_norm, Layers.hpp:1003-1021: per-row form.  gamma has
 * `cols` entries (NULL -> no scale, i.e. gamma == 1 without the multiply). */
int oracle_rmsnorm_rows(const float* x, int64_t rows, int64_t cols,
                        const float* gamma, float eps, float* y);

/* Residual add followed by per-row RMSNorm: h = add_forward(x, residual)
 * (LayerOps.hpp:142-199, equal sizes) then Normalization::rms_norm of h
 * (Layers.hpp:1003-1021).  Writes h to residual_out and the normed h to y. */
int oracle_add_rmsnorm(const float* x, const float* residual, int64_t rows,
                       int64_t cols, const float* gamma, float eps,
                       float* residual_out, float* y);

/* LayerOps::add_forward, LayerOps.hpp:142-199 (equal / scalar / repeat). */
int oracle_add(const float* a, int64_t na, const float* b, int64_t nb, float* y);

/* LayerOps::multiply_forward, LayerOps.hpp:205-230. */
int oracle_mul(const float* a, int64_t na, const float* b, int64_t nb, float* y);

/* Softmax modes. */
#define ORACLE_SOFTMAX_DIV_EPS 0 /* LayerOps::softmax_inplace, LayerOps.hpp:952-974 */
#define ORACLE_SOFTMAX_MUL_INV 1 /* LayerOps::softmax_forward, LayerOps.hpp:325-361 */
#define ORACLE_SOFTMAX_LOG     2 /* same, LogSoftmax branch, LayerOps.hpp:345-353 */

/* Row softmax over `rows` rows of `cols` elements in the given mode. */
int oracle_softmax_rows(const float* x, int64_t rows, int64_t cols, int mode, float* y);

/* LayerOps::gelu_forward, LayerOps.hpp:556-568 (tanh approximation). */
void oracle_gelu(const float* x, int64_t n, float* y);
/* LayerOps::silu_forward, LayerOps.hpp:570-581. */
void oracle_silu(const float* x, int64_t n, float* y);
/* multiply_forward(silu_forward(gate), up): LayerOps.hpp:570-581 then :205-230. */
void oracle_silu_mul(const float* gate, const float* up, int64_t n, float* y);
/* multiply_forward(gelu_forward(gate), up): LayerOps.hpp:556-568 then :205-230. */
void oracle_gelu_mul(const float* gate, const float* up, int64_t n, float* y);

/* Embedding gather, inline in Model.cpp:1152-1205 (int ids).  vocab and dim
 * are clamped to >= 1; the table must hold vocab*dim floats; out is zero-filled
 * and rows for padding / out-of-range ids stay zero. */
int oracle_embedding_i32(const int32_t* ids, int64_t n_ids, const float* table,
                         int64_t table_len, int32_t vocab, int32_t dim,
                         int32_t padding_idx, float* y);

/* Float-id form, Model.cpp:5301-5334: id = (int) llround((double) x[t]). */
int oracle_embedding_f32(const float* ids, int64_t n_ids, const float* table,
                         int64_t table_len, int32_t vocab, int32_t dim,
                         int32_t padding_idx, float* y);

/* Rotary table (no reference): inv_freq_i = 1 / theta^(2i/D), angle = p*inv_freq_i,
 * both in double; cos/sin rounded once to float.  Shape [rows x D/2]. */
int oracle_rope_table(int64_t rows, int64_t head_dim, double theta,
                      float* cos_tab, float* sin_tab);

/* Rotate-half RoPE on x laid out [B, S, H, D]; position = pos_offset + s.
 * y[i] = x[i]*c - x[i+D/2]*s;  y[i+D/2] = x[i+D/2]*c + x[i]*s  (float32). */
int oracle_rope(const float* x, float* y, int64_t B, int64_t S, int64_t H,
                int64_t D, int64_t pos_offset, const float* cos_tab,
                const float* sin_tab, int64_t table_rows);

/* ---- Backward (Model::backwardPass branches, Model.cpp:7305-9153) ---- */

/* accumulate_grad, Model.cpp:7329-7341: dst[i] += src[i]. */
void oracle_accumulate(float* dst, const float* src, int64_t n);

/* LayerNorm branch, Model.cpp:7719-7821.  Groups of n = in_features (or N);
 * gamma NULL when the layer is not affine.  dx is written; grad_params (the
 * [dgamma | dbeta] block, feat*(1+has_bias) floats) is added to, as the
 * reference adds into Layer::grad_weights. */
int oracle_layernorm_bwd(const float* x, const float* dy, int64_t N, int64_t in_features,
                         const float* gamma, int has_bias, float eps, float* dx,
                         float* grad_params);

/* GELU branch, Model.cpp:9026-9051; SiLU branch, Model.cpp:7993-8032. */
void oracle_gelu_bwd(const float* x, const float* dy, int64_t n, float* dx);
void oracle_silu_bwd(const float* x, const float* dy, int64_t n, float* dx);

/* Multiply branch, Model.cpp:7647-7665. */
void oracle_mul_bwd(const float* a, const float* b, const float* dy, int64_t n, float* da,
                    float* db);

/* Add branch, Model.cpp:7541-7601: gradient of the broadcast operand
 * (n_small == 1: the sum of dy; else sums over the n_big/n_small tiles). */
int oracle_add_bwd_small(const float* dy, int64_t n_big, int64_t n_small, float* d_small);

/* Embedding branch, Model.cpp:7429-7461 (ids as int32 or as floats rounded
 * with llround): grad_table rows += dy rows in token order. */
int oracle_embedding_bwd_i32(const int32_t* ids, int64_t n_ids, const float* dy,
                             float* grad_table, int64_t table_len, int32_t vocab, int32_t dim,
                             int32_t padding_idx);
int oracle_embedding_bwd_f32(const float* ids, int64_t n_ids, const float* dy, float* grad_table,
                             int64_t table_len, int32_t vocab, int32_t dim, int32_t padding_idx);

/* ---- Attention core (the softmax between QK^T and PV) ---- */

/* The core of LayerOps::self_attention_forward (LayerOps.hpp:1045-1089) and
 * cross_attention_forward (:1163-1209): softmax(Q K^T * scale, causal mask
 * j > i) V over `batch` independent sequences of q_len queries and kv_len
 * keys.  Q rows have stride ld_q, K and V rows stride ld_kv (so Q, K, V may be
 * the column blocks of one fused QKV buffer), output rows stride ld_out; head
 * h owns columns [h*head_dim, (h+1)*head_dim).  The reference's scale is
 * 1.0f / sqrtf((float) head_dim) (:1047). */
int oracle_attention(const float* q, int64_t ld_q, const float* k, const float* v, int64_t ld_kv,
                     float* out, int64_t ld_out, int64_t batch, int64_t q_len, int64_t kv_len,
                     int64_t heads, int64_t head_dim, float scale, int causal);

/* The per-head core of the reference's backward_self_attention /
 * backward_cross_attention (Model.cpp:6892-7028, 7122-7246): from q, k, v
 * (laid out as for oracle_attention) and dout, the gradient of the attended
 * heads, writes dq (rows ld_dq), dk and dv (rows ld_dkv). */
int oracle_attention_bwd(const float* q, int64_t ld_q, const float* k, const float* v, int64_t ld_kv,
                         const float* dout, int64_t ld_dout, float* dq, int64_t ld_dq, float* dk, float* dv,
                         int64_t ld_dkv, int64_t batch, int64_t q_len, int64_t kv_len, int64_t heads,
                         int64_t head_dim, float scale, int causal);

#ifdef __cplusplus
}
#endif

#endif
