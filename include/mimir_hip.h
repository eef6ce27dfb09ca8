/*
 * mimir_hip.h -- C ABI of the MI355X (gfx950) backend for Mimir's fused
 * elementwise and row-reduction layer path.
 *
 * The library (libmimir_hip.so) replaces the CPU forward entry points listed
 * next to each function below (file:line in brit45/mimir-framework).  All
 * tensors are fp32 (ids int32), row-major and contiguous, and live in device
 * memory: every `float*` / `int32_t*` argument of an op is a DEVICE pointer
 * (from mimir_malloc, hipMalloc or any other HIP allocation on the context's
 * device).  Ops never allocate and never synchronise: they enqueue on the
 * context's stream and return.  Stream order is the only ordering;
 * mimir_sync() and the download copy are the blocking calls.
 *
 * Status codes: every function returns MIMIR_OK or one of the codes below.
 * Argument errors are detected on the host before anything is enqueued (the
 * cases where the reference throws std::runtime_error), and the message is
 * available from mimir_last_error(ctx).
 *
 * Threading: one context per host thread; a context is not safe for
 * concurrent use without external locking.
 */
#ifndef MIMIR_HIP_H
#define MIMIR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIMIR_OK 0
#define MIMIR_EINVAL 1  /* invalid shape / argument; the reference throws here */
#define MIMIR_ENOMEM 2  /* device allocation failed or exceeded the context cap */
#define MIMIR_EDEVICE 3 /* HIP runtime error or no usable device */
#define MIMIR_EBUSY 4   /* a per-GPU resource is held by another context (mimir_layernorm_bwd_noalloc) */

typedef struct mimir_ctx mimir_ctx;
typedef struct mimir_event mimir_event;

/* ---------------------------------------------------------------------------
 * Context, memory, ordering.  These replace the host-side storage the
 * reference ops read and write (std::vector<float> activations in
 * Model::tensor_store, Model.hpp:608-610; weight blocks via Layer::getWeights,
 * Layers.hpp:232-240; RuntimeAllocator::allocate_tensor,
 * RuntimeAllocator.hpp:191-226) with device-resident buffers.
 * ------------------------------------------------------------------------- */

/* Create a context on HIP device `device` with its own (default-priority)
 * stream. */
int mimir_ctx_create(int device, mimir_ctx** out);
int mimir_ctx_destroy(mimir_ctx* ctx);
/* Enqueue on an existing HIP stream (hipStream_t passed as void*) instead of
 * the context's own; NULL restores the context's stream.  Waits for the work
 * already enqueued on the previous stream (the context's scratch memory is
 * reused in stream order). */
int mimir_ctx_set_stream(mimir_ctx* ctx, void* hip_stream);
void* mimir_ctx_stream(mimir_ctx* ctx);
/* Cap on the bytes mimir_malloc may hold at once (0 = no cap).  Mirrors
 * MemoryGuard::setLimit (MemoryGuard.hpp:75-130): over the cap -> ENOMEM. */
int mimir_ctx_set_alloc_limit(mimir_ctx* ctx, size_t bytes);
/* Output store policy of the ops enqueued after this call.  0 (default):
 * outputs are streamed to HBM with non-temporal stores, the fastest form
 * for an op whose result is not read again soon.  1: plain stores, which
 * leave the output in L2 / the Infinity Cache (256 MiB), so an op launched
 * next that reads it finds much of it there -- a chain of layers.  The
 * device-resident runtime (mimir_store_run) sets it for every layer but the
 * last.  No counterpart in the reference (its ops run on host vectors). */
int mimir_ctx_set_output_caching(mimir_ctx* ctx, int keep);
/* Message for the last non-OK status returned on this context. */
const char* mimir_last_error(const mimir_ctx* ctx);

int mimir_malloc(mimir_ctx* ctx, size_t bytes, void** dptr);
int mimir_free(mimir_ctx* ctx, void* dptr);
/* Stream-ordered copies.  Upload returns once the source may be reused;
 * download returns once the data is on the host. */
int mimir_upload(mimir_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
int mimir_download(mimir_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);
/* Device-to-device copy (a plain streaming-copy kernel; n bytes, any alignment). */
int mimir_copy(mimir_ctx* ctx, void* dst_dev, const void* src_dev, size_t bytes);
/* Fill `n` floats with `value` (a fill kernel, so it is safe under graph capture). */
int mimir_fill_f32(mimir_ctx* ctx, float* dst_dev, int64_t n, float value);
int mimir_sync(mimir_ctx* ctx);

/* Stream-ordered timing events on the context's current stream. */
int mimir_event_create(mimir_ctx* ctx, mimir_event** out);
int mimir_event_destroy(mimir_event* ev);
int mimir_event_record(mimir_ctx* ctx, mimir_event* ev);
/* Milliseconds between two recorded events (waits for `stop`). */
int mimir_event_elapsed_ms(mimir_event* start, mimir_event* stop, float* ms);

/* ---------------------------------------------------------------------------
 * Normalisation
 * ------------------------------------------------------------------------- */

/* LayerOps::layernorm_forward, LayerOps.hpp:264-319.
 * x and y hold `groups * n` floats; each group of n is normalised with the
 * two-pass mean / variance: y = (x - mean) / sqrt(var + eps) [* gamma[i]
 * [+ beta[i]]].  gamma == NULL is the non-affine layer; beta == NULL is
 * use_bias == false; beta without gamma is EINVAL (the reference adds the
 * bias only inside the affine branch).  The reference's group size is
 * `in_features > 0 ? in_features : N`; n <= 0 is EINVAL.  y may alias x. */
int mimir_layernorm_fwd(mimir_ctx* ctx, const float* x, const float* gamma, const float* beta,
                        float* y, int64_t groups, int64_t n, float eps);

/* RMSNorm over `rows` rows of `cols`: y = x / sqrt(sum(x^2)/cols + eps) * w[c].
 * rows == 1, cols == N is the reference layer LayerOpsExt::rms_norm_forward
 * (LayerOpsExt.hpp:345-378), which normalises the WHOLE input as one group
 * and multiplies element c by w[c] only while c < w_len.  rows > 1 is the
 * per-row form Normalization::rms_norm (Layers.hpp:1003-1021), with
 * w_len == cols.  w == NULL (or w_len == 0) -> no scale.  y may alias x. */
int mimir_rmsnorm_fwd(mimir_ctx* ctx, const float* x, const float* w, int64_t w_len, float* y,
                      int64_t rows, int64_t cols, float eps);

/* Residual add fused with per-row RMSNorm, one HBM pass:
 *   h = x + residual   (LayerOps::add_forward, LayerOps.hpp:142-169)
 *   residual_out = h;  y = h / sqrt(sum(h^2)/cols + eps) * w[c]
 *                      (Normalization::rms_norm, Layers.hpp:1003-1021).
 * The reference has no fused op; it runs the two calls back to back.
 * residual_out may alias residual (in-place residual update); y must not
 * alias residual_out.  w may be NULL. */
int mimir_add_rmsnorm_fwd(mimir_ctx* ctx, const float* x, const float* residual,
                          float* residual_out, const float* w, float* y, int64_t rows,
                          int64_t cols, float eps);

/* ---------------------------------------------------------------------------
 * Softmax
 * ------------------------------------------------------------------------- */

/* y[j] = e[j] / (sum + 1e-9f): LayerOps::softmax_inplace, LayerOps.hpp:952-974
 * (the row softmax used by attention). */
#define MIMIR_SOFTMAX_DIV_EPS 0
/* y[j] = e[j] * (1.0f / sum): LayerOps::softmax_forward, LayerOps.hpp:325-361
 * (the Softmax layer; the layer itself is rows == 1, cols == N). */
#define MIMIR_SOFTMAX_MUL_INV 1
/* y[j] = (x[j] - max) - log(sum): LogSoftmax branch, LayerOps.hpp:345-353. */
#define MIMIR_SOFTMAX_LOG 2

/* Max-subtracted softmax of each of `rows` rows of `cols` (cols >= 1), with
 * e[j] = exp(x[j] - max).  -inf entries give exactly 0.  y may alias x. */
int mimir_softmax_fwd(mimir_ctx* ctx, const float* x, float* y, int64_t rows, int64_t cols,
                      int mode);

/* ---------------------------------------------------------------------------
 * Elementwise
 * ------------------------------------------------------------------------- */

/* LayerOps::gelu_forward, LayerOps.hpp:556-568 (tanh form):
 * y = x * 0.5f*(1 + tanh(sqrt(2/pi)*(x + 0.044715f*x^3))).  y may alias x. */
int mimir_gelu_fwd(mimir_ctx* ctx, const float* x, float* y, int64_t n);
/* LayerOps::silu_forward, LayerOps.hpp:570-581: y = x * (1/(1+exp(-x))). */
int mimir_silu_fwd(mimir_ctx* ctx, const float* x, float* y, int64_t n);
/* SiLU-gated product in one pass: y = silu(gate) * up, i.e.
 * multiply_forward(silu_forward(gate), up) (LayerOps.hpp:570-581, 205-230). */
int mimir_silu_mul_fwd(mimir_ctx* ctx, const float* gate, const float* up, float* y, int64_t n);
/* GELU-gated product: multiply_forward(gelu_forward(gate), up). */
int mimir_gelu_mul_fwd(mimir_ctx* ctx, const float* gate, const float* up, float* y, int64_t n);
/* LayerOps::add_forward, LayerOps.hpp:142-199.  Output has max(na, nb) floats:
 * equal sizes -> elementwise; the shorter operand of size 1 -> scalar
 * broadcast; the longer size a multiple of the shorter -> repeat
 * (y[i] = big[i] + small[i % small_n]); otherwise EINVAL; either size 0 ->
 * EINVAL.  Bit-identical to the reference (one IEEE add per element). */
int mimir_add_fwd(mimir_ctx* ctx, const float* a, int64_t na, const float* b, int64_t nb,
                  float* y);
/* LayerOps::multiply_forward, LayerOps.hpp:205-230: na != nb -> EINVAL. */
int mimir_mul_fwd(mimir_ctx* ctx, const float* a, int64_t na, const float* b, int64_t nb,
                  float* y);

/* Branch merge operations: the reference's MergeOperation (Layers.hpp:72-80). */
#define MIMIR_MERGE_ADD 0
#define MIMIR_MERGE_MULTIPLY 1
#define MIMIR_MERGE_CONCATENATE 2
#define MIMIR_MERGE_MAX 3
#define MIMIR_MERGE_AVERAGE 4
#define MIMIR_MERGE_GATED 5
#define MIMIR_MERGE_ATTENTION_WEIGHTED 6
/* Model::computeBranchMerge(branch1 = a, branch2 = b, output = y, merge_op),
 * Model.cpp:4344-4479, the training-mode residual merge.  y holds na floats
 * (na + nb for CONCATENATE: a then b).  ADD, and GATED / ATTENTION_WEIGHTED
 * (the reference's default branch, copy then +=): a[i] + b[i]; MULTIPLY:
 * a[i] * b[i]; AVERAGE: (a[i] + b[i]) * 0.5f; MAX: for i below na rounded
 * down to a multiple of 8, the AVX2 body's vmaxps (a[i] > b[i] ? a[i] :
 * b[i]), past it the scalar tail's std::max (a[i] < b[i] ? b[i] : a[i]) --
 * the two differ only for NaN and signed zeros.  Bit-identical to the
 * reference.  The reference reads b past its end when nb < na; that is
 * EINVAL here. */
int mimir_branch_merge_fwd(mimir_ctx* ctx, const float* a, int64_t na, const float* b, int64_t nb,
                           float* y, int merge_op);

/* ---------------------------------------------------------------------------
 * Embedding gather and rotary position embedding
 * ------------------------------------------------------------------------- */

/* Token-embedding gather, inline in Model::forwardPassView (int ids),
 * Model.cpp:1152-1205.  vocab and dim are clamped to >= 1 (Model.cpp:1176-1177);
 * table_len < vocab*dim is EINVAL (:1181-1182).  y is [n_ids x dim]; the row of
 * an id equal to padding_idx (when padding_idx >= 0) or outside [0, vocab) is
 * all zeros (silently, as in the reference); every other row is a bit-exact
 * copy of table[id]. */
int mimir_embedding_fwd(mimir_ctx* ctx, const int32_t* ids, int64_t n_ids, const float* table,
                        int64_t table_len, int32_t vocab, int32_t dim, int32_t padding_idx,
                        float* y);
/* Float-id form, Model.cpp:5301-5334: id = (int) llround((double) ids[t]),
 * including the x86-64 conversion of non-finite / huge values (id 0) and
 * the wrap of the 64-bit result to int. */
int mimir_embedding_f32ids_fwd(mimir_ctx* ctx, const float* ids, int64_t n_ids,
                               const float* table, int64_t table_len, int32_t vocab, int32_t dim,
                               int32_t padding_idx, float* y);

/* Host-side rotary table (the reference has no RoPE): for p in [0, rows),
 * i in [0, head_dim/2): inv_freq = 1 / theta^(2i/head_dim), a = p*inv_freq in
 * double; cos_tab/sin_tab[p*head_dim/2 + i] = (float)cos(a) / (float)sin(a).
 * cos_tab and sin_tab are HOST arrays of rows*head_dim/2 floats. */
int mimir_rope_table(int64_t rows, int64_t head_dim, double theta, float* cos_tab,
                     float* sin_tab);

/* Rotate-half RoPE on q and k in one launch, both laid out
 * [batch, seq, heads, head_dim] (k may have its own head count k_heads;
 * k == NULL skips it).  For position p = pos_offset + s and pair i < D/2:
 *   y[i]     = x[i]*cos[p,i] - x[i+D/2]*sin[p,i]
 *   y[i+D/2] = x[i+D/2]*cos[p,i] + x[i]*sin[p,i]
 * cos_tab / sin_tab are DEVICE tables of table_rows x D/2 (mimir_rope_table);
 * pos_offset + seq > table_rows is EINVAL.  head_dim must be even.
 * q_out may alias q and k_out may alias k (in place). */
int mimir_rope_fwd(mimir_ctx* ctx, const float* q, float* q_out, int64_t q_heads, const float* k,
                   float* k_out, int64_t k_heads, int64_t batch, int64_t seq, int64_t head_dim,
                   int64_t pos_offset, const float* cos_tab, const float* sin_tab,
                   int64_t table_rows);

/* The attention core with the softmax fused between QK^T and PV: replaces
 * steps 3-5 of LayerOps::self_attention_forward (LayerOps.hpp:1045-1089,
 * called by the SelfAttention / MultiHeadAttention layers, Model.cpp:
 * 5904-5934 and :1291-1310) and the same core of cross_attention_forward
 * (:1163-1209).  For each of `batch` independent sequences, head h and query i:
 *   s_j = (Q_i . K_j) * scale, j in [0, kv_len); causal: keys j > i excluded
 *   out_i = sum_j exp(s_j - max) V_j / (sum_j exp(s_j - max) + 1e-9)
 * Query i of sequence b is row b*q_len + i of q (stride ld_q floats) and of
 * out (stride ld_out); key j is row b*kv_len + j of k and v (stride ld_kv),
 * so q / k / v may be the three column blocks of one fused QKV buffer
 * (ld = 3 * heads * head_dim).  Head h owns columns [h*head_dim,
 * (h+1)*head_dim).  The reference's scale is 1.0f / sqrtf(head_dim).
 * head_dim <= 2048 (above 128 a plain fp32 vector kernel runs instead of the
 * matrix-core one).  fp32 throughout (fp32 matrix-core products), no score
 * matrix in memory.  out must not overlap q, k or v.  kv_len == 0 gives zeros;
 * batch == 0 or q_len == 0 is a no-op.  Device pointers, stream order. */
int mimir_attention_fwd(mimir_ctx* ctx, const float* q, int64_t ld_q, const float* k, const float* v,
                        int64_t ld_kv, float* out, int64_t ld_out, int64_t batch, int64_t q_len,
                        int64_t kv_len, int64_t heads, int64_t head_dim, float scale, int causal);

/* The SelfAttention / MultiHeadAttention layer: LayerOps::self_attention_forward
 * (LayerOps.hpp:1004-1097; MultiHeadAttention calls it, :1100-1113), as
 * Model.cpp:5904-5934 dispatches it.  input [seq_len x embed_dim]; weights =
 * the layer's block [qkv_weight (embed_dim x 3 embed_dim) | out_weight
 * (embed_dim x embed_dim)], row-major as the reference's matmul reads them,
 * at least 4 embed_dim^2 floats (the reference reads past a shorter block; it
 * is refused here); out [seq_len x embed_dim].  The projections are fp32
 * library GEMMs, the core is mimir_attention_fwd with the reference's
 * scale 1/sqrtf(head_dim).  head_dim <= 2048.  Uses the context's scratch
 * (4 seq_len embed_dim floats).  out must not overlap input or weights. */
int mimir_self_attention_fwd(mimir_ctx* ctx, const float* input, int64_t seq_len, int64_t embed_dim,
                             int64_t num_heads, int causal, const float* weights, int64_t weights_len,
                             float* out);

/* The CrossAttention layer: LayerOps::cross_attention_forward
 * (LayerOps.hpp:1116-1216) as Model.cpp:5936-5990 dispatches it.
 * query_input [query_len x embed_dim], kv_input [kv_len x embed_dim];
 * weights = [q_weight (E x E) | kv_weight (E x 2E) | out_weight (E x E)],
 * at least 4 E^2 floats; out [query_len x embed_dim].  Scratch: 2 (query_len
 * + kv_len) E floats. */
int mimir_cross_attention_fwd(mimir_ctx* ctx, const float* query_input, int64_t query_len,
                              const float* kv_input, int64_t kv_len, int64_t embed_dim, int64_t num_heads,
                              int causal, const float* weights, int64_t weights_len, float* out);

/* Backward of the attention core: the per-head part of the reference's
 * backward_self_attention / backward_cross_attention (Model.cpp:6892-7028,
 * 7122-7246).  From q, k, v (laid out as for mimir_attention_fwd) and dout,
 * the gradient of the core's output (ld_dout), writes
 *   dv = P^T dout,  dq = scale dS k,  dk = scale dS^T q,
 *   dS = P (dout v^T - rowsum(P * (dout v^T))), 0 on masked keys,
 * with P the core's probabilities (causal j > i masked to -1e9, max from
 * -1e30, p = e / (sum + 1e-9)).  dq rows have ld_dq, dk and dv rows ld_dkv
 * (dk and dv may be column blocks of one buffer, as the reference's dqkv).
 * Overwrites dq / dk / dv.  P and dS are materialised per group of heads
 * in the context's scratch (2 q_len kv_len floats per head, groups capped at
 * 1 GiB, one head at least), beside K^T and V^T of one sequence (2 kv_len
 * heads head_dim floats); the products are fp32 library GEMMs, the row
 * passes (mask + softmax, softmax backward) and the transposes hand-written
 * kernels.
 * kv_len == 0: dq = 0.  Outputs must not overlap the inputs. */
int mimir_attention_bwd(mimir_ctx* ctx, const float* q, int64_t ld_q, const float* k, const float* v,
                        int64_t ld_kv, const float* dout, int64_t ld_dout, float* dq, int64_t ld_dq, float* dk,
                        float* dv, int64_t ld_dkv, int64_t batch, int64_t q_len, int64_t kv_len, int64_t heads,
                        int64_t head_dim, float scale, int causal);

/* backward_self_attention (Model.cpp:6847-7062), as Model::backwardPass's
 * SelfAttention / MultiHeadAttention branch calls it (:8034-8072): input
 * [seq_len x E] (the layer's forward input), grad_out [seq_len x E], the
 * weight block as for mimir_self_attention_fwd.  Adds dWqkv / dWout into
 * grad_weights (same layout as weights; skipped when NULL) and writes the
 * input gradient dx = dqkv Wqkv^T to grad_input, or adds it there when
 * accumulate (accumulate_grad's add).  grad_input may be grad_out itself
 * (it is written last).  Scratch: 8 seq_len E floats plus the core's. */
int mimir_self_attention_bwd(mimir_ctx* ctx, const float* input, const float* grad_out, int64_t seq_len,
                             int64_t embed_dim, int64_t num_heads, int causal, const float* weights,
                             int64_t weights_len, float* grad_weights, float* grad_input, int accumulate);

/* backward_cross_attention (Model.cpp:7068-7300), as the CrossAttention
 * branch calls it (:8074-8130): adds dWq / dWkv / dWout into grad_weights
 * (skipped when NULL), then writes (or, with the accumulate flags, adds) the
 * query gradient into grad_query and after it the key/value gradient into
 * grad_kv; either may be grad_out's buffer and the two may be one buffer
 * (inputs that share a name).  Scratch: 4 (query_len + kv_len) E floats plus
 * the core's. */
int mimir_cross_attention_bwd(mimir_ctx* ctx, const float* query_input, int64_t query_len, const float* kv_input,
                              int64_t kv_len, const float* grad_out, int64_t embed_dim, int64_t num_heads,
                              int causal, const float* weights, int64_t weights_len, float* grad_weights,
                              float* grad_query, int accumulate_query, float* grad_kv, int accumulate_kv);

/* ---------------------------------------------------------------------------
 * Backward of the path's ops: the branches of the reference's
 * Model::backwardPass (Model.cpp:7305-9153).  Device pointers, stream order.
 *
 * Gradient outputs follow the reference's accumulate_grad (Model.cpp:
 * 7329-7341): with `accumulate` 0 the gradient is written (the name had no
 * gradient yet), with 1 it is added onto what the buffer holds.  Products
 * and sums are rounded where the reference rounds them (no FMA
 * contraction), so Multiply / Add gradients and the accumulation itself are
 * bit-identical; the Embedding scatter-add adds in token order and is
 * bit-identical too.  Reductions over tokens (dgamma, dbeta, the broadcast
 * operand of Add) are deterministic: the same inputs give the same bits.
 * Scratch for partial sums is the context's (reused in stream order).
 * ------------------------------------------------------------------------- */

/* LayerNorm branch, Model.cpp:7719-7821, over `groups` groups of n
 * (n = in_features, or the whole input).  gamma NULL when the layer is not
 * affine.  dx gets the input gradient ((+)= per `accumulate`); dgamma /
 * dbeta (n floats each, or NULL) are ADDED to, as the reference adds into
 * Layer::grad_weights (:7809-7819); dbeta needs dgamma, dgamma needs gamma.
 * dx may alias dy. */
int mimir_layernorm_bwd(mimir_ctx* ctx, const float* x, const float* dy, const float* gamma, float* dx,
                        float* dgamma, float* dbeta, int64_t groups, int64_t n, float eps, int accumulate);
/* mimir_layernorm_bwd that allocates nothing.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving and training loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and bits as mimir_layernorm_bwd, but
 * its scratch (the dgamma / dbeta partial-sum slots, the long-row partials)
 * is a fixed 32 MiB device array that the library reserves per GPU for the
 * life of the process.  A call that needs more (e.g. width 4096 takes 17.3 MB
 * with dgamma, a width above ~7900 takes more than 32 MiB) returns EINVAL
 * before any launch.  One context per GPU uses that array at a time: the
 * first context to call this entry point on a GPU holds it until the context
 * is destroyed, and a call from another context on that GPU returns
 * MIMIR_EBUSY before any launch.  The holder's calls run in its stream's
 * order (mimir_ctx_set_stream waits for the old stream), so they cannot
 * overlap.  The check is host-side only: it allocates nothing and records
 * nothing into a captured graph. */
int mimir_layernorm_bwd_noalloc(mimir_ctx* ctx, const float* x, const float* dy, const float* gamma, float* dx,
                                float* dgamma, float* dbeta, int64_t groups, int64_t n, float eps, int accumulate);

/* GELU branch, Model.cpp:9026-9051 (tanh approximation): dx (+)= dy * gelu'(x). */
int mimir_gelu_bwd(mimir_ctx* ctx, const float* x, const float* dy, float* dx, int64_t n, int accumulate);

/* SiLU branch, Model.cpp:7993-8032: dx (+)= dy * (s + x*s*(1-s)), s = sigmoid(x). */
int mimir_silu_bwd(mimir_ctx* ctx, const float* x, const float* dy, float* dx, int64_t n, int accumulate);

/* Multiply branch, Model.cpp:7647-7665: da (+)= dy*b, db (+)= dy*a, both
 * products formed before either accumulation.  da or db may be NULL.  When
 * da == db (a tensor times itself) the second accumulation adds onto the
 * first. */
int mimir_mul_bwd(mimir_ctx* ctx, const float* a, const float* b, const float* dy, float* da, float* db,
                  int64_t n, int acc_a, int acc_b);

/* Add branch, Model.cpp:7541-7601, for add_forward(a[na], b[nb]) whose output
 * gradient dy has max(na, nb) floats.  Equal sizes: da (+)= dy, then
 * db (+)= dy.  Broadcast: the big operand's gradient (+)= dy, then the small
 * operand's (+)= the sum of dy over the tiles (nb == 1: over all of it).
 * Accumulations run in the reference's order and see each other where the
 * buffers alias (dy, da, db may be the same buffer, as names can be in the
 * reference's gradient map).  da or db may be NULL. */
int mimir_add_bwd(mimir_ctx* ctx, const float* dy, int64_t na, int64_t nb, float* da, float* db, int acc_a,
                  int acc_b);

/* Embedding branch, Model.cpp:7429-7461: grad_table[id*dim + d] += dy[t*dim + d]
 * for every token t in order; the padding id and ids outside [0, vocab) are
 * skipped.  grad_table holds at least vocab*dim floats (table_len); dy holds
 * n_ids*dim. */
int mimir_embedding_bwd(mimir_ctx* ctx, const int32_t* ids, int64_t n_ids, const float* dy,
                        float* grad_table, int64_t table_len, int32_t vocab, int32_t dim,
                        int32_t padding_idx);
/* Same with float ids rounded by llround (Model.cpp:7453). */
int mimir_embedding_f32ids_bwd(mimir_ctx* ctx, const float* ids, int64_t n_ids, const float* dy,
                               float* grad_table, int64_t table_len, int32_t vocab, int32_t dim,
                               int32_t padding_idx);

/* ---------------------------------------------------------------------------
 * Device-resident runtime: a named tensor store and a layer runner with the
 * routing of the reference's Model::forwardPassNamed (Model.cpp:1352-1408,
 * forwardPassView Model.cpp:4621-6824) for the layer types of this path.
 * Replaces Model::tensor_store / tensor_store_int (Model.hpp:608-610), which
 * hold every activation as a host std::vector, with device buffers, so
 * consecutive layers never leave HBM.  Inference only (training=false).
 * Buffers are pooled per store and reused in stream order: once a graph has
 * run, running it again allocates nothing.
 * ------------------------------------------------------------------------- */

typedef struct mimir_store mimir_store;

#define MIMIR_DTYPE_F32 0
#define MIMIR_DTYPE_I32 1

/* Layer types (the reference's LayerType names, LayerTypes.hpp:13-120). */
#define MIMIR_LAYER_LAYERNORM 1  /* LayerOps::layernorm_forward, LayerOps.hpp:264-319 */
#define MIMIR_LAYER_RMSNORM 2    /* LayerOpsExt::rms_norm_forward (whole vector) */
#define MIMIR_LAYER_SOFTMAX 3    /* LayerOps::softmax_forward (whole vector) */
#define MIMIR_LAYER_LOGSOFTMAX 4 /* LayerOps::softmax_forward, LogSoftmax branch */
#define MIMIR_LAYER_GELU 5       /* LayerOps::gelu_forward */
#define MIMIR_LAYER_SILU 6       /* LayerOps::silu_forward */
#define MIMIR_LAYER_ADD 7        /* LayerOps::add_forward (inputs[0], inputs[1]) */
#define MIMIR_LAYER_MULTIPLY 8   /* LayerOps::multiply_forward */
#define MIMIR_LAYER_EMBEDDING 9  /* inline gather, Model.cpp:5301-5334 */
#define MIMIR_LAYER_IDENTITY 10  /* LayerOps::identity_forward */
#define MIMIR_LAYER_DROPOUT 11   /* LayerOps::dropout_forward at inference: identity */
/* The attention layers (Model.cpp:5904-5990): projections + the fused core,
 * mimir_self_attention_fwd / mimir_cross_attention_fwd; in
 * mimir_store_backward, mimir_self_attention_bwd / mimir_cross_attention_bwd
 * (Model.cpp:8034-8130). */
#define MIMIR_LAYER_SELF_ATTENTION 12      /* LayerOps::self_attention_forward */
#define MIMIR_LAYER_MULTIHEAD_ATTENTION 13 /* LayerOps::multihead_attention_forward (the same) */
#define MIMIR_LAYER_CROSS_ATTENTION 14     /* LayerOps::cross_attention_forward (inputs: query, key_value) */

/* One layer: the fields of the reference's `Layer` (Layers.hpp:86-309) this
 * path reads.  `weights` is a DEVICE pointer to the layer's weight block
 * (Layer::getWeights) of `weights_len` floats (Layer::getWeightsSize). */
typedef struct mimir_layer {
    int32_t type;
    const char* name;           /* used in error messages */
    const char* const* inputs;  /* n_inputs names; n_inputs == 0 -> {"x"} */
    int32_t n_inputs;
    const char* output;         /* NULL or "" -> "x" */
    const float* weights;
    int64_t weights_len;
    float eps;
    int32_t affine;
    int32_t use_bias;
    int32_t in_features;
    int32_t vocab_size;
    int32_t embed_dim;
    int32_t padding_idx;
    int32_t seq_len;
    float* grad_weights;        /* DEVICE, weights_len floats, or NULL: the layer's
                                   Layer::grad_weights for mimir_store_backward
                                   (added to, as the reference adds into it) */
    /* Branch fields (Layers.hpp:214-219), read by mimir_store_run_training
     * only, as forwardPassView reads them only with training=true
     * (Model.cpp:4729-4732, 6676-6685).  Zero-initialised = no branch. */
    int32_t branch_type;              /* Layer::branch_type (BranchType, Layers.hpp:59-69) */
    int32_t merge_op;                 /* Layer::merge_op, a MIMIR_MERGE_* value */
    const int32_t* branch_sources;    /* host array, Layer::branch_sources */
    int32_t n_branch_sources;
    /* Attention fields (Layers.hpp:174-178), read by the attention layers. */
    int32_t num_heads;                /* Layer::num_heads (the reference's default is 8) */
    int32_t head_dim;                 /* Layer::head_dim (CrossAttention: embed_dim = head_dim * num_heads when 0) */
    int32_t causal;                   /* Layer::causal */
} mimir_layer;

/* BranchType values (Layers.hpp:59-69) that the runtime acts on. */
#define MIMIR_BRANCH_NONE 0
#define MIMIR_BRANCH_RESIDUAL 1

int mimir_store_create(mimir_ctx* ctx, mimir_store** out);
int mimir_store_destroy(mimir_store* store);
/* Drop every name (buffers go back to the store's pool). */
int mimir_store_clear(mimir_store* store);
/* Upload `n` elements of `dtype` from host memory under `name` (replacing a
 * tensor of that name and dtype). */
int mimir_store_put(mimir_store* store, const char* name, int dtype, const void* host, int64_t n);
/* Device pointer and element count of a stored tensor (EINVAL if absent). */
int mimir_store_info(mimir_store* store, const char* name, int dtype, void** dptr, int64_t* n);
/* Download a stored tensor into `host` (cap elements); *n gets its size. */
int mimir_store_get(mimir_store* store, const char* name, int dtype, void* host, int64_t cap,
                    int64_t* n);
/* The input setup of Model::forwardPassNamed(float_inputs, int_inputs):
 * clears both stores, stores "x" and "__input__" = float_inputs["x"] (else
 * float_inputs["__input__"], else empty), the int inputs (an int "seq" also
 * under "text_ids", "__input__" and "x"), then every float input.  Host data. */
int mimir_store_set_inputs(mimir_store* store, const char* const* fnames, const float* const* fdata,
                           const int64_t* fsizes, int32_t nf, const char* const* inames,
                           const int32_t* const* idata, const int64_t* isizes, int32_t ni);
/* Run layers in order (Model::forwardPassView's layer loop): inputs by name
 * from the float store (Embedding input 0 also from the int store, read as
 * float ids, else seq_len padding ids stored under that name), output stored
 * under layer.output or "x".  Errors where the reference throws: EINVAL with
 * the message, e.g. "Missing input tensor: <name>". */
int mimir_store_run(mimir_store* store, const mimir_layer* layers, int32_t n_layers);

/* Inference fusion for mimir_store_run (and what mimir_store_capture
 * records), off by default.  No counterpart in the reference, which stores
 * every layer's output.  When on, a group of consecutive layers in which
 * each reads the previous one's output runs as one kernel:
 *   - [Add (equal sizes) ->] LayerNorm [-> elementwise chain]: the
 *     LayerNorm kernel adds its input first and applies the chain to the
 *     normalised values before storing (rows the register-resident kernel
 *     takes: widths that are multiples of 4 up to 16384 floats, aligned
 *     parameters, no LayerNorm shape override);
 *   - an elementwise chain alone: GELU, SiLU, and Add / Multiply of equal
 *     sizes.
 * Every tensor the group reads crosses HBM once.  An intermediate output is
 * written only when a layer after the group reads its name (or it is "x"
 * and the group does not write "x" again); the other intermediates' names
 * are left unbound, so mimir_store_get on them fails.  "x" and every name a
 * later layer reads hold the unfused run's values bit for bit.  The second
 * operand of a fused Add / Multiply in a chain must be bound when the group
 * starts.  Training runs never fuse. */
int mimir_store_set_fusion(mimir_store* store, int enable);

/* mimir_store_run with the reference's training bookkeeping (forwardPassView
 * with training=true, Model.cpp:4723-4878): each layer's inputs are kept for
 * mimir_store_backward.  The store never writes a tensor in place, so the
 * snapshots are references to its buffers, not copies.  Dropout is refused
 * (its training form draws a random mask).  The snapshots live until the
 * next run, set_inputs or clear.
 * Residual merges (Model.cpp:6676-6685 -> executeBranchComputation :4550-4582):
 * after a layer with branch_type RESIDUAL and a branch source s (its first
 * entry) with 0 <= s <= the layer's index, the layer's output is replaced by
 * mimir_branch_merge_fwd(output, the output layer s produced in this run,
 * merge_op) under the same name; that merged tensor is also what a later
 * merge reads as this layer's output.  Other sources merge nothing, as in
 * the reference.  The backward ignores merges, as Model::backwardPass does
 * (backpropThroughBranch, Model.cpp:4584-4613, is never called). */
int mimir_store_run_training(mimir_store* store, const mimir_layer* layers, int32_t n_layers);

/* The int-ids forward, Model::forwardPassView(const std::vector<int>&
 * input_ids, bool training) (Model.cpp:1030-1349; Model::forwardPass(ids)
 * :1026-1028), the Lua Mimir.Model.forward path.  set_input_ids is its input
 * setup: both stores cleared, the ids (host data) stored as the int tensors
 * "x" and "__input__" (:1046-1049). */
int mimir_store_set_input_ids(mimir_store* store, const int32_t* ids, int64_t n);
/* Its layer loop (:1143-1346).  An Embedding reads its first input from the
 * int store and gathers the ids as ints (EINVAL "Int tensor not found: <name>"
 * when absent; no padding fallback); every other layer reads float inputs
 * (EINVAL "Tensor not found: <name>").  The int path's switch is narrower
 * than forwardPassView(float)'s: of this path's types it runs LayerNorm,
 * GELU, Softmax, LogSoftmax, Dropout, Add and Embedding, and refuses RMSNorm,
 * SiLU, Multiply and Identity with the reference's strict-mode error
 * "forwardPass(int): layer type not supported in int path: <type>"
 * (:1311-1319); an Add with one input is "Add requires 2 inputs" (:1285).
 * Outputs go to layer.output or "x"; with layers, the result must be the
 * float tensor "x" (EINVAL "Tensor not found: x" otherwise, :1348).
 * training=1 keeps the snapshots mimir_store_backward needs (Dropout is then
 * refused, as in mimir_store_run_training); the int path has no residual
 * merges. */
int mimir_store_run_ids(mimir_store* store, const mimir_layer* layers, int32_t n_layers, int training);

/* Model::backwardPass(loss_gradient), Model.cpp:7307-9153, over the layers of
 * the last mimir_store_run_training or training mimir_store_run_ids (the
 * same array): the gradient map starts
 * as {"x": loss_grad} (n_grad host floats) and each layer, last to first,
 * routes its output's gradient to its inputs with the branches of the
 * mimir_*_bwd entry points and accumulate_grad's copy-or-add (an input named
 * like the output adds onto that same gradient, as in the reference).
 * Layer parameter gradients are added into layers[i].grad_weights (skipped
 * when NULL).  Layers whose types have no backward branch in the reference
 * (RMSNorm, Softmax, LogSoftmax) pass the gradient through when the sizes
 * match, as its fallback does (:9133-9140); shape mismatches that the
 * reference skips with a warning are skipped. */
int mimir_store_backward(mimir_store* store, const mimir_layer* layers, int32_t n_layers, const float* loss_grad,
                         int64_t n_grad);
/* mimir_store_backward with loss_grad in device memory (n_grad floats,
 * copied into the store like the host form's upload).  No counterpart in
 * the reference, whose loss gradient is a host vector: for a device-resident
 * training step whose loss gradient is computed on the GPU. */
int mimir_store_backward_dev(mimir_store* store, const mimir_layer* layers, int32_t n_layers, const float* loss_grad,
                             int64_t n_grad);

/* ---------------------------------------------------------------------------
 * Captured forwards: a mimir_store_run recorded once as a HIP graph and
 * replayed with one launch.  No counterpart in the reference, whose layers
 * run one host call after another: for callers that run the same graph of
 * small layers many times (serving, evaluation loops), where launching the
 * kernels one by one costs more than running them.
 *
 *   mimir_store_set_inputs(store, ...);        // the tensors the graph reads
 *   mimir_store_capture(store, layers, n, &g); // runs once eagerly (so every
 *                                              // buffer exists), then records
 *                                              // the same run and launches it
 *   for (...) {
 *       mimir_store_graph_set_input(g, "x", MIMIR_DTYPE_F32, host, n);
 *       mimir_store_graph_launch(g);
 *       mimir_store_graph_get(g, "x", MIMIR_DTYPE_F32, out, cap, &n_out);
 *   }
 *   mimir_store_graph_destroy(g);
 *
 * The graph holds every buffer its run uses (its inputs are the tensors
 * bound at capture, its outputs the bindings the run left), so the store may
 * run other work between launches; they are ordered on the context's
 * stream.  While any graph is alive the context keeps the scratch and
 * library workspace addresses it captured (growing either allocates a new
 * one beside the old).  Inference runs only (mimir_store_run).  The
 * context's stream must not be the null stream.  Destroying the store
 * destroys its graphs.
 * ------------------------------------------------------------------------- */
typedef struct mimir_store_graph mimir_store_graph;

int mimir_store_capture(mimir_store* store, const mimir_layer* layers, int32_t n_layers, mimir_store_graph** out);
/* Replay on the context's stream (asynchronous). */
int mimir_store_graph_launch(mimir_store_graph* graph);
/* Write n host elements into the input `name` (bound when the graph was
 * captured; EINVAL for another name or size). */
int mimir_store_graph_set_input(mimir_store_graph* graph, const char* name, int dtype, const void* host,
                                int64_t n);
/* Download a tensor the graph's run left bound (at most cap elements; *n
 * gets its size).  Waits for the launches before it. */
int mimir_store_graph_get(mimir_store_graph* graph, const char* name, int dtype, void* host, int64_t cap,
                          int64_t* n);
int mimir_store_graph_destroy(mimir_store_graph* graph);

/* A gradient of the last mimir_store_backward by tensor name ("__input__"
 * for Model::getLastInputGradient): device pointer and size, or a download
 * of at most cap floats (*n = its size).  EINVAL when no gradient reached
 * that name. */
int mimir_store_grad_info(mimir_store* store, const char* name, void** dptr, int64_t* n);
int mimir_store_grad_get(mimir_store* store, const char* name, float* host, int64_t cap, int64_t* n);

/* ---------------------------------------------------------------------------
 * SafeTensors checkpoints read straight into device memory: the reference's
 * Mimir::Serialization::load_checkpoint for the SafeTensors format
 * (Serialization.hpp:114; SafeTensorsReader.cpp).  The header is parsed
 * with the reference's checks; tensor bytes go from the file to HBM through
 * pinned staging buffers on the context's stream (reads overlap the DMA).
 * ------------------------------------------------------------------------- */
typedef struct mimir_safetensors mimir_safetensors;

/* dtype codes, the reference's DType (Serialization.hpp:29-36). */
#define MIMIR_ST_F32 0
#define MIMIR_ST_F16 1
#define MIMIR_ST_I32 2
#define MIMIR_ST_I16 3
#define MIMIR_ST_U16 4
#define MIMIR_ST_U8 5

/* Open and parse the header (SafeTensorsReader::parse_header, :52-166):
 * 8-byte little-endian length (0 < len <= 100 MiB), JSON object of entries
 * {dtype, shape, data_offsets} plus "__metadata__"; EINVAL with the
 * reference's message for a missing / unknown dtype, missing shape or
 * data_offsets, bad offsets or (end - begin) != prod(shape) * dtype size.
 * JSON is read as the reference's nlohmann::json 3.11.2 reads it (strict
 * syntax, well-formed UTF-8, a NUL between tokens ends the header, the last
 * of duplicate keys); entries are visited and numbered in byte order of their
 * names.  Refused where the reference's size arithmetic would wrap: negative
 * or out-of-range sizes, and tensor data past the end of the file.
 * ctx may be NULL to inspect a file without a device (no reads then);
 * mimir_safetensors_error reports the message in that case. */
int mimir_safetensors_open(mimir_ctx* ctx, const char* path, mimir_safetensors** out);
int mimir_safetensors_close(mimir_safetensors* f);
/* Number of tensor entries (metadata excluded), -1 for NULL. */
int64_t mimir_safetensors_count(const mimir_safetensors* f);
/* Entry i: name (valid until close), dtype code, up to max_dims dims of its
 * shape, the number of dims and its byte size. */
int mimir_safetensors_entry(const mimir_safetensors* f, int64_t i, const char** name, int32_t* dtype,
                            int64_t* shape, int32_t max_dims, int32_t* ndims, int64_t* nbytes);
/* Index of the entry named `name`, or -1. */
int64_t mimir_safetensors_find(const mimir_safetensors* f, const char* name);
/* The last error of this file (also in mimir_last_error when it has a ctx);
 * with f == NULL, the message of this thread's last failed open. */
const char* mimir_safetensors_error(const mimir_safetensors* f);
/* Copy tensor `name`'s bytes into device memory (SafeTensorsReader::
 * load_tensor_data, :168-216); EINVAL if they exceed dst_bytes.  Returns
 * once the data is on the device. */
int mimir_safetensors_read(mimir_safetensors* f, const char* name, void* dst_device, size_t dst_bytes);
/* The weight loop of SafeTensorsReader::apply_tensors_to_model (:263-317):
 * for every layer with a weight block (weights != NULL, weights_len > 0),
 * tensor "<name>/weights" must have weights_len elements and is copied into
 * the layer's DEVICE weights; a missing tensor is skipped, or EINVAL
 * ("Missing tensor in strict mode: ...") when strict. */
int mimir_safetensors_load_layers(mimir_safetensors* f, const mimir_layer* layers, int32_t n_layers, int strict);

#ifdef __cplusplus
}
#endif

#endif /* MIMIR_HIP_H */
