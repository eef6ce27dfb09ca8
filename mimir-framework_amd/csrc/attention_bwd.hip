// attention_bwd.hip -- the gradient of the attention layers.
//
// Reference: backward_self_attention (Model.cpp:6847-7062) and
// backward_cross_attention (:7068-7300), called from Model::backwardPass's
// SelfAttention / MultiHeadAttention and CrossAttention branches
// (:8034-8127).  Per head h, with S = scale Q K^T (causal j > i masked to
// -1e9), P = softmax(S) (max from -1e30, inv = 1 / (sum + 1e-9)) and dO the
// gradient of the attended heads (dY Wout^T):
//   dV = P^T dO,   dP = dO V^T,   dS = P * (dP - rowsum(P * dP)) (masked: 0),
//   dQ = scale dS K,   dK = scale dS^T Q,
// then the projections' gradients dW += X^T dG and dX = dG W^T.
//
// The reference recomputes P from the layer's input and keeps it whole
// ([heads, q_len, kv_len]).  Here too: P and dS are materialised per group
// of heads in the context's scratch (capped at kWorkBytes, one head at
// least), the five per-head products run as strided-batched library GEMMs
// over the group's heads straight on the Q / K / V columns of the projection
// output (head h is the column block h*head_dim of each row, so consecutive
// heads sit head_dim floats apart), and the two row passes between them --
// mask + softmax, and the softmax backward -- are the kernels below, one wave
// per score row.  The gradients of Q, K and V land in place in one [rows,
// 3E] (or [rows, 2E]) buffer, the layout the weight-gradient product reads.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

#include <algorithm>
#include <cmath>

using namespace mimir;

namespace {

constexpr int kRowWaves = 4;  // score rows per 256-thread workgroup, one wave each
constexpr float kMaskedScore = -1e9f;
// Scratch cap for the materialised P and dS of one group of heads.
constexpr int64_t kWorkBytes = int64_t{1} << 30;

// Keys a row scores: causal row i sees keys 0..i (Model.cpp:6902, 7131).
__device__ __forceinline__ int live_keys(int64_t row, int32_t q_len, int32_t kv_len, int32_t causal) {
    const int i = static_cast<int>(row % q_len);
    return causal ? min(kv_len, i + 1) : kv_len;
}

// Mask + softmax of one score row in place: s_j -> p_j (Model.cpp:6892-6920).
// NV > 0: the row (at most 64*NV keys) is held in registers, key j in lane
// j % 64, slot j / 64.  NV == 0: any length, three passes over the row.
// Masked keys take -1e9 in the max, as in the reference, and exp(-1e9 - max)
// is 0, so their probability is written as 0 without reading them.
template <int NV>
__global__ __launch_bounds__(kRowWaves * kWave) void attn_probs_kernel(float* __restrict__ s, int64_t rows,
                                                                       int32_t q_len, int32_t kv_len,
                                                                       int32_t causal) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave;
    if (row >= rows) return;  // whole waves only: no barrier below
    const int lane = threadIdx.x & (kWave - 1);
    float* p = s + row * kv_len;
    const int live = live_keys(row, q_len, kv_len, causal);
    float m = live < kv_len ? kMaskedScore : -1e30f;
    float sum = 0.0f;
    if constexpr (NV > 0) {
        float e[NV];
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int j = lane + kWave * c;
            e[c] = j < live ? p[j] : -INFINITY;
            m = fmaxf(m, e[c]);
        }
        m = wave_max(m);
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            e[c] = expf(e[c] - m);
            sum += e[c];
        }
        const float inv = 1.0f / (wave_sum(sum) + 1e-9f);
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int j = lane + kWave * c;
            if (j < kv_len) p[j] = e[c] * inv;
        }
    } else {
        for (int j = lane; j < live; j += kWave) m = fmaxf(m, p[j]);
        m = wave_max(m);
        for (int j = lane; j < live; j += kWave) sum += expf(p[j] - m);
        const float inv = 1.0f / (wave_sum(sum) + 1e-9f);
        for (int j = lane; j < kv_len; j += kWave) p[j] = j < live ? expf(p[j] - m) * inv : 0.0f;
    }
}

// Softmax backward of one row in place: dp_j -> ds_j = (dp_j - sum_k p_k dp_k)
// p_j, masked keys 0 (Model.cpp:6991-7005; softmax_row_dot :6841-6845).  The
// masked keys' p is 0, so the dot runs over the live keys only.
template <int NV>
__global__ __launch_bounds__(kRowWaves * kWave) void attn_dsoftmax_kernel(const float* __restrict__ p_all,
                                                                          float* __restrict__ g, int64_t rows,
                                                                          int32_t q_len, int32_t kv_len,
                                                                          int32_t causal) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = threadIdx.x & (kWave - 1);
    const float* p = p_all + row * kv_len;
    float* d = g + row * kv_len;
    const int live = live_keys(row, q_len, kv_len, causal);
    float dot = 0.0f;
    if constexpr (NV > 0) {
        float pv[NV], dv[NV];
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int j = lane + kWave * c;
            pv[c] = j < live ? p[j] : 0.0f;
            dv[c] = j < live ? d[j] : 0.0f;
            dot += dv[c] * pv[c];
        }
        dot = wave_sum(dot);
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int j = lane + kWave * c;
            if (j < kv_len) d[j] = j < live ? (dv[c] - dot) * pv[c] : 0.0f;
        }
    } else {
        for (int j = lane; j < live; j += kWave) dot += d[j] * p[j];
        dot = wave_sum(dot);
        for (int j = lane; j < kv_len; j += kWave) d[j] = j < live ? (d[j] - dot) * p[j] : 0.0f;
    }
}

// The two row passes in one, for rows held in registers: mask + softmax of
// the score row s in place (attn_probs_kernel's arithmetic), then, with dP
// already in g, dS = (dP - sum_k p_k dP_k) p in place (attn_dsoftmax_kernel's,
// on the same p values it would read back).  The row's dP is loaded with its
// scores, so one read of each matrix and one write of each replace the two
// passes' three reads and two writes, with the same arithmetic in the
// same order.
template <int NV>
__global__ __launch_bounds__(kRowWaves * kWave) void attn_probs_dsoftmax_kernel(float* __restrict__ s,
                                                                                float* __restrict__ g, int64_t rows,
                                                                                int32_t q_len, int32_t kv_len,
                                                                                int32_t causal) {
    static_assert(NV > 0, "register rows only");
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave;
    if (row >= rows) return;  // whole waves only: no barrier below
    const int lane = threadIdx.x & (kWave - 1);
    float* p = s + row * kv_len;
    float* d = g + row * kv_len;
    const int live = live_keys(row, q_len, kv_len, causal);
    float m = live < kv_len ? kMaskedScore : -1e30f;
    float e[NV], dv[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int j = lane + kWave * c;
        e[c] = j < live ? p[j] : -INFINITY;
        dv[c] = j < live ? d[j] : 0.0f;
        m = fmaxf(m, e[c]);
    }
    m = wave_max(m);
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        e[c] = expf(e[c] - m);
        sum += e[c];
    }
    const float inv = 1.0f / (wave_sum(sum) + 1e-9f);
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int j = lane + kWave * c;
        e[c] = e[c] * inv;  // p_j, 0 for masked keys
        if (j < kv_len) p[j] = e[c];
        dot += dv[c] * (j < live ? e[c] : 0.0f);
    }
    dot = wave_sum(dot);
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int j = lane + kWave * c;
        if (j < kv_len) d[j] = j < live ? (dv[c] - dot) * e[c] : 0.0f;
    }
}

__global__ __launch_bounds__(kBlock) void zero_rows_kernel(float* __restrict__ y, int64_t rows, int64_t cols,
                                                           int64_t ld) {
    const int64_t n = rows * cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; t < n; t += stride)
        y[(t / cols) * ld + t % cols] = 0.0f;
}

// dst[t * ld + h * D + d] = src[(h * T + t) * D + d]: n heads' [T x D]
// blocks, stored one after another, into the rows of interleaved heads.
// Eight floats (two 16-byte vectors) per thread when D % 4 == 0 and the
// pointers and ld allow, else one float.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void heads_to_rows_kernel(const float* __restrict__ src, int64_t n, int64_t T,
                                                               int64_t D, float* __restrict__ dst, int64_t ld) {
    const int64_t w = VEC ? D / 4 : D;  // elements (vectors or floats) per head row
    const int64_t total = n * T * w;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride) {
        const int64_t h = i / (T * w), r = i % (T * w), t = r / w, c = r % w;
        if constexpr (VEC)
            *reinterpret_cast<f4*>(dst + t * ld + h * D + 4 * c) = reinterpret_cast<const f4*>(src)[i];
        else
            dst[t * ld + h * D + c] = src[i];
    }
}

int heads_to_rows(mimir_ctx* ctx, const float* src, int64_t n, int64_t T, int64_t D, float* dst, int64_t ld) {
    if (n == 0 || T == 0) return MIMIR_OK;
    const bool vec = D % 4 == 0 && ld % 4 == 0 && aligned16(src) && aligned16(dst);
    unsigned blocks = 0;
    if (!grid_for(n * T * (vec ? D / 4 : D), kBlock, kBlock, &blocks))
        return fail(ctx, MIMIR_EINVAL, "attention backward: grid too large");
    blocks = std::min(blocks, 16384u);
    if (vec)
        heads_to_rows_kernel<true><<<blocks, kBlock, 0, ctx->stream>>>(src, n, T, D, dst, ld);
    else
        heads_to_rows_kernel<false><<<blocks, kBlock, 0, ctx->stream>>>(src, n, T, D, dst, ld);
    return launched(ctx, "heads_to_rows_kernel");
}

// dst[c][r] = src[r][c] for a [rows x cols] block of rows ld_src apart; dst
// is [cols x rows] dense.  32 x 32 tiles through LDS (one padding column so
// the transposed reads hit distinct banks).
constexpr int kTile = 32;
__global__ __launch_bounds__(kTile * 8) void transpose_kernel(const float* __restrict__ src, int64_t ld_src,
                                                              int64_t rows, int64_t cols, float* __restrict__ dst) {
    __shared__ float t[kTile][kTile + 1];
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kTile, r0 = static_cast<int64_t>(blockIdx.y) * kTile;
    const int tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
    for (int i = ty; i < kTile; i += 8)
        if (r0 + i < rows && c0 + tx < cols) t[i][tx] = src[(r0 + i) * ld_src + c0 + tx];
    __syncthreads();
    for (int i = ty; i < kTile; i += 8)
        if (c0 + i < cols && r0 + tx < rows) dst[(c0 + i) * rows + r0 + tx] = t[tx][i];
}

int transpose(mimir_ctx* ctx, const float* src, int64_t ld_src, int64_t rows, int64_t cols, float* dst) {
    const int64_t gx = (cols + kTile - 1) / kTile, gy = (rows + kTile - 1) / kTile;
    if (!dispatch_fits(gx, kTile * 8) || gy > 65535)
        return fail(ctx, MIMIR_EINVAL, "attention backward: transpose grid too large");
    transpose_kernel<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)), kTile * 8, 0, ctx->stream>>>(
        src, ld_src, rows, cols, dst);
    return launched(ctx, "transpose_kernel");
}

int zero_rows(mimir_ctx* ctx, float* y, int64_t rows, int64_t cols, int64_t ld) {
    if (rows == 0 || cols == 0) return MIMIR_OK;
    unsigned blocks = 0;
    if (!grid_for(rows * cols, kBlock, kBlock, &blocks)) return fail(ctx, MIMIR_EINVAL, "attention: grid too large");
    zero_rows_kernel<<<std::min(blocks, 8192u), kBlock, 0, ctx->stream>>>(y, rows, cols, ld);
    return launched(ctx, "zero_rows_kernel");
}

int probs(mimir_ctx* ctx, float* s, int64_t rows, int32_t q_len, int32_t kv_len, int32_t causal) {
    unsigned blocks = 0;
    if (!grid_for(rows, kRowWaves, kRowWaves * kWave, &blocks)) return fail(ctx, MIMIR_EINVAL, "attention backward: grid too large");
    const dim3 grid(blocks), block(kRowWaves * kWave);
    if (kv_len <= 4 * kWave)
        attn_probs_kernel<4><<<grid, block, 0, ctx->stream>>>(s, rows, q_len, kv_len, causal);
    else if (kv_len <= 16 * kWave)
        attn_probs_kernel<16><<<grid, block, 0, ctx->stream>>>(s, rows, q_len, kv_len, causal);
    else if (kv_len <= 64 * kWave)
        attn_probs_kernel<64><<<grid, block, 0, ctx->stream>>>(s, rows, q_len, kv_len, causal);
    else
        attn_probs_kernel<0><<<grid, block, 0, ctx->stream>>>(s, rows, q_len, kv_len, causal);
    return launched(ctx, "attn_probs_kernel");
}

// Whether probs_dsoftmax applies: rows the register forms hold.
bool fused_rows(int32_t kv_len) { return kv_len <= 64 * kWave; }

int probs_dsoftmax(mimir_ctx* ctx, float* s, float* g, int64_t rows, int32_t q_len, int32_t kv_len,
                   int32_t causal) {
    unsigned blocks = 0;
    if (!grid_for(rows, kRowWaves, kRowWaves * kWave, &blocks)) return fail(ctx, MIMIR_EINVAL, "attention backward: grid too large");
    const dim3 grid(blocks), block(kRowWaves * kWave);
    if (kv_len <= 4 * kWave)
        attn_probs_dsoftmax_kernel<4><<<grid, block, 0, ctx->stream>>>(s, g, rows, q_len, kv_len, causal);
    else if (kv_len <= 16 * kWave)
        attn_probs_dsoftmax_kernel<16><<<grid, block, 0, ctx->stream>>>(s, g, rows, q_len, kv_len, causal);
    else
        attn_probs_dsoftmax_kernel<64><<<grid, block, 0, ctx->stream>>>(s, g, rows, q_len, kv_len, causal);
    return launched(ctx, "attn_probs_dsoftmax_kernel");
}

int dsoftmax(mimir_ctx* ctx, const float* p, float* g, int64_t rows, int32_t q_len, int32_t kv_len,
             int32_t causal) {
    unsigned blocks = 0;
    if (!grid_for(rows, kRowWaves, kRowWaves * kWave, &blocks)) return fail(ctx, MIMIR_EINVAL, "attention backward: grid too large");
    const dim3 grid(blocks), block(kRowWaves * kWave);
    if (kv_len <= 4 * kWave)
        attn_dsoftmax_kernel<4><<<grid, block, 0, ctx->stream>>>(p, g, rows, q_len, kv_len, causal);
    else if (kv_len <= 16 * kWave)
        attn_dsoftmax_kernel<16><<<grid, block, 0, ctx->stream>>>(p, g, rows, q_len, kv_len, causal);
    else if (kv_len <= 64 * kWave)
        attn_dsoftmax_kernel<64><<<grid, block, 0, ctx->stream>>>(p, g, rows, q_len, kv_len, causal);
    else
        attn_dsoftmax_kernel<0><<<grid, block, 0, ctx->stream>>>(p, g, rows, q_len, kv_len, causal);
    return launched(ctx, "attn_dsoftmax_kernel");
}

// One backward of the core.  att (optional): also write the attended heads
// P V, which the layers' output-projection gradient reads.
struct CoreBwd {
    const float* q;
    int64_t ld_q;
    const float* k;
    const float* v;
    int64_t ld_kv;
    const float* dout;
    int64_t ld_dout;
    float* dq;
    int64_t ld_dq;
    float* dk;
    float* dv;
    int64_t ld_dkv;
    float* att;
    int64_t ld_att;
    int64_t batch, q_len, kv_len, heads, head_dim;
    float scale;
    int causal;
};

// Heads per group (a tuning override may lower it), and the scratch floats
// of one group (P and dS).
int64_t heads_per_group(const mimir_ctx* ctx, const CoreBwd& a) {
    const int64_t per_head = 2 * a.q_len * a.kv_len * static_cast<int64_t>(sizeof(float));
    int64_t hc = std::min<int64_t>(a.heads, kWorkBytes / std::max<int64_t>(per_head, 1));
    if (ctx->tune.attn_bwd_heads > 0) hc = std::min<int64_t>(hc, ctx->tune.attn_bwd_heads);
    return std::max<int64_t>(1, hc);
}
// P and dS of a head group, then either the group's dQ / dK / dV in head-
// major blocks (hipBLASLt) or K^T and V^T of a sequence (rocBLAS only).
int64_t work_floats(mimir_ctx* ctx, const CoreBwd& a) {
    const int64_t hc = heads_per_group(ctx, a);
    return 2 * hc * a.q_len * a.kv_len + (gemm_lt(ctx) ? hc * a.head_dim * (a.q_len + 2 * a.kv_len)
                                                       : 2 * a.heads * a.head_dim * a.kv_len);
}

int core_bwd(mimir_ctx* ctx, const CoreBwd& a, float* work) {
    const int64_t D = a.head_dim, Tq = a.q_len, Tk = a.kv_len, TT = Tq * Tk;
    if (a.batch == 0 || Tq == 0) return MIMIR_OK;
    if (Tk == 0) {  // no keys: the attended heads and dQ are 0, dK / dV empty
        for (int64_t b = 0; b < a.batch; ++b) {
            if (int st = zero_rows(ctx, a.dq + b * Tq * a.ld_dq, Tq, a.heads * D, a.ld_dq)) return st;
            if (a.att)
                if (int st = zero_rows(ctx, a.att + b * Tq * a.ld_att, Tq, a.heads * D, a.ld_att)) return st;
        }
        return MIMIR_OK;
    }
    const int64_t hc = heads_per_group(ctx, a);
    const int64_t width = a.heads * D;
    float* P = work;
    float* G = work + hc * TT;
    // The score products S = Q K^T and dP = dO V^T read K and V in place as
    // transposed operands through hipBLASLt.  With rocBLAS only, whose
    // transposed-operand form runs at about half the plain one's rate on
    // these shapes, they read K^T and V^T of the sequence, [width x kv_len],
    // as plain (NN) operands.  hipBLASLt writes the group's dQ, dK and dV as
    // head-major [n][T][D] blocks (batches that do not overlap, which its
    // split reductions need), copied into the interleaved heads after.
    const bool lt = gemm_lt(ctx);
    float* KT = G + hc * TT;
    float* VT = KT + width * Tk;
    float* SQ = G + hc * TT;
    float* SK = SQ + hc * Tq * D;
    float* SV = SK + hc * Tk * D;
    // Causal: the products may run over blocks of bq queries (S, P V, dP,
    // dQ) or bk keys (dV, dK), so the key columns past a query block's
    // diagonal -- masked, P = dS = 0 there -- are not multiplied ((nblk + 1)
    // / (2 nblk) of the full work).  Measured at 32 heads of 1024 x 1024 x
    // 128: hipBLASLt keeps its rate on two query blocks for S and dP (3/4 of
    // the work in 77 us, against 92 us whole), rocBLAS runs the query-side dQ
    // faster on two blocks (80 against 87 us) but the key-side products
    // slower (110 against 85 us); rocBLAS's plain S is slower on any split.
    // hipBLASLt takes dV / dK on two key blocks in 62 us and dQ on two query
    // blocks in 64 us.  A tuning override sets one count for all.
    auto block_size = [&](int64_t want) {
        const int64_t nblk = a.causal ? std::max<int64_t>(1, std::min<int64_t>(want, Tq / 256)) : 1;
        return nblk > 1 ? ((Tq + nblk - 1) / nblk + 63) / 64 * 64 : std::max(Tq, Tk);
    };
    const int64_t over = ctx->tune.attn_bwd_blocks;
    const int64_t bq = block_size(over > 0 ? over : (lt ? 2 : 1));  // S, P V, dP
    const int64_t bdq = block_size(over > 0 ? over : 2);            // dQ
    const int64_t bk = block_size(over > 0 ? over : (lt ? 2 : 1));  // dV, dK
    auto live = [&](int64_t q1) { return a.causal ? std::min(q1, Tk) : Tk; };  // keys queries < q1 see
    for (int64_t b = 0; b < a.batch; ++b) {
        const float* qb = a.q + b * Tq * a.ld_q;
        const float* kb = a.k + b * Tk * a.ld_kv;
        const float* vb = a.v + b * Tk * a.ld_kv;
        const float* ob = a.dout + b * Tq * a.ld_dout;
        float* dqb = a.dq + b * Tq * a.ld_dq;
        float* dkb = a.dk + b * Tk * a.ld_dkv;
        float* dvb = a.dv + b * Tk * a.ld_dkv;
        float* attb = a.att ? a.att + b * Tq * a.ld_att : nullptr;
        if (!lt) {
            if (int st = transpose(ctx, kb, a.ld_kv, Tk, width, KT)) return st;
            if (int st = transpose(ctx, vb, a.ld_kv, Tk, width, VT)) return st;
        }
        for (int64_t h0 = 0; h0 < a.heads; h0 += hc) {
            const int64_t n = std::min(hc, a.heads - h0), off = h0 * D;
            const int64_t rows = n * Tq;
            const auto q32 = static_cast<int32_t>(Tq), k32 = static_cast<int32_t>(Tk);
            // Row-blocked products (S, attended, dP, dQ): query block [q0, q1)
            // reads keys [0, live(q1)).
            for (int64_t q0 = 0; q0 < Tq; q0 += bq) {
                const int64_t m = std::min(bq, Tq - q0), kl = live(q0 + m);
                // S = scale Q K^T (:6892-6905)
                if (int st = lt ? gemm_f32_ex(ctx, false, true, m, kl, D, a.scale, qb + q0 * a.ld_q + off, a.ld_q, D,
                                              kb + off, a.ld_kv, D, 0.0f, P + q0 * Tk, Tk, TT, n)
                                : gemm_f32_ex(ctx, false, false, m, kl, D, a.scale, qb + q0 * a.ld_q + off, a.ld_q, D,
                                              KT + off * Tk, Tk, D * Tk, 0.0f, P + q0 * Tk, Tk, TT, n))
                    return st;
            }
            // P = softmax(mask(S)) in place (:6906-6920) and dS in place
            // (:6991-7005); every key column of both is written (0 where
            // masked), so the key-blocked products below may read whole
            // columns of a block.  Rows held in registers take both passes in
            // one kernel after dP; longer rows take them one before and one
            // after it.
            const bool fuse = fused_rows(k32);
            if (!fuse)
                if (int st = probs(ctx, P, rows, q32, k32, a.causal)) return st;
            auto attended = [&](int64_t q0, int64_t m, int64_t kl) {  // attended = P V (:6922-6930)
                return gemm_f32_ex(ctx, false, false, m, D, kl, 1.0f, P + q0 * Tk, Tk, TT, vb + off, a.ld_kv, D, 0.0f,
                                   attb + q0 * a.ld_att + off, a.ld_att, D, n);
            };
            for (int64_t q0 = 0; q0 < Tq; q0 += bq) {
                const int64_t m = std::min(bq, Tq - q0), kl = live(q0 + m);
                if (attb && !fuse)
                    if (int st = attended(q0, m, kl)) return st;
                // dP = dO V^T (:6979-6989)
                if (int st = lt ? gemm_f32_ex(ctx, false, true, m, kl, D, 1.0f, ob + q0 * a.ld_dout + off, a.ld_dout,
                                              D, vb + off, a.ld_kv, D, 0.0f, G + q0 * Tk, Tk, TT, n)
                                : gemm_f32_ex(ctx, false, false, m, kl, D, 1.0f, ob + q0 * a.ld_dout + off, a.ld_dout,
                                              D, VT + off * Tk, Tk, D * Tk, 0.0f, G + q0 * Tk, Tk, TT, n))
                    return st;
            }
            if (fuse) {
                if (int st = probs_dsoftmax(ctx, P, G, rows, q32, k32, a.causal)) return st;
                if (attb)
                    for (int64_t q0 = 0; q0 < Tq; q0 += bq) {
                        const int64_t m = std::min(bq, Tq - q0);
                        if (int st = attended(q0, m, live(q0 + m))) return st;
                    }
            } else if (int st = dsoftmax(ctx, P, G, rows, q32, k32, a.causal)) {
                return st;
            }
            for (int64_t q0 = 0; q0 < Tq; q0 += bdq) {  // dQ = scale dS K (:7007-7016)
                const int64_t m = std::min(bdq, Tq - q0), kl = live(q0 + m);
                if (int st = lt ? gemm_f32_ex(ctx, false, false, m, D, kl, a.scale, G + q0 * Tk, Tk, TT, kb + off,
                                              a.ld_kv, D, 0.0f, SQ + q0 * D, D, Tq * D, n)
                                : gemm_f32_ex(ctx, false, false, m, D, kl, a.scale, G + q0 * Tk, Tk, TT, kb + off,
                                              a.ld_kv, D, 0.0f, dqb + q0 * a.ld_dq + off, a.ld_dq, D, n))
                    return st;
            }
            if (lt)
                if (int st = heads_to_rows(ctx, SQ, n, Tq, D, dqb + off, a.ld_dq)) return st;
            // Key-blocked products (dV, dK): key block [k0, k1) is seen by
            // queries [first(k0), Tq); a block no query sees gets zeros.
            for (int64_t k0 = 0; k0 < Tk; k0 += bk) {
                const int64_t m = std::min(bk, Tk - k0), qs = a.causal ? k0 : 0;
                if (qs >= Tq) {
                    if (!lt) {
                        if (int st = zero_rows(ctx, dvb + k0 * a.ld_dkv + off, m, n * D, a.ld_dkv)) return st;
                        if (int st = zero_rows(ctx, dkb + k0 * a.ld_dkv + off, m, n * D, a.ld_dkv)) return st;
                        continue;
                    }
                    for (int64_t h = 0; h < n; ++h) {  // the head-major blocks' rows
                        if (int st = zero_rows(ctx, SV + (h * Tk + k0) * D, m, D, D)) return st;
                        if (int st = zero_rows(ctx, SK + (h * Tk + k0) * D, m, D, D)) return st;
                    }
                    continue;
                }
                float* dvo = lt ? SV + k0 * D : dvb + k0 * a.ld_dkv + off;
                float* dko = lt ? SK + k0 * D : dkb + k0 * a.ld_dkv + off;
                const int64_t ldo = lt ? D : a.ld_dkv, so = lt ? Tk * D : D;
                // dV = P^T dO (:6967-6977)
                if (int st = gemm_f32_ex(ctx, true, false, m, D, Tq - qs, 1.0f, P + qs * Tk + k0, Tk, TT,
                                         ob + qs * a.ld_dout + off, a.ld_dout, D, 0.0f, dvo, ldo, so, n))
                    return st;
                // dK = scale dS^T Q (:7018-7028)
                if (int st = gemm_f32_ex(ctx, true, false, m, D, Tq - qs, a.scale, G + qs * Tk + k0, Tk, TT,
                                         qb + qs * a.ld_q + off, a.ld_q, D, 0.0f, dko, ldo, so, n))
                    return st;
            }
            if (lt) {
                if (int st = heads_to_rows(ctx, SV, n, Tk, D, dvb + off, a.ld_dkv)) return st;
                if (int st = heads_to_rows(ctx, SK, n, Tk, D, dkb + off, a.ld_dkv)) return st;
            }
        }
    }
    return MIMIR_OK;
}

int check_core(mimir_ctx* ctx, const CoreBwd& a) {
    MIMIR_REQUIRE(ctx, a.batch >= 0 && a.q_len >= 0 && a.kv_len >= 0 && a.heads >= 1 && a.head_dim >= 1,
                  "attention backward: invalid shape (batch=%lld q_len=%lld kv_len=%lld heads=%lld head_dim=%lld)",
                  (long long)a.batch, (long long)a.q_len, (long long)a.kv_len, (long long)a.heads,
                  (long long)a.head_dim);
    const int64_t width = a.heads * a.head_dim;
    MIMIR_REQUIRE(ctx, a.ld_q >= width && a.ld_kv >= width && a.ld_dout >= width && a.ld_dq >= width &&
                           a.ld_dkv >= width,
                  "attention backward: row strides below heads * head_dim = %lld", (long long)width);
    MIMIR_REQUIRE(ctx, a.q_len < (int64_t{1} << 30) && a.kv_len < (int64_t{1} << 30) && width <= INT32_MAX,
                  "attention backward: sequence or width too large");
    MIMIR_REQUIRE(ctx, std::isfinite(a.scale), "attention backward: scale must be finite");
    return MIMIR_OK;
}

}  // namespace

extern "C" {

int mimir_attention_bwd(mimir_ctx* ctx, const float* q, int64_t ld_q, const float* k, const float* v,
                        int64_t ld_kv, const float* dout, int64_t ld_dout, float* dq, int64_t ld_dq, float* dk,
                        float* dv, int64_t ld_dkv, int64_t batch, int64_t q_len, int64_t kv_len, int64_t heads,
                        int64_t head_dim, float scale, int causal) {
    if (!ctx) return MIMIR_EINVAL;
    const CoreBwd a{q, ld_q, k, v, ld_kv, dout, ld_dout, dq, ld_dq, dk, dv, ld_dkv, nullptr, 0,
                    batch, q_len, kv_len, heads, head_dim, scale, causal ? 1 : 0};
    if (int st = check_core(ctx, a)) return st;
    if (batch == 0 || q_len == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, q && dout && dq && (kv_len == 0 || (k && v && dk && dv)), "attention backward: null pointer");
    MIMIR_ENTER(ctx);
    void* w = nullptr;
    if (kv_len > 0)
        if (int st = ensure_scratch(ctx, sizeof(float) * static_cast<size_t>(work_floats(ctx, a)), &w)) return st;
    return core_bwd(ctx, a, static_cast<float*>(w));
}

// backward_self_attention (Model.cpp:6847-7062): qkv = x Wqkv; the core's
// backward on dAtt = dY Wout^T; dWout += att^T dY; dWqkv += x^T dqkv;
// dx = dqkv Wqkv^T.  Scratch: qkv [T, 3E], att [T, E], dAtt [T, E],
// dqkv [T, 3E], then the core's P / dS.  grad_input is written last, so it
// may be grad_out's own buffer (the reference adds dx into grad_store, which
// holds grad_out when the layer's input and output share a name).
int mimir_self_attention_bwd(mimir_ctx* ctx, const float* input, const float* grad_out, int64_t seq_len,
                             int64_t embed_dim, int64_t num_heads, int causal, const float* weights,
                             int64_t weights_len, float* grad_weights, float* grad_input, int accumulate) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, embed_dim >= 1 && num_heads >= 1 && embed_dim % num_heads == 0,
                  "SelfAttention backward: embed_dim must be divisible by num_heads");
    MIMIR_REQUIRE(ctx, seq_len >= 0, "SelfAttention backward: invalid seq_len");
    const int64_t e = embed_dim, T = seq_len;
    MIMIR_REQUIRE(ctx, weights_len >= 4 * e * e, "SelfAttention backward: weight block of %lld floats, %lld needed",
                  (long long)weights_len, (long long)(4 * e * e));
    if (T == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, input && grad_out && weights && grad_input, "SelfAttention backward: null pointer");
    const int64_t hd = e / num_heads;
    const float* wqkv = weights;
    const float* wout = weights + 3 * e * e;
    CoreBwd a{nullptr, 3 * e, nullptr, nullptr, 3 * e, nullptr, e, nullptr, 3 * e, nullptr, nullptr, 3 * e,
              nullptr, e, 1, T, T, num_heads, hd, 1.0f / std::sqrt(static_cast<float>(hd)), causal ? 1 : 0};
    if (int st = check_core(ctx, a)) return st;
    MIMIR_ENTER(ctx);
    const int64_t acts = 8 * T * e;
    void* s = nullptr;
    if (int st = ensure_scratch(ctx, sizeof(float) * static_cast<size_t>(acts + work_floats(ctx, a)), &s)) return st;
    float* qkv = static_cast<float*>(s);
    float* att = qkv + 3 * T * e;
    float* datt = att + T * e;
    float* dqkv = datt + T * e;
    a.q = qkv;
    a.k = qkv + e;
    a.v = qkv + 2 * e;
    a.dout = datt;
    a.dq = dqkv;
    a.dk = dqkv + e;
    a.dv = dqkv + 2 * e;
    a.att = att;
    if (int st = gemm_f32(ctx, T, 3 * e, e, input, e, wqkv, 3 * e, qkv, 3 * e)) return st;  // :6868-6880
    if (int st = gemm_f32_ex(ctx, false, true, T, e, e, 1.0f, grad_out, e, 0, wout, e, 0, 0.0f, datt, e, 0, 1))
        return st;  // :6935-6947
    if (int st = core_bwd(ctx, a, qkv + acts)) return st;
    if (grad_weights) {
        if (int st = gemm_f32_ex(ctx, true, false, e, e, T, 1.0f, att, e, 0, grad_out, e, 0, 1.0f,
                                 grad_weights + 3 * e * e, e, 0, 1))
            return st;  // dWout, :6949-6958
        if (int st = gemm_f32_ex(ctx, true, false, e, 3 * e, T, 1.0f, input, e, 0, dqkv, 3 * e, 0, 1.0f, grad_weights,
                                 3 * e, 0, 1))
            return st;  // dWqkv, :7041-7050
    }
    // dx, :7052-7061
    return gemm_f32_ex(ctx, false, true, T, e, 3 * e, 1.0f, dqkv, 3 * e, 0, wqkv, 3 * e, 0, accumulate ? 1.0f : 0.0f,
                       grad_input, e, 0, 1);
}

// backward_cross_attention (Model.cpp:7068-7300): Q = xq Wq, KV = xkv Wkv;
// the core's backward on dAtt = dY Wout^T; dWout += att^T dY; dWq += xq^T dQ,
// dxq = dQ Wq^T; dWkv += xkv^T dKV, dxkv = dKV Wkv^T, in that order (the
// input gradients last, dxq before dxkv, so either may be grad_out's buffer
// and both may be one buffer, as when the two inputs share a name).
int mimir_cross_attention_bwd(mimir_ctx* ctx, const float* query_input, int64_t query_len, const float* kv_input,
                              int64_t kv_len, const float* grad_out, int64_t embed_dim, int64_t num_heads,
                              int causal, const float* weights, int64_t weights_len, float* grad_weights,
                              float* grad_query, int accumulate_query, float* grad_kv, int accumulate_kv) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, embed_dim >= 1 && num_heads >= 1 && embed_dim % num_heads == 0,
                  "CrossAttention backward: embed_dim must be divisible by num_heads");
    MIMIR_REQUIRE(ctx, query_len > 0 && kv_len > 0, "CrossAttention backward: invalid dimensions");
    const int64_t e = embed_dim, Tq = query_len, Tk = kv_len;
    MIMIR_REQUIRE(ctx, weights_len >= 4 * e * e, "CrossAttention backward: weight block of %lld floats, %lld needed",
                  (long long)weights_len, (long long)(4 * e * e));
    MIMIR_REQUIRE(ctx, query_input && kv_input && grad_out && weights && grad_query && grad_kv,
                  "CrossAttention backward: null pointer");
    const int64_t hd = e / num_heads;
    const float* wq = weights;
    const float* wkv = weights + e * e;
    const float* wout = weights + 3 * e * e;
    CoreBwd a{nullptr, e, nullptr, nullptr, 2 * e, nullptr, e, nullptr, e, nullptr, nullptr, 2 * e,
              nullptr, e, 1, Tq, Tk, num_heads, hd, 1.0f / std::sqrt(static_cast<float>(hd)), causal ? 1 : 0};
    if (int st = check_core(ctx, a)) return st;
    MIMIR_ENTER(ctx);
    const int64_t acts = 4 * Tq * e + 4 * Tk * e;
    void* s = nullptr;
    if (int st = ensure_scratch(ctx, sizeof(float) * static_cast<size_t>(acts + work_floats(ctx, a)), &s)) return st;
    float* qp = static_cast<float*>(s);  // [Tq, E]
    float* att = qp + Tq * e;           // [Tq, E]
    float* datt = att + Tq * e;         // [Tq, E]
    float* dqp = datt + Tq * e;         // [Tq, E]
    float* kv = dqp + Tq * e;           // [Tk, 2E]
    float* dkv = kv + 2 * Tk * e;       // [Tk, 2E]
    a.q = qp;
    a.k = kv;
    a.v = kv + e;
    a.dout = datt;
    a.dq = dqp;
    a.dk = dkv;
    a.dv = dkv + e;
    a.att = att;
    if (int st = gemm_f32(ctx, Tq, e, e, query_input, e, wq, e, qp, e)) return st;           // :7095-7105
    if (int st = gemm_f32(ctx, Tk, 2 * e, e, kv_input, e, wkv, 2 * e, kv, 2 * e)) return st;  // :7106-7116
    if (int st = gemm_f32_ex(ctx, false, true, Tq, e, e, 1.0f, grad_out, e, 0, wout, e, 0, 0.0f, datt, e, 0, 1))
        return st;  // :7163-7174
    if (int st = core_bwd(ctx, a, qp + acts)) return st;
    if (grad_weights) {
        if (int st = gemm_f32_ex(ctx, true, false, e, e, Tq, 1.0f, att, e, 0, grad_out, e, 0, 1.0f,
                                 grad_weights + 3 * e * e, e, 0, 1))
            return st;  // dWout, :7175-7184
        if (int st = gemm_f32_ex(ctx, true, false, e, e, Tq, 1.0f, query_input, e, 0, dqp, e, 0, 1.0f, grad_weights, e,
                                 0, 1))
            return st;  // dWq, :7249-7258
    }
    if (int st = gemm_f32_ex(ctx, false, true, Tq, e, e, 1.0f, dqp, e, 0, wq, e, 0, accumulate_query ? 1.0f : 0.0f,
                             grad_query, e, 0, 1))
        return st;  // dxq, :7259-7268
    if (grad_weights)
        if (int st = gemm_f32_ex(ctx, true, false, e, 2 * e, Tk, 1.0f, kv_input, e, 0, dkv, 2 * e, 0, 1.0f,
                                 grad_weights + e * e, 2 * e, 0, 1))
            return st;  // dWkv, :7279-7288
    return gemm_f32_ex(ctx, false, true, Tk, e, 2 * e, 1.0f, dkv, 2 * e, 0, wkv, 2 * e, 0,
                       accumulate_kv ? 1.0f : 0.0f, grad_kv, e, 0, 1);  // dxkv, :7290-7300
}

}  // extern "C"
