// rope.hip -- rotary position embedding (rotate-half form) for gfx950, with
// q and k processed by one launch.
//
// The reference has no RoPE; the convention is the RoFormer / GPT-NeoX
// "rotate-half" one: for a head row x of D floats at position p and pair
// i < D/2, y[i] = x[i]*cos(p*f_i) - x[i+D/2]*sin(p*f_i),
// y[i+D/2] = x[i+D/2]*cos(p*f_i) + x[i]*sin(p*f_i), f_i = theta^(-2i/D).
// cos/sin come from a [rows x D/2] fp32 table built on the host in double
// (mimir_rope_table), which stays L2-resident while q and k stream through.
//
// Work unit ("slot"): 4 consecutive pairs of one head row -- a 16-byte vector
// from the first half, the matching one from the second half, and the two
// table vectors.  Q = D/8 slots per head row; q's slots come first, then k's.
// Each thread handles PPT slots spaced one workgroup-width apart (PPT = 4 by
// default), so a wave instruction reads 4 head rows' half-rows (4 x 256 B
// for D = 128).
#include "common.hpp"
#include "fastdiv.hpp"
#include "internal.hpp"

#include <math.h>

using namespace mimir;

namespace {

struct RopeArgs {
    const float* q;
    float* q_out;
    const float* k;
    float* k_out;
    const float* cos_tab;
    const float* sin_tab;
    uint32_t q_heads;
    uint32_t k_heads;
    uint32_t seq;
    uint32_t half;        // D / 2
    FastDiv q_div, k_div, seq_div;  // the same three divisors for the vector kernel (rows < 2^32)
    int64_t q_slots;      // q head rows * Q
    int64_t total_slots;  // (q + k head rows) * Q
    int64_t pos_offset;
};

__device__ __forceinline__ void rotate(f4& x0, f4& x1, f4 c, f4 s) {
    const f4 y0 = x0 * c - x1 * s;
    const f4 y1 = x1 * c + x0 * s;
    x0 = y0;
    x1 = y1;
}

// KEEP: outputs through the caches (mimir_ctx_set_output_caching).
// BS: the workgroup size (rows.hpp rope_block).
template <int LOG2Q, int PPT, bool KEEP, int BS = kBlock>
__global__ __launch_bounds__(BS) void rope_vec(RopeArgs a) {
    constexpr int Q = 1 << LOG2Q;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * PPT * BS + threadIdx.x;
    const int64_t D = 2 * static_cast<int64_t>(a.half);
    f4 x0[PPT], x1[PPT], c[PPT], s[PPT];
    float* out[PPT];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        const int64_t slot = first + static_cast<int64_t>(j) * BS;
        out[j] = nullptr;
        if (slot < a.total_slots) {
            const bool is_q = slot < a.q_slots;
            const int64_t local = is_q ? slot : slot - a.q_slots;
            const uint32_t hr = static_cast<uint32_t>(local >> LOG2Q);  // head row (the host checks < 2^32)
            const int64_t i4 = 4 * (local & (Q - 1));                   // first pair of the slot
            const uint32_t tok = fastdiv(hr, is_q ? a.q_div : a.k_div);
            const int64_t pos = a.pos_offset + static_cast<int64_t>(fastmod(tok, a.seq_div));
            const float* src = (is_q ? a.q : a.k) + static_cast<int64_t>(hr) * D + i4;
            out[j] = (is_q ? a.q_out : a.k_out) + static_cast<int64_t>(hr) * D + i4;
            x0[j] = ld4<true>(src);
            x1[j] = ld4<true>(src + a.half);
            c[j] = *reinterpret_cast<const f4*>(a.cos_tab + pos * a.half + i4);
            s[j] = *reinterpret_cast<const f4*>(a.sin_tab + pos * a.half + i4);
        }
    }
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
        if (out[j]) {
            rotate(x0[j], x1[j], c[j], s[j]);
            // Write-through stores: RoPE writes as much as it reads.
            st_out<KEEP, kStoreThrough>(out[j], x0[j]);
            st_out<KEEP, kStoreThrough>(out[j] + a.half, x1[j]);
        }
    }
}

// Any head_dim / alignment: one thread per pair.
__global__ __launch_bounds__(kBlock) void rope_scalar(RopeArgs a, int64_t q_pairs, int64_t total_pairs) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t D = 2 * static_cast<int64_t>(a.half);
    for (int64_t p = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; p < total_pairs; p += stride) {
        const bool is_q = p < q_pairs;
        const int64_t local = is_q ? p : p - q_pairs;
        const int64_t hr = local / a.half;
        const int64_t i = local % a.half;
        const int64_t tok = hr / (is_q ? a.q_heads : a.k_heads);
        const int64_t pos = a.pos_offset + tok % a.seq;
        const float* src = (is_q ? a.q : a.k) + hr * D;
        float* dst = (is_q ? a.q_out : a.k_out) + hr * D;
        const float x0 = src[i];
        const float x1 = src[i + a.half];
        const float cv = a.cos_tab[pos * a.half + i];
        const float sv = a.sin_tab[pos * a.half + i];
        dst[i] = x0 * cv - x1 * sv;
        dst[i + a.half] = x1 * cv + x0 * sv;
    }
}

template <int LOG2Q, int PPT>
int launch_ppt(mimir_ctx* ctx, const RopeArgs& a) {
    return with_block(rope_block(ctx->tune), [&](auto bsc) {
        constexpr int BS = decltype(bsc)::value;
        unsigned blocks;
        if (!grid_for(a.total_slots, static_cast<int64_t>(PPT) * BS, BS, &blocks))
            return fail(ctx, MIMIR_EINVAL, "RoPE: tensor exceeds the grid limit");
        if (ctx->keep_outputs) rope_vec<LOG2Q, PPT, true, BS><<<blocks, BS, 0, ctx->stream>>>(a);
        else rope_vec<LOG2Q, PPT, false, BS><<<blocks, BS, 0, ctx->stream>>>(a);
        return launched(ctx, "rope_vec");
    });
}

// Four slots per thread (a workgroup-width apart) measured best on MI355X at
// configs[3] (332 us against 334 us for one and 341 us for two); 1 and 2
// stay for sweeps (MIMIR_TUNE rope=1 / rope=2).
template <int LOG2Q>
int launch_vec(mimir_ctx* ctx, const RopeArgs& a) {
    switch (ctx->tune.rope_ppt) {
        case 1: return launch_ppt<LOG2Q, 1>(ctx, a);
        case 2: return launch_ppt<LOG2Q, 2>(ctx, a);
        default: return launch_ppt<LOG2Q, 4>(ctx, a);
    }
}

}  // namespace

extern "C" {

int mimir_rope_table(int64_t rows, int64_t head_dim, double theta, float* cos_tab,
                     float* sin_tab) {
    if (rows < 0 || head_dim <= 0 || (head_dim & 1) || !(theta > 0.0)) return MIMIR_EINVAL;
    if (rows > 0 && (!cos_tab || !sin_tab)) return MIMIR_EINVAL;
    const int64_t half = head_dim / 2;
    for (int64_t p = 0; p < rows; ++p) {
        for (int64_t i = 0; i < half; ++i) {
            const double inv_freq = 1.0 / pow(theta, static_cast<double>(2 * i) / static_cast<double>(head_dim));
            const double ang = static_cast<double>(p) * inv_freq;
            cos_tab[p * half + i] = static_cast<float>(cos(ang));
            sin_tab[p * half + i] = static_cast<float>(sin(ang));
        }
    }
    return MIMIR_OK;
}

int mimir_rope_fwd(mimir_ctx* ctx, const float* q, float* q_out, int64_t q_heads, const float* k,
                   float* k_out, int64_t k_heads, int64_t batch, int64_t seq, int64_t head_dim,
                   int64_t pos_offset, const float* cos_tab, const float* sin_tab,
                   int64_t table_rows) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, batch >= 0 && seq >= 0 && q_heads >= 0 && head_dim > 0 && (head_dim % 2) == 0,
                  "RoPE: invalid shape (batch=%lld seq=%lld heads=%lld head_dim=%lld)", (long long)batch,
                  (long long)seq, (long long)q_heads, (long long)head_dim);
    MIMIR_REQUIRE(ctx, !k || k_heads >= 0, "RoPE: k_heads < 0");
    MIMIR_REQUIRE(ctx, pos_offset >= 0 && (seq == 0 || pos_offset + seq <= table_rows),
                  "RoPE: positions [%lld, %lld) exceed the %lld-row table", (long long)pos_offset,
                  (long long)(pos_offset + seq), (long long)table_rows);
    const int64_t qh = q ? q_heads : 0;
    const int64_t kh = k ? k_heads : 0;
    const int64_t q_rows = batch * seq * qh;
    const int64_t k_rows = batch * seq * kh;
    if (q_rows + k_rows == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, cos_tab && sin_tab && (!q || q_out) && (!k || k_out), "RoPE: null tensor");
    MIMIR_REQUIRE(ctx, q_rows + k_rows < (int64_t(1) << 32) && qh < (int64_t(1) << 31) &&
                           kh < (int64_t(1) << 31) && seq < (int64_t(1) << 31),
                  "RoPE: tensor too large");
    MIMIR_ENTER(ctx);
    const int64_t half = head_dim / 2;
    RopeArgs a{q, q_out, k, k_out, cos_tab, sin_tab,
               static_cast<uint32_t>(qh ? qh : 1), static_cast<uint32_t>(kh ? kh : 1),
               static_cast<uint32_t>(seq), static_cast<uint32_t>(half), {}, {}, {}, 0, 0, pos_offset};
    a.q_div = make_fastdiv(a.q_heads);
    a.k_div = make_fastdiv(a.k_heads);
    a.seq_div = make_fastdiv(a.seq ? a.seq : 1);
    bool vec = (half % 4) == 0 && aligned16(cos_tab) && aligned16(sin_tab) &&
               (!q || (aligned16(q) && aligned16(q_out))) && (!k || (aligned16(k) && aligned16(k_out)));
    const int64_t Q = half / 4;
    if (vec && Q >= 1 && Q <= 64 && (Q & (Q - 1)) == 0) {
        a.q_slots = q_rows * Q;
        a.total_slots = (q_rows + k_rows) * Q;
        switch (Q) {
            case 1: return launch_vec<0>(ctx, a);
            case 2: return launch_vec<1>(ctx, a);
            case 4: return launch_vec<2>(ctx, a);
            case 8: return launch_vec<3>(ctx, a);
            case 16: return launch_vec<4>(ctx, a);
            case 32: return launch_vec<5>(ctx, a);
            default: return launch_vec<6>(ctx, a);
        }
    }
    const int64_t q_pairs = q_rows * half;
    const int64_t total = (q_rows + k_rows) * half;
    const int64_t b = (total + kBlock - 1) / kBlock;
    rope_scalar<<<static_cast<unsigned>(b > 65536 ? 65536 : b), kBlock, 0, ctx->stream>>>(a, q_pairs, total);
    return launched(ctx, "rope_scalar");
}

}  // extern "C"
