// rows.hpp -- launch shapes for the row kernels (LayerNorm, RMSNorm, add +
// RMSNorm, softmax) and the tuning override shared by every kernel family.
//
// A row of `cols` fp32 is held in VGPRs by TPR threads, each owning VPT
// 16-byte vectors at float4 columns t, t+TPR, ..., in workgroups of BS
// threads (BS/TPR rows per workgroup).  The shapes below were chosen by
// measurement on MI355X: one or two vectors per thread with many waves in
// flight streams better than deep per-thread unrolling.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace mimir {

struct RowShape {
    int tpr;
    int vpt;
    int bs;
};

// Every (TPR, VPT, BS) the row kernels are compiled for.  X(tpr, vpt, bs).
#define MIMIR_ROW_SHAPES(X) \
    X(64, 1, 64)            \
    X(64, 1, 256)           \
    X(64, 2, 64)            \
    X(64, 2, 256)           \
    X(64, 4, 64)            \
    X(64, 4, 256)           \
    X(128, 1, 256)          \
    X(128, 2, 128)          \
    X(128, 2, 256)          \
    X(128, 2, 512)          \
    X(128, 4, 512)          \
    X(256, 1, 256)          \
    X(256, 2, 256)          \
    X(256, 4, 256)          \
    X(256, 4, 1024)         \
    X(512, 1, 512)          \
    X(512, 2, 512)          \
    X(512, 2, 1024)         \
    X(512, 4, 512)          \
    X(1024, 1, 1024)        \
    X(1024, 2, 1024)        \
    X(1024, 4, 1024)

// Tuning override, read once per context from MIMIR_TUNE, e.g.
//   MIMIR_TUNE="norm=1024x1x1024,layernorm=512x2x512,softmax=64x4x64,ew=1,gather=1024,rope=1,
//               lnbwd=512x2x512,lnbwd_grid=512,chain=0,attnbwd_heads=4,attnbwd_blocks=2,
//               embmerge=0,embsort=0,embruns=0,emb1pass=0,blas=0,lnbwd_narrow=0,lrcpw=2,ewbs=128,
//               lrapply=256x4,lrpart=256"
// Each entry selects among the compiled variants above; an entry that does
// not fit a call (row too wide for it) is ignored for that call.  Unset, the
// measured defaults apply.  Used for sweeps; results are identical.
struct Tuning {
    RowShape layernorm{0, 0, 0};
    RowShape rmsnorm{0, 0, 0};  // RMSNorm and add + RMSNorm
    RowShape softmax{0, 0, 0};
    int ew_vpt = 0;
    int gather_tpt = 0;
    int rope_ppt = 0;
    RowShape lnbwd{0, 0, 0};  // LayerNorm backward
    int lnbwd_grid = 0;       // its persistent grid (workgroups)
    int chain_streamed = 0;   // chain=0: the runtime streams every layer's output (no kept outputs)
    int attn_bwd_heads = 0;   // heads per group of the attention backward (0: what 1 GiB of P / dS holds)
    int attn_bwd_blocks = 0;  // causal attention backward: query / key blocks of the products (0: default)
    int embed_bwd_merged = -1;  // embedding backward: rows + segment partials in one launch (1) or two (0)
    int embed_bwd_sort = -1;    // embedding backward: counting sort where it applies (-1, 1) or rocPRIM's (0)
    int embed_bwd_runs = -1;    // embedding backward: rows kernel over the counting sort's run list (-1, 1) or
                                // over the sorted positions (0)
    int embed_bwd_onepass = -1; // embedding backward: the counting sort in one launch where it applies (-1, 1) or
                                // in three (0)
    int blas_lt = -1;           // library products: hipBLASLt first (-1, 1) or rocBLAS only (0)
    int lnbwd_narrow = -1;      // LayerNorm backward, rows <= 64 floats: several rows per wave (-1, 1) or not (0)
    int lr_cpw = 0;             // long rows: 4096-float chunks per workgroup of the first pass (1, 2, 4; 0: measured default)
    int ew_bs = 0;              // workgroup size of the one-float4-per-thread streaming kernels (64 .. 1024; 0: default)
    int lr_apply_bs = 0;        // long rows' apply pass shape (lrapply=256x4: the chunk shape)
    int lr_apply_vpt = 0;
    int lr_part_bs = 0;         // long rows' first pass: threads per 4096-float chunk (lrpart=256/512; 0: default)
};

inline bool parse_shape(const char* v, RowShape* s) {
    int a = 0, b = 0, c = 0;
    char* end = nullptr;
    a = static_cast<int>(std::strtol(v, &end, 10));
    if (*end != 'x') return false;
    b = static_cast<int>(std::strtol(end + 1, &end, 10));
    if (*end != 'x') return false;
    c = static_cast<int>(std::strtol(end + 1, &end, 10));
    *s = RowShape{a, b, c};
    return true;
}

inline Tuning read_tuning() {
    Tuning t;
    const char* env = std::getenv("MIMIR_TUNE");
    if (!env) return t;
    char buf[512];
    std::strncpy(buf, env, sizeof buf - 1);
    buf[sizeof buf - 1] = 0;
    for (char* tok = std::strtok(buf, ","); tok; tok = std::strtok(nullptr, ",")) {
        char* eq = std::strchr(tok, '=');
        if (!eq) continue;
        *eq = 0;
        const char* k = tok;
        const char* v = eq + 1;
        if (!std::strcmp(k, "layernorm")) parse_shape(v, &t.layernorm);
        else if (!std::strcmp(k, "norm")) parse_shape(v, &t.rmsnorm);
        else if (!std::strcmp(k, "softmax")) parse_shape(v, &t.softmax);
        else if (!std::strcmp(k, "ew")) t.ew_vpt = std::atoi(v);
        else if (!std::strcmp(k, "gather")) t.gather_tpt = std::atoi(v);
        else if (!std::strcmp(k, "rope")) t.rope_ppt = std::atoi(v);
        else if (!std::strcmp(k, "lnbwd")) parse_shape(v, &t.lnbwd);
        else if (!std::strcmp(k, "lnbwd_grid")) t.lnbwd_grid = std::atoi(v);
        else if (!std::strcmp(k, "chain")) t.chain_streamed = std::atoi(v) == 0;
        else if (!std::strcmp(k, "attnbwd_heads")) t.attn_bwd_heads = std::atoi(v);
        else if (!std::strcmp(k, "attnbwd_blocks")) t.attn_bwd_blocks = std::atoi(v);
        else if (!std::strcmp(k, "embmerge")) t.embed_bwd_merged = std::atoi(v);
        else if (!std::strcmp(k, "embsort")) t.embed_bwd_sort = std::atoi(v);
        else if (!std::strcmp(k, "embruns")) t.embed_bwd_runs = std::atoi(v);
        else if (!std::strcmp(k, "emb1pass")) t.embed_bwd_onepass = std::atoi(v);
        else if (!std::strcmp(k, "blas")) t.blas_lt = std::atoi(v);
        else if (!std::strcmp(k, "lnbwd_narrow")) t.lnbwd_narrow = std::atoi(v);
        else if (!std::strcmp(k, "lrcpw")) t.lr_cpw = std::atoi(v);
        else if (!std::strcmp(k, "ewbs")) t.ew_bs = std::atoi(v);
        else if (!std::strcmp(k, "lrpart")) t.lr_part_bs = std::atoi(v);
        else if (!std::strcmp(k, "lrapply")) {
            char* end = nullptr;
            t.lr_apply_bs = static_cast<int>(std::strtol(v, &end, 10));
            t.lr_apply_vpt = *end == 'x' ? std::atoi(end + 1) : 0;
        }
    }
    return t;
}

// Default shapes by row width in float4 (c4 = cols / 4), from the sweeps.
inline RowShape default_norm_shape(int64_t c4) {
    if (c4 <= 64) return {64, 1, 256};
    if (c4 <= 128) return {128, 1, 256};
    if (c4 <= 256) return {64, 4, 64};
    if (c4 <= 512) return {512, 1, 512};
    if (c4 <= 1024) return {512, 2, 512};
    if (c4 <= 2048) return {512, 4, 512};
    if (c4 <= 4096) return {1024, 4, 1024};
    return {0, 0, 0};
}

// LayerNorm reduces twice per wave and combines (mean, M2) pairs across the
// row's waves, so it favours fewer, fuller waves per row at 4096 floats.
inline RowShape default_layernorm_shape(int64_t c4) {
    if (c4 > 512 && c4 <= 1024) return {256, 4, 256};
    return default_norm_shape(c4);
}

// Rows of 1024 floats: one row per 128-thread workgroup, 81.6-81.8%
// of 8 TB/s on MI355X against 80.6-81.2% with four rows per 512 threads (the
// same per-row arithmetic, so the same bits).
inline RowShape default_softmax_shape(int64_t c4) {
    if (c4 <= 64) return {64, 1, 64};
    if (c4 <= 128) return {64, 2, 64};
    if (c4 <= 256) return {128, 2, 128};
    if (c4 <= 512) return {128, 4, 512};
    if (c4 <= 1024) return {1024, 1, 1024};
    if (c4 <= 2048) return {1024, 2, 1024};
    if (c4 <= 4096) return {1024, 4, 1024};
    return {0, 0, 0};
}

// Workgroup size of the streaming kernels that move one float4 per thread
// (unary_vec / binary_vec, dact_vec, mul_bwd_vec, add_bwd_vec,
// fused_chain_vec, copy16_kernel): the tuned value if it is one of the
// compiled sizes, else the default.  Measured on MI355X at configs[4]
// (% of 8 TB/s for 64 / 128 / 256 threads): add 82.0 / 82.0 / 79.3,
// SiLU-gated product 83.5 / 83.3 / 81.5, multiply backward 80.6 / 81.7 / 75.9,
// add backward 79.2 / 80.6 / 78.0, GELU backward 83.3 / 83.0 / 81.4, GELU
// 84.5 / 84.2 / 84.3: the same stream in workgroups of 128 threads instead of
// 256 gains up to 6 points.  RoPE (four slots per thread) keeps 256 threads
// (82.4 against 80.6 at 128; rope_block).
constexpr int kEwBlock = 128;
inline int ew_block(const Tuning& t) {
    return t.ew_bs == 64 || t.ew_bs == 128 || t.ew_bs == 256 || t.ew_bs == 512 || t.ew_bs == 1024 ? t.ew_bs
                                                                                                  : kEwBlock;
}
inline int rope_block(const Tuning& t) { return t.ew_bs ? ew_block(t) : 256; }

// Calls f(std::integral_constant<int, BS>{}) for the workgroup size `bs`
// (one of 64, 128, 256, 512, 1024).
template <class Fn>
inline auto with_block(int bs, Fn&& f) {
    switch (bs) {
        case 64: return f(std::integral_constant<int, 64>{});
        case 128: return f(std::integral_constant<int, 128>{});
        case 512: return f(std::integral_constant<int, 512>{});
        case 1024: return f(std::integral_constant<int, 1024>{});
        default: return f(std::integral_constant<int, 256>{});
    }
}

inline bool shape_fits(const RowShape& s, int64_t c4) {
    return s.tpr > 0 && static_cast<int64_t>(s.tpr) * s.vpt >= c4;
}

// Whether `blocks` workgroups of `threads` fit one grid dimension: HIP takes
// at most 2^31 - 1 workgroups, and the dispatch packet counts the grid in
// work-items in 32 bits, so blocks * threads must stay below 2^32.
inline bool dispatch_fits(int64_t blocks, int64_t threads) {
    return blocks > 0 && blocks <= 0x7fffffffLL && blocks * threads <= 0xffffffffLL;
}

// Number of workgroups of `threads` for `units` work items of `per_block`
// each, refusing grids beyond the dispatch limits above.
inline bool grid_for(int64_t units, int64_t per_block, int threads, unsigned* blocks) {
    const int64_t b = (units + per_block - 1) / per_block;
    if (!dispatch_fits(b, threads)) return false;
    *blocks = static_cast<unsigned>(b);
    return true;
}

}  // namespace mimir
