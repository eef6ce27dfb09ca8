// attention.hip -- the attention core softmax(Q K^T * scale) V with the
// softmax fused between the two products, fp32 on the gfx950 matrix cores.
//
// Reference: the core of LayerOps::self_attention_forward (LayerOps.hpp:
// 1045-1089) and cross_attention_forward (:1163-1209), which materialise one
// score row per query (s = dot * scale; causal j > i masked to -1e9; max from
// -1e30; e = exp(s - max); p = e / (sum + 1e-9); out = sum_j p_j V_j).  Here
// no score row is ever stored: each workgroup streams K / V tiles through LDS
// and keeps a running max / sum per query ("online softmax"; Milakov and
// Gimelshein 2018, as used by FlashAttention, Dao et al. 2022), rescaling its
// partial output when the max grows, and divides by (sum + 1e-9) at the end.
// Q is multiplied by scale * log2(e) once, so the scores come out of the
// matrix core in base-2 units and each probability is one v_exp_f32.
//
// Matrix-core mapping.  v_mfma_f32_32x32x2_f32 computes D[32x32] += A[32x2] *
// B[2x32]; lane l supplies A[l%32][l/32] and B[l/32][l%32] and receives
// D[8*(r/4) + 4*(l/32) + r%4][l%32] in accumulator register r (r = 0..15).
// - Scores: S^T = K Q^T, keys as rows, queries as columns.  A = K (row = the
//   key, k index = one head dimension), B = Q^T, so lane l owns query l%32 and
//   16 of the 32 keys of the tile.  The head dimensions are split between the
//   two lane halves: at step s the half h = l/32 supplies dimension
//   h*DP/2 + s, so each lane reads four steps of K with one 16-byte LDS read
//   and holds its query's DP/2 Q values in registers for the whole kernel.
// - Softmax: per lane over its 16 keys; the running max is shared with the
//   other half (lane l ^ 32, same query) once per tile.
// - Output: O^T = V^T P^T.  The accumulator register r of S^T already holds
//   P^T[key(r, h)][query] in the layout of the B operand when the MFMA's two
//   k-slots are the keys key(r, 0), key(r, 1), key(r, h) = 8*(r/4) + 4h + r%4,
//   so the probabilities feed the second product without a lane exchange.
//   The A operand row i of dimension block db is head dimension (DP/32)*i + db,
//   so a lane reads its DP/32 values of one V row with one LDS read, and its
//   output rows come out as DP/32 consecutive dimensions (one 16-byte store
//   for DP = 128).
//
// Pipeline.  A wave issues its instructions in order, and a v_mfma holds the
// matrix pipe for 64 cycles, so the softmax's vector work only overlaps the
// matrix core if it sits between independent MFMAs.  Iteration t therefore
// computes the scores of tile t+1 (S_next = K_{t+1} Q^T) interleaved
// instruction by instruction with the softmax of tile t (whose scores came
// from iteration t-1), then O += V_t^T P_t.  K runs one tile ahead of V: LDS
// holds a K ring and a V ring of two tiles each; iteration t reads K_{t+1}
// and V_t and refills the slots of K_t and V_{t-1} with K_{t+2} and V_{t+1},
// whose global loads were issued at the start of the iteration, then one
// barrier.
//
// Workgroup: 4 waves, 32 queries each (128 queries of one (sequence, head)).
// Causal: a workgroup stops at its last query's diagonal, a wave skips the
// tiles past its own diagonal and masks inside its last tile only (the
// diagonal, or the sequence's ragged end).
// Grid: the hardware deals workgroups to the 8 XCDs round-robin.  When the
// (sequence, head) count divides by 8, each XCD owns an eighth of them (their
// K and V stay in that XCD's L2) and runs its query blocks longest first
// across all of its heads, so the short causal blocks fill the tail.
#include "common.hpp"
#include "internal.hpp"

#include <math.h>

#include <cmath>

using namespace mimir;

namespace {

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f2 __attribute__((ext_vector_type(2)));

constexpr int kQPerWave = 32;
constexpr int kWaves = 4;
constexpr int kQPerBlock = kQPerWave * kWaves;  // 128
constexpr int kKeyTile = 32;
constexpr int kThreads = kWaves * kWave;        // 256
constexpr int kXcds = 8;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
    const float* q;
    const float* k;
    const float* v;
    float* out;
    int64_t ld_q, ld_kv, ld_out;  // row strides (floats)
    int32_t q_len, kv_len, heads, head_dim;
    int32_t n_qblocks;            // ceil(q_len / 128)
    uint32_t total_blocks;        // batch * heads * n_qblocks
    float qscale;                 // scale * log2(e), applied to Q
    int32_t causal;
};

// LDS: the K ring [2][32][DP + 4] (the pad staggers the rows across banks for
// the column-wise reads), then the V ring [2][32][DP].
template <int DP>
struct Lds {
    static constexpr int kLd = DP + 4;
    static constexpr int vLd = DP;
    static constexpr int kTile = kKeyTile * kLd;
    static constexpr int vTile = kKeyTile * vLd;
    static constexpr int vRing = 2 * kTile;
    static constexpr int total = 2 * kTile + 2 * vTile;
    static constexpr int f4PerRow = DP / 4;
    static constexpr int loads = kKeyTile * f4PerRow / kThreads;  // float4 per thread per tile
    static_assert(loads >= 1 && kKeyTile * f4PerRow == loads * kThreads, "tile / block mismatch");
};

// 4 floats of a row at column c (a multiple of 4), zero past `valid` columns.
// VEC: head_dim, the strides and the base pointers are 16-byte multiples.
template <bool VEC>
__device__ __forceinline__ f4 load4(const float* row, int c, int valid) {
    if constexpr (VEC) {
        if (c < valid) return *reinterpret_cast<const f4*>(row + c);
        return f4{0.f, 0.f, 0.f, 0.f};
    } else {
        f4 r;
        r.x = c + 0 < valid ? row[c + 0] : 0.f;
        r.y = c + 1 < valid ? row[c + 1] : 0.f;
        r.z = c + 2 < valid ? row[c + 2] : 0.f;
        r.w = c + 3 < valid ? row[c + 3] : 0.f;
        return r;
    }
}

// Scalar-path tile load: four loads from clamped, always valid columns
// (< head_dim); the caller clamps the row below kv_len.  What lies outside
// the tile's valid rows / columns is replaced by zeros when the values are
// written to LDS (zero_outside).
__device__ __forceinline__ f4 load4_clamped(const float* row, int c, int head_dim) {
    f4 r;
    r.x = row[min(c + 0, head_dim - 1)];
    r.y = row[min(c + 1, head_dim - 1)];
    r.z = row[min(c + 2, head_dim - 1)];
    r.w = row[min(c + 3, head_dim - 1)];
    return r;
}

// Word 3 of a raw (stride 0) buffer descriptor on gfx9-family GPUs: 32-bit
// data format, no swizzle; out-of-range offsets return zeros.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ f4 zero_outside(f4 x, bool row_ok, int c, int head_dim) {
    x.x = row_ok && c + 0 < head_dim ? x.x : 0.f;
    x.y = row_ok && c + 1 < head_dim ? x.y : 0.f;
    x.z = row_ok && c + 2 < head_dim ? x.z : 0.f;
    x.w = row_ok && c + 3 < head_dim ? x.w : 0.f;
    return x;
}

// Workgroup -> (sequence * heads + head, query block): see the file comment.
__device__ __forceinline__ void block_coords(const AttnArgs& a, uint32_t bid, uint32_t* bh, int* qb) {
    const uint32_t n_bh = a.total_blocks / static_cast<uint32_t>(a.n_qblocks);
    uint32_t first = 0, owned = n_bh, idx = bid;
    if (n_bh % kXcds == 0) {
        owned = n_bh / kXcds;
        first = (bid % kXcds) * owned;
        idx = bid / kXcds;
    }
    *qb = a.n_qblocks - 1 - static_cast<int>(idx / owned);
    *bh = first + idx % owned;
}

template <int DP, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void attention_fwd_mfma(AttnArgs a) {
    using L = Lds<DP>;
    constexpr int kHalf = DP / 2;  // dimensions per lane half = MFMA k-steps of S
    constexpr int kDb = DP / 32;   // output dimension blocks
    __shared__ __attribute__((aligned(16))) float lds[L::total];

    uint32_t bh;
    int qb;
    block_coords(a, blockIdx.x, &bh, &qb);
    const int64_t b = bh / static_cast<uint32_t>(a.heads);
    const int64_t hd_off = static_cast<int64_t>(bh % static_cast<uint32_t>(a.heads)) * a.head_dim;
    const float* qbase = a.q + b * a.q_len * a.ld_q + hd_off;
    const float* kbase = a.k + b * a.kv_len * a.ld_kv + hd_off;
    const float* vbase = a.v + b * a.kv_len * a.ld_kv + hd_off;
    float* obase = a.out + b * a.q_len * a.ld_out + hd_off;

    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int li = lane % 32;  // query column / MFMA row index
    const int hf = lane / 32;  // lane half
    const int q0 = qb * kQPerBlock;
    const int qw0 = q0 + wave * kQPerWave;
    const int my_q = qw0 + li;

    // Tiles this workgroup streams, and the ones this wave computes.
    int key_end = a.kv_len;
    int wave_key_end = a.kv_len;
    if (a.causal) {
        key_end = min(key_end, min(q0 + kQPerBlock, a.q_len));
        wave_key_end = min(wave_key_end, min(qw0 + kQPerWave, a.q_len));
    }
    if (qw0 >= a.q_len) wave_key_end = 0;
    const int n_tiles = (key_end + kKeyTile - 1) / kKeyTile;
    const int wave_tiles = (wave_key_end + kKeyTile - 1) / kKeyTile;
    // Keys of this lane's query: the rest of its last tile is masked
    // (causal: key > query; all: key >= kv_len).
    const int lane_key_end = min(a.kv_len, a.causal ? my_q + 1 : a.kv_len);

    // This lane's Q values, times scale*log2(e): query my_q, dimensions
    // hf*kHalf + [0, kHalf).
    float qreg[kHalf];
    {
        const float* qrow = qbase + static_cast<int64_t>(min(my_q, a.q_len - 1)) * a.ld_q;
        const int valid = my_q < a.q_len ? a.head_dim : 0;
#pragma unroll
        for (int j = 0; j < kHalf / 4; ++j) {
            const f4 t = load4<VEC>(qrow, hf * kHalf + 4 * j, valid);
            qreg[4 * j + 0] = t.x * a.qscale;
            qreg[4 * j + 1] = t.y * a.qscale;
            qreg[4 * j + 2] = t.z * a.qscale;
            qreg[4 * j + 3] = t.w * a.qscale;
        }
    }

    // Cooperative tile load: thread tid moves float4 number tid + 256*r of a
    // tile (row = key within the tile, column group c).  VEC: buffer loads
    // through a descriptor based at the tile's first row whose range ends
    // after the sequence's last row, so rows past kv_len read as zeros
    // without a memory access; the per-thread byte offsets are loop
    // invariants (no address registers recycled while the loads are in
    // flight).  Columns are clamped below head_dim (never past the row).
    f4 kst[L::loads], vst[L::loads];
    uint32_t voff[L::loads];
    if constexpr (VEC) {
#pragma unroll
        for (int r = 0; r < L::loads; ++r) {
            const int f = tid + r * kThreads;
            const int row = f / L::f4PerRow;
            const int c = min(4 * (f % L::f4PerRow), a.head_dim - 4);
            voff[r] = static_cast<uint32_t>((row * a.ld_kv + c) * 4);
        }
    }
    auto fetch = [&](const float* base, int tile, f4* dst) {
        if constexpr (VEC) {
            const int64_t first = static_cast<int64_t>(tile) * kKeyTile * a.ld_kv;
            const int rows = min(kKeyTile, a.kv_len - tile * kKeyTile);
            const int bytes = static_cast<int>(rows * a.ld_kv * 4);
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base + first), 0, bytes, kBufferWord3);
#pragma unroll
            for (int r = 0; r < L::loads; ++r)
                dst[r] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff[r], 0, 0));
        } else {
#pragma unroll
            for (int r = 0; r < L::loads; ++r) {
                const int f = tid + r * kThreads;
                const int row = f / L::f4PerRow;
                const int c = 4 * (f % L::f4PerRow);
                const int64_t off = static_cast<int64_t>(min(tile * kKeyTile + row, a.kv_len - 1)) * a.ld_kv;
                dst[r] = load4_clamped(base + off, c, a.head_dim);
            }
        }
    };
    auto stash = [&](const f4* src, int tile, float* dst, int ld) {
#pragma unroll
        for (int r = 0; r < L::loads; ++r) {
            const int f = tid + r * kThreads;
            const int row = f / L::f4PerRow;
            const int c = 4 * (f % L::f4PerRow);
            const bool row_ok = tile * kKeyTile + row < a.kv_len;
            *reinterpret_cast<f4*>(dst + row * ld + c) = zero_outside(src[r], row_ok, c, a.head_dim);
        }
    };
    float* const kring = lds;
    float* const vring = lds + L::vRing;

    // S^T = K Q^T over the head dimension, K from ring slot `slot`.
    auto scores = [&](int slot) {
        f16v s = f16v{};
        const float* krow = kring + slot * L::kTile + li * L::kLd + hf * kHalf;
#pragma unroll
        for (int j = 0; j < kHalf / 4; ++j) {
            const f4 kv = *reinterpret_cast<const f4*>(krow + 4 * j);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qreg[4 * j + 0], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qreg[4 * j + 1], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qreg[4 * j + 2], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qreg[4 * j + 3], s, 0, 0, 0);
        }
        return s;
    };

    f16v o[kDb];
#pragma unroll
    for (int d = 0; d < kDb; ++d) o[d] = f16v{};
    float m_run = -1e30f;  // running max (base-2 units); the reference starts at -1e30 (LayerOps.hpp:1052)
    float l_run = 0.f;     // this half's share of the running sum

    // Online softmax of one tile's scores (in place: s becomes P), rescale of
    // O and the running sum, then O^T += V^T P^T with V from ring slot
    // `slot`.  mask: keys at or past lane_key_end are excluded.
    auto softmax_pv = [&](f16v& s, int slot, bool mask, int key0) {
        if (mask) {
            const int lim = lane_key_end - key0 - 4 * hf;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 8 * (r / 4) + (r % 4) < lim ? s[r] : -INFINITY;
        }
        float tmax = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
        tmax = fmaxf(tmax, fmaxf(fmaxf(fmaxf(s[8], s[9]), fmaxf(s[10], s[11])),
                                 fmaxf(fmaxf(s[12], s[13]), fmaxf(s[14], s[15]))));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = __builtin_amdgcn_exp2f(s[r] - m_new);  // exp2(-inf) = 0: masked keys
            psum += s[r];
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int d = 0; d < kDb; ++d) o[d] *= alpha;
        const float* vl = vring + slot * L::vTile;
        // k-slot h of step r is key(r, h) = 8*(r/4) + 4h + r%4.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float* vrow = vl + (8 * (r / 4) + 4 * hf + (r % 4)) * L::vLd + kDb * li;
            if constexpr (kDb == 4) {
                const f4 vv = *reinterpret_cast<const f4*>(vrow);
                o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, s[r], o[0], 0, 0, 0);
                o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, s[r], o[1], 0, 0, 0);
                o[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, s[r], o[2], 0, 0, 0);
                o[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, s[r], o[3], 0, 0, 0);
            } else if constexpr (kDb == 2) {
                const f2 vv = *reinterpret_cast<const f2*>(vrow);
                o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, s[r], o[0], 0, 0, 0);
                o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, s[r], o[1], 0, 0, 0);
            } else {
                o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[0], s[r], o[0], 0, 0, 0);
            }
        }
    };

    // Prologue: K_0, V_0 and K_1 in LDS, S_0 computed.
    if (n_tiles > 0) {
        fetch(kbase, 0, kst);
        fetch(vbase, 0, vst);
        stash(kst, 0, kring, L::kLd);
        stash(vst, 0, vring, L::vLd);
    }
    if (n_tiles > 1) {
        fetch(kbase, 1, kst);
        stash(kst, 1, kring + L::kTile, L::kLd);
    }
    __syncthreads();
    f16v s_cur = f16v{};
    if (wave_tiles > 0) s_cur = scores(0);
    // Iteration 0 refills K_0's slot: every wave must have read it first
    // (later refills are ordered by the previous iteration's barrier).
    __syncthreads();

    for (int t = 0; t < n_tiles; ++t) {
        // Global loads of K_{t+2} and V_{t+1} (clamped to the last tile; the
        // slots they fill are not read again once they would be past it).
        fetch(kbase, min(t + 2, n_tiles - 1), kst);
        fetch(vbase, min(t + 1, n_tiles - 1), vst);
        if (t + 1 < wave_tiles) {
            // S_{t+1} interleaved with the softmax of S_t; a tile before the
            // wave's last one is never masked.
            const f16v s_next = scores((t + 1) & 1);
            softmax_pv(s_cur, t & 1, false, t * kKeyTile);
#pragma unroll
            for (int i = 0; i < kHalf / 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read (K)
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // four score MFMAs
                __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six softmax VALU ops
            }
            s_cur = s_next;
        } else if (t < wave_tiles) {
            const bool mask = (t + 1) * kKeyTile > a.kv_len || (a.causal && (t + 1) * kKeyTile - 1 > qw0);
            if (mask) softmax_pv(s_cur, t & 1, true, t * kKeyTile);
            else softmax_pv(s_cur, t & 1, false, t * kKeyTile);
        }
        stash(kst, min(t + 2, n_tiles - 1), kring + (t & 1) * L::kTile, L::kLd);
        stash(vst, min(t + 1, n_tiles - 1), vring + ((t + 1) & 1) * L::vTile, L::vLd);
        __syncthreads();
    }

    // out = O / (sum + 1e-9) (LayerOps.hpp:1076-1079), rows of DP/32 dims.
    if (my_q < a.q_len) {
        const float l_tot = l_run + __shfl_xor(l_run, 32);
        const float inv = 1.0f / (l_tot + 1e-9f);
        float* orow = obase + static_cast<int64_t>(my_q) * a.ld_out;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int d0 = kDb * (8 * (r / 4) + 4 * hf + (r % 4));
            if (d0 >= a.head_dim) continue;
            if constexpr (kDb == 4) {
                const f4 val{o[0][r] * inv, o[1][r] * inv, o[2][r] * inv, o[3][r] * inv};
                if constexpr (VEC) {
                    *reinterpret_cast<f4*>(orow + d0) = val;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < a.head_dim) orow[d0 + e] = val[e];
                }
            } else if constexpr (kDb == 2) {
                orow[d0] = o[0][r] * inv;
                if (d0 + 1 < a.head_dim) orow[d0 + 1] = o[1][r] * inv;
            } else {
                orow[d0] = o[0][r] * inv;
            }
        }
    }
}

// Heads wider than 128 (up to 2048): one wave per query, the head's
// dimensions spread over the lanes (CH per lane, lane + 64 c), each score a
// DPP wave sum, the same online softmax (base-2 scores, running max and
// sum) and the same division by (sum + 1e-9).  Plain fp32 vector code: the
// reference accepts any head size, the matrix-core kernel's register layout
// stops at 128.  Keys are read row by row through L2 by all four waves of a
// workgroup (four queries).
constexpr int kGenericWaves = 4;
template <int CH>
__global__ __launch_bounds__(kGenericWaves * kWave) void attention_fwd_generic(AttnArgs a) {
    const int lane = threadIdx.x % kWave;
    const int64_t qi = static_cast<int64_t>(blockIdx.y) * kGenericWaves + threadIdx.x / kWave;
    if (qi >= a.q_len) return;  // whole waves leave: no barrier below
    const uint32_t bh = blockIdx.x;
    const int64_t b = bh / static_cast<uint32_t>(a.heads);
    const int64_t hd_off = static_cast<int64_t>(bh % static_cast<uint32_t>(a.heads)) * a.head_dim;
    const float* qrow = a.q + (b * a.q_len + qi) * a.ld_q + hd_off;
    const float* kb = a.k + b * a.kv_len * a.ld_kv + hd_off;
    const float* vb = a.v + b * a.kv_len * a.ld_kv + hd_off;
    float q[CH], acc[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int d = lane + c * kWave;
        q[c] = d < a.head_dim ? qrow[d] * a.qscale : 0.f;
        acc[c] = 0.f;
    }
    const int64_t key_end = a.causal ? (qi + 1 < a.kv_len ? qi + 1 : a.kv_len) : a.kv_len;
    float m_run = -1e30f, l_run = 0.f;
    for (int64_t j = 0; j < key_end; ++j) {
        const float* krow = kb + j * a.ld_kv;
        const float* vrow = vb + j * a.ld_kv;
        float part = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int d = lane + c * kWave;
            if (d < a.head_dim) part += q[c] * krow[d];
        }
        const float s = wave_sum(part);  // wave-uniform
        const float m_new = fmaxf(m_run, s);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        const float p = __builtin_amdgcn_exp2f(s - m_new);
        m_run = m_new;
        l_run = l_run * alpha + p;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int d = lane + c * kWave;
            acc[c] = acc[c] * alpha + (d < a.head_dim ? p * vrow[d] : 0.f);
        }
    }
    const float inv = 1.0f / (l_run + 1e-9f);
    float* orow = a.out + (b * a.q_len + qi) * a.ld_out + hd_off;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int d = lane + c * kWave;
        if (d < a.head_dim) orow[d] = acc[c] * inv;
    }
}

template <int CH>
int launch_generic(mimir_ctx* ctx, const AttnArgs& a, int64_t batch, int64_t heads) {
    const dim3 grid(static_cast<unsigned>(batch * heads),
                    static_cast<unsigned>((a.q_len + kGenericWaves - 1) / kGenericWaves));
    attention_fwd_generic<CH><<<grid, kGenericWaves * kWave, 0, ctx->stream>>>(a);
    return launched(ctx, "attention_fwd_generic");
}

template <int DP>
int launch(mimir_ctx* ctx, const AttnArgs& a, bool vec) {
    if (vec) attention_fwd_mfma<DP, true><<<a.total_blocks, kThreads, 0, ctx->stream>>>(a);
    else attention_fwd_mfma<DP, false><<<a.total_blocks, kThreads, 0, ctx->stream>>>(a);
    return launched(ctx, "attention_fwd_mfma");
}

}  // namespace

extern "C" {

int mimir_attention_fwd(mimir_ctx* ctx, const float* q, int64_t ld_q, const float* k, const float* v,
                        int64_t ld_kv, float* out, int64_t ld_out, int64_t batch, int64_t q_len,
                        int64_t kv_len, int64_t heads, int64_t head_dim, float scale, int causal) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, batch >= 0 && q_len >= 0 && kv_len >= 0 && heads >= 1 && head_dim >= 1,
                  "attention: invalid shape (batch=%lld q_len=%lld kv_len=%lld heads=%lld head_dim=%lld)",
                  (long long)batch, (long long)q_len, (long long)kv_len, (long long)heads, (long long)head_dim);
    MIMIR_REQUIRE(ctx, head_dim <= 2048, "attention: head_dim %lld > 2048 is not supported", (long long)head_dim);
    const int64_t width = heads * head_dim;
    MIMIR_REQUIRE(ctx, ld_q >= width && ld_kv >= width && ld_out >= width,
                  "attention: row strides (%lld, %lld, %lld) below heads * head_dim = %lld", (long long)ld_q,
                  (long long)ld_kv, (long long)ld_out, (long long)width);
    MIMIR_REQUIRE(ctx, q_len < (int64_t{1} << 30) && kv_len < (int64_t{1} << 30) && heads < (int64_t{1} << 30),
                  "attention: sequence or head count too large");
    MIMIR_REQUIRE(ctx, std::isfinite(scale), "attention: scale must be finite");
    if (batch == 0 || q_len == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, q && out && (kv_len == 0 || (k && v)), "attention: null pointer");
    const int64_t nqb = (q_len + kQPerBlock - 1) / kQPerBlock;
    MIMIR_REQUIRE(ctx, dispatch_fits(batch * heads * nqb, kThreads), "attention: grid of %lld workgroups exceeds the limit",
                  (long long)(batch * heads * nqb));
    if (int st = enter(ctx)) return st;
    AttnArgs a;
    a.q = q;
    a.k = kv_len ? k : q;  // never read when kv_len == 0
    a.v = kv_len ? v : q;
    a.out = out;
    a.ld_q = ld_q;
    a.ld_kv = ld_kv;
    a.ld_out = ld_out;
    a.q_len = static_cast<int32_t>(q_len);
    a.kv_len = static_cast<int32_t>(kv_len);
    a.heads = static_cast<int32_t>(heads);
    a.head_dim = static_cast<int32_t>(head_dim);
    a.n_qblocks = static_cast<int32_t>(nqb);
    a.total_blocks = static_cast<uint32_t>(batch * heads * nqb);
    a.qscale = scale * kLog2e;
    a.causal = causal ? 1 : 0;
    // The vector path's buffer descriptors span one 32-row tile: 32 rows of
    // ld_kv floats must stay below 2^31 bytes.
    const bool vec = head_dim % 4 == 0 && ld_q % 4 == 0 && ld_kv % 4 == 0 && ld_out % 4 == 0 && aligned16(q) &&
                     aligned16(a.k) && aligned16(a.v) && aligned16(out) &&
                     ld_kv < (int64_t{1} << 31) / (4 * kKeyTile);
    if (head_dim <= 32) return launch<32>(ctx, a, vec);
    if (head_dim <= 64) return launch<64>(ctx, a, vec);
    if (head_dim <= 128) return launch<128>(ctx, a, vec);
    MIMIR_REQUIRE(ctx, dispatch_fits(batch * heads, kGenericWaves * kWave) && (q_len + kGenericWaves - 1) / kGenericWaves <= 65535,
                  "attention: grid exceeds the limit of the wide-head kernel");
    if (head_dim <= 256) return launch_generic<4>(ctx, a, batch, heads);
    if (head_dim <= 512) return launch_generic<8>(ctx, a, batch, heads);
    if (head_dim <= 1024) return launch_generic<16>(ctx, a, batch, heads);
    return launch_generic<32>(ctx, a, batch, heads);
}

// The attention layers (Model.cpp:5904-5934, 5936-5990): the projections as
// library GEMMs (gemm.hip), the fused core between them on the projection's
// output in place (no split copies).  Scratch: the projections' outputs and
// the attended heads, reused in stream order.
int mimir_self_attention_fwd(mimir_ctx* ctx, const float* input, int64_t seq_len, int64_t embed_dim,
                             int64_t num_heads, int causal, const float* weights, int64_t weights_len, float* out) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, embed_dim >= 1 && num_heads >= 1 && embed_dim % num_heads == 0,
                  "SelfAttention: embed_dim must be divisible by num_heads");
    MIMIR_REQUIRE(ctx, seq_len >= 0, "SelfAttention: input size mismatch");
    const int64_t e = embed_dim;
    MIMIR_REQUIRE(ctx, weights_len >= 4 * e * e, "SelfAttention: weight block of %lld floats, %lld needed",
                  (long long)weights_len, (long long)(4 * e * e));
    MIMIR_REQUIRE(ctx, e / num_heads <= 2048, "attention: head_dim %lld > 2048 is not supported",
                  (long long)(e / num_heads));
    if (seq_len == 0) return MIMIR_OK;
    MIMIR_REQUIRE(ctx, input && weights && out, "SelfAttention: null pointer");
    MIMIR_ENTER(ctx);
    void* s = nullptr;
    if (int st = ensure_scratch(ctx, sizeof(float) * static_cast<size_t>(seq_len) * 4 * e, &s)) return st;
    float* qkv = static_cast<float*>(s);  // [seq, 3E]: Q | K | V
    float* att = qkv + seq_len * 3 * e;   // [seq, E]
    const int64_t hd = e / num_heads;
    if (int st = gemm_f32(ctx, seq_len, 3 * e, e, input, e, weights, 3 * e, qkv, 3 * e)) return st;  // :1027-1028
    if (int st = mimir_attention_fwd(ctx, qkv, 3 * e, qkv + e, qkv + 2 * e, 3 * e, att, e, 1, seq_len, seq_len,
                                     num_heads, hd, 1.0f / std::sqrt(static_cast<float>(hd)), causal))
        return st;
    return gemm_f32(ctx, seq_len, e, e, att, e, weights + 3 * e * e, e, out, e);  // :1093-1094
}

int mimir_cross_attention_fwd(mimir_ctx* ctx, const float* query_input, int64_t query_len, const float* kv_input,
                              int64_t kv_len, int64_t embed_dim, int64_t num_heads, int causal,
                              const float* weights, int64_t weights_len, float* out) {
    if (!ctx) return MIMIR_EINVAL;
    MIMIR_REQUIRE(ctx, embed_dim >= 1 && num_heads >= 1 && embed_dim % num_heads == 0,
                  "CrossAttention: embed_dim must be divisible by num_heads");
    MIMIR_REQUIRE(ctx, query_len > 0 && kv_len > 0, "CrossAttention: invalid dimensions");
    const int64_t e = embed_dim;
    MIMIR_REQUIRE(ctx, weights_len >= 4 * e * e, "CrossAttention: weight block of %lld floats, %lld needed",
                  (long long)weights_len, (long long)(4 * e * e));
    MIMIR_REQUIRE(ctx, e / num_heads <= 2048, "attention: head_dim %lld > 2048 is not supported",
                  (long long)(e / num_heads));
    MIMIR_REQUIRE(ctx, query_input && kv_input && weights && out, "CrossAttention: null pointer");
    MIMIR_ENTER(ctx);
    void* s = nullptr;
    if (int st = ensure_scratch(ctx, sizeof(float) * static_cast<size_t>(2 * query_len + 2 * kv_len) * e, &s))
        return st;
    float* qp = static_cast<float*>(s);  // [query_len, E]
    float* kv = qp + query_len * e;      // [kv_len, 2E]: K | V
    float* att = kv + kv_len * 2 * e;    // [query_len, E]
    const int64_t hd = e / num_heads;
    if (int st = gemm_f32(ctx, query_len, e, e, query_input, e, weights, e, qp, e)) return st;  // :1146-1147
    if (int st = gemm_f32(ctx, kv_len, 2 * e, e, kv_input, e, weights + e * e, 2 * e, kv, 2 * e)) return st;
    if (int st = mimir_attention_fwd(ctx, qp, e, kv, kv + e, 2 * e, att, e, 1, query_len, kv_len, num_heads, hd,
                                     1.0f / std::sqrt(static_cast<float>(hd)), causal))
        return st;
    return gemm_f32(ctx, query_len, e, e, att, e, weights + 3 * e * e, e, out, e);  // :1213-1214
}

}  // extern "C"
