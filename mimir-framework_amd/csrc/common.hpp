// common.hpp -- device helpers shared by the gfx950 kernels of libmimir_hip.
//
// Wave64 throughout.  Reductions run inside one wavefront with DPP lane moves
// (quad_perm, row_half_mirror, row_mirror) and finish with four readlanes, so
// the reduced value is wave-uniform (held in an SGPR) and bitwise identical
// for every lane.  LDS is used only to combine the per-wave partials of a
// multi-wave row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mimir {

constexpr int kWave = 64;
constexpr int kBlock = 256;  // workgroup size of the streaming kernels (row kernels pick their own)

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// memory: 128-bit global accesses.  `nt` selects the non-temporal variants
// (the data is streamed once; keep it out of the way of reused lines).
// ---------------------------------------------------------------------------
template <bool NT>
__device__ __forceinline__ f4 ld4(const float* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
    else return *reinterpret_cast<const f4*>(p);
}

// Streaming stores: data written once and not read again by this kernel,
// with one of two cache policies, chosen per kernel by measurement:
//   kStoreNt       `nt`: the line enters the XCD's L2 with a streaming hint
//                  and reaches HBM when L2 writes it back;
//   kStoreThrough  `sc1 nt`: device scope, so L2 writes the line through to
//                  memory at once and holds no dirty copy.  Measured on
//                  MI355X it lifts write-heavy streams (RoPE, GELU, the add
//                  backward's two outputs) by 1-3 points and costs the
//                  read-heavy ones (add, SiLU-gated product, the row ops) 1-2.
// The non-temporal form is the compiler's store with its non-temporal hint.
// The hint is metadata that loop-invariant code motion drops when it sinks
// a store out of a one-trip loop (a VPT = 1 kernel), so the address first
// passes through an empty volatile asm, which no pass can move or see
// through.  The write-through form has no builtin and is inline assembly;
// the compiler does not count it in its waits, and a gfx9 wave's vmcnt is
// in order, so a later wait for a load issued before such a store also
// waits for the store: use it where every load precedes every store.
enum : int { kStoreNt = 0, kStoreThrough = 1 };

// A pointer into global memory (address space 1), so stores through it are
// global_store, not flat_store.
template <typename T>
using gptr = __attribute__((address_space(1))) T*;

template <int POL = kStoreNt>
__device__ __forceinline__ void st_stream(void* p, u4 v) {
    if constexpr (POL == kStoreThrough) {
        asm volatile("global_store_dwordx4 %0, %1, off sc1 nt" : : "v"(p), "v"(v) : "memory");
    } else {
        gptr<u4> g = (gptr<u4>)p;
        asm volatile("" : "+v"(g));
        __builtin_nontemporal_store(v, g);
    }
}

template <int POL = kStoreNt>
__device__ __forceinline__ void st_stream(float* p, f4 v) {
    st_stream<POL>(static_cast<void*>(p), __builtin_bit_cast(u4, v));
}
template <int POL = kStoreNt>
__device__ __forceinline__ void st_stream(f4* p, f4 v) {
    st_stream<POL>(static_cast<void*>(p), __builtin_bit_cast(u4, v));
}

template <int POL = kStoreNt>
__device__ __forceinline__ void st_stream(float* p, float v) {
    if constexpr (POL == kStoreThrough) {
        asm volatile("global_store_dword %0, %1, off sc1 nt" : : "v"(p), "v"(v) : "memory");
    } else {
        gptr<float> g = (gptr<float>)p;
        asm volatile("" : "+v"(g));
        __builtin_nontemporal_store(v, g);
    }
}

template <bool NT>
__device__ __forceinline__ void st4(float* p, f4 v) {
    if constexpr (NT) st_stream(p, v);
    else *reinterpret_cast<f4*>(p) = v;
}

// An op's output: streamed unless KEEP, in which case a plain store leaves
// the line in L2 / the Infinity Cache for the op launched next.  Measured on
// MI355X, producer -> consumer through a 128 MiB tensor: 79 us with kept
// outputs, 92 us streamed; an op whose output is not read next is ~3% faster
// streamed.  KEEP is a template parameter, chosen per launch: a run-time
// flag lets the compiler merge the two stores into one plain store and drop
// the streaming policy.
template <bool KEEP, int POL = kStoreNt>
__device__ __forceinline__ void st_out(float* p, f4 v) {
    if constexpr (KEEP) *reinterpret_cast<f4*>(p) = v;
    else st_stream<POL>(p, v);
}

// ---------------------------------------------------------------------------
// DPP wave reductions
// ---------------------------------------------------------------------------
enum : int {
    kDppQuadXor1 = 0xB1,      // quad_perm [1,0,3,2]
    kDppQuadXor2 = 0x4E,      // quad_perm [2,3,0,1]
    kDppRowHalfMirror = 0x141,
    kDppRowMirror = 0x140,
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes.  Every lane of a 16-lane row first holds its row
// sum (4 DPP steps), then the four row sums are combined in a fixed order.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<kDppQuadXor1>(v);
    v += dpp<kDppQuadXor2>(v);
    v += dpp<kDppRowHalfMirror>(v);
    v += dpp<kDppRowMirror>(v);
    return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

// Sum over aligned groups of W lanes (W = 16: a DPP row; W = 32: two rows):
// every lane of a group ends with the same value, since each step adds a
// partner's value to its own symmetrically.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(W == 16 || W == 32, "groups of 16 or 32 lanes");
    v += dpp<kDppQuadXor1>(v);
    v += dpp<kDppQuadXor2>(v);
    v += dpp<kDppRowHalfMirror>(v);
    v += dpp<kDppRowMirror>(v);
    if constexpr (W == 32) v += __shfl_xor(v, 16);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kDppQuadXor1>(v));
    v = fmaxf(v, dpp<kDppQuadXor2>(v));
    v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp<kDppRowMirror>(v));
    return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

// Reductions for a row spread over NW waves of a workgroup that holds
// several rows (row `sub` owns waves sub*NW .. sub*NW+NW-1).  `lds` holds one
// float per wave of the workgroup.  REUSE adds a leading barrier, needed when
// the same `lds` array served an earlier reduction of the kernel.
template <int NW, bool REUSE = true>
__device__ __forceinline__ float row_sum(float v, float* lds, int sub) {
    const float w = wave_sum(v);
    if constexpr (NW == 1) {
        return w;
    } else {
        if constexpr (REUSE) __syncthreads();
        if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = w;
        __syncthreads();
        float s = lds[sub * NW];
#pragma unroll
        for (int i = 1; i < NW; ++i) s += lds[sub * NW + i];
        return s;
    }
}

template <int NW>
__device__ __forceinline__ float row_max(float v, float* lds, int sub) {
    const float w = wave_max(v);
    if constexpr (NW == 1) {
        return w;
    } else {
        __syncthreads();
        if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = w;
        __syncthreads();
        float s = lds[sub * NW];
#pragma unroll
        for (int i = 1; i < NW; ++i) s = fmaxf(s, lds[sub * NW + i]);
        return s;
    }
}

// Whole-workgroup reductions (one row per workgroup of NW waves).
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* lds) {
    return row_sum<NW>(v, lds, 0);
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float* lds) {
    return row_max<NW>(v, lds, 0);
}

}  // namespace mimir
