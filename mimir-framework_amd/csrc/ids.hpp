// ids.hpp -- token ids as the reference reads them, shared by the gather
// (gather.hip) and its backward scatter-add (backward.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.hpp"

namespace mimir {

// static_cast<int>(std::llround(static_cast<double>(f))) as compiled for
// x86-64 with glibc (Model.cpp:5321, 7453): llround rounds half away from
// zero; values whose magnitude reaches 2^63, and NaN, convert to the x86
// "integer indefinite" 0x8000000000000000, whose low 32 bits are 0; the
// 64-bit result is then narrowed to int by keeping its low 32 bits.
__device__ __forceinline__ int32_t float_id(float f) {
    const double d = static_cast<double>(f);
    if (!(fabs(d) < 9223372036854775808.0)) return 0;
    const long long r = static_cast<long long>(round(d));
    return static_cast<int32_t>(static_cast<uint32_t>(static_cast<unsigned long long>(r)));
}

// Id modes: int32 ids (Model.cpp:1152-1205); float ids (Model.cpp:5301-5334);
// int32 ids read as float first, as the forwardPassView float path does when
// an Embedding's input comes from the int store (Model.cpp:4836-4840).
// The id a 32-bit word of the ids array holds (every mode reads 32 bits).
template <int MODE>
__device__ __forceinline__ int32_t id_from_word(uint32_t w) {
    if constexpr (MODE == kIdsF32) return float_id(__uint_as_float(w));
    else if constexpr (MODE == kIdsI32AsF32) return float_id(static_cast<float>(static_cast<int32_t>(w)));
    else return static_cast<int32_t>(w);
}

template <int MODE>
__device__ __forceinline__ int32_t load_id(const void* ids, int64_t t) {
    return id_from_word<MODE>(static_cast<const uint32_t*>(ids)[t]);
}

}  // namespace mimir
