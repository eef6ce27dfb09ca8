// pointwise.hpp -- the per-element functions of the path's activation layers
// and of fused elementwise chains, shared by every kernel that applies them
// (elementwise.hip, and the LayerNorm epilogue in norm.hip), so a value has
// the same bits whichever kernel computes it.
#pragma once

#include "common.hpp"
#include "internal.hpp"

#include <math.h>

namespace mimir {

// LayerOps::gelu_forward, LayerOps.hpp:556-568, computes
//   y = x * 0.5f*(1 + tanhf(u)),  u = sqrt(2/pi)*(x + 0.044715f*x^3)
// with the float sqrt of the float quotient as the constant.  Since
// 0.5*(1 + tanh(u)) = 1/(1 + exp(-2u)) exactly, this evaluates the
// logistic form: one expf and one hardware reciprocal (v_rcp_f32, 1 ulp)
// instead of the branchy tanhf, which left the op compute-bound on MI355X.
// It is also the better-conditioned form: the reference's 1 + tanhf(u)
// cancels for x < -3 (absolute error <= 1.5e-7 there), so the two agree to
// the path's tolerance everywhere, including the -0 / +-inf / NaN cases
// (exp overflow gives x * 0).
__device__ __forceinline__ float gelu1(float x) {
    const float k = __builtin_sqrtf(2.0f / 3.14159265359f);
    const float u = k * (x + 0.044715f * x * x * x);
    return x * __builtin_amdgcn_rcpf(1.0f + expf(-2.0f * u));
}

// LayerOps::silu_forward, LayerOps.hpp:570-581: y = x * (1/(1 + exp(-x))),
// with the reciprocal taken by v_rcp_f32 (1 ulp).
__device__ __forceinline__ float silu1(float x) {
    const float sigmoid = __builtin_amdgcn_rcpf(1.0f + expf(-x));
    return x * sigmoid;
}

// One step of a fused chain on four consecutive elements: GELU / SiLU of
// the value, or the value plus / times the operand (an Add or Multiply
// layer's single IEEE operation, whichever input the value was).
__device__ __forceinline__ f4 fuse_step4(int32_t kind, f4 v, f4 w) {
    switch (kind) {
        case kFuseGelu: return f4{gelu1(v.x), gelu1(v.y), gelu1(v.z), gelu1(v.w)};
        case kFuseSilu: return f4{silu1(v.x), silu1(v.y), silu1(v.z), silu1(v.w)};
        case kFuseAdd: return f4{v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w};
        default: return f4{v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w};
    }
}

__device__ __forceinline__ float fuse_step1(int32_t kind, float v, float w) {
    switch (kind) {
        case kFuseGelu: return gelu1(v);
        case kFuseSilu: return silu1(v);
        case kFuseAdd: return v + w;
        default: return v * w;
    }
}

}  // namespace mimir
