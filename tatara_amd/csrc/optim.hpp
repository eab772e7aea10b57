// Element-wise optimizer arithmetic shared by every optimizer kernel.
//
// Follows crates/gpu-kernels/src/pointwise/radam_step.rs:116-149 (radam_step_cpu)
// and crates/gpu-kernels/src/pointwise/ranger_step.rs:52-59 (lookahead lerp)
// operation for operation; the library is built with -ffp-contract=off so no
// multiply-add is fused and the result is bit-identical to that CPU code.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tatara {

// Per-step scalars of one parameter group (host pre-computed).
struct OptScalars {
    float lr;         // scheduled lr x group lr_mult
    float step_size;  // RAdam rectified step size (AdamW: 1)
    int32_t denom;    // 1: divide by sqrt(v)+eps
    float decay;      // decoupled weight decay
    float beta1, beta2, eps;
    float min_w, max_w;
    int32_t lookahead;  // 1: apply the Ranger lerp after the update this step
    float alpha;        // lerp coefficient
};

struct OptState4 {
    float4 w, m, v;
};

__device__ __forceinline__ float radam_elem(float& w, float& m, float& v, float g,
                                            const OptScalars& s) {
    const float rate = s.lr * s.step_size;
    float p = w;
    p *= 1.0f - s.decay * rate;
    const float mi = s.beta1 * m + (1.0f - s.beta1) * g;
    const float vi = s.beta2 * v + (1.0f - s.beta2) * g * g;
    m = mi;
    v = vi;
    float val = mi;
    if (s.denom != 0) val /= sqrtf(vi) + s.eps;  // correctly rounded (llvm.sqrt.f32); __fsqrt_rn is native
    p -= rate * val;
    p = p < s.min_w ? s.min_w : (p > s.max_w ? s.max_w : p);
    w = p;
    return p;
}

__device__ __forceinline__ void lerp_elem(float& w, float& slow, float alpha) {
    const float nw = alpha * w + (1.0f - alpha) * slow;
    w = nw;
    slow = nw;
}

}  // namespace tatara
