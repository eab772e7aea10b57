// Per-position loss and output gradient, shared by the LayerStack and Simple
// output kernels.
//
// Restates loss_wdl_cpu (crates/gpu-kernels/src/pointwise/loss_wdl.rs) and
// loss_wrm_cpu (crates/gpu-kernels/src/pointwise/loss_wrm.rs, the plain and the
// extended form) operation for operation; LossKind is
// crates/nnue-train/src/trainer.rs:89-221.  The library is built with
// -ffp-contract=off and every exp is ref_expf (glibc's expf, what the
// reference's CPU path calls), so for the same net output the sigmoid, the
// WRM transforms, the error and the plain losses' gradient are the reference
// CPU values bit for bit; powf (extended WRM only) is the device library's.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ref_expf.hpp"

namespace tatara {

// Loss selection, mirroring LossKind.
struct LossParams {
    int32_t kind;  // 0 sigmoid-MSE, 1 WRM
    float scale;   // sigmoid
    float nnue2score, in_scaling, in_offset, target_offset, target_scaling;
    float pow_exp, qp_asymmetry, w1, w2;
    int32_t extended;  // WRM extended form (pow != 2 || asym != 0 || w1 != 0)
};

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + ref_expf(-x)); }

// Extended-WRM position weight (wrm_weight_sum, native_kernels.cu:520-544).
__device__ __forceinline__ float wrm_weight_dev(float s, const LossParams& lp) {
    const float tp = 1.0f / (1.0f + ref_expf(-((s - lp.target_offset) / lp.target_scaling)));
    const float tn = 1.0f / (1.0f + ref_expf(-((-s - lp.target_offset) / lp.target_scaling)));
    const float t = 0.5f * (1.0f + tp - tn);
    const float wb = (t - 0.5f) * (t - 0.5f) * t * (1.0f - t);
    return 1.0f + (powf(2.0f, lp.w1) - 1.0f) * powf(wb, lp.w2);
}

// Loss contribution of one position (what the reference adds to its f64
// accumulator) and the gradient of the loss with respect to the net output.
// weight_sum is the extended-WRM sum of position weights over the batch.
__device__ __forceinline__ double position_loss(float net, float sc, float wd, float lam,
                                                const LossParams& lp, float per_pos_norm,
                                                const double* weight_sum, uint32_t batch,
                                                float& dy) {
    if (lp.kind == 0) {
        const float p = sigmoidf_(net * lp.scale);
        const float ys = sigmoidf_(sc * lp.scale);
        const float y = lam * wd + (1.0f - lam) * ys;
        const float err = p - y;
        dy = 2.0f * err * p * (1.0f - p) * lp.scale * per_pos_norm;
        return (double)err * (double)err;
    }
    const float tp = 1.0f / (1.0f + ref_expf(-((sc - lp.target_offset) / lp.target_scaling)));
    const float tn = 1.0f / (1.0f + ref_expf(-((-sc - lp.target_offset) / lp.target_scaling)));
    const float twrm = 0.5f * (1.0f + tp - tn);
    const float target = lam * wd + (1.0f - lam) * twrm;
    const float sn = net * lp.nnue2score;
    const float q = 1.0f / (1.0f + ref_expf(-((sn - lp.in_offset) / lp.in_scaling)));
    const float qm = 1.0f / (1.0f + ref_expf(-((-sn - lp.in_offset) / lp.in_scaling)));
    const float pred = 0.5f * (1.0f + q - qm);
    const float err = pred - target;
    if (!lp.extended) {
        dy = err * (lp.nnue2score / lp.in_scaling) * (q * (1.0f - q) + qm * (1.0f - qm)) * per_pos_norm;
        return (double)err * (double)err;
    }
    const float wb = (twrm - 0.5f) * (twrm - 0.5f) * twrm * (1.0f - twrm);
    const float weight = 1.0f + (powf(2.0f, lp.w1) - 1.0f) * powf(wb, lp.w2);
    const float asym = pred > target ? 1.0f + lp.qp_asymmetry : 1.0f;
    const float ae = fabsf(err);
    const float ap = powf(ae, lp.pow_exp - 1.0f);
    const float sp = err < 0.0f ? -ap : ap;
    const float inv = (float)(1.0 / weight_sum[0]);
    const float pg = 0.5f * (lp.nnue2score / lp.in_scaling) * (q * (1.0f - q) + qm * (1.0f - qm));
    dy = (weight * inv) * (asym * lp.pow_exp * sp) * pg;
    return (double)(asym * powf(ae, lp.pow_exp) * weight * (float)batch * inv);
}

}  // namespace tatara
