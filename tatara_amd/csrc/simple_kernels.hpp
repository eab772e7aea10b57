// Host launchers of the Simple-architecture dense kernels (see simple_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "loss.hpp"
#include "optim.hpp"

namespace tatara {

// The Simple dense shapes with kernels: l1 (first hidden layer) in
// {8, 16, 32}, l2 (second) in {16, 32, 64}; "512x2-8-64" is (8, 64).
constexpr const char* kSimpleDenseShapes = "Simple l1 must be 8, 16 or 32 and l2 16, 32 or 64";
inline bool simple_dense_shape_ok(int64_t l1, int64_t l2) {
    return (l1 == 8 || l1 == 16 || l1 == 32) && (l2 == 16 || l2 == 32 || l2 == 64);
}

// Per-workgroup gradient partials of the Simple output kernel, in this order:
// l2_w [l1][l2], l2_b [l2], l3_w [l2], l3_b [1], l1_b [l1].
struct SimpleTailDims {
    uint32_t l1, l2;
    __host__ __device__ uint32_t off_w2() const { return 0; }
    __host__ __device__ uint32_t off_b2() const { return l1 * l2; }
    __host__ __device__ uint32_t off_w3() const { return off_b2() + l2; }
    __host__ __device__ uint32_t off_b3() const { return off_w3() + l2; }
    __host__ __device__ uint32_t off_b1() const { return off_b3() + 1; }
    __host__ __device__ uint32_t cells() const { return off_b1() + l1; }
};

constexpr uint32_t kSimpleChunkRows = 256;   // rows per L1 weight-gradient chunk
// rows per L1-input/FT-post workgroup: 64 keeps twice the waves of 128 in
// flight (Simple 256x2-32-32, b = 65536: dense backward 0.145 against
// 0.187 ms; 32 rows, 0.149 ms plus the larger partial reduction)
constexpr uint32_t kSimplePostRows = 64;

struct SimpleDenseArgs {
    uint32_t batch, ft_out, l1, l2;
    const float* combined;  // [batch][2*ft_out] CReLU of both perspectives
    const float* ft_stm;    // [batch][ft_out] FT sums with the bias added
    const float* ft_nstm;
    float* l1_pre;          // [batch][l1]
    float* dl1;             // [batch][l1] gradient at the L1 pre-activation
    float* net_output;      // [batch]
    float* dft;             // chunk-major [ceil(ft_out/256)][2*batch][256]
    const float* score;
    const float* wdl;
    float per_pos_norm, wdl_lambda;
    LossParams loss;
    const double* weight_sum;
    const float* l1_w;  // [2*ft_out][l1]
    const float* l1_b;  // [l1]
    const float* l2_w;  // [l1][l2]
    const float* l2_b;  // [l2]
    const float* l3_w;  // [l2]
    const float* l3_b;  // [1]
    float* tail_partial;   // [n_tail][cells]
    double* loss_partial;  // [n_tail]
    float* w1_partial;     // [n_chunks][2*ft_out*l1]
    float* ftb_partial;    // [n_post][ft_out]
    float* tail_sum;       // [cells]
    float* w1_sum;         // [2*ft_out*l1]
    float* ftb_sum;        // [ft_out]
    double* loss_out;
};

uint32_t simple_tail_workgroups(uint32_t batch);
uint32_t simple_chunks(uint32_t batch);
uint32_t simple_post_workgroups(uint32_t batch);

// L1 forward (MFMA): l1_pre = combined . l1_w + l1_b.
int32_t launch_simple_l1_forward(const SimpleDenseArgs& a, hipStream_t stream);
// CReLU, L2, CReLU, L3, loss; with train, the backward to dl1 and the
// per-workgroup partials of the l2/l3/l1-bias gradients.
int32_t launch_simple_tail(const SimpleDenseArgs& a, int32_t train, hipStream_t stream);
// L1 weight-gradient chunk partials (MFMA).
int32_t launch_simple_l1_weight_grad(const SimpleDenseArgs& a, hipStream_t stream);
// dcombined = dl1 . l1_w^T fused with the CReLU gradient into dft and the
// ft_b gradient partials.
int32_t launch_simple_l1_input_post(const SimpleDenseArgs& a, hipStream_t stream);

struct SimpleDenseGroup {
    float *w, *m, *v, *slow, *grad;
    uint64_t n;
    float min_w, max_w;
    int32_t kind;  // 1 dense, 2 bias
};
// Reduces the partials and applies the optimizer to ft_b, l1_w, l1_b, l2_w,
// l2_b, l3_w, l3_b (in that order in groups[7]).
int32_t launch_simple_dense_finalize(const SimpleDenseArgs& a, SimpleDenseGroup* groups,
                                     const OptScalars& dense, const OptScalars& bias,
                                     int32_t keep_grads, hipStream_t stream);

}  // namespace tatara
