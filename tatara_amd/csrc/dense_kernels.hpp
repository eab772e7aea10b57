// Host launchers of the LayerStack dense-layer kernels (see dense_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "loss.hpp"
#include "optim.hpp"

namespace tatara {

// The LayerStack dense shapes with kernels: l1 (L1 outputs, the last one the
// skip output) in {8, 16, 32}, l2 (L2 outputs) in {16, 32, 64}.
constexpr const char* kLsDenseShapes = "LayerStack l1 must be 8, 16 or 32 and l2 16, 32 or 64";
inline bool ls_dense_shape_ok(int64_t l1, int64_t l2) {
    return (l1 == 8 || l1 == 16 || l1 == 32) && (l2 == 16 || l2 == 32 || l2 == 64);
}

// Layout of the per-workgroup gradient partials written by the tail kernel.
struct TailDims {
    uint32_t l1, l2, nb;
    __host__ __device__ uint32_t l2_in() const { return 2 * (l1 - 1); }
    // cells per bucket: W2 (l2*l2_in), b2 (l2), W3 (l2), b3 (1), b1 (l1)
    __host__ __device__ uint32_t cells() const { return l2 * l2_in() + l2 + l2 + 1 + l1; }
    __host__ __device__ uint32_t off_w2() const { return 0; }
    __host__ __device__ uint32_t off_b2() const { return l2 * l2_in(); }
    __host__ __device__ uint32_t off_w3() const { return off_b2() + l2; }
    __host__ __device__ uint32_t off_b3() const { return off_w3() + l2; }
    __host__ __device__ uint32_t off_b1() const { return off_b3() + 1; }
};

constexpr uint32_t kChunkTiles = 16;     // 16-row tiles per L1 weight-gradient chunk
constexpr uint32_t kPostTiles = 4;       // 16-row tiles per L1-input/FT-post row block

struct LsDenseArgs {
    // shapes
    uint32_t batch, padded_b, ft_out, l1, l2, nb;
    // bucket sort
    const int32_t* perm;        // [padded_b] sorted row -> original row, -1 padding
    const int32_t* sorted_bin;  // [padded_b] bin (nb = invalid bucket), -1 padding
    const uint32_t* bin_start;  // [nb + 2]
    const uint32_t* bin_count;  // [nb + 1]
    // chunk table for the L1 weight gradient
    uint32_t* chunk_info;       // [max_chunks][3] (bin, first tile, n tiles); [max_chunks*3] = count,
                                // then [nb + 2] first chunk of each bin (last = count)
    uint32_t max_chunks;
    // activations
    const float* combined;      // [batch][ft_out]
    // TF32-class L1 products (the reference's --tf32; gfx950 has no TF32
    // matrix instructions): when non-null, `combined` is held as f16 here
    // (read instead of `combined`) and the L1 forward multiplies f16
    // operands (combined, f16-rounded weights) on the matrix cores with f32
    // sums; the L1 weight gradient takes the f16 `combined` with f32 dl1,
    // and the input gradient stays f32.
    const uint16_t* combined16;
    const float* ft_stm;        // [batch][ft_out] raw FT sums
    const float* ft_nstm;
    float* l1_sorted;           // [padded_b][2*l1]  bucket part | shared part (biases added)
    float* dl1_sorted;          // [padded_b][l1]
    float* net_output;          // [batch]
    float* dft;                 // chunk-major [ceil(ft_out/256)][2*batch][256]
    // f16 FT activations (the reference's --ft-fp16-out): raw sums read as f16,
    // dft written as f16(clamp(g * dft_scale, +-65504)) with every clamp counted
    const uint16_t* ft_stm16;   // [batch][ft_out], used instead of ft_stm / ft_nstm when non-null
    const uint16_t* ft_nstm16;
    uint16_t* dft16;            // chunk-major like dft, written instead of dft when non-null
    float dft_scale;
    unsigned long long* clamp_counter;
    // inputs
    const float* score;
    const float* wdl;
    float per_pos_norm;
    float wdl_lambda;
    LossParams loss;
    double* weight_sum;         // [1] extended WRM sum of weights
    // weights
    const float* ft_b;
    const float* l1_w;          // [nb][l1][ft_out]
    const float* l1_b;          // [nb][l1]
    const float* l1s_w;         // [ft_out][l1]
    const float* l1s_b;         // [l1]
    // the TF32 forward's weight operands (combined16 set), written from l1_w
    // and l1s_w at the start of each forward: f16 copies, l1s_w transposed
    // so that a lane's K values are consecutive
    uint16_t* l1_w16;           // [nb][l1][ft_out] f16
    uint16_t* l1s_wt16;         // [l1][ft_out] f16
    const float* l2_w;          // [nb][l2][l2_in]
    const float* l2_b;          // [nb][l2]
    const float* l3_w;          // [nb][l2]
    const float* l3_b;          // [nb]
    float ft_post_scale, l1_sqr_scale;
    // partials
    float* tail_partial;        // [n_tiles][cells], written for tiles of a valid bucket
    uint32_t* tail_seg;         // [nb + 1] first tile of each bin (bin nb: end of the last bucket)
    float* b1s_partial;         // [n_tiles][l1]
    double* loss_partial;       // [n_tiles]
    float* w1_partial;          // [max_chunks][l1][ft_out]
    float* ftb_partial;         // [n_post_wg][2][ft_out]
    double* loss_out;           // [1] reduced loss
    // fixed-order reductions of the partials
    float* tail_sum;            // [nb][cells]
    float* b1s_sum;             // [l1]
    float* ftb_sum;             // [2][ft_out]
    float* w1_seg;              // [nb + 1][l1][ft_out]
};

uint32_t ls_tail_workgroups(uint32_t padded_b);
uint32_t ls_post_workgroups(uint32_t padded_b);
uint32_t ls_max_chunks(uint32_t padded_b, uint32_t nb);

// Forward: L1 (bucket + shared) on sorted tiles.
int32_t launch_ls_l1_forward(const LsDenseArgs& a, hipStream_t stream);
// Extended WRM: sum of position weights (before the tail).
int32_t launch_wrm_weight_sum(const float* score, uint32_t n, const LossParams& lp, double* out,
                              double* scratch, hipStream_t stream);
// Tail: L1 glue, L2, L3, loss, and (train) their backward with gradient partials.
int32_t launch_ls_tail(const LsDenseArgs& a, int32_t train, hipStream_t stream);
// Backward: L1 weight-gradient partials (chunk table built on device).
int32_t launch_ls_l1_weight_grad(const LsDenseArgs& a, hipStream_t stream);
// Backward: L1 input gradient fused with the FT-post gradient -> dft, ft_b partials.
int32_t launch_ls_l1_input_post(const LsDenseArgs& a, hipStream_t stream);

// Reduces every dense-group gradient from its partials and applies the
// optimizer.  grads_out receives the gradients (keep_grads) or zeros.
struct LsDenseGroup {
    float *w, *m, *v, *slow, *grad;
    uint64_t n;
    float min_w, max_w;
    int32_t kind;  // 0 ft (unused here), 1 dense, 2 bias
};
int32_t launch_ls_dense_finalize(const LsDenseArgs& a, LsDenseGroup* groups /*9*/,
                                 const OptScalars& dense, const OptScalars& bias,
                                 int32_t apply_update, int32_t keep_grads, hipStream_t stream);
// Sums the tail loss partials into a.loss_out (deterministic order).
int32_t launch_ls_loss_reduce(const LsDenseArgs& a, hipStream_t stream);

// Deterministic column sums of a row-major partial matrix P[n_rows][n_cols]:
// out[s][c] = sum of P[r][c] over segment s, whose rows are
// [seg_rows[s], seg_rows[s+1]) (device array) or all rows when seg_rows is
// null (n_seg must then be 1).  The summation order is fixed.
int32_t launch_reduce_rows(const float* P, uint32_t n_rows, uint32_t n_cols,
                           const uint32_t* seg_rows, uint32_t n_seg, float* out, hipStream_t stream);
// out[0] = sum of partial[0..n) in index order (f64).
int32_t launch_sum_f64(const double* partial, uint32_t n, double* out, hipStream_t stream);

}  // namespace tatara
