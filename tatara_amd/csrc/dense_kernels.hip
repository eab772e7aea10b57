// LayerStack dense layers for gfx950.
//
// The batch is processed in the bucket-sorted order produced by the stable
// bin sort (every 16-row tile belongs to one bucket), as the reference's
// sorted L1 kernels do (crates/cuda-native-runtime/kernels/native_kernels.cu:
// 2394-2432, 2502-2589).  Per-row arithmetic follows the reference CPU
// functions in crates/gpu-kernels/src/layerstack/ (dense_mm.rs,
// dense_mm_bucket.rs, crelu.rs, abs_pow2_scale.rs, concat_l1sqr_main.rs,
// elementwise.rs, slice2d.rs, ft_post_perspective.rs) and the loss kernels in
// crates/gpu-kernels/src/pointwise/{loss_wdl,loss_wrm}.rs; the launch order is
// the one of GpuTrainer::forward/backward (bins/nnue_train/src/
// trainer_layerstack.rs:2038-3936).
//
// MFMA (v_mfma_f32_16x16x4_f32) is used for the FT->L1 contraction only: the
// L1 forward (bucket + shared weights, K = ft_out) and the L1 weight gradient
// (K = rows of the batch).  Everything reduced over the batch goes through
// per-workgroup partials that are summed in a fixed order, so a step is
// bit-reproducible run to run (no float atomics anywhere).
#include "dense_kernels.hpp"

#include "common.hpp"
#include "ft_kernels.hpp"

namespace tatara {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));


// ---------------------------------------------------------------------------
// L1 forward.  One wave per 16-row sorted tile (two with one bucket, the
// f32 form).
//   bucket part: l1_b[g] + combined . l1_w[g]^T   (accumulator starts at the bias,
//                as dense_mm_fwd_bucket_tiled_l1_sorted does); 0 for an invalid bucket
//   shared part: combined . l1s_w + l1s_b         (bias after the sum, as the
//                reference's sgemm + bias_add_per_row)
// MFMA operand layout (16x16x4 f32): lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; the result holds D[4*(l/16)+r][l%16] in element r.  Each lane
// loads float4 column runs and feeds their components to four successive
// MFMAs, which permutes the K order consistently for A and B.
// ---------------------------------------------------------------------------
// T (1 or 2) consecutive tiles of bucket `bin`: the weights of each K-block
// are loaded once for all T tiles.  NJ (1 or 2) blocks of 16 L1 outputs:
// lane i computes outputs i and 16 + i (l1 = 32) from the same row loads.
template <int T, int NJ>
__device__ __forceinline__ void ls_l1_fwd_tiles(const LsDenseArgs& a, uint32_t tile0, int32_t bin, uint32_t lane) {
    const uint32_t i = lane % 16, q = lane / 16;
    const uint32_t ft_out = a.ft_out, l1 = a.l1;
    const bool bvalid = (uint32_t)bin < a.nb;
    // Operands are loaded unconditionally from always-valid addresses (row 0,
    // bucket 0, column l1-1) and masked afterwards: a guarded load would be
    // split into predicated dword loads and lose the 16-byte accesses.
    bool jvalid[NJ], wbvalid[NJ];
    const float4* W1[NJ];
    const float* Ws[NJ];
    float binit[NJ];
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
        const uint32_t j = 16 * jt + i;
        jvalid[jt] = j < l1;
        wbvalid[jt] = bvalid && jvalid[jt];
        const uint32_t ic = jvalid[jt] ? j : l1 - 1;
        W1[jt] = reinterpret_cast<const float4*>(a.l1_w + ((uint64_t)(bvalid ? bin : 0) * l1 + ic) * ft_out);
        Ws[jt] = a.l1s_w + ic;
        binit[jt] = wbvalid[jt] ? a.l1_b[bin * l1 + j] : 0.0f;
    }
    const float4* X[T];
    bool xvalid[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int32_t orig = a.perm[(tile0 + t) * 16 + i];
        xvalid[t] = orig >= 0;
        X[t] = reinterpret_cast<const float4*>(a.combined + (uint64_t)(orig >= 0 ? orig : 0) * ft_out);
    }
    floatx4 accb[T][NJ], accs[T][NJ];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt) {
            accb[t][jt] = floatx4{binit[jt], binit[jt], binit[jt], binit[jt]};
            accs[t][jt] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // ft_out % 64 == 0: whole groups of kU K-blocks; a group's operands are
    // loaded before its MFMAs so each wave keeps several loads in flight
    const uint32_t nk = ft_out / 16;
    constexpr uint32_t kU = T * NJ == 1 ? 4 : 2;
    for (uint32_t kb0 = 0; kb0 < nk; kb0 += kU) {
        float4 x[kU][T], wb[kU][NJ];
        float ws[kU][NJ][4];
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) {
            const uint32_t kb = kb0 + u;
#pragma unroll
            for (int t = 0; t < T; ++t) x[u][t] = X[t][kb * 4 + q];
            const uint32_t k = kb * 16 + 4 * q;
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                wb[u][jt] = W1[jt][kb * 4 + q];
#pragma unroll
                for (int c = 0; c < 4; ++c) ws[u][jt][c] = Ws[jt][(uint64_t)(k + c) * l1];
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                const float4 wv = wbvalid[jt] ? wb[u][jt] : zero4;
                const bool jv = jvalid[jt];
                const float w0 = jv ? ws[u][jt][0] : 0.f, w1 = jv ? ws[u][jt][1] : 0.f;
                const float w2 = jv ? ws[u][jt][2] : 0.f, w3 = jv ? ws[u][jt][3] : 0.f;
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const float4 xv = xvalid[t] ? x[u][t] : zero4;
                    accb[t][jt] = mfma4(xv.x, wv.x, accb[t][jt]);
                    accs[t][jt] = mfma4(xv.x, w0, accs[t][jt]);
                    accb[t][jt] = mfma4(xv.y, wv.y, accb[t][jt]);
                    accs[t][jt] = mfma4(xv.y, w1, accs[t][jt]);
                    accb[t][jt] = mfma4(xv.z, wv.z, accb[t][jt]);
                    accs[t][jt] = mfma4(xv.z, w2, accs[t][jt]);
                    accb[t][jt] = mfma4(xv.w, wv.w, accb[t][jt]);
                    accs[t][jt] = mfma4(xv.w, w3, accs[t][jt]);
                }
            }
    }
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
        const uint32_t j = 16 * jt + lane % 16;
        if (j >= l1) continue;
        const float bs = a.l1s_b[j];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint64_t row = (uint64_t)(tile0 + t) * 16 + 4 * q + r;
                float* o = a.l1_sorted + row * 2 * l1;
                o[j] = bvalid ? accb[t][jt][r] : 0.0f;
                o[l1 + j] = accs[t][jt][r] + bs;
            }
    }
}

// The TF32 L1 forward's weight operands, once per forward: f16 copies of
// l1_w and of l1s_w transposed ([l1][ft_out], a lane's K values
// consecutive).  Thread i: bucket weight i, and shared weight i when
// i < l1 * ft_out (nb >= 1).  (The f32 forward reads the weights as they
// are: the transposed copy cost more than the strided loads it saved.)
__global__ __launch_bounds__(256) void ls_l1_weights_f16_kernel(LsDenseArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t n_w = (uint64_t)a.nb * a.l1 * a.ft_out, n_s = (uint64_t)a.l1 * a.ft_out;
    if (i >= n_w) return;
    reinterpret_cast<_Float16*>(a.l1_w16)[i] = (_Float16)a.l1_w[i];
    if (i < n_s) {
        const uint64_t j = i / a.ft_out, k = i % a.ft_out;  // transposed [j][k] <- [k][j]
        reinterpret_cast<_Float16*>(a.l1s_wt16)[i] = (_Float16)a.l1s_w[k * a.l1 + j];
    }
}

// One wave per pair of 16-row sorted tiles: both in one pass when they
// belong to one bucket, else (at a bucket boundary) one pass each; a tile
// of bin -1 (all padding) is skipped.
template <int NJ>
__global__ __launch_bounds__(256) void ls_l1_fwd_kernel(LsDenseArgs a) {
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t tile0 = (blockIdx.x * 4 + wave) * 2;
    const uint32_t n_tiles = (uint32_t)(a.padded_b / 16);
    if (tile0 >= n_tiles) return;
    const int32_t bin0 = scalar_load(a.sorted_bin + (uint64_t)tile0 * 16);
    const int32_t bin1 = tile0 + 1 < n_tiles ? scalar_load(a.sorted_bin + (uint64_t)(tile0 + 1) * 16) : -1;
    if (bin0 >= 0 && bin0 == bin1) {
        ls_l1_fwd_tiles<2, NJ>(a, tile0, bin0, lane);
    } else {
        if (bin0 >= 0) ls_l1_fwd_tiles<1, NJ>(a, tile0, bin0, lane);
        if (bin1 >= 0) ls_l1_fwd_tiles<1, NJ>(a, tile0 + 1, bin1, lane);
    }
}

// ---------------------------------------------------------------------------
// L1 forward with TF32-class products: f16 operands on the matrix cores
// (v_mfma_f32_16x16x32_f16, f32 sums).  Lane l supplies A[l%16][8(l/16)+e]
// (row l%16 of the tile, 8 consecutive K from the f16 `combined`, one
// 16-byte load) and B[8(l/16)+e][l%16] (output l%16: 8 consecutive K of its
// bucket weight row, rounded to f16, and 8 strided shared weights).  As the
// reference's tf32 path (per-bucket sgemm, then the bias,
// trainer_layerstack.rs:2388-2480) the bucket bias is added after the sum.
// ---------------------------------------------------------------------------
template <int NJ>
__global__ __launch_bounds__(256) void ls_l1_fwd_tf32_kernel(LsDenseArgs a) {
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t tile = blockIdx.x * 4 + wave;
    if ((uint64_t)tile * 16 >= a.padded_b) return;
    const int32_t bin = a.sorted_bin[tile * 16];
    if (bin < 0) return;  // trailing all-padding tile
    const uint32_t i = lane % 16, q = lane / 16;
    const uint32_t ft_out = a.ft_out, l1 = a.l1;
    const int32_t orig = a.perm[tile * 16 + i];
    const bool bvalid = (uint32_t)bin < a.nb;
    // unconditional loads from always-valid addresses, masked afterwards
    const bool xvalid = orig >= 0;
    const half8* X = reinterpret_cast<const half8*>(
        reinterpret_cast<const _Float16*>(a.combined16) + (uint64_t)(orig >= 0 ? orig : 0) * ft_out);
    bool jvalid[NJ], wbvalid[NJ];
    const half8 *W1[NJ], *Ws[NJ];
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
        const uint32_t j = 16 * jt + i;
        jvalid[jt] = j < l1;
        wbvalid[jt] = bvalid && jvalid[jt];
        const uint32_t ic = jvalid[jt] ? j : l1 - 1;
        W1[jt] = reinterpret_cast<const half8*>(reinterpret_cast<const _Float16*>(a.l1_w16) +
                                                ((uint64_t)(bvalid ? bin : 0) * l1 + ic) * ft_out);
        Ws[jt] = reinterpret_cast<const half8*>(reinterpret_cast<const _Float16*>(a.l1s_wt16) + (uint64_t)ic * ft_out);
    }
    floatx4 accb[NJ], accs[NJ];
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) accb[jt] = accs[jt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const half8 zero8 = {};
    // ft_out % 64 == 0: K blocks of 32, four loaded before their MFMAs
    const uint32_t nk = ft_out / 32;
    constexpr uint32_t kU = 4;
    for (uint32_t kb0 = 0; kb0 < nk; kb0 += kU) {
        half8 x[kU], wb[kU][NJ], wsh[kU][NJ];
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) {
            const uint32_t k8 = (kb0 + u) * 4 + q;
            x[u] = X[k8];
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                wb[u][jt] = W1[jt][k8];
                wsh[u][jt] = Ws[jt][k8];
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) {
            const half8 xv = xvalid ? x[u] : zero8;
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                accb[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, wbvalid[jt] ? wb[u][jt] : zero8, accb[jt], 0, 0, 0);
                accs[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv, jvalid[jt] ? wsh[u][jt] : zero8, accs[jt], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
        const uint32_t j = 16 * jt + lane % 16;
        if (j >= l1) continue;
        const float bb = bvalid ? a.l1_b[bin * l1 + j] : 0.0f;
        const float bs = a.l1s_b[j];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint64_t row = (uint64_t)tile * 16 + 4 * q + r;
            float* o = a.l1_sorted + row * 2 * l1;
            o[j] = bvalid ? accb[jt][r] + bb : 0.0f;
            o[l1 + j] = accs[jt][r] + bs;
        }
    }
}

// ---------------------------------------------------------------------------
// Extended-WRM weight sum (wrm_weight_sum, native_kernels.cu:520-544), as a
// deterministic two-level f64 reduction in position order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void wrm_weight_partial_kernel(const float* __restrict__ score,
                                                                 uint32_t n, LossParams lp,
                                                                 double* __restrict__ partial) {
    __shared__ double s[256];
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    s[threadIdx.x] = i < n ? (double)wrm_weight_dev(score[i], lp) : 0.0;
    __syncthreads();
    if (threadIdx.x == 0) {
        double acc = 0.0;
        for (int k = 0; k < 256; ++k) acc += s[k];
        partial[blockIdx.x] = acc;
    }
}

// out[0] = sum of partial[0..n): thread t adds t, t + 256, ... in order, then
// the 256 thread sums are combined by a fixed pairwise tree (deterministic).
__global__ __launch_bounds__(256) void sum_partials_f64_kernel(const double* __restrict__ partial,
                                                               uint32_t n, double* __restrict__ out) {
    __shared__ double s[256];
    const uint32_t t = threadIdx.x;
    double acc = 0.0;
    for (uint32_t k = t; k < n; k += 256) acc += partial[k];
    s[t] = acc;
    __syncthreads();
    for (uint32_t w = 128; w > 0; w >>= 1) {
        if (t < w) s[t] = s[t] + s[t + w];
        __syncthreads();
    }
    if (t == 0) *out = s[0];
}

// ---------------------------------------------------------------------------
// Tail: one 64-lane workgroup per sorted 16-row tile (one bucket, the tile's
// rows being bucket-sorted and 16-aligned).  Lane l serves row r = l % 16 with
// quarter q = l / 16: its eight L2 outputs o = 8q..8q+7 in the forward, the
// L2 inputs k = q, q+4, .. in the backward, the L1 outputs k = q, q+4, .. of
// the L1-tail gradient.  The bucket's L2/L3 weights are staged in LDS.  Every
// per-row sum keeps the reference order (k ascending for L2, o ascending for
// L3 and for the L2 input gradient); the gradient partials are per tile, rows
// in order, and are reduced per bucket over the bucket's tiles.
// ---------------------------------------------------------------------------
template <int L1, int L2>
__global__ __launch_bounds__(64) void ls_tail_kernel(LsDenseArgs a, int32_t train) {
    constexpr int LE = L1 - 1;
    constexpr int LIN = 2 * LE;
    constexpr int OQ = L2 / 4;             // L2 outputs per lane
    constexpr int KQ = (LIN + 3) / 4;      // L2 inputs per lane (backward)
    constexpr int JQ = L1 / 4;             // L1 outputs per lane (backward)
    static_assert(L2 % 4 == 0 && L1 % 4 == 0, "quarters");
    __shared__ float sW2[L2 * LIN];
    __shared__ float sB2[L2], sW3[L2];
    __shared__ float s_l2in[16][LIN + 1];
    __shared__ float s_l2a[16][L2 + 1];
    __shared__ float s_dl2o[16][L2 + 1];
    __shared__ float s_dl2pre[16][LIN + 1];
    __shared__ float s_dl1[16][L1 + 1];
    __shared__ float s_dy[16];
    __shared__ double s_loss[16];
    __shared__ int32_t s_real[16];

    const uint32_t lane = threadIdx.x;
    const uint32_t r = lane % 16, q = lane / 16;
    const uint64_t tile = blockIdx.x;
    const uint64_t row = tile * 16 + r;
    // the tile's bucket: its first row is real unless the tile is all padding
    const int32_t orig0 = a.perm[tile * 16];
    const int32_t bin = orig0 >= 0 ? a.sorted_bin[tile * 16] : -1;
    const bool bvalid = bin >= 0 && (uint32_t)bin < a.nb;
    const int g = bvalid ? bin : 0;
    if (bvalid) {
        const float* W2 = a.l2_w + (uint64_t)g * L2 * LIN;
        for (uint32_t i = lane; i < (uint32_t)(L2 * LIN); i += 64) sW2[i] = W2[i];
        if (lane < (uint32_t)L2) {
            sB2[lane] = a.l2_b[g * L2 + lane];
            sW3[lane] = a.l3_w[g * L2 + lane];
        }
    }
    const float b3 = bvalid ? a.l3_b[g] : 0.0f;
    const int32_t orig = a.perm[row];
    const bool real = orig >= 0;

    float l1t[L1], l2pre[LIN], l2in[LIN];
    float skip = 0.0f;
    if (real) {
        const float* l1v = a.l1_sorted + row * 2 * L1;
#pragma unroll
        for (int o = 0; o < L1; ++o) l1t[o] = l1v[o] + l1v[L1 + o];  // elementwise_add
        skip = l1t[L1 - 1];                                          // slice_extract_2d
#pragma unroll
        for (int k = 0; k < LE; ++k) {
            const float mk = l1t[k];
            l2pre[k] = mk * mk * a.l1_sqr_scale;  // abs_pow2_scale_fwd
            l2pre[LE + k] = mk;                   // concat_l1sqr_main_fwd
        }
#pragma unroll
        for (int k = 0; k < LIN; ++k) l2in[k] = crelu01(l2pre[k]);
    } else {
#pragma unroll
        for (int o = 0; o < L1; ++o) l1t[o] = 0.0f;
#pragma unroll
        for (int k = 0; k < LIN; ++k) l2pre[k] = l2in[k] = 0.0f;
    }
    __syncthreads();  // staged weights visible
    // L2 (dense_mm_fwd_bucket: the sum starts at the bias, k ascending) + CReLU
    float l2o[OQ];
#pragma unroll
    for (int j = 0; j < OQ; ++j) {
        const int o = OQ * q + j;
        float acc = bvalid ? sB2[o] : 0.0f;
        if (bvalid) {
#pragma unroll
            for (int k = 0; k < LIN; ++k) acc += l2in[k] * sW2[o * LIN + k];
        }
        l2o[j] = bvalid ? acc : 0.0f;
        s_l2a[r][o] = real ? crelu01(l2o[j]) : 0.0f;
    }
    if (q == 0) {
#pragma unroll
        for (int k = 0; k < LIN; ++k) s_l2in[r][k] = l2in[k];
        s_real[r] = real ? 1 : 0;
    }
    __syncthreads();
    if (q == 0) {
        // L3 (o ascending from the bias), net = l3 + skip, loss
        double loss_c = 0.0;
        float dy = 0.0f;
        if (real) {
            float l3 = 0.0f;
            if (bvalid) {
                l3 = b3;
#pragma unroll
                for (int o = 0; o < L2; ++o) l3 += s_l2a[r][o] * sW3[o];
            }
            const float net = l3 + skip;
            a.net_output[orig] = net;
            loss_c = position_loss(net, a.score[orig], a.wdl[orig], a.wdl_lambda, a.loss, a.per_pos_norm,
                                   a.weight_sum, a.batch, dy);
        }
        s_dy[r] = dy;
        s_loss[r] = loss_c;
    }
    __syncthreads();
    if (lane == 0) {
        double acc = 0.0;
        for (int k = 0; k < 16; ++k) acc += s_loss[k];
        a.loss_partial[tile] = acc;
    }
    if (!train) return;

    // backward: L3 input gradient and the L2 CReLU mask for this lane's outputs
    const float dy = s_dy[r];
#pragma unroll
    for (int j = 0; j < OQ; ++j) {
        const int o = OQ * q + j;
        float acc = 0.0f;  // dense_mm_bwd_input_bucket, out_dim 1
        if (bvalid) acc += dy * sW3[o];
        const float d = (l2o[j] > 0.0f && l2o[j] < 1.0f) ? acc : 0.0f;  // crelu_grad
        s_dl2o[r][o] = real ? d : 0.0f;
    }
    __syncthreads();
    // L2 input gradient for this lane's inputs (o ascending), masked by the L1-tail CReLU
#pragma unroll
    for (int i = 0; i < KQ; ++i) {
        const int k = (int)q + 4 * i;
        if (k >= LIN) break;
        float acc = 0.0f;
        if (bvalid) {
#pragma unroll
            for (int o = 0; o < L2; ++o) acc += s_dl2o[r][o] * sW2[o * LIN + k];
        }
        s_dl2pre[r][k] = (l2pre[k] > 0.0f && l2pre[k] < 1.0f) ? acc : 0.0f;
    }
    __syncthreads();
    // L1-tail gradient for this lane's L1 outputs
#pragma unroll
    for (int i = 0; i < JQ; ++i) {
        const int k = (int)q + 4 * i;
        float d = 0.0f;
        if (real) {
            if (k < LE) {
                const float from_sqr = 2.0f * l1t[k] * a.l1_sqr_scale * s_dl2pre[r][k];  // abs_pow2_scale_grad
                d = s_dl2pre[r][LE + k] + from_sqr;                                        // elementwise_add
            } else {
                d = dy;  // slice_scatter_2d of the skip gradient
            }
        }
        a.dl1_sorted[row * L1 + k] = d;
        s_dl1[r][k] = d;
    }
    __syncthreads();

    // per-tile gradient partials, rows in order (real rows only)
    if (bvalid) {
        const TailDims td{(uint32_t)L1, (uint32_t)L2, a.nb};
        const uint32_t cells = td.cells();
        float* part = a.tail_partial + tile * cells;
        for (uint32_t c = lane; c < cells; c += 64) {
            float acc = 0.0f;
            if (c < td.off_b2()) {
                const uint32_t o = c / LIN, k = c % LIN;
                for (int rr = 0; rr < 16; ++rr)
                    if (s_real[rr]) acc += s_l2in[rr][k] * s_dl2o[rr][o];
            } else if (c < td.off_w3()) {
                const uint32_t o = c - td.off_b2();
                for (int rr = 0; rr < 16; ++rr)
                    if (s_real[rr]) acc += s_dl2o[rr][o];
            } else if (c < td.off_b3()) {
                const uint32_t o = c - td.off_w3();
                for (int rr = 0; rr < 16; ++rr)
                    if (s_real[rr]) acc += s_l2a[rr][o] * s_dy[rr];
            } else if (c < td.off_b1()) {
                for (int rr = 0; rr < 16; ++rr)
                    if (s_real[rr]) acc += s_dy[rr];
            } else {
                const uint32_t o = c - td.off_b1();
                for (int rr = 0; rr < 16; ++rr)
                    if (s_real[rr]) acc += s_dl1[rr][o];
            }
            part[c] = acc;
        }
    }
    // shared L1 bias: every real row, including rows of an invalid bucket
    if (lane < (uint32_t)L1) {
        float acc = 0.0f;
        for (int rr = 0; rr < 16; ++rr)
            if (s_real[rr]) acc += s_dl1[rr][lane];
        a.b1s_partial[tile * L1 + lane] = acc;
    }
    // the bucket segments of the tile partials (first tile of each bin)
    if (tile == 0 && lane <= a.nb) a.tail_seg[lane] = a.bin_start[lane] / 16;
}

// ---------------------------------------------------------------------------
// Chunk table for the L1 weight gradient: every bin (including the invalid
// bin nb, whose rows still feed the shared weight) is split into chunks of at
// most kChunkTiles 16-row tiles.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ls_chunk_table_kernel(const uint32_t* __restrict__ bin_start,
                                                             const uint32_t* __restrict__ bin_count, uint32_t nb,
                                                             uint32_t max_chunks, uint32_t* __restrict__ info) {
    // the bins' tile ranges and first chunks (at most 17 bins: nb <= 16 plus
    // the invalid bin), then one thread per chunk entry
    __shared__ uint32_t s_t0[17], s_t1[17], s_first[18];
    const uint32_t t = threadIdx.x;
    if (t <= nb) {
        s_t0[t] = bin_start[t] / 16;
        s_t1[t] = (bin_start[t] + bin_count[t] + 15) / 16;
    }
    __syncthreads();
    if (t == 0) {
        uint32_t c = 0;
        for (uint32_t g = 0; g <= nb; ++g) {
            s_first[g] = c;
            const uint32_t n = s_t1[g] > s_t0[g] ? (s_t1[g] - s_t0[g] + kChunkTiles - 1) / kChunkTiles : 0u;
            c = c + n < max_chunks ? c + n : max_chunks;
        }
        s_first[nb + 1] = c;
    }
    __syncthreads();
    const uint32_t total = s_first[nb + 1];
    for (uint32_t ci = t; ci < total; ci += blockDim.x) {
        uint32_t g = 0;
        while (g < nb && s_first[g + 1] <= ci) ++g;  // the bin whose chunks hold ci
        const uint32_t tile = s_t0[g] + (ci - s_first[g]) * kChunkTiles;
        info[3 * ci + 0] = g;
        info[3 * ci + 1] = tile;
        info[3 * ci + 2] = min(kChunkTiles, s_t1[g] - tile);
    }
    uint32_t* seg = info + 3 * max_chunks + 1;  // seg[g] = first chunk of bin g, seg[nb+1] = end
    if (t <= nb + 1) seg[t] = s_first[t];
    if (t == 0) info[3 * max_chunks] = total;
}

// ---------------------------------------------------------------------------
// Deterministic column sums of a partial matrix P[rows][n_cols]:
// out[seg][c] = sum over the segment's rows of P[r][c].  Thread (c, phase)
// sums rows phase, phase + PH, ... sequentially; the PH phase sums are then
// combined by a fixed pairwise tree.  Segment s covers rows
// [seg_rows[s], seg_rows[s+1]) when seg_rows is given, else all rows.
// ---------------------------------------------------------------------------

// COLS columns per workgroup and 1024 / COLS phases: 64 columns (16 phases)
// for wide matrices, 16 columns (64 phases) for tall narrow ones.
template <uint32_t COLS>
__global__ __launch_bounds__(1024) void reduce_rows_kernel(const float* __restrict__ P, uint32_t n_rows,
                                                           uint32_t n_cols, const uint32_t* __restrict__ seg_rows,
                                                           float* __restrict__ out) {
    constexpr uint32_t PH = 1024 / COLS;
    __shared__ float part[PH][COLS];
    const uint32_t lane = threadIdx.x % COLS, phase = threadIdx.x / COLS;
    const uint32_t c = blockIdx.x * COLS + lane;
    const uint32_t seg = blockIdx.y;
    const uint32_t r0 = seg_rows ? seg_rows[seg] : 0;
    const uint32_t r1 = seg_rows ? seg_rows[seg + 1] : n_rows;
    float acc = 0.0f;
    if (c < n_cols) {
#pragma unroll 8
        for (uint32_t r = r0 + phase; r < r1; r += PH) acc += P[(uint64_t)r * n_cols + c];
    }
    part[phase][lane] = acc;
    __syncthreads();
    for (uint32_t w = PH / 2; w > 0; w >>= 1) {
        if (phase < w) part[phase][lane] = part[phase][lane] + part[phase + w][lane];
        __syncthreads();
    }
    if (phase == 0 && c < n_cols) out[(uint64_t)seg * n_cols + c] = part[0][lane];
}

// The reduce_rows_kernel shape for a matrix n_cols wide: 16-column
// workgroups for narrow matrices, and for tall ones whose 64-column
// workgroups would not fill the chip (fewer rows per thread).
void reduce_rows(const float* P, uint32_t n_rows, uint32_t n_cols, const uint32_t* seg_rows, uint32_t n_seg,
                 float* out, hipStream_t stream) {
    // (n_rows: all segments' rows; 0 when unknown on the host)
    const bool tall = n_rows >= 256ull * n_seg && (uint64_t)ceil_div(n_cols, 64) * n_seg < 256;
    if (n_cols <= 16 || tall)
        reduce_rows_kernel<16><<<dim3(ceil_div(n_cols, 16), n_seg), 1024, 0, stream>>>(P, n_rows, n_cols, seg_rows,
                                                                                      out);
    else
        reduce_rows_kernel<64><<<dim3(ceil_div(n_cols, 64), n_seg), 1024, 0, stream>>>(P, n_rows, n_cols, seg_rows,
                                                                                      out);
}

// ---------------------------------------------------------------------------
// L1 weight gradient partials: P[chunk][o][k] = sum over the chunk's rows of
// dl1[row][o] * combined[row][k].  One wave owns 64 columns; lane (k, q) loads
// a float4 of combined so block c of its four MFMAs holds columns k0+4k+c.
// TF32: `combined` read as f16 (as the forward stored it); dl1 and the
// products stay f32.
// ---------------------------------------------------------------------------
template <bool TF32, int NJ>
__global__ __launch_bounds__(256) void ls_l1_wgrad_kernel(LsDenseArgs a) {
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t n_chunks = a.chunk_info[3 * a.max_chunks];
    const uint32_t chunk = blockIdx.x;
    if (chunk >= n_chunks) return;
    const uint32_t k0 = (blockIdx.y * 4 + wave) * 64;
    if (k0 >= a.ft_out) return;
    const uint32_t t0 = a.chunk_info[3 * chunk + 1], nt = a.chunk_info[3 * chunk + 2];
    const uint32_t o = lane % 16, q = lane / 16, kk = lane % 16;
    const uint32_t l1 = a.l1, ft_out = a.ft_out;
    const bool kvalid = k0 + 4 * kk < ft_out;
    // NJ blocks of 16 L1 outputs (lane o: outputs o and 16 + o)
    bool ovalid[NJ];
    uint32_t oc[NJ];
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
        ovalid[jt] = 16 * jt + o < l1;
        oc[jt] = ovalid[jt] ? 16 * jt + o : 0;
    }
    floatx4 acc[NJ][4];
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[jt][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const uint32_t kc = kvalid ? k0 + 4 * kk : 0;  // always-valid column, masked below
    for (uint32_t tt = 0; tt < nt; ++tt) {
        // the tile's 16 rows are loaded before its 16 MFMAs (unconditional
        // loads from valid addresses, masked after the load)
        float4 xs[4];
        float ds[4][NJ];
        bool rvs[4];
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) {
            const uint64_t row = (uint64_t)(t0 + tt) * 16 + 4 * s + q;
            const int32_t orig = a.perm[row];
            rvs[s] = orig >= 0;
            const uint64_t xo = (uint64_t)(orig >= 0 ? orig : 0) * ft_out + kc;
            if constexpr (TF32) {
                typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                const h4 h = *reinterpret_cast<const h4*>(reinterpret_cast<const _Float16*>(a.combined16) + xo);
                xs[s] = make_float4((float)h.x, (float)h.y, (float)h.z, (float)h.w);
            } else {
                xs[s] = *reinterpret_cast<const float4*>(a.combined + xo);
            }
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) ds[s][jt] = a.dl1_sorted[row * l1 + oc[jt]];
        }
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) {
            const float4 x = (rvs[s] && kvalid) ? xs[s] : zero4;
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                const float d = ovalid[jt] ? ds[s][jt] : 0.0f;
                acc[jt][0] = mfma4(d, x.x, acc[jt][0]);
                acc[jt][1] = mfma4(d, x.y, acc[jt][1]);
                acc[jt][2] = mfma4(d, x.z, acc[jt][2]);
                acc[jt][3] = mfma4(d, x.w, acc[jt][3]);
            }
        }
    }
    if (!kvalid) return;
    float* P = a.w1_partial + (uint64_t)chunk * l1 * ft_out;
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t oo = 16 * jt + 4 * q + r;
            if (oo >= l1) continue;
            float* dst = P + (uint64_t)oo * ft_out + k0 + 4 * kk;
            dst[0] = acc[jt][0][r];
            dst[1] = acc[jt][1][r];
            dst[2] = acc[jt][2][r];
            dst[3] = acc[jt][3][r];
        }
}

// ---------------------------------------------------------------------------
// L1 input gradient fused with the FT-post gradient.
// dcombined[c] = sum_o dl1[o] * l1_w[g][o][c]  +  sum_o dl1[o] * l1s_w[c][o]
// (the reference's two input-gradient kernels, added as in
// ft_post_perspective_grad_fused), then the pairwise CReLU gradient into dft
// (native_kernels.cu:2260-2302).  Grid (column block, row block): a lane owns
// its columns of the combined output over kPostTiles sorted tiles (the L1
// gradient row is wave-uniform, the weights stay in registers) and writes
// its ft_b gradient partials per perspective for that row block.  The f16
// variant reads f16 raw sums and writes the f16 dft, scaled by dft_scale and
// clamped to +-65504 with a count of every clamp
// (ft_post_perspective_grad_fused_fp16, native_kernels.cu:2304-2352); the
// ft_b gradient stays unscaled f32.  For the f32 dft, two columns per lane
// with rows loaded four at a time measured 5% faster than one column per
// lane with all 16 rows loaded ahead (0.555 against 0.586 ms for the whole
// dense backward at ft_out 1536, b 65536), and faster than four columns per
// lane (193 VGPRs) or one workgroup per full row; for the f16 dft the
// one-column form stays faster (0.44 against 0.48 ms per launch).  The two
// 16-term input-gradient sums use
// fused multiply-adds (these layers are checked within tolerance, and their
// reference GPU kernels contract too).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float clamp_f16_range(float v, uint32_t& clamps) {
    if (v > 65504.0f) {
        ++clamps;
        return 65504.0f;
    }
    if (v < -65504.0f) {
        ++clamps;
        return -65504.0f;
    }
    return v;
}

// Each lane owns CPL consecutive combined columns c..c+CPL-1 (all on one
// perspective's half); a 128-lane block covers 128 * CPL columns
// (ft_out % (128 * CPL) == 0).  A tile's rows are taken in groups of RB, an
// even number of groups per tile.  A tile's row ids, dl1 rows and bin are
// loaded one tile ahead (lane r holds row r's id, lane i float4 i of the
// dl1 rows; readlane hands each lane a row's values, which are the same for
// every lane), and each group's raw-sum pairs are loaded while the group
// before it is computed (two register sets; the loads are unconditional,
// from row 0 where a row is padding, so the wait before a group counts only
// the loads issued after it).  H16: f16 raw sums and dft.
template <int L1, int CPL, int RB, bool H16>
__global__ __launch_bounds__(128) void ls_l1_input_post_c_kernel(LsDenseArgs a) {
    static_assert(16 % RB == 0 && (16 / RB) % 2 == 0, "an even number of RB-row groups per tile");
    constexpr int G = 16 / RB;
    constexpr int DL = 16 * L1 / 4;          // float4 of a tile's dl1 rows
    constexpr int NDL = (DL + 63) / 64;      // of them per lane
    static_assert(L1 % 4 == 0, "whole float4 of dl1 per row");
    const uint32_t ft_out = a.ft_out, half = ft_out / 2;
    const uint64_t batch = a.batch;
    const uint32_t c = (blockIdx.x * 128 + threadIdx.x) * CPL;
    if (c >= ft_out) return;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t persp = c < half ? 0 : 1;
    const uint32_t p = c - persp * half;
    const _Float16* ft16 = reinterpret_cast<const _Float16*>(persp ? a.ft_nstm16 : a.ft_stm16);
    const float* ft32 = persp ? a.ft_nstm : a.ft_stm;
    const uint64_t cstride = 2 * batch * kDftChunk;
    const uint64_t off_a = (uint64_t)(p / kDftChunk) * cstride + persp * batch * kDftChunk + p % kDftChunk;
    const uint64_t off_b =
        (uint64_t)((p + half) / kDftChunk) * cstride + persp * batch * kDftChunk + (p + half) % kDftChunk;
    float ws[CPL][L1];
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int o = 0; o < L1; ++o) ws[j][o] = a.l1s_w[(uint64_t)(c + j) * L1 + o];
    float ba[CPL], bb[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        ba[j] = a.ft_b[p + j];
        bb[j] = a.ft_b[p + half + j];
    }
    float w1[CPL][L1];
    int32_t cur_bin = -2;
    bool bvalid = false;
    float acc_a[CPL] = {}, acc_b[CPL] = {};
    uint32_t clamps = 0;
    const uint32_t tile0 = blockIdx.y * kPostTiles;
    const uint32_t tiles_total = (uint32_t)(a.padded_b / 16);
    const uint32_t n_tiles = tile0 < tiles_total ? min((uint32_t)kPostTiles, tiles_total - tile0) : 0u;
    auto tile_perm = [&](uint32_t tile) -> int32_t { return a.perm[(uint64_t)tile * 16 + (lane & 15u)]; };
    struct Dl1 {
        float4 v[NDL];
    };
    // float4 f of the tile's dl1 rows is element f / 64 of lane f % 64
    auto tile_dl1 = [&](uint32_t tile) -> Dl1 {
        Dl1 d;
        const float4* src = reinterpret_cast<const float4*>(a.dl1_sorted + (uint64_t)tile * 16 * L1);
#pragma unroll
        for (int k = 0; k < NDL; ++k) d.v[k] = src[(64 * k + lane) % DL];
        return d;
    };
    auto bcast_i = [](int32_t v, int l) -> int32_t { return __builtin_amdgcn_readlane(v, l); };
    auto bcast_f = [](float v, int l) -> float {
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
    };
    float xr[2][RB][CPL], yr[2][RB][CPL];
    // group G0's raw-sum pairs (row ids from PERMV) into register set BUF
#define TATARA_POST_LOAD(BUF, PERMV, G0)                                                      \
    _Pragma("unroll") for (int r = 0; r < RB; ++r) {                                         \
        const int32_t o_ = bcast_i((PERMV), (G0) * RB + r);                                  \
        const uint64_t base = (uint64_t)(o_ >= 0 ? o_ : 0) * ft_out + p;                      \
        if constexpr (CPL == 1) {                                                             \
            xr[BUF][r][0] = H16 ? (float)ft16[base] : ft32[base];                             \
            yr[BUF][r][0] = H16 ? (float)ft16[base + half] : ft32[base + half];               \
        } else if constexpr (H16) {                                                           \
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));                          \
            const h2 x_ = *reinterpret_cast<const h2*>(ft16 + base);                          \
            const h2 y_ = *reinterpret_cast<const h2*>(ft16 + base + half);                   \
            xr[BUF][r][0] = (float)x_.x;                                                      \
            xr[BUF][r][1] = (float)x_.y;                                                      \
            yr[BUF][r][0] = (float)y_.x;                                                      \
            yr[BUF][r][1] = (float)y_.y;                                                      \
        } else {                                                                              \
            const float2 x_ = *reinterpret_cast<const float2*>(ft32 + base);                  \
            const float2 y_ = *reinterpret_cast<const float2*>(ft32 + base + half);           \
            xr[BUF][r][0] = x_.x;                                                             \
            xr[BUF][r][1] = x_.y;                                                             \
            yr[BUF][r][0] = y_.x;                                                             \
            yr[BUF][r][1] = y_.y;                                                             \
        }                                                                                     \
    }
    int32_t perm_c = 0, bin_c = -1;
    Dl1 dl1_c = {};
    if (n_tiles) {
        perm_c = tile_perm(tile0);
        dl1_c = tile_dl1(tile0);
        bin_c = scalar_load(a.sorted_bin + (uint64_t)tile0 * 16);
        TATARA_POST_LOAD(0, perm_c, 0)
    }
    for (uint32_t t = 0; t < n_tiles; ++t) {
        const uint32_t tile = tile0 + t;
        const bool has_next = t + 1 < n_tiles;
        const uint32_t tn = has_next ? tile + 1 : tile;  // the last tile re-reads itself, unused
        const int32_t perm_n = tile_perm(tn);
        const Dl1 dl1_n = tile_dl1(tn);
        const int32_t bin_n = has_next ? scalar_load(a.sorted_bin + (uint64_t)tn * 16) : -1;
        const int32_t bin = bin_c;  // < 0: a trailing all-padding tile
        if (bin >= 0 && bin != cur_bin) {
            cur_bin = bin;
            bvalid = (uint32_t)bin < a.nb;
#pragma unroll
            for (int o = 0; o < L1; ++o) {
                const uint64_t i = ((uint64_t)bin * L1 + o) * ft_out + c;
                if constexpr (CPL == 2) {
                    const float2 w = bvalid ? *reinterpret_cast<const float2*>(a.l1_w + i) : make_float2(0.0f, 0.0f);
                    w1[0][o] = w.x;
                    w1[1][o] = w.y;
                } else {
                    w1[0][o] = bvalid ? a.l1_w[i] : 0.0f;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            // the next group's loads first: of this tile, or the next tile's first
            if (g + 1 < G) {
                TATARA_POST_LOAD((g + 1) & 1, perm_c, g + 1)
            } else {
                TATARA_POST_LOAD(0, perm_n, 0)
            }
            if (bin < 0) continue;
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const int row_in_tile = g * RB + r;
                const int32_t orig = bcast_i(perm_c, row_in_tile);
                if (orig < 0) continue;
                float d[L1];
#pragma unroll
                for (int o = 0; o < L1; ++o) {
                    const int e = row_in_tile * L1 + o, f4 = e >> 2;
                    const float4& v = dl1_c.v[f4 / 64];
                    const float comp = (e & 3) == 0 ? v.x : (e & 3) == 1 ? v.y : (e & 3) == 2 ? v.z : v.w;
                    d[o] = bcast_f(comp, f4 % 64);
                }
                float ga[CPL], gb[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    float da = 0.0f;
                    if (bvalid) {
#pragma unroll
                        for (int o = 0; o < L1; ++o) da = __builtin_fmaf(d[o], w1[j][o], da);
                    }
                    float db = 0.0f;
#pragma unroll
                    for (int o = 0; o < L1; ++o) db = __builtin_fmaf(d[o], ws[j][o], db);
                    const float dy = da + db;
                    const float xa = xr[g & 1][r][j] + ba[j], xb = yr[g & 1][r][j] + bb[j];
                    const float ya = crelu01(xa), yb = crelu01(xb);
                    ga[j] = (xa > 0.0f && xa < 1.0f) ? dy * yb * a.ft_post_scale : 0.0f;
                    gb[j] = (xb > 0.0f && xb < 1.0f) ? dy * ya * a.ft_post_scale : 0.0f;
                    acc_a[j] += ga[j];
                    acc_b[j] += gb[j];
                }
                const uint64_t row = (uint64_t)orig * kDftChunk;
                if constexpr (H16) {
                    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                    const float sc = a.dft_scale;
                    _Float16* d16 = reinterpret_cast<_Float16*>(a.dft16);
                    if constexpr (CPL == 2) {
                        h2 va, vb;
                        va.x = (_Float16)clamp_f16_range(ga[0] * sc, clamps);
                        va.y = (_Float16)clamp_f16_range(ga[1] * sc, clamps);
                        vb.x = (_Float16)clamp_f16_range(gb[0] * sc, clamps);
                        vb.y = (_Float16)clamp_f16_range(gb[1] * sc, clamps);
                        *reinterpret_cast<h2*>(d16 + off_a + row) = va;
                        *reinterpret_cast<h2*>(d16 + off_b + row) = vb;
                    } else {
                        d16[off_a + row] = (_Float16)clamp_f16_range(ga[0] * sc, clamps);
                        d16[off_b + row] = (_Float16)clamp_f16_range(gb[0] * sc, clamps);
                    }
                } else if constexpr (CPL == 2) {
                    *reinterpret_cast<float2*>(a.dft + off_a + row) = make_float2(ga[0], ga[1]);
                    *reinterpret_cast<float2*>(a.dft + off_b + row) = make_float2(gb[0], gb[1]);
                } else {
                    a.dft[off_a + row] = ga[0];
                    a.dft[off_b + row] = gb[0];
                }
            }
        }
        perm_c = perm_n;
        dl1_c = dl1_n;
        bin_c = bin_n;
    }
#undef TATARA_POST_LOAD
    float* pp = a.ftb_partial + ((uint64_t)blockIdx.y * 2 + persp) * ft_out;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        pp[p + j] = acc_a[j];
        pp[p + half + j] = acc_b[j];
    }
    if (H16 && clamps) atomicAdd(a.clamp_counter, (unsigned long long)clamps);
}

// ---------------------------------------------------------------------------
// Dense gradient finalize + optimizer: one thread per parameter element of
// the nine non-FT groups (uniform_optim_group_layout order,
// trainer_layerstack.rs:676-705).
// ---------------------------------------------------------------------------
struct GroupTable {
    LsDenseGroup g[9];
    uint64_t start[10];
};

__global__ __launch_bounds__(256) void ls_dense_finalize_kernel(LsDenseArgs a, GroupTable gt,
                                                                OptScalars dense, OptScalars bias,
                                                                int32_t apply_update,
                                                                int32_t keep_grads) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= gt.start[9]) return;
    int gi = 0;
    while (i >= gt.start[gi + 1]) ++gi;
    const uint64_t e = i - gt.start[gi];
    const uint32_t l1 = a.l1, l2 = a.l2, nb = a.nb, ft_out = a.ft_out;
    const TailDims td{l1, l2, nb};
    const uint32_t cells = td.cells();
    float grad = 0.0f;
    auto tail_sum = [&](uint32_t g, uint32_t cell) { return a.tail_sum[(uint64_t)g * cells + cell]; };
    switch (gi) {
        case 0:  // ft_b: stm sum then nstm sum
            grad = a.ftb_sum[e] + a.ftb_sum[ft_out + e];
            break;
        case 1:  // l1_w [nb][l1][ft_out]: bucket segments of the chunk partials
            grad = a.w1_seg[e];
            break;
        case 2: {  // l1_b [nb][l1]
            grad = tail_sum((uint32_t)(e / l1), td.off_b1() + (uint32_t)(e % l1));
            break;
        }
        case 3: {  // l1s_w [ft_out][l1]: every bin's segment, invalid bin included
            const uint32_t k = (uint32_t)(e / l1), o = (uint32_t)(e % l1);
            float s = 0.0f;
            for (uint32_t g = 0; g <= nb; ++g) s += a.w1_seg[((uint64_t)g * l1 + o) * ft_out + k];
            grad = s;
            break;
        }
        case 4:  // l1s_b [l1]
            grad = a.b1s_sum[e];
            break;
        case 5: {  // l2_w [nb][l2][l2_in]
            const uint32_t per = l2 * td.l2_in();
            grad = tail_sum((uint32_t)(e / per), td.off_w2() + (uint32_t)(e % per));
            break;
        }
        case 6:  // l2_b [nb][l2]
            grad = tail_sum((uint32_t)(e / l2), td.off_b2() + (uint32_t)(e % l2));
            break;
        case 7:  // l3_w [nb][l2]
            grad = tail_sum((uint32_t)(e / l2), td.off_w3() + (uint32_t)(e % l2));
            break;
        default:  // l3_b [nb]
            grad = tail_sum((uint32_t)e, td.off_b3());
            break;
    }
    const LsDenseGroup& G = gt.g[gi];
    if (!apply_update) {
        G.grad[e] = grad;
        return;
    }
    OptScalars s = G.kind == 2 ? bias : dense;
    s.min_w = G.min_w;
    s.max_w = G.max_w;
    float W = G.w[e], M = G.m[e], V = G.v[e];
    radam_elem(W, M, V, grad, s);
    if (s.lookahead) {
        float S = G.slow[e];
        lerp_elem(W, S, s.alpha);
        G.slow[e] = S;
    }
    G.w[e] = W;
    G.m[e] = M;
    G.v[e] = V;
    G.grad[e] = keep_grads ? grad : 0.0f;
}

}  // namespace

uint32_t ls_tail_workgroups(uint32_t padded_b) { return ceil_div(padded_b, 16); }
uint32_t ls_post_workgroups(uint32_t padded_b) { return ceil_div(padded_b / 16, kPostTiles); }
uint32_t ls_max_chunks(uint32_t padded_b, uint32_t nb) {
    return ceil_div(padded_b / 16, kChunkTiles) + nb + 1;
}

int32_t launch_ls_l1_forward(const LsDenseArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(a.l1 >= 2 && a.l1 <= 32, "l1 must be in [2, 32]");
    TATARA_REQUIRE(a.ft_out % 64 == 0, "ft_out must be a multiple of 64");
    const bool two = a.l1 > 16;  // two blocks of 16 outputs
    TATARA_REQUIRE(!a.combined16 || (a.l1_w16 && a.l1s_wt16), "the TF32 L1 forward needs its f16 weights");
    const uint32_t tiles = a.padded_b / 16;
    if (tiles == 0) return kOk;
    if (a.combined16) {
        const uint64_t n_w = (uint64_t)a.nb * a.l1 * a.ft_out;
        ls_l1_weights_f16_kernel<<<ceil_div(n_w, 256), 256, 0, stream>>>(a);
        TATARA_LAUNCHED("ls_l1_weights_f16");
        if (two)
            ls_l1_fwd_tf32_kernel<2><<<ceil_div(tiles, 4), 256, 0, stream>>>(a);
        else
            ls_l1_fwd_tf32_kernel<1><<<ceil_div(tiles, 4), 256, 0, stream>>>(a);
    } else if (two) {
        ls_l1_fwd_kernel<2><<<ceil_div(tiles, 8), 256, 0, stream>>>(a);
    } else {
        ls_l1_fwd_kernel<1><<<ceil_div(tiles, 8), 256, 0, stream>>>(a);
    }
    TATARA_LAUNCHED("ls_l1_forward");
    return kOk;
}

int32_t launch_wrm_weight_sum(const float* score, uint32_t n, const LossParams& lp, double* out,
                              double* scratch, hipStream_t stream) {
    const uint32_t blocks = ceil_div(n, 256);
    if (blocks) {
        wrm_weight_partial_kernel<<<blocks, 256, 0, stream>>>(score, n, lp, scratch);
        TATARA_LAUNCHED("wrm_weight_sum");
    }
    sum_partials_f64_kernel<<<1, 256, 0, stream>>>(scratch, blocks, out);
    TATARA_LAUNCHED("wrm_weight_sum_reduce");
    return kOk;
}

int32_t launch_ls_tail(const LsDenseArgs& a, int32_t train, hipStream_t stream) {
    TATARA_REQUIRE(a.nb <= 16, "num_buckets must be <= 16");
    TATARA_REQUIRE(a.padded_b % 16 == 0, "the sorted batch is whole 16-row tiles");
    const uint32_t blocks = ls_tail_workgroups(a.padded_b);
    if (blocks == 0) return kOk;
    // one instantiation per accepted (l1, l2)
#define TATARA_TAIL(L1_, L2_)                                            \
    if (a.l1 == L1_ && a.l2 == L2_) {                                    \
        ls_tail_kernel<L1_, L2_><<<blocks, 64, 0, stream>>>(a, train);   \
        TATARA_LAUNCHED("ls_tail");                                      \
        return kOk;                                                      \
    }
    TATARA_TAIL(8, 16)
    TATARA_TAIL(8, 32)
    TATARA_TAIL(8, 64)
    TATARA_TAIL(16, 16)
    TATARA_TAIL(16, 32)
    TATARA_TAIL(16, 64)
    TATARA_TAIL(32, 16)
    TATARA_TAIL(32, 32)
    TATARA_TAIL(32, 64)
#undef TATARA_TAIL
    TATARA_REQUIRE(false, kLsDenseShapes);
    return kOk;
}

int32_t launch_ls_l1_weight_grad(const LsDenseArgs& a, hipStream_t stream) {
    ls_chunk_table_kernel<<<1, 256, 0, stream>>>(a.bin_start, a.bin_count, a.nb, a.max_chunks,
                                               a.chunk_info);
    TATARA_LAUNCHED("ls_chunk_table");
    dim3 grid(a.max_chunks, ceil_div(a.ft_out, 256));
    TATARA_REQUIRE(a.l1 >= 2 && a.l1 <= 32, "l1 must be in [2, 32]");
    const bool two = a.l1 > 16;
    if (a.combined16)
        (two ? ls_l1_wgrad_kernel<true, 2> : ls_l1_wgrad_kernel<true, 1>)<<<grid, 256, 0, stream>>>(a);
    else
        (two ? ls_l1_wgrad_kernel<false, 2> : ls_l1_wgrad_kernel<false, 1>)<<<grid, 256, 0, stream>>>(a);
    TATARA_LAUNCHED("ls_l1_weight_grad");
    return kOk;
}

int32_t launch_ls_l1_input_post(const LsDenseArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(!a.dft16 || (a.ft_stm16 && a.ft_nstm16 && a.clamp_counter),
                   "an f16 dft needs the f16 raw sums and a clamp counter");
    const uint32_t rows = ls_post_workgroups(a.padded_b);
    if (rows == 0) return kOk;
    TATARA_REQUIRE(a.ft_out % 128 == 0, "ft_out must be a multiple of 128");
    TATARA_REQUIRE(a.l1 == 8 || a.l1 == 16 || a.l1 == 32, kLsDenseShapes);
    // two columns per lane (f32, l1 <= 16) where the 256-column blocks tile
    // ft_out; l1 = 32 keeps one column per lane (its 64 weights per column
    // stay in registers)
    const bool two = !a.dft16 && a.ft_out % 256 == 0 && a.l1 <= 16;
    const dim3 grid(a.ft_out / (two ? 256 : 128), rows);
    // f32: two columns per lane, rows four at a time; f16: one column per
    // lane, all 16 rows of a tile ahead (each measured fastest for its type)
    auto kernel = a.dft16 ? (a.l1 == 32   ? ls_l1_input_post_c_kernel<32, 1, 8, true>
                             : a.l1 == 16 ? ls_l1_input_post_c_kernel<16, 1, 8, true>
                                          : ls_l1_input_post_c_kernel<8, 1, 8, true>)
                  : two   ? (a.l1 == 16 ? ls_l1_input_post_c_kernel<16, 2, 4, false>
                                        : ls_l1_input_post_c_kernel<8, 2, 4, false>)
                          : (a.l1 == 32   ? ls_l1_input_post_c_kernel<32, 1, 4, false>
                             : a.l1 == 16 ? ls_l1_input_post_c_kernel<16, 1, 4, false>
                                          : ls_l1_input_post_c_kernel<8, 1, 4, false>);
    kernel<<<grid, 128, 0, stream>>>(a);
    TATARA_LAUNCHED("ls_l1_input_post");
    return kOk;
}

int32_t launch_ls_dense_finalize(const LsDenseArgs& a, LsDenseGroup* groups,
                                 const OptScalars& dense, const OptScalars& bias,
                                 int32_t apply_update, int32_t keep_grads, hipStream_t stream) {
    GroupTable gt;
    gt.start[0] = 0;
    for (int k = 0; k < 9; ++k) {
        gt.g[k] = groups[k];
        gt.start[k + 1] = gt.start[k] + groups[k].n;
    }
    const uint64_t n = gt.start[9];
    const TailDims td{a.l1, a.l2, a.nb};
    const uint32_t n_tail = ls_tail_workgroups(a.padded_b);
    const uint32_t n_post = ls_post_workgroups(a.padded_b);
    // bucket g's tile partials are the rows [tail_seg[g], tail_seg[g + 1])
    reduce_rows(a.tail_partial, n_tail, td.cells(), a.tail_seg, a.nb, a.tail_sum, stream);
    reduce_rows(a.b1s_partial, n_tail, a.l1, nullptr, 1, a.b1s_sum, stream);
    reduce_rows(a.ftb_partial, n_post, 2 * a.ft_out, nullptr, 1, a.ftb_sum, stream);
    reduce_rows(a.w1_partial, 0, a.l1 * a.ft_out, a.chunk_info + 3 * a.max_chunks + 1, a.nb + 1, a.w1_seg, stream);
    TATARA_LAUNCHED("reduce_rows");
    ls_dense_finalize_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(a, gt, dense, bias, apply_update,
                                                                    keep_grads);
    TATARA_LAUNCHED("ls_dense_finalize");
    return kOk;
}

int32_t launch_ls_loss_reduce(const LsDenseArgs& a, hipStream_t stream) {
    return launch_sum_f64(a.loss_partial, ls_tail_workgroups(a.padded_b), a.loss_out, stream);
}

int32_t launch_reduce_rows(const float* P, uint32_t n_rows, uint32_t n_cols,
                           const uint32_t* seg_rows, uint32_t n_seg, float* out, hipStream_t stream) {
    TATARA_REQUIRE(seg_rows || n_seg == 1, "reduce_rows: n_seg must be 1 without segments");
    if (n_cols == 0 || n_seg == 0) return kOk;
    reduce_rows(P, n_rows, n_cols, seg_rows, n_seg, out, stream);
    TATARA_LAUNCHED("reduce_rows");
    return kOk;
}

int32_t launch_sum_f64(const double* partial, uint32_t n, double* out, hipStream_t stream) {
    sum_partials_f64_kernel<<<1, 256, 0, stream>>>(partial, n, out);
    TATARA_LAUNCHED("sum_f64");
    return kOk;
}

}  // namespace tatara
