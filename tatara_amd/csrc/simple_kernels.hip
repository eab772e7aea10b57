// Simple architecture (FT -> L1 -> L2 -> L3 with CReLU) dense layers for gfx950.
//
// Forward/backward follow SimpleGpuTrainer::run_forward_kernels /
// run_backward_kernels (bins/nnue_train/src/trainer_simple.rs:857-2347):
// combined = [crelu(ft_stm + b), crelu(ft_nstm + b)] of width 2*ft_out, then
// row-major x . W + bias layers (W stored [in][out], as the cuBLAS row-major
// wrappers of trainer_common.rs:752-860 read it), the loss, and the chain rule
// back to dft.  Per-element arithmetic restates the CPU functions the
// reference pins those layers to (crates/gpu-kernels/src/layerstack/
// dense_mm.rs, crelu.rs; loss_wdl.rs / loss_wrm.rs): a dense sum starts at the
// bias and adds k in ascending order.
//
// MFMA (v_mfma_f32_16x16x4_f32) carries the two FT->L1 contractions (the L1
// forward, K = 2*ft_out, and the L1 weight gradient, K = rows); the tiny L2/L3
// layers run one 64-lane workgroup per 16-row tile, four lanes per row.  Batch reductions go through per-workgroup
// partials summed in a fixed order: no float atomics, bit-reproducible steps.
#include "simple_kernels.hpp"

#include "common.hpp"
#include "dense_kernels.hpp"
#include "ft_kernels.hpp"

namespace tatara {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// L1 forward: one wave per 16-row tile, ceil(L1/16) output blocks of 16
// columns (l1 = 8: the lanes of outputs 8..15 load column 7 and drop it).
// MFMA operand layout (16x16x4 f32): lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; element r of the result is D[4*(l/16)+r][l%16].  Lane (i, q)
// loads a float4 of row i at k = 16*kb + 4q and feeds its components to four
// successive MFMAs with the matching rows k..k+3 of W.
// ---------------------------------------------------------------------------
template <int L1>
__global__ __launch_bounds__(256) void simple_l1_fwd_kernel(SimpleDenseArgs a) {
    constexpr int NB = (L1 + 15) / 16;
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t tile = blockIdx.x * 4 + wave;
    const uint32_t batch = a.batch;
    if (tile * 16 >= batch) return;
    const uint32_t i = lane % 16, q = lane / 16;
    const uint32_t K = 2 * a.ft_out;
    const uint32_t row_a = tile * 16 + i;
    // rows past the batch load row 0 (always valid) and are zeroed after the
    // load: a guarded load would be split into predicated dword loads
    const bool xvalid = row_a < batch;
    const float4* X = reinterpret_cast<const float4*>(a.combined + (uint64_t)(xvalid ? row_a : 0) * K);
    // lane i's output in block nb (always-valid column; outputs >= L1 are
    // computed from zeroed weights and not stored)
    const uint32_t ic = i < (uint32_t)L1 ? i : L1 - 1;
    const bool ivalid = i < (uint32_t)L1;
    floatx4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const float b = a.l1_b[16 * nb + ic];  // dense_mm_fwd_cpu: the sum starts at the bias
        acc[nb] = floatx4{b, b, b, b};
    }
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // K / 16 is a multiple of kU (ft_out % 32 == 0); a group's operands are
    // loaded before its MFMAs so each wave keeps several loads in flight
    const uint32_t nk = K / 16;
    constexpr uint32_t kU = 4;
    for (uint32_t kb0 = 0; kb0 < nk; kb0 += kU) {
        float4 x[kU];
        float w[kU][4][NB];
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) {
            const uint32_t kb = kb0 + u;
            x[u] = X[kb * 4 + q];
            const float* wp = a.l1_w + (uint64_t)(kb * 16 + 4 * q) * L1 + ic;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const float wv = wp[c * L1 + 16 * nb];
                    w[u][c][nb] = (L1 % 16 == 0 || ivalid) ? wv : 0.0f;
                }
        }
#pragma unroll
        for (uint32_t u = 0; u < kU; ++u) {
            const float4 xv = xvalid ? x[u] : zero4;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                acc[nb] = mfma4(xv.x, w[u][0][nb], acc[nb]);
                acc[nb] = mfma4(xv.y, w[u][1][nb], acc[nb]);
                acc[nb] = mfma4(xv.z, w[u][2][nb], acc[nb]);
                acc[nb] = mfma4(xv.w, w[u][3][nb], acc[nb]);
            }
        }
    }
    // the bias seeded every row of column i; lane (j = i, q) holds rows 4q + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t row = tile * 16 + 4 * q + r;
        if (row >= batch) continue;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            if (L1 % 16 == 0 || ivalid) a.l1_pre[(uint64_t)row * L1 + 16 * nb + i] = acc[nb][r];
    }
}

// ---------------------------------------------------------------------------
// Tail: one 64-lane workgroup per 16-row tile.  Lane l serves row r = l % 16
// with quarter q = l / 16: L2 outputs o = 8q..8q+7 in the forward, L1 inputs
// k = q, q+4, .. in the backward.  The weights are staged in LDS.  Every
// per-row sum keeps the reference order (k ascending for L2, o ascending for
// L3 and the L2 input gradient); the gradient partials are per tile, rows in
// order.
// ---------------------------------------------------------------------------
template <int L1, int L2>
__global__ __launch_bounds__(64) void simple_tail_kernel(SimpleDenseArgs a, int32_t train) {
    constexpr int OQ = L2 / 4;  // L2 outputs per lane
    constexpr int KQ = L1 / 4;  // L1 inputs per lane (backward)
    static_assert(L1 % 4 == 0 && L2 % 4 == 0, "quarters");
    __shared__ float sW2[L1 * L2];
    __shared__ float sB2[L2], sW3[L2];
    __shared__ float s_l1p[16][L1 + 1];
    __shared__ float s_l1a[16][L1 + 1];
    __shared__ float s_l2a[16][L2 + 1];
    __shared__ float s_dl2[16][L2 + 1];
    __shared__ float s_dl1[16][L1 + 1];
    __shared__ float s_dy[16];
    __shared__ double s_loss[16];

    const uint32_t lane = threadIdx.x;
    const uint32_t r = lane % 16, q = lane / 16;
    const uint64_t tile = blockIdx.x;
    const uint64_t row = tile * 16 + r;
    const bool real = row < a.batch;
    for (uint32_t i = lane; i < (uint32_t)(L1 * L2); i += 64) sW2[i] = a.l2_w[i];
    if (lane < (uint32_t)L2) {
        sB2[lane] = a.l2_b[lane];
        sW3[lane] = a.l3_w[lane];
    }
    // the tile's L1 pre-activations, read once and coalesced; padding rows are zero
    const float* src = a.l1_pre + tile * 16 * L1;
    for (uint32_t i = lane; i < (uint32_t)(16 * L1); i += 64) {
        const uint32_t rr = i / L1, k = i % L1;
        const float v = tile * 16 + rr < a.batch ? src[i] : 0.0f;
        s_l1p[rr][k] = v;
        s_l1a[rr][k] = crelu01(v);
    }
    __syncthreads();  // staged weights and activations visible
    // k outermost: every output's sum still adds k in ascending order
    float l2p[OQ];
#pragma unroll
    for (int j = 0; j < OQ; ++j) l2p[j] = sB2[OQ * q + j];
#pragma unroll 4
    for (int k = 0; k < L1; ++k) {
        const float x = s_l1a[r][k];
        const float* w = sW2 + k * L2 + OQ * q;
#pragma unroll
        for (int j = 0; j < OQ; ++j) l2p[j] += x * w[j];
    }
#pragma unroll
    for (int j = 0; j < OQ; ++j) s_l2a[r][OQ * q + j] = real ? crelu01(l2p[j]) : 0.0f;
    __syncthreads();
    if (q == 0) {
        double loss_c = 0.0;
        float dy = 0.0f;
        if (real) {
            float net = a.l3_b[0];
#pragma unroll
            for (int k = 0; k < L2; ++k) net += s_l2a[r][k] * sW3[k];
            a.net_output[row] = net;
            loss_c = position_loss(net, a.score[row], a.wdl[row], a.wdl_lambda, a.loss, a.per_pos_norm,
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

    const float dy = s_dy[r];
#pragma unroll
    for (int j = 0; j < OQ; ++j) {
        const int o = OQ * q + j;
        const float g = dy * sW3[o];                                  // x . W^T with out_dim 1
        const float d = (l2p[j] > 0.0f && l2p[j] < 1.0f) ? g : 0.0f;  // crelu_grad
        s_dl2[r][o] = real ? d : 0.0f;
    }
    __syncthreads();
    // o outermost: every input's sum still adds o in ascending order
    float g1[KQ];
#pragma unroll
    for (int i = 0; i < KQ; ++i) g1[i] = 0.0f;
#pragma unroll 4
    for (int o = 0; o < L2; ++o) {
        const float d = s_dl2[r][o];
#pragma unroll
        for (int i = 0; i < KQ; ++i) g1[i] += d * sW2[((int)q + 4 * i) * L2 + o];
    }
#pragma unroll
    for (int i = 0; i < KQ; ++i) {
        const int k = (int)q + 4 * i;
        const float p = s_l1p[r][k];
        const float d = (real && p > 0.0f && p < 1.0f) ? g1[i] : 0.0f;
        if (real) a.dl1[row * L1 + k] = d;
        s_dl1[r][k] = d;
    }
    __syncthreads();

    const SimpleTailDims td{(uint32_t)L1, (uint32_t)L2};
    const uint32_t cells = td.cells();
    const int nreal = a.batch - tile * 16 < 16 ? (int)(a.batch - tile * 16) : 16;  // real rows come first
    float* part = a.tail_partial + tile * cells;
    for (uint32_t c = lane; c < cells; c += 64) {
        float acc = 0.0f;
        if (c < td.off_b2()) {
            const uint32_t k = c / L2, o = c % L2;
            for (int rr = 0; rr < nreal; ++rr) acc += s_l1a[rr][k] * s_dl2[rr][o];
        } else if (c < td.off_w3()) {
            const uint32_t o = c - td.off_b2();
            for (int rr = 0; rr < nreal; ++rr) acc += s_dl2[rr][o];
        } else if (c < td.off_b3()) {
            const uint32_t o = c - td.off_w3();
            for (int rr = 0; rr < nreal; ++rr) acc += s_l2a[rr][o] * s_dy[rr];
        } else if (c < td.off_b1()) {
            for (int rr = 0; rr < nreal; ++rr) acc += s_dy[rr];
        } else {
            const uint32_t k = c - td.off_b1();
            for (int rr = 0; rr < nreal; ++rr) acc += s_dl1[rr][k];
        }
        part[c] = acc;
    }
}

// ---------------------------------------------------------------------------
// L1 weight-gradient partials: P[chunk][k][o] = sum over the chunk's rows of
// combined[row][k] * dl1[row][o].  One wave owns 64 columns k; lane (o, q)
// supplies dl1 of row 4s + q as the A operand and lane (q, kk) a float4 of
// combined at k0 + 4kk as B, so block c of its four MFMAs holds k0 + 4kk + c.
// ---------------------------------------------------------------------------
template <int L1>
__global__ __launch_bounds__(256) void simple_l1_wgrad_kernel(SimpleDenseArgs a) {
    constexpr int NB = (L1 + 15) / 16;  // l1 = 8: outputs 8..15 of the block are zero and dropped
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t K = 2 * a.ft_out;
    const uint32_t k0 = (blockIdx.y * 4 + wave) * 64;
    if (k0 >= K) return;
    const uint32_t chunk = blockIdx.x;
    const uint32_t r0 = chunk * kSimpleChunkRows;
    const uint32_t r1 = min(r0 + kSimpleChunkRows, a.batch);
    const uint32_t o = lane % 16, q = lane / 16, kk = lane % 16;
    const bool kvalid = k0 + 4 * kk < K;
    floatx4 acc[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[nb][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const uint32_t kc = kvalid ? k0 + 4 * kk : 0;  // always-valid column for the masked lanes
    for (uint32_t base = r0; base < r1; base += 4) {
        const uint32_t row = base + q;
        const bool rv = row < r1;
        const uint32_t rc = rv ? row : r0;  // always-valid row, masked below
        const float4 xl = *reinterpret_cast<const float4*>(a.combined + (uint64_t)rc * K + kc);
        const float4 x = (rv && kvalid) ? xl : zero4;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const bool ov = L1 % 16 == 0 || o < (uint32_t)L1;
            const float dl = a.dl1[(uint64_t)rc * L1 + 16 * nb + (ov ? o : 0)];
            const float d = (rv && ov) ? dl : 0.0f;
            acc[nb][0] = mfma4(d, x.x, acc[nb][0]);
            acc[nb][1] = mfma4(d, x.y, acc[nb][1]);
            acc[nb][2] = mfma4(d, x.z, acc[nb][2]);
            acc[nb][3] = mfma4(d, x.w, acc[nb][3]);
        }
    }
    if (!kvalid) return;
    float* P = a.w1_partial + (uint64_t)chunk * K * L1;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (L1 % 16 == 0 || 4 * q + r < (uint32_t)L1)
                    P[(uint64_t)(k0 + 4 * kk + c) * L1 + 16 * nb + 4 * q + r] = acc[nb][c][r];
}

// ---------------------------------------------------------------------------
// L1 input gradient fused with the FT CReLU gradient.  Thread c owns FT
// column c of both perspectives: dcombined[row][p*ft_out + c] =
// sum_o dl1[row][o] * l1_w[p*ft_out + c][o] (o ascending, from 0), then
// dft_p[row][c] passes it where 0 < x < 1 (simple_bwd_ft_act_crelu_fused,
// native_kernels.cu:1452).  The ft_b partial adds stm + nstm per row, rows in
// order (simple_bias_grad_dual, native_kernels.cu:1572).
// ---------------------------------------------------------------------------
template <int L1>
__global__ __launch_bounds__(256) void simple_l1_input_post_kernel(SimpleDenseArgs a) {
    constexpr int R = kSimplePostRows;
    __shared__ float s_d[R][L1];
    const uint32_t ft_out = a.ft_out;
    const uint32_t batch = a.batch;
    const uint32_t r0 = blockIdx.y * R;
    const uint32_t nr = min((uint32_t)R, batch - r0);
    for (uint32_t e = threadIdx.x; e < nr * L1; e += 256)
        s_d[e / L1][e % L1] = a.dl1[(uint64_t)r0 * L1 + e];
    __syncthreads();
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    if (c >= ft_out) return;
    float ws[L1], wn[L1];
#pragma unroll
    for (int o = 0; o < L1; ++o) {
        ws[o] = a.l1_w[(uint64_t)c * L1 + o];
        wn[o] = a.l1_w[(uint64_t)(ft_out + c) * L1 + o];
    }
    // chunk-major dft: column c of row r at (c / 256) * 2*batch*256 + r * 256 + c % 256
    const uint64_t cbase = (uint64_t)(c / kDftChunk) * 2 * batch * kDftChunk + c % kDftChunk;
    float* dft_s = a.dft + cbase;
    float* dft_n = a.dft + cbase + (uint64_t)batch * kDftChunk;
    float acc = 0.0f;
    for (uint32_t r = 0; r < nr; ++r) {
        const uint64_t i = (uint64_t)(r0 + r) * ft_out + c;
        const uint64_t di = (uint64_t)(r0 + r) * kDftChunk;
        float da = 0.0f, db = 0.0f;
#pragma unroll
        for (int o = 0; o < L1; ++o) {
            da += s_d[r][o] * ws[o];
            db += s_d[r][o] * wn[o];
        }
        const float xs = a.ft_stm[i], xn = a.ft_nstm[i];
        const float gs = (xs > 0.0f && xs < 1.0f) ? da : 0.0f;
        const float gn = (xn > 0.0f && xn < 1.0f) ? db : 0.0f;
        dft_s[di] = gs;
        dft_n[di] = gn;
        acc += gs + gn;
    }
    a.ftb_partial[(uint64_t)blockIdx.y * ft_out + c] = acc;
}

// ---------------------------------------------------------------------------
// Dense gradients from the reduced partials + RAdam/Ranger/AdamW, one thread
// per element of ft_b, l1_w, l1_b, l2_w, l2_b, l3_w, l3_b.
// ---------------------------------------------------------------------------
struct SimpleGroupTable {
    SimpleDenseGroup g[7];
    uint64_t start[8];
};

__global__ __launch_bounds__(256) void simple_dense_finalize_kernel(SimpleDenseArgs a,
                                                                    SimpleGroupTable gt,
                                                                    OptScalars dense,
                                                                    OptScalars bias,
                                                                    int32_t keep_grads) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= gt.start[7]) return;
    int gi = 0;
    while (i >= gt.start[gi + 1]) ++gi;
    const uint64_t e = i - gt.start[gi];
    const SimpleTailDims td{a.l1, a.l2};
    float grad;
    switch (gi) {
        case 0: grad = a.ftb_sum[e]; break;
        case 1: grad = a.w1_sum[e]; break;
        case 2: grad = a.tail_sum[td.off_b1() + e]; break;
        case 3: grad = a.tail_sum[td.off_w2() + e]; break;
        case 4: grad = a.tail_sum[td.off_b2() + e]; break;
        case 5: grad = a.tail_sum[td.off_w3() + e]; break;
        default: grad = a.tail_sum[td.off_b3()]; break;
    }
    const SimpleDenseGroup& G = gt.g[gi];
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

uint32_t simple_tail_workgroups(uint32_t batch) { return ceil_div(batch, 16); }
uint32_t simple_chunks(uint32_t batch) { return ceil_div(batch, kSimpleChunkRows); }
uint32_t simple_post_workgroups(uint32_t batch) { return ceil_div(batch, kSimplePostRows); }

static int32_t check_dims(const SimpleDenseArgs& a) {
    TATARA_REQUIRE(simple_dense_shape_ok(a.l1, a.l2), kSimpleDenseShapes);
    TATARA_REQUIRE(a.ft_out % 32 == 0, "Simple ft_out must be a multiple of 32");
    return kOk;
}

// kernel<L1>(...) for the accepted l1
#define TATARA_BY_L1(KERNEL, GRID, BLOCK, ...)                                  \
    do {                                                                        \
        if (a.l1 == 32)                                                         \
            KERNEL<32><<<GRID, BLOCK, 0, stream>>>(__VA_ARGS__);                \
        else if (a.l1 == 16)                                                    \
            KERNEL<16><<<GRID, BLOCK, 0, stream>>>(__VA_ARGS__);                \
        else                                                                    \
            KERNEL<8><<<GRID, BLOCK, 0, stream>>>(__VA_ARGS__);                 \
    } while (0)

int32_t launch_simple_l1_forward(const SimpleDenseArgs& a, hipStream_t stream) {
    int32_t st = check_dims(a);
    if (st) return st;
    const uint32_t tiles = ceil_div(a.batch, 16);
    if (tiles == 0) return kOk;
    TATARA_BY_L1(simple_l1_fwd_kernel, ceil_div(tiles, 4), 256, a);
    TATARA_LAUNCHED("simple_l1_forward");
    return kOk;
}

int32_t launch_simple_tail(const SimpleDenseArgs& a, int32_t train, hipStream_t stream) {
    int32_t st = check_dims(a);
    if (st) return st;
    const uint32_t blocks = simple_tail_workgroups(a.batch);
    if (blocks == 0) return kOk;
    // one instantiation per accepted (l1, l2)
#define TATARA_TAIL(L1_, L2_)                                                 \
    if (a.l1 == L1_ && a.l2 == L2_) {                                         \
        simple_tail_kernel<L1_, L2_><<<blocks, 64, 0, stream>>>(a, train);    \
        TATARA_LAUNCHED("simple_tail");                                       \
        return kOk;                                                           \
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
    TATARA_REQUIRE(false, kSimpleDenseShapes);
    return kOk;
}

int32_t launch_simple_l1_weight_grad(const SimpleDenseArgs& a, hipStream_t stream) {
    int32_t st = check_dims(a);
    if (st) return st;
    const uint32_t chunks = simple_chunks(a.batch);
    if (chunks == 0) return kOk;
    const dim3 grid(chunks, ceil_div(2 * a.ft_out, 256));
    TATARA_BY_L1(simple_l1_wgrad_kernel, grid, 256, a);
    TATARA_LAUNCHED("simple_l1_weight_grad");
    return kOk;
}

int32_t launch_simple_l1_input_post(const SimpleDenseArgs& a, hipStream_t stream) {
    int32_t st = check_dims(a);
    if (st) return st;
    const uint32_t rows = simple_post_workgroups(a.batch);
    if (rows == 0) return kOk;
    const dim3 grid(ceil_div(a.ft_out, 256), rows);
    TATARA_BY_L1(simple_l1_input_post_kernel, grid, 256, a);
    TATARA_LAUNCHED("simple_l1_input_post");
    return kOk;
}

int32_t launch_simple_dense_finalize(const SimpleDenseArgs& a, SimpleDenseGroup* groups,
                                     const OptScalars& dense, const OptScalars& bias,
                                     int32_t keep_grads, hipStream_t stream) {
    int32_t st = check_dims(a);
    if (st) return st;
    const SimpleTailDims td{a.l1, a.l2};
    const uint32_t K = 2 * a.ft_out;
    if ((st = launch_reduce_rows(a.tail_partial, simple_tail_workgroups(a.batch), td.cells(), nullptr,
                                 1, a.tail_sum, stream)))
        return st;
    if ((st = launch_reduce_rows(a.w1_partial, simple_chunks(a.batch), K * a.l1, nullptr, 1, a.w1_sum,
                                 stream)))
        return st;
    if ((st = launch_reduce_rows(a.ftb_partial, simple_post_workgroups(a.batch), a.ft_out, nullptr, 1,
                                 a.ftb_sum, stream)))
        return st;
    SimpleGroupTable gt;
    gt.start[0] = 0;
    for (int k = 0; k < 7; ++k) {
        gt.g[k] = groups[k];
        gt.start[k + 1] = gt.start[k] + groups[k].n;
    }
    simple_dense_finalize_kernel<<<ceil_div(gt.start[7], 256), 256, 0, stream>>>(a, gt, dense, bias,
                                                                                 keep_grads);
    TATARA_LAUNCHED("simple_dense_finalize");
    return kOk;
}

}  // namespace tatara
