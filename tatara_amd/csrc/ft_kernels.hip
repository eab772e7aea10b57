// Feature-transformer (FT) kernels for gfx950: the sparse gather forward with
// the FT post activation fused into its store, the deterministic backward
// (sorted occurrence lists + one sequential accumulator per weight cell) with
// the RAdam/Ranger update and the factorizer fold fused in, and the
// scheduling sorts they rely on.
//
// Reference semantics:
//   forward   crates/gpu-kernels/src/sparse/sparse_ft_forward.rs:100-122
//   post      crates/gpu-kernels/src/layerstack/ft_post_perspective.rs (fwd)
//             crates/cuda-native-runtime/kernels/native_kernels.cu:1406-1427 (Simple)
//   backward  crates/gpu-kernels/src/sparse/sparse_ft_backward.rs:247-267 in the
//             trainer's stm-then-nstm order (gpu_cpu_equivalence_tests.rs:4257-4275)
//   reduce    crates/gpu-kernels/src/sparse/ft_factorize.rs (ft_reduce_virtual_grad_cpu)
//   fold      crates/gpu-kernels/src/sparse/ft_factorize.rs (ft_fold_virtual_cpu)
//   optimizer crates/gpu-kernels/src/pointwise/radam_step.rs:116-149
#include "ft_kernels.hpp"

#include <hipcub/hipcub.hpp>

#include "common.hpp"
#include "optim.hpp"

namespace tatara {

namespace {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kMaxActive = 64;  // one index per lane
// Floats per lane in the FT gradient gather (a wave covers 64 * this columns).
#ifndef TATARA_FT_GRAD_LANE_FLOATS
#define TATARA_FT_GRAD_LANE_FLOATS 4
#endif
constexpr int kFtGradLaneFloats = TATARA_FT_GRAD_LANE_FLOATS;

__device__ __forceinline__ float4 f4add(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// Streamed data (outputs written once, optimizer state touched once per step)
// uses non-temporal accesses so it does not evict the gathered rows from L2.
typedef float nt_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void st_nt(float4* p, float4 v) {
    nt_f4 x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<nt_f4*>(p));
}

// Loads the position's active indices into per-wave LDS in slot order,
// keeping only valid ones (slot < nnz and 0 <= idx < cols), and returns how
// many there are.  Skipping invalid slots here matches the reference, which
// skips them in the sum (adding nothing).
__device__ __forceinline__ int compact_indices(const int32_t* __restrict__ idx_row, int nnz,
                                               uint32_t cols, uint32_t max_active, int* s_idx) {
    const int lane = __lane_id();
    const int n = nnz < (int)max_active ? nnz : (int)max_active;  // never read past the row
    int v = -1;
    if (lane < n) v = idx_row[lane];
    const bool ok = lane < n && v >= 0 && (uint32_t)v < cols;
    const uint64_t mask = __ballot(ok);
    const int rank = __popcll(mask & ((1ull << lane) - 1ull));
    if (ok) s_idx[rank] = v;
    __builtin_amdgcn_wave_barrier();
    return __popcll(mask);
}

// Sums rows idx[0..nv) of W (row length ft_out) at float4 column q (and q2 if
// TWO), in slot order, starting from +0.0.  Loads of UNROLL rows are issued
// before their adds so that many 16-byte loads are in flight per lane.
template <bool TWO, int UNROLL>
__device__ __forceinline__ void gather_rows(const float* __restrict__ W, uint64_t ft_out,
                                            const int* s_idx, int nv, uint32_t q, uint32_t q2,
                                            bool active, float4& a0, float4& a1) {
    a0 = make_float4(0.f, 0.f, 0.f, 0.f);
    a1 = a0;
    if (!active) return;
    const float4* __restrict__ W4 = reinterpret_cast<const float4*>(W);
    const uint64_t row4 = ft_out / 4;
    int k = 0;
    for (; k + UNROLL <= nv; k += UNROLL) {
        float4 w0[UNROLL], w1[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t r = (uint32_t)__builtin_amdgcn_readfirstlane(s_idx[k + u]);
            w0[u] = W4[r * row4 + q];
            if (TWO) w1[u] = W4[r * row4 + q2];
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            a0 = f4add(a0, w0[u]);
            if (TWO) a1 = f4add(a1, w1[u]);
        }
    }
    for (; k < nv; ++k) {
        const uint64_t r = (uint32_t)__builtin_amdgcn_readfirstlane(s_idx[k]);
        const float4 w0 = W4[r * row4 + q];
        a0 = f4add(a0, w0);
        if (TWO) {
            const float4 w1 = W4[r * row4 + q2];
            a1 = f4add(a1, w1);
        }
    }
}

// ---------------------------------------------------------------------------
// Forward gather.
//
// One wave = one task (position, column chunk); each lane owns one float4
// column, so a task reads 1 KB of every gathered row.  RAW/CONCAT: lane j of
// chunk c owns column q = 64c + j.  PAIR: chunk c covers 32 CReLU pairs; lane
// j < 32 owns q = 32c + j of the first half and lane j + 32 its partner
// q + ft_out/8, and the pair meets with one cross-lane swap.  Tasks are enumerated
// (perspective, chunk, position-in-schedule) and the schedule lists positions
// grouped by king block, so concurrently running waves read rows of the same
// king block (a few MB) and hit in L2; the XCD swizzle keeps neighbouring
// tasks on one XCD.
// ---------------------------------------------------------------------------

enum FwdMode : int { kRaw = 0, kPair = 1, kConcat = 2 };

template <int MODE>
__global__ __launch_bounds__(256) void ft_forward_kernel(
    const float* __restrict__ W, const int32_t* __restrict__ idx_stm,
    const int32_t* __restrict__ idx_nstm, const int32_t* __restrict__ nnz,
    const int32_t* __restrict__ schedule,  // [n_persp][batch] position order, or null
    const float* __restrict__ bias, float* __restrict__ out_stm, float* __restrict__ out_nstm,
    float* __restrict__ combined, uint32_t batch, uint32_t ft_out, uint32_t cols,
    uint32_t max_active, uint32_t n_chunks, uint32_t n_persp, float scale) {
    __shared__ int s_idx_all[kWavesPerBlock][kMaxActive];
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint64_t task = (uint64_t)bid * kWavesPerBlock + wave;
    const uint64_t per_persp = (uint64_t)n_chunks * batch;
    if (task >= per_persp * n_persp) return;
    const uint32_t persp = (uint32_t)(task / per_persp);
    const uint64_t rem = task - (uint64_t)persp * per_persp;
    const uint32_t chunk = (uint32_t)(rem / batch);
    const uint32_t slot = (uint32_t)(rem - (uint64_t)chunk * batch);
    const uint32_t pos = schedule ? (uint32_t)schedule[(uint64_t)persp * batch + slot] : slot;
    if (pos >= batch) return;  // a schedule always lists every position once

    const int32_t* idx = persp == 0 ? idx_stm : idx_nstm;
    float* out = persp == 0 ? out_stm : out_nstm;
    int* s_idx = s_idx_all[wave];
    const int nv = compact_indices(idx + (uint64_t)pos * max_active, nnz[pos], cols, max_active, s_idx);

    const uint32_t half4 = ft_out / 8;
    const uint32_t row4 = ft_out / 4;
    float4 a0, a1;
    if (MODE == kPair) {
        const uint32_t j = lane & 31u;
        const uint32_t qp = chunk * 32 + j;  // pair index
        const bool active = qp < half4;
        const uint32_t q = lane < 32 ? qp : qp + half4;
        gather_rows<false, 8>(W, ft_out, s_idx, nv, q, 0, active, a0, a1);
        // first-half lanes receive their partner's sums from lane + 32
        float4 p;
        p.x = __shfl_xor(a0.x, 32);
        p.y = __shfl_xor(a0.y, 32);
        p.z = __shfl_xor(a0.z, 32);
        p.w = __shfl_xor(a0.w, 32);
        if (!active) return;
        float4* o4 = reinterpret_cast<float4*>(out + (uint64_t)pos * ft_out);
        st_nt(o4 + q, a0);
        if (lane >= 32) return;
        const float4 b0 = reinterpret_cast<const float4*>(bias)[qp];
        const float4 b1 = reinterpret_cast<const float4*>(bias)[qp + half4];
        float4 c;
        c.x = crelu01(a0.x + b0.x) * crelu01(p.x + b1.x) * scale;
        c.y = crelu01(a0.y + b0.y) * crelu01(p.y + b1.y) * scale;
        c.z = crelu01(a0.z + b0.z) * crelu01(p.z + b1.z) * scale;
        c.w = crelu01(a0.w + b0.w) * crelu01(p.w + b1.w) * scale;
        st_nt(reinterpret_cast<float4*>(combined + (uint64_t)pos * ft_out + persp * (ft_out / 2)) + qp, c);
    } else {
        const uint32_t q = chunk * kWave + lane;
        const bool active = q < row4;
        gather_rows<false, 8>(W, ft_out, s_idx, nv, q, 0, active, a0, a1);
        if (!active) return;
        if (MODE == kRaw) {
            reinterpret_cast<float4*>(out + (uint64_t)pos * ft_out)[q] = a0;
        } else {
            // Simple: ft_out += bias in place, combined[off + c] = crelu(x).
            const float4 b0 = reinterpret_cast<const float4*>(bias)[q];
            const float4 x = f4add(a0, b0);
            reinterpret_cast<float4*>(out + (uint64_t)pos * ft_out)[q] = x;
            float4 c;
            c.x = crelu01(x.x);
            c.y = crelu01(x.y);
            c.z = crelu01(x.z);
            c.w = crelu01(x.w);
            reinterpret_cast<float4*>(combined + (uint64_t)pos * 2 * ft_out + persp * ft_out)[q] = c;
        }
    }
}

// ---------------------------------------------------------------------------
// Forward schedule keys: item p*batch + b gets key p*n_bins + (king block of
// position b in perspective p), where the king block is the first valid
// index divided by piece_inputs.  A stable bin sort of these keys yields,
// per perspective, the positions grouped by king block in ascending order.
// ---------------------------------------------------------------------------

__global__ void king_block_keys_kernel(const int32_t* __restrict__ idx_stm,
                                       const int32_t* __restrict__ idx_nstm,
                                       const int32_t* __restrict__ nnz, uint8_t* __restrict__ keys,
                                       uint32_t batch, uint32_t max_active, uint32_t cols,
                                       uint32_t piece_inputs, uint32_t n_bins) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 2ull * batch) return;
    const uint32_t persp = i >= batch ? 1u : 0u;
    const uint32_t b = (uint32_t)(i - (uint64_t)persp * batch);
    const int32_t* row = (persp ? idx_nstm : idx_stm) + (uint64_t)b * max_active;
    const int n = nnz[b] < (int)max_active ? nnz[b] : (int)max_active;
    uint32_t k = 0;
    for (int s = 0; s < n; ++s) {
        const int32_t v = row[s];
        if (v >= 0 && (uint32_t)v < cols) {
            k = piece_inputs ? (uint32_t)v / piece_inputs : 0u;
            if (k >= n_bins) k = n_bins - 1;
            break;
        }
    }
    keys[i] = (uint8_t)(persp * n_bins + k);
}

// ---------------------------------------------------------------------------
// Occurrence lists for the backward: key = 2*feature + perspective, value =
// perspective*batch + position (a row of the concatenated [2][batch][ft_out]
// dft buffer).  Items are emitted in (perspective, position, slot) order and
// sorted stably, so each key's list is in ascending position order: the same
// order in which the reference CPU backward accumulates.
// ---------------------------------------------------------------------------

__global__ void build_occurrence_keys_kernel(const int32_t* __restrict__ idx_stm,
                                             const int32_t* __restrict__ idx_nstm,
                                             const int32_t* __restrict__ nnz,
                                             uint32_t* __restrict__ keys,
                                             uint32_t* __restrict__ vals, uint32_t batch,
                                             uint32_t max_active, uint32_t cols) {
    const uint64_t per = (uint64_t)batch * max_active;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= 2 * per) return;
    const uint32_t persp = i >= per ? 1u : 0u;
    const uint64_t j = i - persp * per;
    const uint32_t b = (uint32_t)(j / max_active);
    const uint32_t slot = (uint32_t)(j - (uint64_t)b * max_active);
    const int32_t v = (persp ? idx_nstm : idx_stm)[j];
    const bool ok = (int)slot < nnz[b] && v >= 0 && (uint32_t)v < cols;
    const uint32_t key = ok ? 2u * (uint32_t)v + persp : 2u * cols;
    keys[i] = key;
    vals[i] = persp * batch + b;
}

// Segment offsets from the sorted keys: offsets[k] = first sorted position
// with key >= k, for k in [0, n_keys]; offsets[n_keys] = n_items.  Each entry
// is written by exactly one thread (the one at the boundary it falls in), so
// no histogram, atomics or scan are needed.
__global__ void occurrence_offsets_kernel(const uint32_t* __restrict__ sorted_keys,
                                          uint64_t n_items, uint32_t n_keys,
                                          uint32_t* __restrict__ offsets) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i > n_items) return;
    const int64_t prev = i == 0 ? -1 : (int64_t)sorted_keys[i - 1];
    const int64_t cur = i == n_items ? (int64_t)n_keys : (int64_t)sorted_keys[i];
    for (int64_t k = prev + 1; k <= cur; ++k) offsets[k] = (uint32_t)i;
}

// ---------------------------------------------------------------------------
// Backward + optimizer, phase A: one wave = one task (column chunk c, real row
// f).  The gradient of row f is the sequential sum, from +0.0, of the dft rows
// listed in its occurrence segment [off[2f], off[2f+2]) - stm occurrences in
// ascending position order, then nstm ones - which is exactly the order of the
// reference CPU backward (sparse_ft_backward_cpu, stm then nstm).  The row is
// then updated with RAdam (+ the Ranger lerp on lookahead steps) and its
// gradient stored for the factorizer's virtual rows (phase B).
// Tasks are chunk-major and swizzled so that an XCD walks consecutive rows of
// one column chunk: those rows share a king block, whose occurrences come from
// the same few thousand (position, perspective) rows, so the gathered dft rows
// stay in L2.  The chunk width bounds that working set: a full king block has
// about 3.3k dft rows, i.e. 3.3 MB at 256 columns but 1.6 MB at 128, and an
// XCD keeps one to two blocks in flight against a 4 MB L2.  A wave covers
// kWave * V columns (V floats per lane).
// ---------------------------------------------------------------------------

template <int V>
using vecf = float __attribute__((ext_vector_type(V)));

template <int V>
__device__ __forceinline__ vecf<V> segment_sum(const vecf<V>* __restrict__ dft, uint64_t row_v,
                                               const uint32_t* __restrict__ vals, uint32_t s,
                                               uint32_t e, uint64_t q) {
    vecf<V> acc = 0.0f;
    constexpr int U = 32 / V;  // 8 (V=4) .. 32 (V=1) loads in flight per lane
    uint32_t i = s;
    for (; i + U <= e; i += U) {
        vecf<V> d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t r = __builtin_amdgcn_readfirstlane(vals[i + u]);
            d[u] = dft[r * row_v + q];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += d[u];
    }
    for (; i < e; ++i) {
        const uint64_t r = __builtin_amdgcn_readfirstlane(vals[i]);
        acc += dft[r * row_v + q];
    }
    return acc;
}

template <int V>
__device__ __forceinline__ void opt_update(float* __restrict__ w, float* __restrict__ m,
                                           float* __restrict__ v, float* __restrict__ slow,
                                           uint64_t off, vecf<V> g, const OptScalars& s) {
    vecf<V>* w_ = reinterpret_cast<vecf<V>*>(w) + off;
    vecf<V>* m_ = reinterpret_cast<vecf<V>*>(m) + off;
    vecf<V>* v_ = reinterpret_cast<vecf<V>*>(v) + off;
    vecf<V> W = __builtin_nontemporal_load(w_);
    vecf<V> M = __builtin_nontemporal_load(m_);
    vecf<V> Q = __builtin_nontemporal_load(v_);
#pragma unroll
    for (int k = 0; k < V; ++k) {
        float a = W[k], b = M[k], c = Q[k];
        radam_elem(a, b, c, g[k], s);
        W[k] = a;
        M[k] = b;
        Q[k] = c;
    }
    if (s.lookahead) {
        vecf<V>* s_ = reinterpret_cast<vecf<V>*>(slow) + off;
        vecf<V> S = __builtin_nontemporal_load(s_);
#pragma unroll
        for (int k = 0; k < V; ++k) {
            float a = W[k], b = S[k];
            lerp_elem(a, b, s.alpha);
            W[k] = a;
            S[k] = b;
        }
        __builtin_nontemporal_store(S, s_);
    }
    __builtin_nontemporal_store(W, w_);
    __builtin_nontemporal_store(M, m_);
    __builtin_nontemporal_store(Q, v_);
}

// dft_row / dft_chunk: the dft strides in floats (chunk = kDftChunk columns).
template <int V>
__global__ __launch_bounds__(256) void ft_grad_update_kernel(
    const float* __restrict__ dft, uint64_t dft_row, uint64_t dft_chunk,
    const uint32_t* __restrict__ occ_vals, const uint32_t* __restrict__ occ_off,
    float* __restrict__ w, float* __restrict__ m, float* __restrict__ v, float* __restrict__ slow,
    float* __restrict__ grad_out,  // gradient per row (may be null without a factorizer)
    uint32_t ft_out, uint32_t rows, uint32_t n_chunks, int32_t apply_update, OptScalars s) {
    constexpr uint32_t kCols = kWave * V;
    static_assert(kDftChunk % kCols == 0, "a wave's columns must lie in one dft chunk");
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint64_t task = (uint64_t)bid * kWavesPerBlock + wave;
    if (task >= (uint64_t)rows * n_chunks) return;
    const uint32_t chunk = (uint32_t)(task / rows);
    const uint32_t f = (uint32_t)(task - (uint64_t)chunk * rows);
    const uint32_t col = chunk * kCols + lane * V;
    const uint32_t s0 = __builtin_amdgcn_readfirstlane(occ_off[2 * f]);
    const uint32_t s1 = __builtin_amdgcn_readfirstlane(occ_off[2 * f + 2]);
    if (col >= ft_out) return;
    const uint64_t q = ((uint64_t)(col / kDftChunk) * dft_chunk + col % kDftChunk) / V;
    const vecf<V> gr = segment_sum<V>(reinterpret_cast<const vecf<V>*>(dft), dft_row / V, occ_vals,
                                      s0, s1, q);
    const uint64_t off = ((uint64_t)f * ft_out + col) / V;
    if (grad_out) __builtin_nontemporal_store(gr, reinterpret_cast<vecf<V>*>(grad_out) + off);
    if (apply_update) opt_update<V>(w, m, v, slow, off, gr, s);
}

// ---------------------------------------------------------------------------
// Backward + optimizer, phase B (factorizer): one wave = (column chunk, piece
// p).  The virtual row's gradient is the sequential sum of the piece's
// king-bucket rows p, p + pi, p + 2 pi, ... (ft_reduce_virtual_grad_cpu's
// order); the virtual row is updated, and the forward table
// comb = w + w_virtual is rewritten for the piece's rows (ft_fold_virtual).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void ft_virtual_fold_kernel(
    float* __restrict__ grad, float* __restrict__ w, float* __restrict__ m, float* __restrict__ v,
    float* __restrict__ slow, float* __restrict__ comb, uint32_t ft_out, uint32_t ft_in,
    uint32_t piece_inputs, uint32_t n_chunks, int32_t apply_update, OptScalars s) {
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t task = (uint64_t)blockIdx.x * kWavesPerBlock + wave;
    if (task >= (uint64_t)piece_inputs * n_chunks) return;
    const uint32_t chunk = (uint32_t)(task / piece_inputs);
    const uint32_t p = (uint32_t)(task - (uint64_t)chunk * piece_inputs);
    const uint32_t row4 = ft_out / 4;
    const uint32_t q = chunk * kWave + lane;
    if (q >= row4) return;
    const uint32_t count = ft_in / piece_inputs;
    const float4* g4 = reinterpret_cast<const float4*>(grad);
    float4 vsum = make_float4(0.f, 0.f, 0.f, 0.f);
    constexpr int U = 8;
    uint32_t j = 0;
    for (; j + U <= count; j += U) {
        float4 d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) d[u] = g4[(uint64_t)(p + (j + u) * piece_inputs) * row4 + q];
#pragma unroll
        for (int u = 0; u < U; ++u) vsum = f4add(vsum, d[u]);
    }
    for (; j < count; ++j) vsum = f4add(vsum, g4[(uint64_t)(p + j * piece_inputs) * row4 + q]);
    const uint64_t voff4 = (uint64_t)(ft_in + p) * row4 + q;
    reinterpret_cast<float4*>(grad)[voff4] = vsum;
    if (!apply_update) return;
    opt_update<4>(w, m, v, slow, voff4, vecf<4>{vsum.x, vsum.y, vsum.z, vsum.w}, s);
    if (!comb) return;
    const float4 wv = reinterpret_cast<const float4*>(w)[voff4];
    for (j = 0; j + U <= count; j += U) {
        float4 wr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) wr[u] = reinterpret_cast<const float4*>(w)[(uint64_t)(p + (j + u) * piece_inputs) * row4 + q];
#pragma unroll
        for (int u = 0; u < U; ++u)
            reinterpret_cast<float4*>(comb)[(uint64_t)(p + (j + u) * piece_inputs) * row4 + q] = f4add(wr[u], wv);
    }
    for (; j < count; ++j) {
        const uint64_t off4 = (uint64_t)(p + j * piece_inputs) * row4 + q;
        reinterpret_cast<float4*>(comb)[off4] = f4add(reinterpret_cast<const float4*>(w)[off4], wv);
    }
}

// Standalone fold / reduce (Base mode), used when they are not fused.
__global__ void ft_fold_kernel(const float* __restrict__ w, float* __restrict__ comb,
                               uint32_t ft_in, uint32_t ft_out, uint32_t piece_inputs) {
    const uint64_t n4 = (uint64_t)ft_in * ft_out / 4;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const uint32_t row4 = ft_out / 4;
    const uint64_t f = i / row4;
    const uint32_t c = (uint32_t)(i - f * row4);
    const uint64_t vrow = ft_in + f % piece_inputs;
    reinterpret_cast<float4*>(comb)[i] =
        f4add(reinterpret_cast<const float4*>(w)[i], reinterpret_cast<const float4*>(w)[vrow * row4 + c]);
}

__global__ void ft_reduce_kernel(float* __restrict__ grad, uint32_t ft_in, uint32_t ft_out,
                                 uint32_t piece_inputs) {
    const uint64_t n = (uint64_t)piece_inputs * ft_out;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t v = i / ft_out;
    const uint32_t c = (uint32_t)(i - v * ft_out);
    float sum = 0.0f;
    for (uint64_t f = v; f < ft_in; f += piece_inputs) sum += grad[f * ft_out + c];
    grad[((uint64_t)ft_in + v) * ft_out + c] = sum;
}

__global__ void radam_kernel(float* __restrict__ w, float* __restrict__ m, float* __restrict__ v,
                             float* __restrict__ g, float* __restrict__ slow, uint64_t n,
                             OptScalars s) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float W = w[i], M = m[i], V = v[i];
    radam_elem(W, M, V, g[i], s);
    if (s.lookahead) {
        float S = slow[i];
        lerp_elem(W, S, s.alpha);
        slow[i] = S;
    }
    w[i] = W;
    m[i] = M;
    v[i] = V;
    g[i] = 0.0f;
}

__global__ void lerp_kernel(float* __restrict__ w, float* __restrict__ slow, uint64_t n,
                            float alpha) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float W = w[i], S = slow[i];
    lerp_elem(W, S, alpha);
    w[i] = W;
    slow[i] = S;
}

}  // namespace

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------

int32_t launch_ft_forward(const FtForwardArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(a.max_active <= (uint32_t)kMaxActive, "max_active must be <= 64");
    TATARA_REQUIRE(a.ft_out % 8 == 0, "ft_out must be a multiple of 8");
    TATARA_REQUIRE(a.n_persp == 1 || a.n_persp == 2, "n_persp must be 1 or 2");
    if (a.batch == 0) return kOk;
    const uint32_t n_chunks = a.mode == kPair ? ceil_div(a.ft_out / 8, 32) : ceil_div(a.ft_out / 4, kWave);
    const uint64_t tasks = (uint64_t)a.n_persp * n_chunks * a.batch;
    const uint32_t blocks = (uint32_t)((tasks + kWavesPerBlock - 1) / kWavesPerBlock);
    switch (a.mode) {
        case kRaw:
            ft_forward_kernel<kRaw><<<blocks, 256, 0, stream>>>(
                a.W, a.idx_stm, a.idx_nstm, a.nnz, a.schedule, a.bias, a.out_stm, a.out_nstm,
                a.combined, a.batch, a.ft_out, a.cols, a.max_active, n_chunks, a.n_persp, a.scale);
            break;
        case kPair:
            ft_forward_kernel<kPair><<<blocks, 256, 0, stream>>>(
                a.W, a.idx_stm, a.idx_nstm, a.nnz, a.schedule, a.bias, a.out_stm, a.out_nstm,
                a.combined, a.batch, a.ft_out, a.cols, a.max_active, n_chunks, a.n_persp, a.scale);
            break;
        case kConcat:
            ft_forward_kernel<kConcat><<<blocks, 256, 0, stream>>>(
                a.W, a.idx_stm, a.idx_nstm, a.nnz, a.schedule, a.bias, a.out_stm, a.out_nstm,
                a.combined, a.batch, a.ft_out, a.cols, a.max_active, n_chunks, a.n_persp, a.scale);
            break;
        default:
            TATARA_REQUIRE(false, "unknown forward mode");
    }
    TATARA_LAUNCHED("ft_forward");
    return kOk;
}

int32_t launch_king_block_keys(const int32_t* idx_stm, const int32_t* idx_nstm,
                               const int32_t* nnz, uint8_t* keys, uint32_t batch,
                               uint32_t max_active, uint32_t cols, uint32_t piece_inputs,
                               uint32_t n_bins, hipStream_t stream) {
    if (batch == 0) return kOk;
    TATARA_REQUIRE(2 * n_bins <= 256, "king block keys: 2*n_bins <= 256");
    king_block_keys_kernel<<<ceil_div(2ull * batch, 256), 256, 0, stream>>>(
        idx_stm, idx_nstm, nnz, keys, batch, max_active, cols, piece_inputs, n_bins);
    TATARA_LAUNCHED("king_block_keys");
    return kOk;
}

uint32_t occurrence_key_bits(uint32_t cols) {
    uint32_t bits = 1;
    while ((1ull << bits) <= 2ull * cols) ++bits;
    return bits;
}

size_t occurrence_sort_temp_bytes(uint64_t n_items, uint32_t cols) {
    size_t bytes = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const uint32_t*)nullptr,
                                             (uint32_t*)nullptr, (const uint32_t*)nullptr,
                                             (uint32_t*)nullptr, (int)n_items, 0,
                                             (int)occurrence_key_bits(cols));
    return bytes;
}

int32_t launch_occurrence_sort(const OccurrenceSortArgs& a, hipStream_t stream) {
    const uint64_t n_items = 2ull * a.batch * a.max_active;
    const uint32_t n_keys = 2 * a.cols + 1;  // keys 0..2*cols (2*cols = invalid slot)
    if (n_items > 0) {
        build_occurrence_keys_kernel<<<ceil_div(n_items, 256), 256, 0, stream>>>(
            a.idx_stm, a.idx_nstm, a.nnz, a.keys_in, a.vals_in, a.batch, a.max_active, a.cols);
        TATARA_LAUNCHED("build_occurrence_keys");
        size_t bytes = a.temp_bytes;
        TATARA_HIP(hipcub::DeviceRadixSort::SortPairs(a.temp, bytes, a.keys_in, a.keys_out,
                                                      a.vals_in, a.vals_out, (int)n_items, 0,
                                                      (int)occurrence_key_bits(a.cols), stream),
                   "occurrence radix sort");
    }
    occurrence_offsets_kernel<<<ceil_div(n_items + 1, 256), 256, 0, stream>>>(a.keys_out, n_items,
                                                                              n_keys, a.offsets);
    TATARA_LAUNCHED("occurrence_offsets");
    return kOk;
}

int32_t launch_ft_grad_update(const FtGradArgs& a, hipStream_t stream) {
    constexpr int V = kFtGradLaneFloats;
    constexpr uint32_t kCols = kWave * V;
    TATARA_REQUIRE(a.ft_out % 4 == 0, "ft_out must be a multiple of 4");
    TATARA_REQUIRE(a.dft_row_stride % 4 == 0 && a.dft_chunk_stride % 4 == 0, "dft strides");
    const uint32_t n_chunks = ceil_div(a.ft_out, kCols);
    const uint64_t tasks = (uint64_t)a.rows * n_chunks;
    if (tasks == 0) return kOk;
    const uint32_t blocks = (uint32_t)((tasks + kWavesPerBlock - 1) / kWavesPerBlock);
    ft_grad_update_kernel<V><<<blocks, 256, 0, stream>>>(a.dft, a.dft_row_stride, a.dft_chunk_stride,
                                                         a.occ_vals, a.occ_off, a.w, a.m, a.v,
                                                         a.slow, a.grad, a.ft_out, a.rows, n_chunks,
                                                         a.apply_update, a.opt);
    TATARA_LAUNCHED("ft_grad_update");
    return kOk;
}

int32_t launch_ft_virtual_fold(const FtGradArgs& a, uint32_t piece_inputs, float* comb,
                               hipStream_t stream) {
    TATARA_REQUIRE(piece_inputs > 0 && a.rows % piece_inputs == 0,
                   "virtual fold: rows must be a multiple of piece_inputs");
    TATARA_REQUIRE(a.grad, "virtual fold needs the real-row gradients");
    const uint32_t n_chunks = ceil_div(a.ft_out / 4, kWave);
    const uint64_t tasks = (uint64_t)piece_inputs * n_chunks;
    const uint32_t blocks = (uint32_t)((tasks + kWavesPerBlock - 1) / kWavesPerBlock);
    ft_virtual_fold_kernel<<<blocks, 256, 0, stream>>>(a.grad, a.w, a.m, a.v, a.slow, comb, a.ft_out,
                                                       a.rows, piece_inputs, n_chunks,
                                                       a.apply_update, a.opt);
    TATARA_LAUNCHED("ft_virtual_fold");
    return kOk;
}

int32_t launch_ft_fold(const float* w, float* comb, uint32_t ft_in, uint32_t ft_out,
                       uint32_t piece_inputs, hipStream_t stream) {
    TATARA_REQUIRE(ft_out % 4 == 0 && piece_inputs > 0, "fold: ft_out%4==0, piece_inputs>0");
    const uint64_t n4 = (uint64_t)ft_in * ft_out / 4;
    if (n4 == 0) return kOk;
    ft_fold_kernel<<<ceil_div(n4, 256), 256, 0, stream>>>(w, comb, ft_in, ft_out, piece_inputs);
    TATARA_LAUNCHED("ft_fold");
    return kOk;
}

int32_t launch_ft_reduce(float* grad, uint32_t ft_in, uint32_t ft_out, uint32_t piece_inputs,
                         hipStream_t stream) {
    TATARA_REQUIRE(piece_inputs > 0, "reduce: piece_inputs > 0");
    const uint64_t n = (uint64_t)piece_inputs * ft_out;
    if (n == 0) return kOk;
    ft_reduce_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(grad, ft_in, ft_out, piece_inputs);
    TATARA_LAUNCHED("ft_reduce");
    return kOk;
}

int32_t launch_radam(float* w, float* m, float* v, float* g, float* slow, uint64_t n,
                     const OptScalars& s, hipStream_t stream) {
    if (n == 0) return kOk;
    radam_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(w, m, v, g, slow, n, s);
    TATARA_LAUNCHED("radam_step");
    return kOk;
}

int32_t launch_lerp(float* w, float* slow, uint64_t n, float alpha, hipStream_t stream) {
    if (n == 0) return kOk;
    lerp_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(w, slow, n, alpha);
    TATARA_LAUNCHED("ranger_lookahead_lerp");
    return kOk;
}

}  // namespace tatara
