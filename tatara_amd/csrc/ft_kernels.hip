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

#include <cmath>
#include <type_traits>
#include <utility>

#include "binsort.hpp"
#include "common.hpp"
#include "optim.hpp"

namespace tatara {

namespace {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kMaxActive = 64;  // one index per lane
// Floats per lane in the FT gradient gather (a wave covers 64 * this columns).
constexpr int kFtGradLaneFloats = 4;

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

// binary16 (f16) values: conversions to f16 round to nearest even
// (__float2half_rn); f16 -> f32 is exact.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 h4_to_f4(h4 h) {
    const nt_f4 f = __builtin_convertvector(h, nt_f4);
    return make_float4(f.x, f.y, f.z, f.w);
}

__device__ __forceinline__ float4 as_f4(float4 v) { return v; }
__device__ __forceinline__ float4 as_f4(h4 v) { return h4_to_f4(v); }

__device__ __forceinline__ h4 f4_to_h4(float4 v) {
    const nt_f4 f = {v.x, v.y, v.z, v.w};
    return __builtin_convertvector(f, h4);
}

// Four consecutive values of a table at float4 index i4, as f32.
template <typename T>
struct Row4;
template <>
struct Row4<float> {
    static __device__ __forceinline__ float4 load(const float* W, uint64_t i4) {
        return reinterpret_cast<const float4*>(W)[i4];
    }
};
template <>
struct Row4<_Float16> {
    static __device__ __forceinline__ float4 load(const _Float16* W, uint64_t i4) {
        return h4_to_f4(reinterpret_cast<const h4*>(W)[i4]);
    }
};

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
// TWO), in slot order, starting from +0.0, in f32 whatever the table's type.
// Loads of UNROLL rows are issued before their adds so that many loads are in
// flight per lane (16 bytes per row for f32 tables, 8 for f16).
template <bool TWO, int UNROLL, typename T>
__device__ __forceinline__ void gather_rows(const T* __restrict__ W, uint64_t ft_out,
                                            const int* s_idx, int nv, uint32_t q, uint32_t q2,
                                            bool active, float4& a0, float4& a1) {
    a0 = make_float4(0.f, 0.f, 0.f, 0.f);
    a1 = a0;
    if (!active) return;
    const uint64_t row4 = ft_out / 4;
    int k = 0;
    for (; k + UNROLL <= nv; k += UNROLL) {
        float4 w0[UNROLL], w1[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint64_t r = (uint32_t)__builtin_amdgcn_readfirstlane(s_idx[k + u]);
            w0[u] = Row4<T>::load(W, r * row4 + q);
            if (TWO) w1[u] = Row4<T>::load(W, r * row4 + q2);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            a0 = f4add(a0, w0[u]);
            if (TWO) a1 = f4add(a1, w1[u]);
        }
    }
    for (; k < nv; ++k) {
        const uint64_t r = (uint32_t)__builtin_amdgcn_readfirstlane(s_idx[k]);
        const float4 w0 = Row4<T>::load(W, r * row4 + q);
        a0 = f4add(a0, w0);
        if (TWO) {
            const float4 w1 = Row4<T>::load(W, r * row4 + q2);
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
// T = _Float16 reads the f16 forward table (sparse_ft_forward_fp16,
// native_kernels.cu:700-780: f16 rows, f32 accumulation); HOUT rounds the raw
// sums to f16 before they are stored and before the pairwise post reads them
// (sparse_ft_forward_fp16_out + ft_post_perspective_fwd_fp16, :762-857).
// ---------------------------------------------------------------------------

enum FwdMode : int { kRaw = 0, kPair = 1, kConcat = 2 };

template <int MODE, typename T, bool HOUT>
__global__ __launch_bounds__(256) void ft_forward_kernel(
    const T* __restrict__ W, const int32_t* __restrict__ idx_stm,
    const int32_t* __restrict__ idx_nstm, const int32_t* __restrict__ nnz,
    const int32_t* __restrict__ schedule,  // [n_persp][batch] position order, or null
    const float* __restrict__ bias, float* __restrict__ out_stm, float* __restrict__ out_nstm,
    _Float16* __restrict__ out16_stm, _Float16* __restrict__ out16_nstm,
    float* __restrict__ combined, _Float16* __restrict__ combined16, uint32_t batch, uint32_t ft_out,
    uint32_t cols, uint32_t max_active, uint32_t n_chunks, uint32_t n_persp, float scale) {
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
    _Float16* out16 = persp == 0 ? out16_stm : out16_nstm;
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
        gather_rows<false, sizeof(T) == 2 ? 16 : 8>(W, ft_out, s_idx, nv, q, 0, active, a0, a1);
        h4 r16;
        if (HOUT) {
            r16 = f4_to_h4(a0);
            a0 = h4_to_f4(r16);
        }
        // first-half lanes receive their partner's sums from lane + 32
        float4 p;
        p.x = __shfl_xor(a0.x, 32);
        p.y = __shfl_xor(a0.y, 32);
        p.z = __shfl_xor(a0.z, 32);
        p.w = __shfl_xor(a0.w, 32);
        if (!active) return;
        if (HOUT) {
            __builtin_nontemporal_store(r16, reinterpret_cast<h4*>(out16 + (uint64_t)pos * ft_out) + q);
        } else {
            float4* o4 = reinterpret_cast<float4*>(out + (uint64_t)pos * ft_out);
            st_nt(o4 + q, a0);
        }
        if (lane >= 32) return;
        const float4 b0 = reinterpret_cast<const float4*>(bias)[qp];
        const float4 b1 = reinterpret_cast<const float4*>(bias)[qp + half4];
        float4 c;
        c.x = crelu01(a0.x + b0.x) * crelu01(p.x + b1.x) * scale;
        c.y = crelu01(a0.y + b0.y) * crelu01(p.y + b1.y) * scale;
        c.z = crelu01(a0.z + b0.z) * crelu01(p.z + b1.z) * scale;
        c.w = crelu01(a0.w + b0.w) * crelu01(p.w + b1.w) * scale;
        const uint64_t co = (uint64_t)pos * ft_out + persp * (ft_out / 2);
        if (combined16)
            __builtin_nontemporal_store(f4_to_h4(c), reinterpret_cast<h4*>(combined16 + co) + qp);
        else
            st_nt(reinterpret_cast<float4*>(combined + co) + qp, c);
    } else {
        const uint32_t q = chunk * kWave + lane;
        const bool active = q < row4;
        gather_rows<false, sizeof(T) == 2 ? 16 : 8>(W, ft_out, s_idx, nv, q, 0, active, a0, a1);
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
// Forward gather from an f16 table, pairwise post (LayerStack).  As the
// kPair mode above, but every lane owns eight columns (one 16-byte f16 load
// per gathered row, half the load instructions of four-column lanes): lane
// j < 32 of chunk c owns columns 8(32c + j) .. +7 of the first half and lane
// j + 32 their partners in the second half.  Sums are f32 in slot order;
// HOUT rounds them to f16 before they are stored and before the post reads
// them.
// ---------------------------------------------------------------------------

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f8v __attribute__((ext_vector_type(8)));

template <bool HOUT>
__global__ __launch_bounds__(256) void ft_forward_pair16_kernel(
    const _Float16* __restrict__ W, const int32_t* __restrict__ idx_stm, const int32_t* __restrict__ idx_nstm,
    const int32_t* __restrict__ nnz, const int32_t* __restrict__ schedule, const float* __restrict__ bias,
    float* __restrict__ out_stm, float* __restrict__ out_nstm, _Float16* __restrict__ out16_stm,
    _Float16* __restrict__ out16_nstm, float* __restrict__ combined, _Float16* __restrict__ combined16,
    uint32_t batch, uint32_t ft_out, uint32_t cols, uint32_t max_active, uint32_t n_chunks, uint32_t n_persp,
    float scale) {
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
    if (pos >= batch) return;

    const int32_t* idx = persp == 0 ? idx_stm : idx_nstm;
    int* s_idx = s_idx_all[wave];
    const int nv = compact_indices(idx + (uint64_t)pos * max_active, nnz[pos], cols, max_active, s_idx);

    const uint32_t half8 = ft_out / 16;  // 8-column groups per half
    const uint32_t row8 = ft_out / 8;
    const uint32_t j = lane & 31u;
    const uint32_t qp = chunk * 32 + j;  // group index within the first half
    const bool active = qp < half8;
    const uint32_t q = lane < 32 ? qp : qp + half8;
    const h8* __restrict__ W8 = reinterpret_cast<const h8*>(W);
    f8v acc = 0.0f;
    if (active) {
        constexpr int U = 8;
        int k = 0;
        for (; k + U <= nv; k += U) {
            h8 w[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint64_t r = (uint32_t)__builtin_amdgcn_readfirstlane(s_idx[k + u]);
                w[u] = W8[r * row8 + q];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) acc += __builtin_convertvector(w[u], f8v);
        }
        for (; k < nv; ++k) {
            const uint64_t r = (uint32_t)__builtin_amdgcn_readfirstlane(s_idx[k]);
            acc += __builtin_convertvector(W8[r * row8 + q], f8v);
        }
    }
    h8 r16;
    if (HOUT) {
        r16 = __builtin_convertvector(acc, h8);
        acc = __builtin_convertvector(r16, f8v);
    }
    f8v p;
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = __shfl_xor(acc[e], 32);
    if (!active) return;
    if (HOUT) {
        _Float16* o = persp == 0 ? out16_stm : out16_nstm;
        __builtin_nontemporal_store(r16, reinterpret_cast<h8*>(o + (uint64_t)pos * ft_out) + q);
    } else {
        float* o = persp == 0 ? out_stm : out_nstm;
        __builtin_nontemporal_store(acc, reinterpret_cast<f8v*>(o + (uint64_t)pos * ft_out) + q);
    }
    if (lane >= 32) return;
    const f8v b0 = reinterpret_cast<const f8v*>(bias)[qp];
    const f8v b1 = reinterpret_cast<const f8v*>(bias)[qp + half8];
    f8v c;
#pragma unroll
    for (int e = 0; e < 8; ++e) c[e] = crelu01(acc[e] + b0[e]) * crelu01(p[e] + b1[e]) * scale;
    const uint64_t co = (uint64_t)pos * ft_out + persp * (ft_out / 2);
    if (combined16)
        __builtin_nontemporal_store(__builtin_convertvector(c, h8), reinterpret_cast<h8*>(combined16 + co) + qp);
    else
        __builtin_nontemporal_store(c, reinterpret_cast<f8v*>(combined + co) + qp);
}

// Element index of (row, col) of a forward table in layout `layout`
// (FtTableLayout); qc: columns per 16-byte quad (4 for f32, 8 for f16).
__host__ __device__ __forceinline__ uint64_t table_index(int layout, uint64_t row, uint32_t col, uint32_t ft_out,
                                                         uint32_t pi, uint32_t qc) {
    if (layout == kTableRows) return row * ft_out + col;
    const uint64_t blk = row / pi;
    const uint64_t f = row - blk * pi;
    const uint32_t h = ft_out / 2, hw = 2 * qc, c = col >= h ? col - h : col, s = c / hw;
    return ((blk * (h / hw) + s) * pi + f) * (4 * qc) + (col >= h ? 2 * qc : 0u) + (c - s * hw);
}

// The king block of rank `rank` when the blocks are ordered by descending
// row count over both perspectives (ties: lower block first), from the
// schedule's bins start[0 .. 2*nb] (perspective-major); up to 128 blocks,
// two per lane.
__device__ __forceinline__ uint32_t block_of_rank(const uint32_t* __restrict__ start, uint32_t nb, uint32_t rank,
                                                  uint32_t lane) {
    auto block_rows = [&](uint32_t k) -> uint32_t {
        return k < nb ? (start[k + 1] - start[k]) + (start[nb + k + 1] - start[nb + k]) : 0u;
    };
    const uint32_t z0 = block_rows(lane), z1 = block_rows(lane + 64);
    uint32_t r0 = 0, r1 = 0;
    for (uint32_t m = 0; m < nb; ++m) {
        const uint32_t zm = m < 64 ? __builtin_amdgcn_readlane(z0, m) : __builtin_amdgcn_readlane(z1, m - 64);
        r0 += (zm > z0 || (zm == z0 && m < lane)) ? 1u : 0u;
        r1 += (zm > z1 || (zm == z1 && m < lane + 64)) ? 1u : 0u;
    }
    const uint64_t h0 = __ballot(lane < nb && r0 == rank);
    const uint64_t h1 = __ballot(lane + 64 < nb && r1 == rank);
    return __builtin_amdgcn_readfirstlane(h0 ? (uint32_t)__builtin_ctzll(h0) : 64u + (uint32_t)__builtin_ctzll(h1));
}

// ---------------------------------------------------------------------------
// Forward gather with the king block's table slice resident in LDS.
//
// For a king-blocked schedule every row of block K reads only rows
// K*pi .. K*pi + pi - 1 of the table.  Workgroup (K, slice) copies those
// rows' slice (64 bytes each: 16 f32 or 32 f16 columns) into LDS once and
// then sums every row of the block from there, so the gather reads LDS (about
// 100 bytes per clock per CU for these 64-byte rows) instead of issuing one
// 16-byte vector-memory request per lane and row (64 bytes per clock per CU
// through the texture-address unit).  A row's four lanes (quads q = 0..3)
// each own one 16-byte quad of the slice: pairwise mode, quads 0-1 hold
// first-half columns and quads 2-3 their partners in the second half;
// concat mode, four consecutive quads.  Each lane sums its row's slots in
// slot order from +0.0, as the row gather does; an empty or invalid slot
// reads a zero row (adding +0.0 to a sum that started at +0.0 changes
// nothing), so the sums are bit-identical to the row gather's.  The slot
// indices are read once per row: slot 4u + q is held by lane q in register
// u and handed to the row's other lanes by a quad permute.  A row with a
// valid index outside its block (possible only when the caller's rows are
// not king-blocked) is summed again by its own lanes from global memory.
//
// Workgroups: (block rank, slice) with blocks by descending row count, and
// four consecutive slices (one 128-byte line of each output row) on one XCD
// at once, so an output line is filled in one L2.
// ---------------------------------------------------------------------------

constexpr uint32_t kFbThreads = 1024;
constexpr uint32_t kFbWaves = kFbThreads / 64;
constexpr uint32_t kFbSlots = 48;           // index slots per row read (12 per lane)
constexpr uint32_t kFbMaxPi = 1791;         // rows of a block slice held in LDS (plus the zero row)
constexpr uint32_t kFbQuadBytes = 16;

struct FtBlockFwd {
    const void* W;  // f32 or f16 table [cols][ft_out]
    const int32_t* idx_stm;
    const int32_t* idx_nstm;
    const int32_t* nnz;
    const int32_t* schedule;
    const uint32_t* sched_start;
    const uint32_t* slot_off;  // [2*batch][4 * NU] LDS byte offset of each slot
    const uint8_t* row_bad;    // [2*batch] row has an index outside its block
    const float* bias;
    float* out_stm;
    float* out_nstm;
    _Float16* out16_stm;
    _Float16* out16_nstm;
    float* combined;
    _Float16* combined16;
    uint32_t batch, ft_out, cols, max_active, n_blocks, piece_inputs, n_slices;
    float scale;
    int w_layout;  // FtTableLayout of W
};

// acc + (f32) the low / high f16 half of h2, rounded once: a mixed-precision
// FMA by 1.0 (the product is exact), one instruction where a conversion and
// an add take two.
__device__ __forceinline__ float add_f16_lo(uint32_t h2, float acc) {
    float d;
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h2), "v"(acc));
    return d;
}
__device__ __forceinline__ float add_f16_hi(uint32_t h2, float acc) {
    float d;
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h2), "v"(acc));
    return d;
}

// A quad-permute broadcast of lane `src` of every group of four lanes.
template <int SRC>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, SRC * 0x55, 0xF, 0xF, true);
}

// NU: slot quads read per row (4 * NU >= max_active; slots past max_active
// are empty and read the zero row).
template <int MODE, typename T, bool HOUT, int NU>
__global__ __launch_bounds__(kFbThreads) void ft_forward_block_kernel(FtBlockFwd a) {
    static_assert(4 * NU <= (int)kFbSlots, "slot quads");
    constexpr bool H16 = sizeof(T) == 2;
    constexpr uint32_t QC = H16 ? 8 : 4;  // columns per quad
    typedef float accv __attribute__((ext_vector_type(QC)));
    typedef T rowv __attribute__((ext_vector_type(QC)));
    static_assert(sizeof(rowv) == kFbQuadBytes, "a quad is 16 bytes");
    __shared__ uint4 s_w[(kFbMaxPi + 1) * 4];  // feature f's quad q at 4f + q; row pi is zero

    const uint32_t lane = threadIdx.x % 64, q = lane & 3u, r = lane >> 2;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t nb = a.n_blocks;
    const uint32_t xcd = blockIdx.x % kNumXcd, j = blockIdx.x / kNumXcd;
    const uint32_t n_sg = (a.n_slices + 3) / 4;
    const uint32_t item = (j / 4) * kNumXcd + xcd;
    if (item >= nb * n_sg) return;
    const uint32_t slice = (item % n_sg) * 4 + j % 4;
    if (slice >= a.n_slices) return;
    const uint32_t K = block_of_rank(a.sched_start, nb, item / n_sg, lane);
    const uint32_t a0 = a.sched_start[K], na = a.sched_start[K + 1] - a0;
    const uint32_t b0 = a.sched_start[nb + K];
    const uint32_t n = na + (a.sched_start[nb + K + 1] - b0);
    if (n == 0) return;

    // the columns of quad q in this slice
    const uint32_t H = a.ft_out / 2;
    auto quad_col = [&](uint32_t qq) -> uint32_t {
        return MODE == kPair ? (qq >= 2 ? H : 0u) + slice * 2 * QC + (qq & 1u) * QC : slice * 4 * QC + qq * QC;
    };
    const uint32_t col = quad_col(q);
    const T* W = reinterpret_cast<const T*>(a.W);
    const uint32_t PI = a.piece_inputs, blk_lo = K * PI;
    const uint32_t nfeat = a.cols > blk_lo ? (a.cols - blk_lo < PI ? a.cols - blk_lo : PI) : 0u;
    // a slice-major table holds this slice as one contiguous run of pi
    // features x 64 bytes (quad i at element i * QC)
    const T* Ws = W + (uint64_t)(K * a.n_slices + slice) * PI * (4 * QC);
    for (uint32_t i = threadIdx.x; i < (PI + 1) * 4; i += kFbThreads) {
        const uint32_t f = i / 4;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (f < nfeat)
            v = a.w_layout != kTableRows
                    ? *reinterpret_cast<const uint4*>(Ws + (uint64_t)i * QC)
                    : *reinterpret_cast<const uint4*>(W + (uint64_t)(blk_lo + f) * a.ft_out + quad_col(i % 4));
        s_w[i] = v;
    }

    // bias of the lane's columns (and of their partners: quad q ^ 2)
    accv b_own, b_par;
    const uint32_t col_par = MODE == kPair ? quad_col(q ^ 2u) : col;
#pragma unroll
    for (uint32_t e = 0; e < QC; ++e) {
        b_own[e] = a.bias[col + e];
        b_par[e] = a.bias[col_par + e];
    }
    __syncthreads();

    // Rows go in groups of 16 (one per four lanes), wave w taking groups w,
    // w + 16, ...  A group's slot offsets are loaded while the wave sums the
    // group before it, and its schedule entry a group earlier still, so the
    // sums never wait for the chain entry -> position -> slots.  Each half
    // iteration issues the position two groups ahead, then the eleven slot
    // loads of the next group (unconditional, so every wait leaves at least
    // eleven loads in flight rather than waiting for the stores).  Group rows
    // past the block's list take its first entry and are empty.
    const uint32_t n_groups = (n + 15) / 16;
    const char* s_bytes = reinterpret_cast<const char*>(s_w);
    auto entry = [&](uint32_t gg) -> uint32_t {
        const uint32_t jr = gg * 16 + r;
        const uint32_t e = (jr < na ? a0 : b0 - na) + jr;
        return jr < n ? e : a0;
    };
    auto row_ptr = [&](uint32_t e, uint32_t pos) -> const int32_t* {
        return (e >= a.batch ? a.idx_nstm : a.idx_stm) + (uint64_t)pos * a.max_active;
    };
    struct Slots {
        uint32_t off[NU];  // slot 4u + q: its row's LDS byte offset
        uint32_t bad;
    };
    auto load_slots = [&](uint32_t e, uint32_t pos, Slots& s) {
        const uint32_t i = (e >= a.batch ? a.batch : 0u) + pos;
        const uint32_t* so = a.slot_off + (uint64_t)i * (4 * NU) + q;
        s.bad = a.row_bad[i];
#pragma unroll
        for (uint32_t u = 0; u < (uint32_t)NU; ++u) s.off[u] = so[4 * u];
    };
    // One group: sums of group gg from its slots s_c (position pos).
    auto group = [&](uint32_t gg, const Slots& s_c, uint32_t pos) {
        const bool live = gg * 16 + r < n;
        const uint32_t e_c = entry(gg);
        const uint32_t persp = e_c >= a.batch ? 1u : 0u;
        // slot 4u + q: its row's byte offset in LDS (the zero row for an
        // empty or invalid slot, and for slots past max_active)
        const uint32_t* off = s_c.off;
        const bool bad = live && s_c.bad != 0;
        accv acc = 0.0f;
        // Slots four at a time: the four reads of slot quad u + 1 are issued
        // before the adds of quad u, so eight reads can be in flight.
        auto read4 = [&](uint32_t u, uint4 (&d)[4]) {
            d[0] = *reinterpret_cast<const uint4*>(s_bytes + quad_bcast<0>(off[u]) + q * kFbQuadBytes);
            d[1] = *reinterpret_cast<const uint4*>(s_bytes + quad_bcast<1>(off[u]) + q * kFbQuadBytes);
            d[2] = *reinterpret_cast<const uint4*>(s_bytes + quad_bcast<2>(off[u]) + q * kFbQuadBytes);
            d[3] = *reinterpret_cast<const uint4*>(s_bytes + quad_bcast<3>(off[u]) + q * kFbQuadBytes);
        };
        auto add4 = [&](const uint4 (&d)[4]) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if constexpr (H16) {
                    acc[0] = add_f16_lo(d[s].x, acc[0]);
                    acc[1] = add_f16_hi(d[s].x, acc[1]);
                    acc[2] = add_f16_lo(d[s].y, acc[2]);
                    acc[3] = add_f16_hi(d[s].y, acc[3]);
                    acc[4] = add_f16_lo(d[s].z, acc[4]);
                    acc[5] = add_f16_hi(d[s].z, acc[5]);
                    acc[6] = add_f16_lo(d[s].w, acc[6]);
                    acc[7] = add_f16_hi(d[s].w, acc[7]);
                } else {
                    acc += __builtin_bit_cast(accv, d[s]);
                }
            }
        };
        uint4 w0[4], w1[4];
        read4(0, w0);
#pragma unroll
        for (uint32_t u = 0; u < (uint32_t)NU; u += 2) {
            if (u + 1 < (uint32_t)NU) read4(u + 1, w1);
            add4(w0);
            if (u + 1 < (uint32_t)NU) {
                if (u + 2 < (uint32_t)NU) read4(u + 2, w0);
                add4(w1);
            }
        }
        // a row with an index outside its block: its lanes sum it again from
        // global memory, valid slots in slot order
        const uint64_t bad_lanes = __ballot(bad);
        if (bad_lanes) {
            if ((bad_lanes >> (4 * r)) & 0xFull) {
                const int32_t* idx = row_ptr(e_c, pos);
                const int32_t nz = a.nnz[pos];
                const uint32_t nv = nz <= 0 ? 0u : ((uint32_t)nz < a.max_active ? (uint32_t)nz : a.max_active);
                acc = 0.0f;
                for (uint32_t k = 0; k < nv; ++k) {
                    const int32_t v = idx[k];
                    if (v < 0 || (uint32_t)v >= a.cols) continue;
                    acc += __builtin_convertvector(
                        *reinterpret_cast<const rowv*>(W + table_index(a.w_layout, (uint32_t)v, col, a.ft_out, PI, QC)),
                        accv);
                }
            }
        }

        if (MODE == kPair) {
            rowv r16;
            if (HOUT) {
                r16 = __builtin_convertvector(acc, rowv);
                acc = __builtin_convertvector(r16, accv);
            }
            // the partner columns' sums, from lane q ^ 2 of the row (each
            // element copied to a scalar first: a bit cast of a vector
            // element reads element 0)
            accv p;
#pragma unroll
            for (uint32_t e2 = 0; e2 < QC; ++e2) {
                const float x = acc[e2];
                p[e2] = __int_as_float(
                    __builtin_amdgcn_mov_dpp(__float_as_int(x), 2 | 3 << 2 | 0 << 4 | 1 << 6, 0xF, 0xF, true));
            }
            if (live) {
                // plain stores: four workgroups fill each 128-byte line, which
                // L2 assembles before it writes the line back
                if (HOUT) {
                    _Float16* o = persp ? a.out16_nstm : a.out16_stm;
                    *reinterpret_cast<rowv*>(o + (uint64_t)pos * a.ft_out + col) = r16;
                } else {
                    float* o = persp ? a.out_nstm : a.out_stm;
                    *reinterpret_cast<accv*>(o + (uint64_t)pos * a.ft_out + col) = acc;
                }
                if (q < 2) {
                    accv c;
#pragma unroll
                    for (uint32_t e2 = 0; e2 < QC; ++e2)
                        c[e2] = crelu01(acc[e2] + b_own[e2]) * crelu01(p[e2] + b_par[e2]) * a.scale;
                    const uint64_t co = (uint64_t)pos * a.ft_out + persp * H + col;
                    if (a.combined16) {
                        typedef _Float16 hv __attribute__((ext_vector_type(QC)));
                        *reinterpret_cast<hv*>(a.combined16 + co) = __builtin_convertvector(c, hv);
                    } else {
                        *reinterpret_cast<accv*>(a.combined + co) = c;
                    }
                }
            }
        } else if (live) {
            // Simple: ft_out += bias in place, combined[off + c] = crelu(x)
            const accv x = acc + b_own;
            float* o = persp ? a.out_nstm : a.out_stm;
            *reinterpret_cast<accv*>(o + (uint64_t)pos * a.ft_out + col) = x;
            accv c;
#pragma unroll
            for (uint32_t e2 = 0; e2 < QC; ++e2) c[e2] = crelu01(x[e2]);
            *reinterpret_cast<accv*>(a.combined + (uint64_t)pos * 2 * a.ft_out + persp * a.ft_out + col) = c;
        }
    };
    // Two register sets: set X sums group g while set Y's slots (group
    // g + 16) are loaded; X's position register is reloaded with group
    // g + 32's first (its old value copied once its load is long done).
    uint32_t g = wave;
    if (g >= n_groups) return;
    uint32_t pA = (uint32_t)a.schedule[entry(g)];
    uint32_t pB = (uint32_t)a.schedule[entry(g + kFbWaves)];
    __builtin_amdgcn_sched_barrier(0);
    Slots sA, sB;
    load_slots(entry(g), pA, sA);
    auto half = [&](uint32_t gg, Slots& sx, uint32_t& px, Slots& sy, const uint32_t& py) {
        const uint32_t pos = px;
        px = (uint32_t)a.schedule[entry(gg + 2 * kFbWaves)];
        __builtin_amdgcn_sched_barrier(0);
        load_slots(entry(gg + kFbWaves), py, sy);
        __builtin_amdgcn_sched_barrier(0);
        group(gg, sx, pos);
    };
    for (;;) {
        half(g, sA, pA, sB, pB);
        g += kFbWaves;
        if (g >= n_groups) break;
        half(g, sB, pB, sA, pA);
        g += kFbWaves;
        if (g >= n_groups) break;
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

// The same keys (a wave per kKeyRowsPerWave rows, lane = slot) and, for the block-resident
// forward, every slot's LDS byte offset in rows of `stride` >= max_active
// slots: (v - k * pi) * 64 for a valid index v of the row's block k, pi * 64
// (the zero row) for an empty or invalid slot, an index outside the block
// and the padding past max_active; row_bad[i] = 1 when the row has a valid
// index outside its block.
constexpr uint32_t kKeyRowsPerWave = 8;

__global__ void king_block_rows_kernel(const int32_t* __restrict__ idx_stm, const int32_t* __restrict__ idx_nstm,
                                       const int32_t* __restrict__ nnz, uint8_t* __restrict__ keys,
                                       uint32_t* __restrict__ slot_off, uint8_t* __restrict__ row_bad,
                                       uint32_t batch, uint32_t max_active, uint32_t stride, uint32_t cols,
                                       uint32_t piece_inputs, uint32_t n_bins) {
    const uint64_t w = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) / 64;
    const uint32_t lane = threadIdx.x % 64;
#pragma unroll
    for (uint32_t rr = 0; rr < kKeyRowsPerWave; ++rr) {
        const uint64_t i = w * kKeyRowsPerWave + rr;
        if (i >= 2ull * batch) return;
        const uint32_t persp = i >= batch ? 1u : 0u;
        const uint32_t b = (uint32_t)(i - (uint64_t)persp * batch);
        const int32_t nz = nnz[b];
        const uint32_t n = nz <= 0 ? 0u : ((uint32_t)nz < max_active ? (uint32_t)nz : max_active);
        const int32_t v = lane < n ? ((persp ? idx_nstm : idx_stm) + (uint64_t)b * max_active)[lane] : -1;
        const bool valid = v >= 0 && (uint32_t)v < cols;
        const uint64_t vm = __ballot(valid);
        uint32_t k = 0;
        if (vm) {
            const uint32_t v0 = (uint32_t)__builtin_amdgcn_readlane(v, (int)__builtin_ctzll(vm));
            k = piece_inputs ? v0 / piece_inputs : 0u;
            if (k >= n_bins) k = n_bins - 1;
        }
        const uint32_t local = (uint32_t)v - k * piece_inputs;
        const bool in_block = valid && local < piece_inputs;
        if (lane < stride) slot_off[i * stride + lane] = (in_block ? local : piece_inputs) * 64u;
        const uint64_t bad = __ballot(valid && !in_block);
        if (lane == 0) {
            keys[i] = (uint8_t)(persp * n_bins + k);
            row_bad[i] = bad ? 1u : 0u;
        }
    }
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
                                             uint32_t max_active, uint32_t cols,
                                             const uint32_t* __restrict__ run_if) {
    if (run_if && __builtin_amdgcn_readfirstlane(*run_if) == 0u) return;
    const uint64_t per = (uint64_t)batch * max_active;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2 * per;
         i += (uint64_t)gridDim.x * blockDim.x) {
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
}

// Segment offsets from the sorted keys: offsets[k] = first sorted position
// with key >= k, for k in [0, n_keys]; offsets[n_keys] = n_items.  Each entry
// is written by exactly one thread (the one at the boundary it falls in), so
// no histogram, atomics or scan are needed.
__global__ void occurrence_offsets_kernel(const uint32_t* __restrict__ sorted_keys,
                                          uint64_t n_items, uint32_t n_keys,
                                          uint32_t* __restrict__ offsets,
                                          const uint32_t* __restrict__ run_if) {
    if (run_if && __builtin_amdgcn_readfirstlane(*run_if) == 0u) return;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i <= n_items;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const int64_t prev = i == 0 ? -1 : (int64_t)sorted_keys[i - 1];
        const int64_t cur = i == n_items ? (int64_t)n_keys : (int64_t)sorted_keys[i];
        for (int64_t k = prev + 1; k <= cur; ++k) offsets[k] = (uint32_t)i;
    }
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
using vech = _Float16 __attribute__((ext_vector_type(V)));

// Sequential sums, from acc, of the dft rows vals[s..e) at vector column q,
// in f32 (V values per lane).  The row ids are wave-uniform, so a row's
// address is a scalar base plus the lane's column.
template <int V>
__device__ __forceinline__ vecf<V> segment_sum(const vecf<V>* __restrict__ dft, uint64_t row_v,
                                               const uint32_t* __restrict__ vals, uint32_t s,
                                               uint32_t e, uint64_t q, vecf<V> acc) {
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

// The same sequential sum over f16 dft rows (V values per lane), in f32.
template <int V>
__device__ __forceinline__ vecf<V> segment_sum_f16(const vech<V>* __restrict__ dft, uint64_t row_v,
                                                   const uint32_t* __restrict__ vals, uint32_t s,
                                                   uint32_t e, uint64_t q, vecf<V> acc) {
    constexpr int U = 64 / V;
    uint32_t i = s;
    for (; i + U <= e; i += U) {
        vech<V> d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t r = __builtin_amdgcn_readfirstlane(vals[i + u]);
            d[u] = dft[r * row_v + q];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += __builtin_convertvector(d[u], vecf<V>);
    }
    for (; i < e; ++i) {
        const uint64_t r = __builtin_amdgcn_readfirstlane(vals[i]);
        acc += __builtin_convertvector(dft[r * row_v + q], vecf<V>);
    }
    return acc;
}

template <int V>
__device__ __forceinline__ void lookahead(vecf<V>& W, float* __restrict__ slow, uint64_t off,
                                          const OptScalars& s) {
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

// The optimizer state of V consecutive cells (f32 weights; f32 moments, or
// f16 moments stored scaled when HSTATE), loaded with non-temporal loads.
template <int V, bool HSTATE>
struct CellState {
    using Mom = typename std::conditional<HSTATE, vech<V>, vecf<V>>::type;
    vecf<V> w;
    Mom m, v;
};

template <int V, bool HSTATE>
__device__ __forceinline__ CellState<V, HSTATE> load_cells(const FtGradArgs& a, uint64_t off) {
    using Mom = typename CellState<V, HSTATE>::Mom;
    CellState<V, HSTATE> c;
    c.w = __builtin_nontemporal_load(reinterpret_cast<vecf<V>*>(a.w) + off);
    if constexpr (HSTATE) {
        c.m = __builtin_nontemporal_load(reinterpret_cast<Mom*>(a.m16) + off);
        c.v = __builtin_nontemporal_load(reinterpret_cast<Mom*>(a.v16) + off);
    } else {
        c.m = __builtin_nontemporal_load(reinterpret_cast<Mom*>(a.m) + off);
        c.v = __builtin_nontemporal_load(reinterpret_cast<Mom*>(a.v) + off);
    }
    return c;
}

// RAdam of the loaded cells with gradient g: the new weights, and the new
// moments in c (f16 moments as radam_step_f16state,
// native_kernels.cu:1118-1170: read back as f16 / scale, stored as
// f16(m * m_scale) clamped to +-65504 and f16(v * v_scale) clamped above at
// 65504, a NaN staying NaN).
// The scales are powers of two (the launchers check it), so x / scale is
// x scaled by an exact power of two: v_ldexp_f32 rounds the same exact value,
// bit for bit, without a division sequence.
template <int V, bool HSTATE>
__device__ __forceinline__ vecf<V> radam_cells(const FtGradArgs& a, vecf<V> g, CellState<V, HSTATE>& c) {
    const OptScalars& s = a.opt;
    vecf<V> W = c.w;
    // scale = 2^(e - 1) with e the frexp exponent
    const int m_shift = 1 - __builtin_amdgcn_frexp_expf(a.m_scale), v_shift = 1 - __builtin_amdgcn_frexp_expf(a.v_scale);
#pragma unroll
    for (int k = 0; k < V; ++k) {
        float w = W[k], m, v;
        if constexpr (HSTATE) {
            m = __builtin_amdgcn_ldexpf((float)c.m[k], m_shift);
            v = __builtin_amdgcn_ldexpf((float)c.v[k], v_shift);
        } else {
            m = c.m[k];
            v = c.v[k];
        }
        radam_elem(w, m, v, g[k], s);
        W[k] = w;
        if constexpr (HSTATE) {
            float sm = m * a.m_scale;
            sm = sm > 65504.0f ? 65504.0f : (sm < -65504.0f ? -65504.0f : sm);
            float sv = v * a.v_scale;
            sv = sv > 65504.0f ? 65504.0f : sv;
            c.m[k] = (_Float16)sm;
            c.v[k] = (_Float16)sv;
        } else {
            c.m[k] = m;
            c.v[k] = v;
        }
    }
    return W;
}

// The Ranger lerp of the new weights W and the slow weights S.
template <int V>
__device__ __forceinline__ void lerp_cells(const FtGradArgs& a, vecf<V>& W, vecf<V>& S) {
#pragma unroll
    for (int k = 0; k < V; ++k) {
        float x = W[k], y = S[k];
        lerp_elem(x, y, a.opt.alpha);
        W[k] = x;
        S[k] = y;
    }
}

// The stores of updated cells: weights, moments, and the f16 mirror of the
// new weights when the forward reads one.
template <int V, bool HSTATE>
__device__ __forceinline__ void store_cells(const FtGradArgs& a, uint64_t off, vecf<V> W,
                                            const CellState<V, HSTATE>& c) {
    using Mom = typename CellState<V, HSTATE>::Mom;
    __builtin_nontemporal_store(W, reinterpret_cast<vecf<V>*>(a.w) + off);
    if constexpr (HSTATE) {
        __builtin_nontemporal_store(c.m, reinterpret_cast<Mom*>(a.m16) + off);
        __builtin_nontemporal_store(c.v, reinterpret_cast<Mom*>(a.v16) + off);
    } else {
        __builtin_nontemporal_store(c.m, reinterpret_cast<Mom*>(a.m) + off);
        __builtin_nontemporal_store(c.v, reinterpret_cast<Mom*>(a.v) + off);
    }
    if (a.mirror16)
        __builtin_nontemporal_store(__builtin_convertvector(W, vech<V>),
                                    reinterpret_cast<vech<V>*>(a.mirror16) + off);
}

// RAdam (+ Ranger lerp every lookahead step) of the loaded cells with
// gradient g, and the stores.
template <int V, bool HSTATE>
__device__ __forceinline__ void apply_cells(const FtGradArgs& a, uint64_t off, vecf<V> g,
                                            CellState<V, HSTATE> c) {
    vecf<V> W = radam_cells<V, HSTATE>(a, g, c);
    if (a.opt.lookahead) {
        vecf<V>* s_ = reinterpret_cast<vecf<V>*>(a.slow) + off;
        vecf<V> S = __builtin_nontemporal_load(s_);
        lerp_cells<V>(a, W, S);
        __builtin_nontemporal_store(S, s_);
    }
    store_cells<V, HSTATE>(a, off, W, c);
}

// The fused update of F feature rows f0 + k * step (k < nf) at the lane's
// columns col .. col + 3, with gradients gfn(k), each row's state loaded D
// rows ahead of its update.  The loads are unconditional (rows past nload >=
// max(nf, 1) re-load row nload - 1, and rows past nf are not stored) and
// come before the earlier rows' stores in program order, so the wave keeps loads in flight and the
// wait before a row's update counts only the loads issued after its own.  A
// row's address is a row base plus the lane's 32-bit column offset (a
// wave-uniform base when f0 is).  LA: this step's Ranger lerp, the slow
// weights loaded with the rest of the state.
template <int F, int D, bool HSTATE, bool LA, typename G>
__device__ __forceinline__ void update_rows_pipelined(const FtGradArgs& a, uint64_t f0, uint32_t step, uint32_t col,
                                                      uint32_t nf, uint32_t nload, G gfn) {
    using Mom = typename CellState<4, HSTATE>::Mom;
    const uint64_t ft_out = a.ft_out;
    // the lane's byte offsets within a row: f32 values and f16 moments
    const uint32_t b32 = col * 4u, b16 = col * 2u;
    auto at = [](auto* base, uint64_t row_elem, uint32_t lane_bytes) {
        using T = typename std::remove_pointer<decltype(base)>::type;
        return reinterpret_cast<T*>(reinterpret_cast<char*>(base + row_elem) + lane_bytes);
    };
    auto row_of = [&](int j) -> uint64_t {
        return (f0 + (uint64_t)((uint32_t)j < nload ? (uint32_t)j : nload - 1) * step) * ft_out;
    };
    CellState<4, HSTATE> cs[F];
    vecf<4> sl[F];
    auto load = [&](int j) {
        const uint64_t r = row_of(j);
        cs[j].w = __builtin_nontemporal_load(reinterpret_cast<const vecf<4>*>(at(a.w, r, b32)));
        if constexpr (HSTATE) {
            cs[j].m = __builtin_nontemporal_load(reinterpret_cast<const Mom*>(at(a.m16, r, b16)));
            cs[j].v = __builtin_nontemporal_load(reinterpret_cast<const Mom*>(at(a.v16, r, b16)));
        } else {
            cs[j].m = __builtin_nontemporal_load(reinterpret_cast<const Mom*>(at(a.m, r, b32)));
            cs[j].v = __builtin_nontemporal_load(reinterpret_cast<const Mom*>(at(a.v, r, b32)));
        }
        if constexpr (LA) sl[j] = __builtin_nontemporal_load(reinterpret_cast<const vecf<4>*>(at(a.slow, r, b32)));
    };
#pragma unroll
    for (int j = 0; j < D && j < F; ++j) load(j);
#pragma unroll
    for (int k = 0; k < F; ++k) {
        if (k + D < F) load(k + D);
        if ((uint32_t)k < nf) {
            const uint64_t r = (f0 + (uint64_t)k * step) * ft_out;
            vecf<4> W = radam_cells<4, HSTATE>(a, gfn(k), cs[k]);
            if constexpr (LA) {
                lerp_cells<4>(a, W, sl[k]);
                __builtin_nontemporal_store(sl[k], reinterpret_cast<vecf<4>*>(at(a.slow, r, b32)));
            }
            __builtin_nontemporal_store(W, reinterpret_cast<vecf<4>*>(at(a.w, r, b32)));
            if constexpr (HSTATE) {
                __builtin_nontemporal_store(cs[k].m, reinterpret_cast<Mom*>(at(a.m16, r, b16)));
                __builtin_nontemporal_store(cs[k].v, reinterpret_cast<Mom*>(at(a.v16, r, b16)));
            } else {
                __builtin_nontemporal_store(cs[k].m, reinterpret_cast<Mom*>(at(a.m, r, b32)));
                __builtin_nontemporal_store(cs[k].v, reinterpret_cast<Mom*>(at(a.v, r, b32)));
            }
            if (a.mirror16)
                __builtin_nontemporal_store(__builtin_convertvector(W, vech<4>),
                                            reinterpret_cast<vech<4>*>(at(a.mirror16, r, b16)));
        }
    }
}

// One cell group's update in the moment format the trainer uses.
template <int V, bool HSTATE>
__device__ __forceinline__ void update_cells(const FtGradArgs& a, uint64_t off, vecf<V> g) {
    apply_cells<V, HSTATE>(a, off, g, load_cells<V, HSTATE>(a, off));
}

// dft_row_stride / dft_chunk_stride: the dft strides in elements (chunk =
// kDftChunk columns).  HDFT: the dft is f16 and each row sum is multiplied by
// dft_inv_scale (gather_and_sum_per_feature_*_fp16, native_kernels.cu:
// 1030-1100).
template <int V, bool HDFT, bool HSTATE>
__device__ __forceinline__ void grad_update_task(const FtGradArgs& a, uint64_t task, uint32_t lane) {
    constexpr uint32_t kCols = kWave * V;
    const uint32_t chunk = (uint32_t)(task / a.rows);
    const uint32_t f = (uint32_t)(task - (uint64_t)chunk * a.rows);
    const uint32_t col = chunk * kCols + lane * V;
    const uint32_t s0 = __builtin_amdgcn_readfirstlane(a.occ_off[2 * f]);
    const uint32_t s1 = __builtin_amdgcn_readfirstlane(a.occ_off[2 * f + 2]);
    if (col >= a.ft_out) return;
    const uint64_t q = ((uint64_t)(col / kDftChunk) * a.dft_chunk_stride + col % kDftChunk) / V;
    const uint64_t off = ((uint64_t)f * a.ft_out + col) / V;
    vecf<V>* grad = reinterpret_cast<vecf<V>*>(a.grad);
    vecf<V> gr = 0.0f;
    if constexpr (HDFT)
        gr = segment_sum_f16<V>(reinterpret_cast<const vech<V>*>(a.dft16), a.dft_row_stride / V, a.occ_vals, s0,
                                s1, q, gr);
    else
        gr = segment_sum<V>(reinterpret_cast<const vecf<V>*>(a.dft), a.dft_row_stride / V, a.occ_vals, s0, s1, q,
                            gr);
    if constexpr (HDFT) gr *= a.dft_inv_scale;
    if (a.grad) __builtin_nontemporal_store(gr, grad + off);
    if (a.apply_update) update_cells<V, HSTATE>(a, off, gr);
}

// One wave per task (feature row, column chunk).  GATED: the launch does
// nothing unless *run_if != 0 and strides its tasks over a bounded grid, so
// it costs little when skipped (the block scan's fallback); otherwise one
// task per wave, which keeps the gather loop's code tight.
template <int V, bool HDFT, bool HSTATE, bool GATED>
__global__ __launch_bounds__(256) void ft_grad_update_kernel(FtGradArgs a, uint32_t n_chunks) {
    constexpr uint32_t kCols = kWave * V;
    static_assert(kDftChunk % V == 0 && (kDftChunk % kCols == 0 || kCols % kDftChunk == 0),
                  "a lane's values must lie in one dft chunk");
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint64_t total = (uint64_t)a.rows * n_chunks;
    if constexpr (GATED) {
        if (__builtin_amdgcn_readfirstlane(*a.run_if) == 0u) return;
        const uint64_t stride = (uint64_t)gridDim.x * kWavesPerBlock;
        for (uint64_t task = (uint64_t)bid * kWavesPerBlock + wave; task < total; task += stride)
            grad_update_task<V, HDFT, HSTATE>(a, task, lane);
    } else {
        const uint64_t task = (uint64_t)bid * kWavesPerBlock + wave;
        if (task < total) grad_update_task<V, HDFT, HSTATE>(a, task, lane);
    }
}

// ---------------------------------------------------------------------------
// FT backward by block scan.
//
// In a king-bucketed feature set every active feature of a perspective lies
// in that perspective's king block [K*PI, (K+1)*PI), so the dft rows that
// contribute to block K's features are exactly the rows the forward schedule
// files under block K: the stm rows of its bin (positions ascending), then
// the nstm rows of its bin.  That is the order in which the reference CPU
// backward visits them (stm pass over positions, then nstm), so walking the
// list once and adding each row to the features that occur in it gives every
// feature the sequential sum of the occurrence-list kernel above, bit for
// bit.
//
// A workgroup owns one 256-column chunk and a group of GS features of one
// block (wave w: 16 of them, accumulated in registers, four columns per
// lane: features g*GS + 16w .. +15, or g*GS + w + 8k when the tables deal
// the group round-robin, FtBlockScan::dealt).  It stages each row's chunk in LDS once
// (a dft row is read once per group instead of once per occurrence) and
// every wave adds it to those of its features whose bit is set in the row's
// hit mask.  Per stage of 32 rows a wave reads 16 feature masks (bit r: the
// stage's row r holds the feature), so feature k's accumulator is a fixed
// register and its rows are added in list order.  The optimizer update of
// the group's cells follows the scan in the same workgroup.
//
// Stage tables (ft_scan_tables_kernel, once per step for all column
// chunks): the blocks' stages numbered consecutively, block K's first at
// sum over k < K of ceil(rows_k / 32); for each stage the dft row of each
// of its 32 slots (perspective * batch + position; slots past the block's
// list repeat its last row) and, for mask word q = g*W + w and feature k,
// a slot mask whose bit r is set when slot r's row holds block feature
// g*GS + 16w + k (dealt: g*GS + w + 8k).  A row with a feature outside its own block, or with one
// feature in two slots, sets *multi; the scan then leaves the step to the
// occurrence-list kernel, which runs only in that case.
// ---------------------------------------------------------------------------

constexpr int kScanWaves = 8;
constexpr int kScanFeat = 16;  // features per wave (low bits of a mask word)
static_assert(kScanFeat <= 32, "a mask word per wave");
constexpr int kScanStage = 32;  // rows per LDS stage

constexpr int kScanMaxWords = 128;  // mask words per row

struct ScanGeom {
    uint32_t n_groups, group_size, words;
};

__host__ __device__ inline ScanGeom scan_geom(uint32_t piece_inputs) {
    const uint32_t cap = (uint32_t)(kScanWaves * kScanFeat);
    ScanGeom g;
    g.n_groups = (piece_inputs + cap - 1) / cap;
    g.group_size = g.n_groups ? (piece_inputs + g.n_groups - 1) / g.n_groups : 0;
    g.words = g.n_groups * kScanWaves;
    return g;
}

__device__ __forceinline__ uint32_t block_of_rank(const FtBlockScan& s, uint32_t rank, uint32_t lane) {
    return block_of_rank(s.sched_start, s.n_blocks, rank, lane);
}

// The first stage of block K in the stage tables: the blocks before it
// hold ceil(rows / 32) stages each (at most 128 blocks, two per lane).
__device__ __forceinline__ uint32_t block_stage_base(const FtBlockScan& s, uint32_t K, uint32_t lane) {
    const uint32_t nb = s.n_blocks;
    auto stages = [&](uint32_t k) -> uint32_t {
        return k < K ? ((s.sched_start[k + 1] - s.sched_start[k]) + (s.sched_start[nb + k + 1] - s.sched_start[nb + k]) +
                        31u) / 32u
                     : 0u;
    };
    uint32_t v = stages(lane) + stages(lane + 64);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return __builtin_amdgcn_readfirstlane(v);
}

// One wave per stage.  Thread 0 of each workgroup numbers the blocks'
// stages (at most 128 blocks); a wave finds its block by binary search,
// loads its 32 slots' schedule entries and feature counts at once (lane =
// slot), then the slots' feature indices four rows at a time (lane =
// feature slot), and sets the slot bits of its feature masks in LDS.
__global__ __launch_bounds__(256) void ft_scan_tables_kernel(FtBlockScan s, ScanGeom geom) {
    static_assert(kScanFeat == 16 && kScanStage == 32, "32 slots per stage, 16 features per mask word");
    __shared__ uint32_t s_base[129];
    __shared__ uint32_t s_t[4][kScanMaxWords * kScanFeat];  // per wave: [mask word][feature]
    const uint32_t nb = s.n_blocks;
    if (threadIdx.x == 0) {
        uint32_t acc = 0;
        for (uint32_t k = 0; k < nb; ++k) {
            s_base[k] = acc;
            const uint32_t rows = (s.sched_start[k + 1] - s.sched_start[k]) +
                                  (s.sched_start[nb + k + 1] - s.sched_start[nb + k]);
            acc += (rows + 31u) / 32u;
        }
        s_base[nb] = acc;
    }
    __syncthreads();
    const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint32_t gs = blockIdx.x * 4 + wave;
    if (gs >= s_base[nb]) return;
    // the block: the last K with s_base[K] <= gs (an empty block shares its
    // base with the next one, so the last is the one the stage belongs to)
    uint32_t lo = 0, hi = nb - 1;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) / 2;
        if (s_base[mid] <= gs) lo = mid;
        else hi = mid - 1;
    }
    const uint32_t K = lo, T = gs - s_base[K];
    const uint32_t a0 = s.sched_start[K], na = s.sched_start[K + 1] - a0;
    const uint32_t b0 = s.sched_start[nb + K];
    const uint32_t n = na + (s.sched_start[nb + K + 1] - b0);  // >= 1: the block has this stage
    const uint32_t W = geom.words, WK = W * kScanFeat;
    uint32_t* st = s_t[wave];
    for (uint32_t i = lane; i < WK; i += 64) st[i] = 0u;
    // slot lane % 32: its row (slots past the block's list repeat its last row)
    const uint32_t slots = n - T * 32u < 32u ? n - T * 32u : 32u;
    const uint32_t jc = T * 32u + ((lane & 31u) < slots ? (lane & 31u) : slots - 1);
    const uint32_t e = jc < na ? a0 + jc : b0 + (jc - na);
    const uint32_t persp = e >= s.batch ? 1u : 0u;
    const uint32_t pos = (uint32_t)s.schedule[e];
    if (lane < 32) s.stage_rows[(uint64_t)gs * 32 + lane] = persp * s.batch + pos;
    const int32_t nz = s.nnz[pos];
    const uint32_t nn = nz <= 0 ? 0u : ((uint32_t)nz < s.max_active ? (uint32_t)nz : s.max_active);
    const int64_t blk_lo = (int64_t)K * s.piece_inputs;
    bool multi = false;
    for (uint32_t r0 = 0; r0 < slots; r0 += 4) {
        int32_t v[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t r = (r0 + u) & 31u;
            const uint32_t pr = __builtin_amdgcn_readlane(pos, r), pp = __builtin_amdgcn_readlane(persp, r);
            const uint32_t nr = __builtin_amdgcn_readlane(nn, r);
            v[u] = (r0 + u < slots && lane < nr) ? (pp ? s.idx_nstm : s.idx_stm)[(uint64_t)pr * s.max_active + lane]
                                                 : -1;
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const int32_t x = v[u];
            if (x < 0 || (uint32_t)x >= s.cols) continue;  // an empty or invalid slot
            const int64_t local = (int64_t)x - blk_lo;
            if (local < 0 || local >= (int64_t)s.piece_inputs) {
                multi = true;  // a feature outside the row's block
                continue;
            }
            const uint32_t g = (uint32_t)local / geom.group_size;
            const uint32_t rr = (uint32_t)local - g * geom.group_size;
            // the group's feature rr: wave rr / 16, entry rr % 16; dealt
            // (s.dealt): wave rr % 8, entry rr / 8
            const uint32_t q = g * kScanWaves + (s.dealt ? rr % kScanWaves : rr / kScanFeat);
            const uint32_t e = s.dealt ? rr / kScanWaves : rr % kScanFeat;
            const uint32_t bit = 1u << (r0 + u);
            const uint32_t old = atomicOr(&st[q * kScanFeat + e], bit);
            if (old & bit) multi = true;  // the feature is in the row twice
        }
    }
    if (multi) {
        atomicOr(s.multi, 1u);
        if (s.multi_sticky) atomicOr(s.multi_sticky, 1u);
    }
    uint32_t* out = s.stage_masks + (uint64_t)gs * WK;
    for (uint32_t i = lane; i < WK; i += 64) out[i] = st[i];
}

// HDFT: the dft is f16 (the --ft-fp16-out mode): rows are staged as f16
// (512 bytes per 256-column chunk), each added value is converted to f32,
// and the sum is multiplied by dft_inv_scale at the end, as the
// occurrence-list kernel does.
//
// DEALT (s.dealt): the tables deal a group's features to the waves
// round-robin, so wave w owns the group's features w, w + 8, w + 16, ...
// and adjacent (often equally frequent) features land on different waves,
// which evens out the hits per wave and stage that the barrier waits for.
template <bool HDFT, bool HSTATE, bool DEALT>
__global__ __launch_bounds__(kScanWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void ft_grad_scan_kernel(
    FtGradArgs a, FtBlockScan s, ScanGeom geom) {
    constexpr int R = kScanStage, RPW = kScanStage / kScanWaves;
    static_assert(R == 32 && (RPW == 2 || RPW == 4), "32 rows per stage, two or four per wave");
    if (__builtin_amdgcn_readfirstlane(*s.multi)) return;  // the occurrence-list kernel runs instead
    using Row4 = typename std::conditional<HDFT, h4, float4>::type;  // a lane's four columns
    __shared__ Row4 s_rows[2][R][64];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t lane = threadIdx.x % 64;
    // Longest king blocks first, spread over the XCDs.  Workgroups x, x + 8,
    // x + 16, ... run on XCD x in that order, so (block, chunk) pair p, pairs
    // ranked by descending block row count, is XCD (p % 8)'s (p / 8)-th pair;
    // a pair's feature groups sit next to each other (they read the same rows
    // through that XCD's L2).  The grid holds a multiple of 8 pairs.
    const uint32_t nb = s.n_blocks;
    const uint32_t n_chunks = (a.ft_out + kDftChunk - 1) / kDftChunk;
    const uint32_t xcd = blockIdx.x % kNumXcd, i_xcd = blockIdx.x / kNumXcd;
    const uint32_t g = i_xcd % geom.n_groups;
    const uint32_t pair = (i_xcd / geom.n_groups) * kNumXcd + xcd;
    if (pair >= nb * n_chunks) return;
    const uint32_t rank = pair / n_chunks, chunk = pair % n_chunks;
    const uint32_t K = block_of_rank(s, rank, lane);
    const uint32_t sb = block_stage_base(s, K, lane);  // its first stage in the stage tables
    const uint32_t PI = s.piece_inputs;
    const uint32_t blk_lo = K * PI;
    const uint32_t blk_n = s.cols > blk_lo ? (s.cols - blk_lo < PI ? s.cols - blk_lo : PI) : 0u;
    // the wave's features: f0 + k * fstep (k < nf)
    const uint32_t g_lo = g * geom.group_size;
    const uint32_t g_hi = (g + 1) * geom.group_size < blk_n ? (g + 1) * geom.group_size : blk_n;
    const uint32_t lo = g_lo + (DEALT ? wave : wave * kScanFeat);
    const uint32_t fstep = DEALT ? kScanWaves : 1u;
    const uint32_t span = g_hi > lo ? (DEALT ? (g_hi - lo + kScanWaves - 1) / kScanWaves : g_hi - lo) : 0u;
    const uint32_t nf = span < (uint32_t)kScanFeat ? span : (uint32_t)kScanFeat;
    const uint32_t f0 = blk_lo + lo;
    // the block's rows: its stm bin, then its nstm bin, as schedule entries
    const uint32_t a0 = s.sched_start[K], na = s.sched_start[K + 1] - a0;
    const uint32_t b0 = s.sched_start[s.n_blocks + K];
    const uint32_t n = na + (s.sched_start[s.n_blocks + K + 1] - b0);
    const Row4* dft4 =
        HDFT ? reinterpret_cast<const Row4*>(reinterpret_cast<const _Float16*>(a.dft16) + (uint64_t)chunk * a.dft_chunk_stride) +
                   lane
             : reinterpret_cast<const Row4*>(a.dft + (uint64_t)chunk * a.dft_chunk_stride) + lane;
    const uint32_t n_stages = (n + R - 1) / R;
    const uint32_t last = n_stages ? n_stages - 1 : 0u;  // stages past the list repeat the last (never summed)
    // Lane l < 32 loads the dft row of slot l and lane k < 16 the wave's
    // mask of feature k (the other lanes repeat them), a stage or two before
    // the stage needs them, so no load is waited for early.
    const uint32_t* srow = s.stage_rows + (uint64_t)sb * R + (lane & 31u);
    const uint32_t* smask =
        s.stage_masks + ((uint64_t)sb * geom.words + g * kScanWaves + wave) * kScanFeat + (lane % kScanFeat);
    auto positions = [&](uint32_t T) -> uint32_t { return srow[(uint64_t)(T < last ? T : last) * R]; };
    auto masks = [&](uint32_t T) -> uint32_t {
        return smask[(uint64_t)(T < last ? T : last) * geom.words * kScanFeat];
    };
    auto dft_row = [&](uint32_t row_lanes, uint32_t j) -> const Row4* {
        return dft4 + (uint64_t)(uint32_t)__builtin_amdgcn_readlane(row_lanes, j % R) * (kDftChunk / 4);
    };

    float4 acc[kScanFeat];
#pragma unroll
    for (int k = 0; k < kScanFeat; ++k) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    // Stage T = rows 32T .. 32T+31 of the list; wave w stages rows 32T + 4w
    // .. +3 in LDS buffer T % 2.  Register sets A / B belong to even / odd
    // stages.  While stage T is summed, the rows of stage T+2 are in flight
    // (issued with row ids loaded a stage earlier, no scalar-load chain), the
    // rows of stage T+1 wait in registers, and loads past the list repeat
    // its last row.
    Row4 sA0, sA1, sA2, sA3, sB0, sB1, sB2, sB3;
    uint32_t ridA = 0, ridB = 0, mA = 0, mB = 0;
#define TATARA_LOAD_ROWS(S, RID, T)                          \
    do {                                                     \
        const uint32_t jb = (T) * R + wave * RPW;            \
        S##0 = *dft_row(RID, jb + 0);                        \
        S##1 = *dft_row(RID, jb + 1);                        \
        if constexpr (RPW == 4) {                            \
            S##2 = *dft_row(RID, jb + 2);                    \
            S##3 = *dft_row(RID, jb + 3);                    \
        }                                                    \
    } while (0)
#define TATARA_STORE_ROWS(BUF, S)                            \
    do {                                                     \
        s_rows[(BUF)][wave * RPW + 0][lane] = S##0;          \
        s_rows[(BUF)][wave * RPW + 1][lane] = S##1;          \
        if constexpr (RPW == 4) {                            \
            s_rows[(BUF)][wave * RPW + 2][lane] = S##2;      \
            s_rows[(BUF)][wave * RPW + 3][lane] = S##3;      \
        }                                                    \
    } while (0)
#define TATARA_SUM_STAGE(BUF, M, T)                                       \
    do {                                                                  \
        if (nf) {                                                         \
            /* the hit loop's latency chain issues ahead of the other     \
               workgroup's staging and update (about 1% of the kernel) */ \
            __builtin_amdgcn_s_setprio(1);                                \
            /* bit k: feature k has a row in the stage (one compare for   \
               all 16, so a feature without one costs a bit test) */      \
            const uint32_t any = (uint32_t)__builtin_amdgcn_ballot_w64((M) != 0u) & 0xFFFFu; \
            _Pragma("unroll") for (int k = 0; k < kScanFeat; ++k) {       \
                if (!(any & (1u << k))) continue;                         \
                /* the stage's rows that hold feature k, ascending */     \
                uint32_t rows = __builtin_amdgcn_readlane((M), k);        \
                do {                                                      \
                    const uint32_t jj = __builtin_ctz(rows);              \
                    rows &= rows - 1u;                                    \
                    acc[k] = f4add(acc[k], as_f4(s_rows[(BUF)][jj][lane])); \
                } while (rows);                                           \
            }                                                             \
            __builtin_amdgcn_s_setprio(0);                                \
        }                                                                 \
    } while (0)
#define TATARA_STAGE(T, X, Y, BUF)                \
    do {                                          \
        rid##Y = positions((T) + 3);              \
        TATARA_LOAD_ROWS(s##X, rid##X, (T) + 2);  \
        TATARA_SUM_STAGE(BUF, m##X, T);           \
        m##X = masks((T) + 2);                    \
        TATARA_STORE_ROWS((BUF) ^ 1, s##Y);       \
        __syncthreads();                          \
    } while (0)
    if (n_stages > 0) {
        // the same issue order as a stage (positions, rows, masks), so the
        // loop is entered with the loads in flight that it expects
        ridA = positions(0);
        ridB = positions(1);
        TATARA_LOAD_ROWS(sA, ridA, 0u);
        mA = masks(0);
        ridA = positions(2);
        TATARA_LOAD_ROWS(sB, ridB, 1u);
        mB = masks(1);
        TATARA_STORE_ROWS(0, sA);
    }
    __syncthreads();
    for (uint32_t t = 0; t < n_stages; t += 2) {
        TATARA_STAGE(t, A, B, 0);
        if (t + 1 >= n_stages) break;
        TATARA_STAGE(t + 1, B, A, 1);
    }
#undef TATARA_LOAD_ROWS
#undef TATARA_STORE_ROWS
#undef TATARA_SUM_STAGE
#undef TATARA_STAGE

    const uint32_t col = chunk * kDftChunk + lane * 4;
    if (col >= a.ft_out) return;
    vecf<4>* grad = reinterpret_cast<vecf<4>*>(a.grad);
    const uint64_t off0 = ((uint64_t)f0 * a.ft_out + col) / 4, row4 = a.ft_out / 4;
    if (nf == 0) return;
    vecf<4> gv[kScanFeat];
#pragma unroll
    for (int k = 0; k < kScanFeat; ++k) {
        gv[k] = vecf<4>{acc[k].x, acc[k].y, acc[k].z, acc[k].w};
        if constexpr (HDFT) gv[k] *= a.dft_inv_scale;
        if (a.grad && (uint32_t)k < nf) __builtin_nontemporal_store(gv[k], grad + off0 + (uint64_t)k * fstep * row4);
    }
    if (!a.apply_update) return;
    // The update loads each row's state two rows ahead of it (one on a
    // lookahead step, which also loads the slow weights).  To make room for
    // that, the gradients of the wave's first kParked rows wait in the stage
    // buffers (free after the last barrier; each wave its own part) while
    // the other rows are updated from registers.
    constexpr int kParked = (int)(sizeof(s_rows) / (kScanWaves * 64 * sizeof(vecf<4>))) < kScanFeat / 2
                                ? (int)(sizeof(s_rows) / (kScanWaves * 64 * sizeof(vecf<4>)))
                                : kScanFeat / 2;
    vecf<4>* parked = reinterpret_cast<vecf<4>*>(&s_rows[0][0][0]) + (uint32_t)wave * kParked * 64 + lane;
#pragma unroll
    for (int k = 0; k < kParked; ++k) parked[k * 64] = gv[k];
    const uint32_t nf_hi = nf > (uint32_t)kParked ? nf - kParked : 0u;
    auto grad_hi = [&](int k) { return gv[kParked + k]; };
    auto grad_lo = [&](int k) { return parked[k * 64]; };
    const uint32_t nf_lo = nf < (uint32_t)kParked ? nf : kParked;
    if (a.opt.lookahead) {
        if (nf_hi)
            update_rows_pipelined<kScanFeat - kParked, 1, HSTATE, true>(a, f0 + kParked * fstep, fstep, col, nf_hi, nf_hi,
                                                                        grad_hi);
        update_rows_pipelined<kParked, 1, HSTATE, true>(a, f0, fstep, col, nf_lo, nf_lo, grad_lo);
    } else {
        if (nf_hi)
            update_rows_pipelined<kScanFeat - kParked, 2, HSTATE, false>(a, f0 + kParked * fstep, fstep, col, nf_hi,
                                                                         nf_hi, grad_hi);
        update_rows_pipelined<kParked, 2, HSTATE, false>(a, f0, fstep, col, nf_lo, nf_lo, grad_lo);
    }
}

// ---------------------------------------------------------------------------
// FT backward from an f16 dft on the matrix cores (the mixed-precision
// trainer).
//
// For king block K, a 256-column chunk and a set of features, the gradient
// rows are G[f][c] = sum over the block's rows e of H[f][e] * D[e][c]: H is
// the 0/1 hit matrix of the masks above and D the block's f16 dft rows, so
// the backward is a GEMM whose K dimension is the block's row list, 32 rows
// per v_mfma_f32_16x16x32_f16.  Products with 0 or 1 are exact and the sums
// are f32, but in the matrix core's order rather than row by row as
// gather_and_sum_per_feature_*_fp16 (native_kernels.cu:1030-1100) adds them:
// a cell equals the sequential sum to within f32 summation error.  Rows past
// the list are zero and the dft is clamped to +-65504, so every zero of H
// multiplies a finite value unless a row of the block holds a NaN or an
// infinity; a wave whose sums come out non-finite then takes the sequential
// per-hit sums instead (below), which keep the value to its row's features.
//
// Workgroups take (block, chunk, feature group, column half) in the block
// scan's order (the two halves of a chunk next to each other).  Wave w of
// the four owns 32 features of the group (mask words 2w, 2w+1) and the 128
// columns of the half: 2 x 8 tiles of 16 x 16, 64 f32 accumulators per lane
// (three waves per SIMD; 128 accumulators and 256 columns allow two, and
// measured 3% slower).  The rows go through LDS in stages of 64: wave w
// loads rows 16w..16w+15 (two columns per lane), transposes them in
// registers and writes them by
// column, so the B operand of a lane (8 rows of one column) is one 16-byte
// read; the stage's mask words sit beside them and the A operand (8 rows of
// one feature) is built from their bits as f16 1.0 / 0.0.  Stage T+1 is
// loaded while stage T is multiplied (two LDS buffers, one barrier per
// stage).  The optimizer update of the workgroup's cells follows.
// ---------------------------------------------------------------------------
constexpr int kMfmaWaves = 4;  // 32 features each
constexpr int kMfmaRows = 64;  // rows per stage: two MFMA steps
// A stage's rows in LDS: 16-byte slots of (column, row octet), each holding
// that column's 8 rows.  Columns come in groups of 16 (octet-major, then
// column); within an octet the 16 columns are rotated by the group index, so
// the 16 slots that 16 lanes write (2 columns apart) or read (16
// consecutive columns) at once fall in 16 distinct groups of the 64 LDS
// banks.
constexpr int kMfmaCols = 128;  // columns per workgroup (half a dft chunk)
__device__ __forceinline__ uint32_t stage_slot(uint32_t col, uint32_t oct) {
    return (col >> 4) * (uint32_t)(kMfmaRows * 2) + oct * 16 + ((col + (col >> 4)) & 15u);
}
constexpr int kMfmaStageHalves = kMfmaCols * kMfmaRows;  // 16 KB per buffer
constexpr int kMfmaUpdRow = 132;                         // floats per update row (128 + padding)
// the update reuses the stage buffers: 8 waves x 16 rows of kMfmaUpdRow floats
constexpr int kMfmaLdsHalves = kMfmaWaves * 16 * kMfmaUpdRow * 2 > 2 * kMfmaStageHalves
                                   ? kMfmaWaves * 16 * kMfmaUpdRow * 2
                                   : 2 * kMfmaStageHalves;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


// A feature's slot bits of 8 rows (bit e: row e) -> its A operand: f16 1.0
// where the bit is set, 0.0 elsewhere (two halves per dword).
__device__ __forceinline__ half8 hit_operand(uint32_t b) {
    auto pair = [&](uint32_t e) -> uint32_t { return (((b >> e) & 1u) | (((b >> (e + 1)) & 1u) << 16)) * 0x3C00u; };
    const u32x4 r = {pair(0), pair(2), pair(4), pair(6)};
    return __builtin_bit_cast(half8, r);
}

template <bool HSTATE>
__global__ __launch_bounds__(kMfmaWaves * 64) void ft_grad_mfma_kernel(FtGradArgs a, FtBlockScan s,
                                                                       ScanGeom geom) {
    constexpr uint32_t R = kMfmaRows, KS = R / 32, RW = R / kMfmaWaves;  // MFMA steps, rows per wave
    if (__builtin_amdgcn_readfirstlane(*s.multi)) return;  // the occurrence-list kernel runs instead
    __shared__ __attribute__((aligned(16))) _Float16 s_lds[kMfmaLdsHalves];  // two stage buffers
    // [K-step][mask word][feature]: the stage's slot masks (bit r: row r of the K-step)
    __shared__ uint32_t s_mt[2][KS * kScanWaves * kScanFeat];
    // the A operand of each slot byte (bit e: row e -> f16 1.0 / 0.0)
    __shared__ __attribute__((aligned(16))) half8 s_hit[256];
    static_assert(kMfmaWaves * 64 == 256, "one operand table entry per thread");
    s_hit[threadIdx.x] = hit_operand(threadIdx.x);
    auto s_d = [&](uint32_t buf, uint32_t slot) -> _Float16* { return s_lds + buf * kMfmaStageHalves + slot * 8; };
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t lane = threadIdx.x % 64;
    // (block, chunk) pairs longest block first, pair p on XCD p % 8, the
    // groups of a pair next to each other (as the block scan)
    const uint32_t n_chunks = (a.ft_out + kDftChunk - 1) / kDftChunk;
    const uint32_t xcd = blockIdx.x % kNumXcd, i_xcd = blockIdx.x / kNumXcd;
    const uint32_t sub = i_xcd % (2 * geom.n_groups);
    const uint32_t g = sub >> 1, half = sub & 1u;
    const uint32_t pair = (i_xcd / (2 * geom.n_groups)) * kNumXcd + xcd;
    if (pair >= s.n_blocks * n_chunks) return;
    const uint32_t K = block_of_rank(s, pair / n_chunks, lane), chunk = pair % n_chunks;
    const uint32_t sb = block_stage_base(s, K, lane);
    const uint32_t PI = s.piece_inputs;
    const uint32_t blk_lo = K * PI;
    const uint32_t blk_n = s.cols > blk_lo ? (s.cols - blk_lo < PI ? s.cols - blk_lo : PI) : 0u;
    const uint32_t a0 = s.sched_start[K], na = s.sched_start[K + 1] - a0;
    const uint32_t b0 = s.sched_start[s.n_blocks + K];
    const uint32_t n = na + (s.sched_start[s.n_blocks + K + 1] - b0);
    const _Float16* d16 =
        reinterpret_cast<const _Float16*>(a.dft16) + (uint64_t)chunk * a.dft_chunk_stride + half * kMfmaCols;
    // Thread t loads slot mask t of a stage: K-step t / 128, mask word
    // (t / 16) % 8 of the group, feature t % 16, from the stage tables (the
    // block's 32-row stages; a K-step past them has no hits).
    static_assert(KS * kScanWaves * kScanFeat == kMfmaWaves * 64, "one slot mask per thread");
    const uint32_t mks = threadIdx.x / (kScanWaves * kScanFeat);
    const uint32_t* tmask = s.stage_masks + (uint64_t)(g * kScanWaves) * kScanFeat + threadIdx.x % (kScanWaves * kScanFeat);
    const uint32_t n32 = (n + 31) / 32;
    const uint32_t* trow = s.stage_rows + (uint64_t)sb * 32;
    const uint32_t n_stages = (n + R - 1) / R;

    // Stage T in registers: wave w's rows RT + RW w + j, the lane's columns
    // 4 lane .. 4 lane + 3 (rows past the list are zero), and the thread's
    // mask words.  Stage T+1's rows are loaded while stage T is multiplied.
    // The positions of a stage's rows are loaded one stage ahead, into the
    // register the row addresses have just been read from: a ring of two
    // position registers needs a copy of a load in flight, and waiting for
    // that load (loads complete in order) waited for the stage's row loads
    // too, before any multiply.  (Deeper register pipelines need the stage
    // loop unrolled, which makes the register allocator copy the
    // accumulators and halves the occupancy.)
    struct Stage {
        uint32_t r[RW];
        uint32_t mt;
    };
    static_assert(R <= 64, "one row id per lane");
    // the dft rows of stage T's slots (slots past the block's stages repeat
    // its last table slot; their rows are zeroed below)
    auto load_pos = [&](uint32_t T) -> uint32_t {
        const uint32_t j = T * R + lane % R;
        return trow[j < 32 * n32 ? j : 32 * n32 - 1];
    };
    auto load_rows = [&](Stage& S, uint32_t pos, uint32_t T) {
#pragma unroll
        for (uint32_t j = 0; j < RW; ++j) {
            const uint32_t jj = T * R + wave * RW + j;
            const uint64_t r = (uint32_t)__builtin_amdgcn_readlane(pos, wave * RW + j);
            S.r[j] = jj < n ? reinterpret_cast<const uint32_t*>(d16 + r * kDftChunk)[lane] : 0u;
        }
        const uint32_t ts = T * KS + mks;
        S.mt = ts < n32 ? tmask[(uint64_t)(sb + ts) * geom.words * kScanFeat] : 0u;
    };
    // registers -> LDS buffer: column 2 lane + c gets this wave's rows
    auto store_rows = [&](const Stage& S, uint32_t buf) {
#pragma unroll
        for (uint32_t o = 0; o < RW / 8; ++o)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                u32x4 v;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    // column c of rows 2k and 2k + 1: low halves (c = 0) or high halves (c = 1)
                    // of the two row words, as one byte permute
                    const uint32_t x0 = S.r[8 * o + 2 * k], x1 = S.r[8 * o + 2 * k + 1];
                    v[k] = __builtin_amdgcn_perm(x1, x0, c == 0 ? 0x05040100u : 0x07060302u);
                }
                *reinterpret_cast<u32x4*>(s_d(buf, stage_slot(lane * 2 + c, wave * (RW / 8) + o))) = v;
            }
        s_mt[buf][threadIdx.x] = S.mt;
    };

    const uint32_t m = lane % 16, oct = lane / 16;
    floatx4 acc[2][8];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    Stage S;
    uint32_t P = 0;  // positions of the next stage to load
    if (n_stages > 0) {
        load_rows(S, load_pos(0), 0);
        P = load_pos(1);
        store_rows(S, 0);
    }
    __syncthreads();
    for (uint32_t t = 0; t < n_stages; ++t) {
        const uint32_t buf = t & 1u;
        const bool more = t + 1 < n_stages;
        if (more) {
            load_rows(S, P, t + 1);
            P = load_pos(t + 2);
        }
#pragma unroll
        for (uint32_t ks = 0; ks < KS; ++ks) {
            half8 A[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                A[i] = s_hit[(s_mt[buf][(ks * kScanWaves + wave * 2 + i) * kScanFeat + m] >> (8 * oct)) & 0xFFu];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const half8 B = *reinterpret_cast<const half8*>(s_d(buf, stage_slot(j * 16 + m, 4 * ks + oct)));
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B, acc[i][j], 0, 0, 0);
            }
        }
        if (more) store_rows(S, buf ^ 1u);
        __syncthreads();
    }

    // A non-finite dft value in one of the block's rows makes its column
    // non-finite in every tile (H multiplies it by 1 or by 0, and 0 x NaN,
    // 0 x Inf are NaN), while finite rows (|D| <= 65504, a few thousand per
    // block) cannot overflow an f32 sum.  A wave that finds one recomputes
    // its cells as the sequential per-hit sums, table stage by stage and row
    // by row (the block scan's order, equal bit for bit to the reference's
    // per-feature gather), so that a NaN reaches only the features of the
    // rows that hold it.
    bool nonfinite = false;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) nonfinite |= !__builtin_isfinite(acc[i][j][r]);
    const bool sequential = __builtin_amdgcn_ballot_w64(nonfinite) != 0;
    // the sequential sums of tile i's cells (feature 4 oct + r of mask word
    // 2 wave + i, column 16 j + m), r and j as in the accumulators
    const uint32_t* mrow = s.stage_masks + (uint64_t)(g * kScanWaves + 2 * wave) * kScanFeat + 4 * oct;
    auto sequential_sums = [&](int i, int r, float (&sum)[8]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) sum[j] = 0.0f;
        for (uint32_t ts = 0; ts < n32; ++ts) {
            uint32_t mk = mrow[(uint64_t)(sb + ts) * geom.words * kScanFeat + i * kScanFeat + r];
            const uint32_t* tr = trow + 32 * ts;
            while (mk) {  // the lane's hits, in row order
                const uint32_t e = __builtin_ctz(mk);
                mk &= mk - 1;
                const _Float16* dr = d16 + (uint64_t)tr[e] * kDftChunk + m;
#pragma unroll
                for (int j = 0; j < 8; ++j) sum[j] += (float)dr[16 * j];
            }
        }
    };

    // Update, 16 features x 128 columns at a time: the wave's tiles go
    // through its own LDS rows so that each lane then updates four
    // consecutive columns of a feature row, four rows' state loaded before
    // any of them is updated.  Lane holds D[4 oct + r][m] of tile (i, j):
    // feature 32w + 16i + 4 oct + r of the group, column 16j + m.
    float* s_u = reinterpret_cast<float*>(s_lds) + wave * 16 * kMfmaUpdRow;
    const uint32_t lo = g * geom.group_size;
    const uint32_t g_hi = (g + 1) * geom.group_size < blk_n ? (g + 1) * geom.group_size : blk_n;
    const uint32_t nf = g_hi > lo ? g_hi - lo : 0u;
    const uint64_t f0 = (uint64_t)blk_lo + lo;
    const uint32_t fw = 32 * wave;
    vecf<4>* grad = reinterpret_cast<vecf<4>*>(a.grad);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        {
            const uint32_t col = chunk * kDftChunk + half * kMfmaCols + 4 * (lane % 32);
            if (sequential) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float sum[8];
                    sequential_sums(i, r, sum);
#pragma unroll
                    for (int j = 0; j < 8; ++j) s_u[(oct * 4 + r) * kMfmaUpdRow + j * 16 + m] = sum[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s_u[(oct * 4 + r) * kMfmaUpdRow + j * 16 + m] = acc[i][j][r];
            }
            __syncthreads();
            // the lane's rows 2 j + lane / 32 of the tile (j < 8): features
            // first + 2 j of the group, nfl of them real (none past the
            // group's end; a lane without any loads the tile's first row)
            const uint32_t tile_lo = fw + i * 16, rsel = lane / 32, first = tile_lo + rsel;
            const uint32_t nfl = first < nf ? min(8u, (nf - first + 1) / 2) : 0u;
            auto gfn = [&](int j) {
                const float4 v =
                    *reinterpret_cast<const float4*>(&s_u[(2 * j + rsel) * kMfmaUpdRow + 4 * (lane % 32)]);
                vecf<4> gr = {v.x, v.y, v.z, v.w};
                return gr * a.dft_inv_scale;
            };
            if (tile_lo < nf && col < a.ft_out) {
                if (a.grad) {
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if ((uint32_t)j < nfl)
                            __builtin_nontemporal_store(gfn(j), grad + ((f0 + first + 2 * j) * a.ft_out + col) / 4);
                }
                if (a.apply_update) {
                    const uint64_t fl = f0 + (nfl ? first : tile_lo);
                    // state loaded two rows ahead (one with the slow weights)
                    if (a.opt.lookahead)
                        update_rows_pipelined<8, 1, HSTATE, true>(a, fl, 2, col, nfl, nfl ? nfl : 1u, gfn);
                    else
                        update_rows_pipelined<8, 2, HSTATE, false>(a, fl, 2, col, nfl, nfl ? nfl : 1u, gfn);
                }
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// Backward + optimizer, phase B (factorizer): one wave = (column chunk, piece
// p).  The virtual row's gradient is the sequential sum of the piece's
// king-bucket rows p, p + pi, p + 2 pi, ... (ft_reduce_virtual_grad_cpu's
// order); the virtual row is updated, and the forward table
// comb = w + w_virtual is rewritten for the piece's rows (ft_fold_virtual).
// ---------------------------------------------------------------------------

// With a slice-major pairwise table (layout kTablePairSlices) a wave takes
// two adjacent pieces: lane 32i + 16h + j holds piece 2u + i, float4 column
// 16c + j of half h, so each store writes two adjacent features' whole
// 64-byte slices, one 128-byte line per slice.
template <bool HSTATE, bool HCOMB>
__global__ __launch_bounds__(256) void ft_virtual_fold_kernel(FtGradArgs a, uint32_t piece_inputs,
                                                              uint32_t n_chunks, float* __restrict__ comb,
                                                              _Float16* __restrict__ comb16, int layout) {
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t task = (uint64_t)blockIdx.x * kWavesPerBlock + wave;
    const bool paired = layout == kTablePairSlices;
    const uint32_t n_units = paired ? (piece_inputs + 1) / 2 : piece_inputs;
    if (task >= (uint64_t)n_units * n_chunks) return;
    const uint32_t chunk = (uint32_t)(task / n_units);
    const uint32_t unit = (uint32_t)(task - (uint64_t)chunk * n_units);
    const uint32_t ft_out = a.ft_out, ft_in = a.rows;
    const uint32_t row4 = ft_out / 4;
    uint32_t q, p;
    if (paired) {
        p = 2 * unit + (lane >> 5);
        const uint32_t qh = chunk * 16 + (lane & 15u);
        if (p >= piece_inputs || qh >= row4 / 2) return;
        q = ((lane >> 4) & 1u ? row4 / 2 : 0u) + qh;
    } else {
        p = unit;
        q = chunk * kWave + lane;
        if (q >= row4) return;
    }
    const uint32_t count = ft_in / piece_inputs;
    const float4* g4 = reinterpret_cast<const float4*>(a.grad);
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
    reinterpret_cast<float4*>(a.grad)[voff4] = vsum;
    if (!a.apply_update) return;
    const vecf<4> g = {vsum.x, vsum.y, vsum.z, vsum.w};
    update_cells<4, HSTATE>(a, voff4, g);  // a factorizer has no f16 mirror
    if (!comb && !comb16) return;
    // the forward rows of this piece: comb = w + w_virtual (f32 add), rounded
    // to f16 for an f16 forward table (ft_fold_virtual_f16, native_kernels.cu:262-300)
    const float4 wv = reinterpret_cast<const float4*>(a.w)[voff4];
    auto put = [&](uint64_t row, float4 wr) {
        const float4 c = f4add(wr, wv);
        const uint64_t t4 = table_index(layout, row, 4 * q, ft_out, piece_inputs, HCOMB ? 8u : 4u) / 4;
        if constexpr (HCOMB)
            reinterpret_cast<h4*>(comb16)[t4] = f4_to_h4(c);
        else
            reinterpret_cast<float4*>(comb)[t4] = c;
    };
    for (j = 0; j + U <= count; j += U) {
        float4 wr[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            wr[u] = reinterpret_cast<const float4*>(a.w)[(uint64_t)(p + (j + u) * piece_inputs) * row4 + q];
#pragma unroll
        for (int u = 0; u < U; ++u) put(p + (uint64_t)(j + u) * piece_inputs, wr[u]);
    }
    for (; j < count; ++j) {
        const uint64_t row = p + (uint64_t)j * piece_inputs;
        put(row, reinterpret_cast<const float4*>(a.w)[row * row4 + q]);
    }
}

// Standalone fold / reduce (Base mode), used when they are not fused.
template <bool HCOMB>
__global__ void ft_fold_kernel(const float* __restrict__ w, float* __restrict__ comb,
                               _Float16* __restrict__ comb16, uint32_t ft_in, uint32_t ft_out,
                               uint32_t piece_inputs, int layout) {
    const uint64_t n4 = (uint64_t)ft_in * ft_out / 4;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const uint32_t row4 = ft_out / 4;
    const uint64_t f = i / row4;
    const uint32_t c = (uint32_t)(i - f * row4);
    const uint64_t vrow = ft_in + f % piece_inputs;
    const float4 x =
        f4add(reinterpret_cast<const float4*>(w)[i], reinterpret_cast<const float4*>(w)[vrow * row4 + c]);
    const uint64_t t4 = table_index(layout, f, 4 * c, ft_out, piece_inputs, HCOMB ? 8u : 4u) / 4;
    if constexpr (HCOMB)
        reinterpret_cast<h4*>(comb16)[t4] = f4_to_h4(x);
    else
        reinterpret_cast<float4*>(comb)[t4] = x;
}

__global__ void cast_f16_kernel(const float* __restrict__ src, _Float16* __restrict__ dst, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = (_Float16)src[i];
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

uint32_t ft_block_slot_stride(uint32_t max_active) { return max_active <= 40 ? 40u : 48u; }

// A slice-major layout needs whole slices: 16-byte quads of 4 (f32) or 8
// (f16) columns, four per slice.
static bool table_layout_ok(int layout, bool f16, uint32_t ft_out) {
    if (layout == kTableRows) return true;
    if (layout == kTablePairSlices) return ft_out % (f16 ? 32u : 16u) == 0;
    return false;
}

bool ft_forward_block_ok(int mode, bool f16_table, uint32_t ft_out, uint32_t piece_inputs, uint32_t max_active) {
    if (piece_inputs == 0 || piece_inputs > kFbMaxPi || max_active > kFbSlots) return false;
    if (mode == kPair) return ft_out % (f16_table ? 32u : 16u) == 0;
    if (mode == kConcat) return !f16_table && ft_out % 16 == 0;
    return false;
}

int32_t launch_ft_forward(const FtForwardArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(a.max_active <= (uint32_t)kMaxActive, "max_active must be <= 64");
    TATARA_REQUIRE(a.ft_out % 8 == 0, "ft_out must be a multiple of 8");
    TATARA_REQUIRE(a.n_persp == 1 || a.n_persp == 2, "n_persp must be 1 or 2");
    const bool h_out = a.out_stm16 != nullptr;
    TATARA_REQUIRE(!h_out || (a.mode == kPair && a.W16), "f16 raw sums need the pairwise mode and an f16 table");
    TATARA_REQUIRE(!a.W16 || a.mode == kPair, "an f16 table is read by the pairwise mode only");
    if (a.batch == 0) return kOk;
    const bool block = a.sched_start && a.schedule && a.slot_off && a.row_bad && a.n_persp == 2 &&
                       a.n_blocks >= 1 && a.n_blocks <= 128 &&
                       ft_forward_block_ok(a.mode, a.W16 != nullptr, a.ft_out, a.piece_inputs, a.max_active);
    TATARA_REQUIRE(a.w_layout == kTableRows ||
                       (block && a.mode == kPair && a.w_layout == kTablePairSlices &&
                        a.cols == a.n_blocks * a.piece_inputs),
                   "a slice-major forward table is read by the pairwise LDS-resident gather only");
    if (block) {
        FtBlockFwd f{};
        f.W = a.W16 ? static_cast<const void*>(a.W16) : static_cast<const void*>(a.W);
        f.idx_stm = a.idx_stm;
        f.idx_nstm = a.idx_nstm;
        f.nnz = a.nnz;
        f.schedule = a.schedule;
        f.sched_start = a.sched_start;
        f.slot_off = a.slot_off;
        f.row_bad = a.row_bad;
        f.bias = a.bias;
        f.out_stm = a.out_stm;
        f.out_nstm = a.out_nstm;
        f.out16_stm = reinterpret_cast<_Float16*>(a.out_stm16);
        f.out16_nstm = reinterpret_cast<_Float16*>(a.out_nstm16);
        f.combined = a.combined;
        f.combined16 = reinterpret_cast<_Float16*>(a.combined16);
        f.batch = a.batch;
        f.ft_out = a.ft_out;
        f.cols = a.cols;
        f.max_active = a.max_active;
        f.n_blocks = a.n_blocks;
        f.piece_inputs = a.piece_inputs;
        f.n_slices = a.ft_out / (a.W16 ? 32u : 16u);
        f.scale = a.scale;
        f.w_layout = a.w_layout;
        const uint32_t items = a.n_blocks * ((f.n_slices + 3) / 4);
        const uint32_t grid = ceil_div(items, kNumXcd) * kNumXcd * 4;
#define TATARA_FB(NU)                                                                         \
    if (a.mode == kConcat)                                                                    \
        ft_forward_block_kernel<kConcat, float, false, NU><<<grid, kFbThreads, 0, stream>>>(f);  \
    else if (!a.W16)                                                                          \
        ft_forward_block_kernel<kPair, float, false, NU><<<grid, kFbThreads, 0, stream>>>(f);    \
    else if (h_out)                                                                           \
        ft_forward_block_kernel<kPair, _Float16, true, NU><<<grid, kFbThreads, 0, stream>>>(f);  \
    else                                                                                      \
        ft_forward_block_kernel<kPair, _Float16, false, NU><<<grid, kFbThreads, 0, stream>>>(f);
        if (a.max_active <= 40) {
            TATARA_FB(10)
        } else {
            TATARA_FB(12)
        }
#undef TATARA_FB
        TATARA_LAUNCHED("ft_forward_block");
        return kOk;
    }
    const uint32_t n_chunks = a.mode == kPair ? ceil_div(a.ft_out / 8, 32) : ceil_div(a.ft_out / 4, kWave);
    const uint64_t tasks = (uint64_t)a.n_persp * n_chunks * a.batch;
    const uint32_t blocks = (uint32_t)((tasks + kWavesPerBlock - 1) / kWavesPerBlock);
    _Float16* o16s = reinterpret_cast<_Float16*>(a.out_stm16);
    _Float16* o16n = reinterpret_cast<_Float16*>(a.out_nstm16);
    const _Float16* W16 = reinterpret_cast<const _Float16*>(a.W16);
    _Float16* c16p = reinterpret_cast<_Float16*>(a.combined16);
    TATARA_REQUIRE(!c16p || a.mode == kPair, "an f16 combined is written by the pairwise mode only");
#define TATARA_FWD(MODE, T, HOUT, WPTR)                                                                      \
    ft_forward_kernel<MODE, T, HOUT><<<blocks, 256, 0, stream>>>(                                          \
        WPTR, a.idx_stm, a.idx_nstm, a.nnz, a.schedule, a.bias, a.out_stm, a.out_nstm, o16s, o16n, a.combined, \
        c16p, a.batch, a.ft_out, a.cols, a.max_active, n_chunks, a.n_persp, a.scale)
    switch (a.mode) {
        case kRaw:
            TATARA_FWD(kRaw, float, false, a.W);
            break;
        case kPair:
            if (W16) {
                // eight columns per lane: a chunk covers 256 pairs
                TATARA_REQUIRE(a.ft_out % 16 == 0, "an f16 table needs ft_out % 16 == 0");
                const uint32_t c16 = ceil_div(a.ft_out / 16, 32);
                const uint64_t t16 = (uint64_t)a.n_persp * c16 * a.batch;
                const uint32_t b16 = (uint32_t)((t16 + kWavesPerBlock - 1) / kWavesPerBlock);
                if (h_out)
                    ft_forward_pair16_kernel<true><<<b16, 256, 0, stream>>>(
                        W16, a.idx_stm, a.idx_nstm, a.nnz, a.schedule, a.bias, a.out_stm, a.out_nstm, o16s, o16n,
                        a.combined, c16p, a.batch, a.ft_out, a.cols, a.max_active, c16, a.n_persp, a.scale);
                else
                    ft_forward_pair16_kernel<false><<<b16, 256, 0, stream>>>(
                        W16, a.idx_stm, a.idx_nstm, a.nnz, a.schedule, a.bias, a.out_stm, a.out_nstm, o16s, o16n,
                        a.combined, c16p, a.batch, a.ft_out, a.cols, a.max_active, c16, a.n_persp, a.scale);
            } else {
                TATARA_FWD(kPair, float, false, a.W);
            }
            break;
        case kConcat:
            TATARA_FWD(kConcat, float, false, a.W);
            break;
        default:
            TATARA_REQUIRE(false, "unknown forward mode");
    }
#undef TATARA_FWD
    TATARA_LAUNCHED("ft_forward");
    return kOk;
}

int32_t launch_king_block_keys(const int32_t* idx_stm, const int32_t* idx_nstm,
                               const int32_t* nnz, uint8_t* keys, uint32_t batch,
                               uint32_t max_active, uint32_t cols, uint32_t piece_inputs,
                               uint32_t n_bins, hipStream_t stream, uint32_t* slot_off, uint8_t* row_bad) {
    if (batch == 0) return kOk;
    TATARA_REQUIRE(2 * n_bins <= 256, "king block keys: 2*n_bins <= 256");
    TATARA_REQUIRE((slot_off == nullptr) == (row_bad == nullptr), "slot offsets and row flags go together");
    if (slot_off) {
        TATARA_REQUIRE(max_active <= 64, "king block rows: max_active <= 64");
        king_block_rows_kernel<<<ceil_div(2ull * batch, 4 * kKeyRowsPerWave), 256, 0, stream>>>(
            idx_stm, idx_nstm, nnz, keys, slot_off, row_bad, batch, max_active, ft_block_slot_stride(max_active),
            cols, piece_inputs, n_bins);
    } else {
        king_block_keys_kernel<<<ceil_div(2ull * batch, 256), 256, 0, stream>>>(
            idx_stm, idx_nstm, nnz, keys, batch, max_active, cols, piece_inputs, n_bins);
    }
    TATARA_LAUNCHED("king_block_keys");
    return kOk;
}

uint32_t occurrence_key_bits(uint32_t cols) {
    uint32_t bits = 1;
    while ((1ull << bits) <= 2ull * cols) ++bits;
    return bits;
}

size_t occurrence_sort_temp_bytes(uint64_t n_items, uint32_t cols) {
    (void)cols;
    // the LSD passes' digit histograms and digit counts
    const uint64_t n = n_items < 0xFFFFFFFFull ? n_items : 0xFFFFFFFFull;
    return 4ull * (256ull * binsort_tiles((uint32_t)n) + 256ull);
}

int32_t launch_occurrence_sort(const OccurrenceSortArgs& a, hipStream_t stream) {
    const uint64_t n_items = 2ull * a.batch * a.max_active;
    const uint32_t n_keys = 2 * a.cols + 1;  // keys 0..2*cols (2*cols = invalid slot)
    TATARA_REQUIRE(n_items <= 0xFFFFFFFFull, "occurrence sort: at most 2^32 - 1 slots");
    // a gated sort strides over small grids, so that skipping it costs
    // little beside the kernels it overlaps (its no-op workgroups still pass
    // through the dispatcher); the rare sort that runs is slower for it
    auto grid = [&](uint64_t n) -> uint32_t {
        const uint64_t g = ceil_div(n, 256);
        return (uint32_t)(a.run_if && g > 256 ? 256 : g);
    };
    if (n_items > 0) {
        // stable LSD passes of 8 bits (the bin-sort kernels), alternating
        // between the two buffer pairs and ending in keys_out / vals_out;
        // their scratch is radix_hist / radix_count, or carved from temp
        uint32_t* hist = a.radix_hist;
        uint32_t* count = a.radix_count;
        if (!hist || !count) {
            TATARA_REQUIRE(a.temp && a.temp_bytes >= occurrence_sort_temp_bytes(n_items, a.cols),
                           "occurrence sort: scratch (occurrence_sort_temp_bytes)");
            hist = static_cast<uint32_t*>(a.temp);
            count = hist + 256ull * binsort_tiles((uint32_t)n_items);
        }
        const uint32_t passes = (occurrence_key_bits(a.cols) + 7) / 8;
        uint32_t *k0 = a.keys_in, *v0 = a.vals_in, *k1 = a.keys_out, *v1 = a.vals_out;
        if (passes % 2 == 0) {
            std::swap(k0, k1);
            std::swap(v0, v1);
        }
        build_occurrence_keys_kernel<<<grid(n_items), 256, 0, stream>>>(a.idx_stm, a.idx_nstm, a.nnz, k0, v0,
                                                                       a.batch, a.max_active, a.cols, a.run_if);
        TATARA_LAUNCHED("build_occurrence_keys");
        for (uint32_t p = 0; p < passes; ++p) {
            RadixPassArgs r{};
            r.keys = k0;
            r.vals = v0;
            r.n_items = (uint32_t)n_items;
            r.shift = 8 * p;
            r.hist = hist;
            r.digit_count = count;
            r.out_keys = k1;
            r.out_vals = v1;
            r.run_if = a.run_if;
            int32_t st = launch_radix_pass(r, stream);
            if (st) return st;
            std::swap(k0, k1);
            std::swap(v0, v1);
        }
    }
    occurrence_offsets_kernel<<<grid(n_items + 1), 256, 0, stream>>>(a.keys_out, n_items, n_keys, a.offsets,
                                                                     a.run_if);
    TATARA_LAUNCHED("occurrence_offsets");
    return kOk;
}

// f16 moments are read back as x / scale by an exact power-of-two scaling
// (radam_cells): the scales must be powers of two with normal reciprocals.
static bool moment_scales_ok(const FtGradArgs& a) {
    auto pow2 = [](float x) {
        int e = 0;
        return x > 0.0f && std::isfinite(x) && std::frexp(x, &e) == 0.5f && e >= -124 && e <= 127;
    };
    return !a.m16 || (pow2(a.m_scale) && pow2(a.v_scale));
}

int32_t launch_ft_grad_update(const FtGradArgs& a, hipStream_t stream) {
    constexpr int V = kFtGradLaneFloats;
    constexpr uint32_t kCols = kWave * V;
    TATARA_REQUIRE(a.ft_out % 4 == 0, "ft_out must be a multiple of 4");
    TATARA_REQUIRE(a.dft_row_stride % 4 == 0 && a.dft_chunk_stride % 4 == 0, "dft strides");
    const bool hdft = a.dft16 != nullptr, hstate = a.m16 != nullptr;
    TATARA_REQUIRE(!hstate || a.v16, "f16 moments need both m16 and v16");
    TATARA_REQUIRE(moment_scales_ok(a), "f16 moment scales must be powers of two");
    const uint32_t n_chunks = ceil_div(a.ft_out, kCols);
    const uint64_t tasks = (uint64_t)a.rows * n_chunks;
    if (tasks == 0) return kOk;
    // a gated launch (the block scan's fallback) strides over a bounded grid
    const uint32_t cap = a.run_if ? 1024u : 0xFFFFFFFFu;
    uint32_t blocks = (uint32_t)((tasks + kWavesPerBlock - 1) / kWavesPerBlock);
    blocks = blocks < cap ? blocks : cap;
    // four f16 values per lane: a wave's rows are 512 bytes, so a king
    // block's dft working set stays half the f32 one (eight values per lane
    // halve the loads but double that working set, and measure slower)
    const uint32_t c4 = ceil_div(a.ft_out, kWave * 4);
    uint32_t b4 = (uint32_t)(((uint64_t)a.rows * c4 + kWavesPerBlock - 1) / kWavesPerBlock);
    b4 = b4 < cap ? b4 : cap;
#define TATARA_GRAD_G(G)                                                                          \
    do {                                                                                          \
        if (hdft && hstate)                                                                       \
            ft_grad_update_kernel<4, true, true, G><<<b4, 256, 0, stream>>>(a, c4);               \
        else if (hdft)                                                                            \
            ft_grad_update_kernel<4, true, false, G><<<b4, 256, 0, stream>>>(a, c4);              \
        else if (hstate)                                                                          \
            ft_grad_update_kernel<V, false, true, G><<<blocks, 256, 0, stream>>>(a, n_chunks);    \
        else                                                                                      \
            ft_grad_update_kernel<V, false, false, G><<<blocks, 256, 0, stream>>>(a, n_chunks);   \
        TATARA_LAUNCHED("ft_grad_update");                                                       \
    } while (0)
    if (a.run_if)
        TATARA_GRAD_G(true);
    else
        TATARA_GRAD_G(false);
#undef TATARA_GRAD_G
    return kOk;
}

uint32_t ft_scan_mask_words(uint32_t piece_inputs) {
    const ScanGeom g = scan_geom(piece_inputs);
    return piece_inputs > 0 && g.words <= (uint32_t)kScanMaxWords ? g.words : 0u;
}

uint64_t ft_scan_max_stages(uint32_t batch, uint32_t n_blocks) {
    return (2ull * batch + kScanStage - 1) / kScanStage + n_blocks;
}

int32_t launch_ft_scan_tables(const FtBlockScan& s, hipStream_t stream) {
    TATARA_REQUIRE(ft_scan_mask_words(s.piece_inputs) > 0, "block scan: piece_inputs out of range");
    TATARA_REQUIRE(s.max_active <= (uint32_t)kMaxActive, "max_active must be <= 64");
    TATARA_REQUIRE(s.n_blocks >= 1 && s.n_blocks <= 128, "block scan: 1 to 128 king blocks");
    TATARA_REQUIRE(s.stage_rows && s.stage_masks && s.multi, "block scan: stage tables and flag");
    int32_t st = launch_fill_i32(reinterpret_cast<int32_t*>(s.multi), 1, 0, stream);
    if (st) return st;
    if (s.batch == 0) return kOk;
    const uint64_t stages = ft_scan_max_stages(s.batch, s.n_blocks);
    ft_scan_tables_kernel<<<(uint32_t)((stages + 3) / 4), 256, 0, stream>>>(s, scan_geom(s.piece_inputs));
    TATARA_LAUNCHED("ft_scan_tables");
    return kOk;
}

int32_t launch_ft_grad_scan(const FtGradArgs& a, const FtBlockScan& s, hipStream_t stream, bool fallback) {
    TATARA_REQUIRE(ft_scan_mask_words(s.piece_inputs) > 0, "block scan: piece_inputs out of range");
    TATARA_REQUIRE(s.stage_rows && s.stage_masks, "block scan: stage tables (launch_ft_scan_tables)");
    TATARA_REQUIRE((a.dft != nullptr) != (a.dft16 != nullptr), "block scan: one dft (f32 or f16)");
    TATARA_REQUIRE(a.dft_row_stride == kDftChunk && a.dft_chunk_stride == 2ull * s.batch * kDftChunk,
                   "block scan: chunk-major dft");
    TATARA_REQUIRE(a.ft_out % 4 == 0 && a.rows == s.cols, "block scan: shapes");
    TATARA_REQUIRE(moment_scales_ok(a), "f16 moment scales must be powers of two");
    const ScanGeom geom = scan_geom(s.piece_inputs);
    TATARA_REQUIRE(s.n_blocks <= 128, "block scan: at most 128 king blocks");
    const uint64_t pairs = (uint64_t)ceil_div(a.ft_out, kDftChunk) * s.n_blocks;
    const uint64_t grid = (pairs + kNumXcd - 1) / kNumXcd * kNumXcd * geom.n_groups;
    if (grid > 0) {
        const uint32_t g = (uint32_t)grid, t = kScanWaves * 64;
#define TATARA_SCAN(D)                                                                  \
    do {                                                                                \
        if (a.dft16 && a.m16)                                                           \
            ft_grad_scan_kernel<true, true, D><<<g, t, 0, stream>>>(a, s, geom);        \
        else if (a.dft16)                                                               \
            ft_grad_scan_kernel<true, false, D><<<g, t, 0, stream>>>(a, s, geom);       \
        else if (a.m16)                                                                 \
            ft_grad_scan_kernel<false, true, D><<<g, t, 0, stream>>>(a, s, geom);       \
        else                                                                            \
            ft_grad_scan_kernel<false, false, D><<<g, t, 0, stream>>>(a, s, geom);      \
    } while (0)
        if (s.dealt)
            TATARA_SCAN(true);
        else
            TATARA_SCAN(false);
#undef TATARA_SCAN
        TATARA_LAUNCHED("ft_grad_scan");
    }
    if (!fallback) return kOk;
    FtGradArgs gated = a;
    gated.run_if = s.multi;
    return launch_ft_grad_update(gated, stream);
}

int32_t launch_ft_grad_mfma(const FtGradArgs& a, const FtBlockScan& s, hipStream_t stream, bool fallback) {
    TATARA_REQUIRE(s.stage_rows && s.stage_masks, "block scan: stage tables (launch_ft_scan_tables)");
    TATARA_REQUIRE(ft_scan_mask_words(s.piece_inputs) > 0, "mfma backward: piece_inputs out of range");
    TATARA_REQUIRE(a.dft16 && !a.dft, "mfma backward: f16 dft only");
    TATARA_REQUIRE(a.dft_row_stride == kDftChunk && a.dft_chunk_stride == 2ull * s.batch * kDftChunk,
                   "mfma backward: chunk-major dft");
    TATARA_REQUIRE(a.ft_out % 4 == 0 && a.rows == s.cols, "mfma backward: shapes");
    TATARA_REQUIRE(moment_scales_ok(a), "f16 moment scales must be powers of two");
    TATARA_REQUIRE(s.n_blocks <= 128, "mfma backward: at most 128 king blocks");
    TATARA_REQUIRE(!s.dealt, "mfma backward: stage tables with contiguous waves");
    const ScanGeom geom = scan_geom(s.piece_inputs);
    TATARA_REQUIRE(geom.group_size <= 128, "mfma backward: at most 128 features per group");
    const uint64_t pairs = (uint64_t)ceil_div(a.ft_out, kDftChunk) * s.n_blocks;
    const uint64_t grid = (pairs + kNumXcd - 1) / kNumXcd * kNumXcd * geom.n_groups * 2;
    if (grid > 0) {
        const uint32_t t = kMfmaWaves * 64;
        if (a.m16)
            ft_grad_mfma_kernel<true><<<(uint32_t)grid, t, 0, stream>>>(a, s, geom);
        else
            ft_grad_mfma_kernel<false><<<(uint32_t)grid, t, 0, stream>>>(a, s, geom);
        TATARA_LAUNCHED("ft_grad_mfma");
    }
    if (!fallback) return kOk;
    FtGradArgs gated = a;
    gated.run_if = s.multi;
    return launch_ft_grad_update(gated, stream);
}

int32_t launch_ft_virtual_fold(const FtGradArgs& a, uint32_t piece_inputs, float* comb, uint16_t* comb16,
                               hipStream_t stream, int layout) {
    TATARA_REQUIRE(piece_inputs > 0 && a.rows % piece_inputs == 0,
                   "virtual fold: rows must be a multiple of piece_inputs");
    TATARA_REQUIRE(a.grad, "virtual fold needs the real-row gradients");
    TATARA_REQUIRE(moment_scales_ok(a), "f16 moment scales must be powers of two");
    TATARA_REQUIRE(!(comb && comb16), "virtual fold writes one forward table");
    TATARA_REQUIRE(table_layout_ok(layout, comb16 != nullptr, a.ft_out), "virtual fold: table layout");
    const uint32_t n_chunks = layout == kTablePairSlices ? ceil_div(a.ft_out / 8, 16) : ceil_div(a.ft_out / 4, kWave);
    const uint64_t tasks = (uint64_t)(layout == kTablePairSlices ? (piece_inputs + 1) / 2 : piece_inputs) * n_chunks;
    const uint32_t blocks = (uint32_t)((tasks + kWavesPerBlock - 1) / kWavesPerBlock);
    _Float16* c16 = reinterpret_cast<_Float16*>(comb16);
    if (a.m16) {
        if (comb16)
            ft_virtual_fold_kernel<true, true><<<blocks, 256, 0, stream>>>(a, piece_inputs, n_chunks, comb, c16, layout);
        else
            ft_virtual_fold_kernel<true, false><<<blocks, 256, 0, stream>>>(a, piece_inputs, n_chunks, comb, c16, layout);
    } else {
        if (comb16)
            ft_virtual_fold_kernel<false, true><<<blocks, 256, 0, stream>>>(a, piece_inputs, n_chunks, comb, c16, layout);
        else
            ft_virtual_fold_kernel<false, false><<<blocks, 256, 0, stream>>>(a, piece_inputs, n_chunks, comb, c16, layout);
    }
    TATARA_LAUNCHED("ft_virtual_fold");
    return kOk;
}

int32_t launch_ft_fold(const float* w, float* comb, uint16_t* comb16, uint32_t ft_in, uint32_t ft_out,
                       uint32_t piece_inputs, hipStream_t stream, int layout) {
    TATARA_REQUIRE(ft_out % 4 == 0 && piece_inputs > 0, "fold: ft_out%4==0, piece_inputs>0");
    TATARA_REQUIRE((comb != nullptr) != (comb16 != nullptr), "fold: exactly one of comb / comb16");
    TATARA_REQUIRE(table_layout_ok(layout, comb16 != nullptr, ft_out) && ft_in % piece_inputs == 0,
                   "fold: table layout");
    const uint64_t n4 = (uint64_t)ft_in * ft_out / 4;
    if (n4 == 0) return kOk;
    if (comb16)
        ft_fold_kernel<true><<<ceil_div(n4, 256), 256, 0, stream>>>(
            w, nullptr, reinterpret_cast<_Float16*>(comb16), ft_in, ft_out, piece_inputs, layout);
    else
        ft_fold_kernel<false><<<ceil_div(n4, 256), 256, 0, stream>>>(w, comb, nullptr, ft_in, ft_out,
                                                                      piece_inputs, layout);
    TATARA_LAUNCHED("ft_fold");
    return kOk;
}

int32_t launch_cast_f16(const float* src, uint16_t* dst, uint64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    const uint32_t blocks = ceil_div(n, 256) < 65536u ? ceil_div(n, 256) : 65536u;
    cast_f16_kernel<<<blocks, 256, 0, stream>>>(src, reinterpret_cast<_Float16*>(dst), n);
    TATARA_LAUNCHED("cast_f32_to_f16");
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
