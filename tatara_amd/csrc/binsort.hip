// Deterministic, stable counting sort of items by a small key (<= 256 bins),
// with optional per-bin alignment of each bin's start (the LayerStack bucket
// sort aligns every bucket to 16 rows so that a 16-row tile never mixes
// buckets, as padded_sort_batch / exclusive_scan_aligned do in the reference:
// bins/nnue_train/src/trainer_common.rs:550-553,
// crates/cuda-native-runtime/kernels/native_kernels.cu:1858-1925).
//
// Unlike the reference's atomic-rank scatter, the rank of an item inside its
// bin is computed without atomics (wave ballots + per-wave counts), so the
// output order is exactly "bin ascending, item index ascending" on every run.
//
//   pass 1  per 1024-item tile: histogram -> hist[bin][tile]
//   pass 2  one workgroup per bin: exclusive scan over its tiles, bin size
//   pass 3  per tile: aligned bin starts (prefix of rounded-up sizes),
//           wave-match ranks + per-wave prefix -> scatter
#include "binsort.hpp"

#include "common.hpp"

namespace tatara {

namespace {

constexpr int kTile = 1024;
constexpr int kWaves = kTile / 64;
constexpr int kMaxBins = 256;

__global__ __launch_bounds__(kTile) void binsort_hist_kernel(const uint8_t* __restrict__ keys,
                                                             uint32_t n_items, uint32_t n_bins,
                                                             uint32_t* __restrict__ hist) {
    __shared__ uint32_t h[kMaxBins];
    const uint32_t t = threadIdx.x;
    for (uint32_t i = t; i < n_bins; i += kTile) h[i] = 0;
    __syncthreads();
    const uint64_t item = (uint64_t)blockIdx.x * kTile + t;
    if (item < n_items) atomicAdd(&h[keys[item]], 1u);
    __syncthreads();
    for (uint32_t i = t; i < n_bins; i += kTile) hist[(uint64_t)i * gridDim.x + blockIdx.x] = h[i];
}

// hist [n_bins][n_tiles] -> each bin's exclusive offsets in place, relative
// to the bin's start; bin_count[bin] = the bin's size.  One workgroup per bin.
constexpr int kScanThreads = 256;

__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t x, uint32_t lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d);
        if (lane >= (uint32_t)d) x += y;
    }
    return x;
}

__global__ __launch_bounds__(kScanThreads) void binsort_scan_kernel(uint32_t* __restrict__ hist,
                                                                    uint32_t n_tiles, uint32_t n_bins,
                                                                    uint32_t* __restrict__ bin_start,
                                                                    uint32_t* __restrict__ bin_count,
                                                                    const uint32_t* __restrict__ run_if) {
    if (run_if && __builtin_amdgcn_readfirstlane(*run_if) == 0u) return;
    constexpr int W = kScanThreads / 64;
    __shared__ uint32_t wsum[W];
    const uint32_t b = blockIdx.x, t = threadIdx.x, lane = t % 64, wave = t / 64;
    uint32_t* row = hist + (uint64_t)b * n_tiles;
    uint32_t carry = 0;
    for (uint32_t k0 = 0; k0 < n_tiles; k0 += kScanThreads) {
        const uint32_t k = k0 + t;
        const uint32_t x = k < n_tiles ? row[k] : 0u;
        const uint32_t incl = wave_inclusive_sum(x, lane);
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        uint32_t before = carry, total = 0;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            before += (uint32_t)w < wave ? wsum[w] : 0u;
            total += wsum[w];
        }
        if (k < n_tiles) row[k] = before + incl - x;
        carry += total;
        __syncthreads();
    }
    if (t == 0) {
        bin_count[b] = carry;
        if (n_tiles == 0 && bin_start) {  // no scatter runs: publish the empty bins here
            bin_start[b] = 0;
            if (b + 1 == n_bins) bin_start[n_bins] = 0;
        }
    }
}

// Bin starts: start[b] = sum over b' < b of size[b'] rounded up to `align`
// (every start is a multiple of align, so rounding each running end up is
// rounding each size up); bin_start[n_bins] = the last bin's end, unrounded.
// Each scatter workgroup computes them; workgroup 0 publishes them.
__global__ __launch_bounds__(kTile) void binsort_scatter_kernel(
    const uint8_t* __restrict__ keys, uint32_t n_items, uint32_t n_bins, uint32_t align,
    const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ bin_count, uint32_t value_mod,
    int32_t* __restrict__ out, int32_t* __restrict__ out_key, uint32_t* __restrict__ bin_start) {
    __shared__ uint32_t wcnt[kWaves][kMaxBins];
    __shared__ uint32_t s_start[kMaxBins];
    __shared__ uint32_t s_wtot[kMaxBins / 64];
    const uint32_t t = threadIdx.x;
    const uint32_t wave = t / 64, lane = t % 64;
    for (uint32_t i = t; i < kWaves * kMaxBins; i += kTile) (&wcnt[0][0])[i] = 0;
    uint32_t cnt = 0, rounded = 0, incl = 0;
    if (t < (uint32_t)kMaxBins) {  // waves 0..3, whole waves
        cnt = t < n_bins ? bin_count[t] : 0u;
        rounded = cnt % align ? cnt + (align - cnt % align) : cnt;
        incl = wave_inclusive_sum(rounded, lane);
        if (lane == 63) s_wtot[wave] = incl;
    }
    __syncthreads();
    if (t < (uint32_t)kMaxBins) {
        uint32_t before = 0;
        for (uint32_t w = 0; w < wave; ++w) before += s_wtot[w];
        const uint32_t start = before + incl - rounded;
        s_start[t] = start;
        if (blockIdx.x == 0 && t < n_bins) {
            bin_start[t] = start;
            if (t + 1 == n_bins) bin_start[n_bins] = start + cnt;
        }
    }
    __syncthreads();
    const uint64_t item = (uint64_t)blockIdx.x * kTile + t;
    const bool ok = item < n_items;
    const uint32_t key = ok ? keys[item] : 0xFFFFFFFFu;
    // lanes with the same key: intersect the ballots of every key bit
    uint64_t match = __ballot(ok);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
        const uint64_t bal = __ballot(ok && ((key >> bit) & 1u));
        match &= ((key >> bit) & 1u) ? bal : ~bal;
    }
    const uint64_t below = (1ull << lane) - 1ull;
    const uint32_t rank = __popcll(match & below);
    // the highest lane of each key group publishes the group's size
    if (ok && (match >> lane) == 1ull) wcnt[wave][key] = __popcll(match);
    __syncthreads();
    if (!ok) return;
    uint32_t before = 0;
    for (uint32_t w = 0; w < wave; ++w) before += wcnt[w][key];
    const uint32_t dst = s_start[key] + offsets[(uint64_t)key * gridDim.x + blockIdx.x] + before + rank;
    out[dst] = (int32_t)(value_mod ? (uint32_t)(item % value_mod) : (uint32_t)item);
    if (out_key) out_key[dst] = (int32_t)key;
}

// One LSD radix pass over (key, value) pairs: the stable counting sort of
// the 8-bit digit (key >> shift) & 255, with the same tiles, scan and
// ballot ranks as the bin sort above.  The kernels do nothing unless
// *run_if != 0 (when run_if is set), and stride over the tiles with a
// bounded grid, so a pass that is skipped costs little.
__global__ __launch_bounds__(kTile) void radix_hist_kernel(const uint32_t* __restrict__ keys, uint32_t n_items,
                                                           uint32_t shift, uint32_t n_tiles,
                                                           uint32_t* __restrict__ hist,
                                                           const uint32_t* __restrict__ run_if) {
    if (run_if && __builtin_amdgcn_readfirstlane(*run_if) == 0u) return;
    __shared__ uint32_t h[kMaxBins];
    const uint32_t t = threadIdx.x;
    for (uint32_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        if (t < (uint32_t)kMaxBins) h[t] = 0;
        __syncthreads();
        const uint64_t item = (uint64_t)tile * kTile + t;
        if (item < n_items) atomicAdd(&h[(keys[item] >> shift) & 255u], 1u);
        __syncthreads();
        if (t < (uint32_t)kMaxBins) hist[(uint64_t)t * n_tiles + tile] = h[t];
        __syncthreads();
    }
}

__global__ __launch_bounds__(kTile) void radix_scatter_kernel(
    const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals, uint32_t n_items, uint32_t shift,
    uint32_t n_tiles, const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ bin_count,
    uint32_t* __restrict__ out_keys, uint32_t* __restrict__ out_vals, const uint32_t* __restrict__ run_if) {
    if (run_if && __builtin_amdgcn_readfirstlane(*run_if) == 0u) return;
    __shared__ uint32_t wcnt[kWaves][kMaxBins];
    __shared__ uint32_t s_start[kMaxBins];
    __shared__ uint32_t s_wtot[kMaxBins / 64];
    const uint32_t t = threadIdx.x;
    const uint32_t wave = t / 64, lane = t % 64;
    uint32_t cnt = 0, incl = 0;
    if (t < (uint32_t)kMaxBins) {  // digit starts: exclusive prefix of the digit sizes
        cnt = bin_count[t];
        incl = wave_inclusive_sum(cnt, lane);
        if (lane == 63) s_wtot[wave] = incl;
    }
    __syncthreads();
    if (t < (uint32_t)kMaxBins) {
        uint32_t before = 0;
        for (uint32_t w = 0; w < wave; ++w) before += s_wtot[w];
        s_start[t] = before + incl - cnt;
    }
    for (uint32_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        for (uint32_t i = t; i < kWaves * kMaxBins; i += kTile) (&wcnt[0][0])[i] = 0;
        __syncthreads();
        const uint64_t item = (uint64_t)tile * kTile + t;
        const bool ok = item < n_items;
        const uint32_t key = ok ? keys[item] : 0u;
        const uint32_t dig = ok ? (key >> shift) & 255u : 0xFFFFFFFFu;
        uint64_t match = __ballot(ok);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const uint64_t bal = __ballot(ok && ((dig >> bit) & 1u));
            match &= ((dig >> bit) & 1u) ? bal : ~bal;
        }
        const uint32_t rank = __popcll(match & ((1ull << lane) - 1ull));
        if (ok && (match >> lane) == 1ull) wcnt[wave][dig] = __popcll(match);
        __syncthreads();
        if (ok) {
            uint32_t before = 0;
            for (uint32_t w = 0; w < wave; ++w) before += wcnt[w][dig];
            const uint32_t dst = s_start[dig] + offsets[(uint64_t)dig * n_tiles + tile] + before + rank;
            out_keys[dst] = key;
            out_vals[dst] = vals[item];
        }
        __syncthreads();
    }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, uint64_t n, int32_t v) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace

uint32_t binsort_tiles(uint32_t n_items) { return ceil_div(n_items, kTile); }

int32_t launch_fill_i32(int32_t* p, uint64_t n, int32_t v, hipStream_t stream) {
    if (n == 0) return kOk;
    fill_i32_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(p, n, v);
    TATARA_LAUNCHED("fill_i32");
    return kOk;
}

int32_t launch_radix_pass(const RadixPassArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(a.shift < 32, "radix pass: shift < 32");
    const uint32_t tiles = binsort_tiles(a.n_items);
    if (tiles == 0) return kOk;
    // a gated pass strides over a small grid (64 workgroups of 1024 lanes):
    // its no-op workgroups cost the kernels it overlaps little
    const uint32_t grid = a.run_if && tiles > 64u ? 64u : tiles;
    radix_hist_kernel<<<grid, kTile, 0, stream>>>(a.keys, a.n_items, a.shift, tiles, a.hist, a.run_if);
    TATARA_LAUNCHED("radix_hist");
    binsort_scan_kernel<<<kMaxBins, kScanThreads, 0, stream>>>(a.hist, tiles, kMaxBins, nullptr, a.digit_count,
                                                               a.run_if);
    TATARA_LAUNCHED("radix_scan");
    radix_scatter_kernel<<<grid, kTile, 0, stream>>>(a.keys, a.vals, a.n_items, a.shift, tiles, a.hist,
                                                     a.digit_count, a.out_keys, a.out_vals, a.run_if);
    TATARA_LAUNCHED("radix_scatter");
    return kOk;
}

int32_t launch_binsort(const BinSortArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(a.n_bins >= 1 && a.n_bins <= (uint32_t)kMaxBins, "binsort: 1 <= n_bins <= 256");
    TATARA_REQUIRE(a.align >= 1, "binsort: align >= 1");
    TATARA_REQUIRE(a.bin_start && a.bin_count, "binsort: bin_start and bin_count are required");
    if (a.out_fill_len) {
        int32_t st = launch_fill_i32(a.out, a.out_fill_len, -1, stream);
        if (st) return st;
        if (a.out_key) {
            st = launch_fill_i32(a.out_key, a.out_fill_len, -1, stream);
            if (st) return st;
        }
    }
    const uint32_t tiles = binsort_tiles(a.n_items);
    if (tiles == 0) {
        // still publish empty bin boundaries
        binsort_scan_kernel<<<a.n_bins, kScanThreads, 0, stream>>>(a.hist, 0, a.n_bins, a.bin_start,
                                                                   a.bin_count, nullptr);
        TATARA_LAUNCHED("binsort_scan");
        return kOk;
    }
    binsort_hist_kernel<<<tiles, kTile, 0, stream>>>(a.keys, a.n_items, a.n_bins, a.hist);
    TATARA_LAUNCHED("binsort_hist");
    binsort_scan_kernel<<<a.n_bins, kScanThreads, 0, stream>>>(a.hist, tiles, a.n_bins, a.bin_start,
                                                               a.bin_count, nullptr);
    TATARA_LAUNCHED("binsort_scan");
    binsort_scatter_kernel<<<tiles, kTile, 0, stream>>>(a.keys, a.n_items, a.n_bins, a.align, a.hist,
                                                       a.bin_count, a.value_mod, a.out, a.out_key,
                                                       a.bin_start);
    TATARA_LAUNCHED("binsort_scatter");
    return kOk;
}

}  // namespace tatara
