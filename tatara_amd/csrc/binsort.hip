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
//   pass 2  one workgroup: exclusive scan in (bin, tile) order, bin alignment
//   pass 3  per tile: wave-match ranks + per-wave prefix -> scatter
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

// hist [n_bins][n_tiles] -> exclusive offsets in place; bin_start[n_bins+1],
// bin_count[n_bins].  Each bin starts at a multiple of `align`.
__global__ __launch_bounds__(1024) void binsort_scan_kernel(uint32_t* __restrict__ hist,
                                                            uint32_t n_tiles, uint32_t n_bins,
                                                            uint32_t align,
                                                            uint32_t* __restrict__ bin_start,
                                                            uint32_t* __restrict__ bin_count) {
    __shared__ uint32_t tot[kMaxBins];
    __shared__ uint32_t start[kMaxBins + 1];
    const uint32_t t = threadIdx.x;
    // per-bin totals: one thread per bin (n_bins <= 256)
    if (t < n_bins) {
        uint32_t s = 0;
        for (uint32_t k = 0; k < n_tiles; ++k) s += hist[(uint64_t)t * n_tiles + k];
        tot[t] = s;
    }
    __syncthreads();
    if (t == 0) {
        uint32_t acc = 0;
        for (uint32_t b = 0; b < n_bins; ++b) {
            const uint32_t r = acc % align;
            if (r) acc += align - r;
            start[b] = acc;
            acc += tot[b];
        }
        start[n_bins] = acc;
    }
    __syncthreads();
    if (t < n_bins) {
        uint32_t acc = start[t];
        for (uint32_t k = 0; k < n_tiles; ++k) {
            const uint64_t i = (uint64_t)t * n_tiles + k;
            const uint32_t x = hist[i];
            hist[i] = acc;
            acc += x;
        }
        bin_count[t] = tot[t];
    }
    if (t <= n_bins) bin_start[t] = start[t];
}

__global__ __launch_bounds__(kTile) void binsort_scatter_kernel(
    const uint8_t* __restrict__ keys, uint32_t n_items, uint32_t n_bins,
    const uint32_t* __restrict__ offsets, uint32_t value_mod, int32_t* __restrict__ out,
    int32_t* __restrict__ out_key) {
    __shared__ uint32_t wcnt[kWaves][kMaxBins];
    const uint32_t t = threadIdx.x;
    const uint32_t wave = t / 64, lane = t % 64;
    for (uint32_t i = t; i < kWaves * kMaxBins; i += kTile) (&wcnt[0][0])[i] = 0;
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
    const uint32_t dst = offsets[(uint64_t)key * gridDim.x + blockIdx.x] + before + rank;
    out[dst] = (int32_t)(value_mod ? (uint32_t)(item % value_mod) : (uint32_t)item);
    if (out_key) out_key[dst] = (int32_t)key;
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

int32_t launch_binsort(const BinSortArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(a.n_bins >= 1 && a.n_bins <= (uint32_t)kMaxBins, "binsort: 1 <= n_bins <= 256");
    TATARA_REQUIRE(a.align >= 1, "binsort: align >= 1");
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
        binsort_scan_kernel<<<1, 1024, 0, stream>>>(a.hist, 0, a.n_bins, a.align, a.bin_start,
                                                   a.bin_count);
        TATARA_LAUNCHED("binsort_scan");
        return kOk;
    }
    binsort_hist_kernel<<<tiles, kTile, 0, stream>>>(a.keys, a.n_items, a.n_bins, a.hist);
    TATARA_LAUNCHED("binsort_hist");
    binsort_scan_kernel<<<1, 1024, 0, stream>>>(a.hist, tiles, a.n_bins, a.align, a.bin_start,
                                               a.bin_count);
    TATARA_LAUNCHED("binsort_scan");
    binsort_scatter_kernel<<<tiles, kTile, 0, stream>>>(a.keys, a.n_items, a.n_bins, a.hist,
                                                       a.value_mod, a.out, a.out_key);
    TATARA_LAUNCHED("binsort_scatter");
    return kOk;
}

}  // namespace tatara
