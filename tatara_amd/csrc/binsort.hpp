// Deterministic stable bin sort (see binsort.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tatara {

struct BinSortArgs {
    const uint8_t* keys;   // [n_items] bin of each item
    uint32_t n_items;
    uint32_t n_bins;       // <= 256
    uint32_t align;        // each bin starts at a multiple of align (1 = packed)
    uint32_t value_mod;    // written value = item % value_mod (0: item)
    uint32_t* hist;        // scratch [n_bins * binsort_tiles(n_items)]
    uint32_t* bin_start;   // [n_bins + 1] first output slot of each bin; [n_bins] = end
    uint32_t* bin_count;   // [n_bins]
    int32_t* out;          // sorted values; slots not written hold -1 when out_fill_len > 0
    int32_t* out_key;      // optional sorted bins (-1 in padding)
    uint64_t out_fill_len; // number of out slots pre-filled with -1 (0: none)
};

// One stable LSD radix pass (8-bit digit (key >> shift) & 255) over
// (key, value) pairs.  With run_if set, every kernel of the pass does
// nothing unless *run_if != 0.
struct RadixPassArgs {
    const uint32_t* keys;
    const uint32_t* vals;
    uint32_t n_items;
    uint32_t shift;
    uint32_t* hist;          // scratch [256 * binsort_tiles(n_items)]
    uint32_t* digit_count;   // scratch [256]
    uint32_t* out_keys;
    uint32_t* out_vals;
    const uint32_t* run_if;  // optional device gate
};

uint32_t binsort_tiles(uint32_t n_items);
int32_t launch_radix_pass(const RadixPassArgs& a, hipStream_t stream);
int32_t launch_binsort(const BinSortArgs& a, hipStream_t stream);
int32_t launch_fill_i32(int32_t* p, uint64_t n, int32_t v, hipStream_t stream);

}  // namespace tatara
