// FT-table quantisation without any device allocation.
//
// tatara_op_quantise_ft allocates the LEB128 path's per-tile byte counts and
// offsets on every call.  Callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc) use tatara_op_quantise_ft_noalloc instead: the same kernels, with
// those arrays in a file-scope device array of fixed size.  Each GPU the
// library runs on holds its own copy of the array (kScratchWords u64, 0.8 MB)
// until the process ends; its device address is looked up once per device
// with hipGetSymbolAddress and used from then on.  Every call on a GPU shares
// that GPU's array, so calls that overlap on one GPU (from several host
// threads) race; nothing in it needs to start at zero (each pass writes every
// entry the next pass reads).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/tatara_hip.h"
#include "common.hpp"
#include "export.hpp"

namespace tatara {
namespace {

// Tiles of 4096 values: up to 2^28 values (an ft_out 3072 halfka-hm-merged
// table has 2.25e8).
constexpr uint64_t kNoAllocMaxTiles = 65536;
// tile offsets (u64, tiles + 1: the total in the last slot), then tile byte
// counts (u32, tiles + 1)
constexpr uint64_t kOffWords = kNoAllocMaxTiles + 1;
constexpr uint64_t kScratchWords = kOffWords + (kNoAllocMaxTiles + 2) / 2;

static __device__ __align__(256) uint64_t scratch[kScratchWords];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on first use).
int32_t device_scratch(uint64_t** out) {
    int dev = 0;
    TATARA_HIP(hipGetDevice(&dev), "hipGetDevice (quantise_ft_noalloc)");
    TATARA_REQUIRE(dev >= 0 && dev < kMaxDevices, "device ordinal out of range for the static scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        TATARA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (quantise_ft_noalloc scratch)");
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<uint64_t*>(g_scratch_ptr[dev]);
    return kOk;
}

}  // namespace
}  // namespace tatara

using namespace tatara;

extern "C" {

int32_t tatara_op_quantise_ft_noalloc(const float* w, uint64_t rows, uint32_t cols, uint32_t piece_inputs,
                                      double scale, int32_t leb128, uint8_t* out, uint64_t out_capacity,
                                      uint64_t* out_bytes) {
    TATARA_REQUIRE(out_bytes, "out_bytes is null");
    TATARA_REQUIRE(rows == 0 || cols == 0 || (w && out), "null device pointer");
    *out_bytes = 0;
    const QuantSource src{w, rows, cols, piece_inputs};
    const uint64_t n = rows * cols;
    if (!leb128) {
        TATARA_REQUIRE(out_capacity >= 2 * n, "out_capacity < 2 * rows * cols");
        int32_t st = launch_quantise_i16(src, scale, reinterpret_cast<int16_t*>(out), 0);
        if (st) return st;
        TATARA_HIP(hipDeviceSynchronize(), "quantise_ft_noalloc");
        *out_bytes = 2 * n;
        return kOk;
    }
    const uint64_t tiles = leb128_tiles(n);
    TATARA_REQUIRE(tiles <= kNoAllocMaxTiles,
                   "quantise_ft_noalloc: the table exceeds the static scratch (at most 65536 tiles of 4096 "
                   "values, 268435456 values); use tatara_op_quantise_ft");
    uint64_t* base = nullptr;
    int32_t st = device_scratch(&base);
    if (st) return st;
    uint64_t* tile_off = base;  // tile offsets, then the total in the last slot
    uint32_t* tile_bytes = reinterpret_cast<uint32_t*>(base + kOffWords);
    if ((st = launch_quantise_leb128(src, scale, tile_bytes, tile_off, tile_off + tiles, nullptr, 0))) return st;
    uint64_t total = 0;
    TATARA_HIP(hipMemcpy(&total, tile_off + tiles, sizeof total, hipMemcpyDeviceToHost), "quantise_ft_noalloc total");
    TATARA_REQUIRE(total <= out_capacity, "out_capacity is smaller than the LEB128 stream");
    if (total && (st = launch_quantise_leb128(src, scale, tile_bytes, tile_off, tile_off + tiles, out, 0)))
        return st;
    TATARA_HIP(hipDeviceSynchronize(), "quantise_ft_noalloc");
    *out_bytes = total;
    return kOk;
}

}  // extern "C"
