// Quantised network export (.bin) for the LayerStack and Simple trainers.
//
// The FT table (the bulk of the file: 73305 x 1536 cells at LS1536) is
// quantised on the GPU where it lives: the factorizer's virtual row is folded
// into each real row, the sum is scaled in f64, rounded half away from zero
// and saturated to i16, and (LayerStack) the values are emitted as a signed
// LEB128 stream.  Only the compressed stream crosses PCIe.  The header, hashes
// and the small dense layers are written on the host.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

namespace tatara {

// An FT-shaped f32 table on the device: `rows` real rows of `cols` floats,
// optionally followed by `piece_inputs` virtual rows that are added to row r
// as row rows + r % piece_inputs (coalesce_ft_factorized, Base mode).
struct QuantSource {
    const float* w = nullptr;
    uint64_t rows = 0;
    uint32_t cols = 0;
    uint32_t piece_inputs = 0;  // 0: no virtual rows
};

// Device launchers.  quantise_leb128 needs `out` with room for 3 bytes per
// value; the byte count lands in *d_total (device).  tile_bytes / tile_off
// hold leb128_tiles(n) entries.
uint64_t leb128_tiles(uint64_t n);
int32_t launch_quantise_i16(const QuantSource& s, double scale, int16_t* out, hipStream_t stream);
int32_t launch_quantise_leb128(const QuantSource& s, double scale, uint32_t* tile_bytes, uint64_t* tile_off,
                               uint64_t* d_total, uint8_t* out, hipStream_t stream);

// Uninitialised host bytes, freed on destruction.  Ordinary pageable memory
// on purpose: the file writer reads these bytes with the CPU, and CPU reads
// of hipHostMalloc memory are uncached (an fwrite of 113 MB from it took
// ~90 ms against ~20 ms from pageable memory, more than the faster D2H
// saves).
struct HostBytes {
    uint8_t* p = nullptr;
    size_t n = 0;
    HostBytes() = default;
    HostBytes(const HostBytes&) = delete;
    HostBytes& operator=(const HostBytes&) = delete;
    ~HostBytes();
    int32_t alloc(size_t bytes);
};

// Host-side wrappers used by the exporters (synchronous on `stream`): the
// quantised table as little-endian i16, or as its LEB128 stream.
int32_t quantise_i16_to_host(const QuantSource& s, double scale, HostBytes& out, hipStream_t stream);
int32_t quantise_leb128_to_host(const QuantSource& s, double scale, HostBytes& out, hipStream_t stream);

// Export identity of a feature set (TATARA_FS_*): arch-string name, feature
// hash and base FT input rows.
struct ExportFeatureSet {
    const char* arch_name;
    uint32_t feature_hash;
    uint64_t ft_in;
};
int32_t export_feature_set(int32_t feature_set, ExportFeatureSet& out);

// LayerStack weights: the FT table and bias on the device, the dense groups
// on the host in the trainer's layouts (l1_w [nb][l1][ft_out],
// l1_shared_weight [ft_out][l1], l2_w [nb][l2][l2_in], l3_w [nb][l2]).
struct LayerStackHost {
    std::vector<float> l1_w, l1_b, l1s_w, l1s_b, l2_w, l2_b, l3_w, l3_b;
};
int32_t write_layerstack_bin(const char* path, const ExportFeatureSet& fs, const QuantSource& ft,
                             const QuantSource& ft_b, uint32_t l1_out, uint32_t l2_out, uint32_t nb,
                             const LayerStackHost& h, bool has_fv, int32_t fv, hipStream_t stream);

// Simple weights (CReLU): l1_w [2*ft_out][l1] and l2_w [l1][l2] in-major, as
// the trainer holds them.
struct SimpleHost {
    std::vector<float> l1_w, l1_b, l2_w, l2_b, l3_w, l3_b;
};
int32_t write_simple_bin(const char* path, const ExportFeatureSet& fs, const QuantSource& ft,
                         const QuantSource& ft_b, uint32_t l1_out, uint32_t l2_out, const SimpleHost& h,
                         int32_t fv, hipStream_t stream);

}  // namespace tatara
