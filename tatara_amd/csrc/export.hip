// Quantised network export (.bin): GPU quantisation of the FT table and the
// host-side file layout.
//
// Reference semantics:
//   LayerStack  crates/nnue-format/src/layerstack_weights.rs:568-829
//               (save_quantised), :120-149 (LEB128), :242-343 (arch string),
//               :351-399 (hashes), :412-491 (coalesce_ft_factorized),
//               :1306-1314 (clamp_i8)
//   Simple      crates/nnue-format/src/simple_weights.rs:374-429
//               (save_quantised), :254-340 (arch string, hashes), :545-690
//               (clamp_round, write_i16_quantised / write_i32_bias /
//               write_i8_weight); trainer_simple.rs:2680-2745 (to_simple_weights:
//               l1_w / l2_w transposed to out-major)
// Numeric semantics follow Rust: f64 round is half away from zero, float ->
// int `as` casts saturate and send NaN to 0.
#include "export.hpp"

#include <hipcub/hipcub.hpp>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <limits>

#include "common.hpp"
#include "psv_kernels.hpp"
#include "../../include/tatara_hip.h"

namespace tatara {

namespace {

constexpr int kQThreads = 256;
constexpr int kQVec = 4;    // consecutive values per thread per step (one float4)
constexpr int kQSteps = 4;  // steps per tile
constexpr uint64_t kQStep = (uint64_t)kQThreads * kQVec;           // values per step
constexpr uint64_t kQTile = kQStep * kQSteps;                      // values per workgroup
constexpr int kScanThreads = 1024;

// Row, column and virtual-row index of cell i.  32-bit division whenever the
// table has < 2^32 cells (every feature set at every supported width).
__device__ __forceinline__ uint64_t virtual_offset(const QuantSource& s, uint64_t i) {
    uint64_t c, p;
    if (s.rows * s.cols < (1ull << 32)) {
        const uint32_t i32 = (uint32_t)i;
        const uint32_t r32 = i32 / s.cols;
        c = i32 - r32 * s.cols;
        p = r32 % s.piece_inputs;
    } else {
        const uint64_t r = i / s.cols;
        c = i - r * s.cols;
        p = r % s.piece_inputs;
    }
    return (s.rows + p) * s.cols + c;
}

// Cell i of the export-shape table: the real row's value plus, with a
// factorizer, its piece's virtual row (an f32 add, as the fold does).
__device__ __forceinline__ float source_value(const QuantSource& s, uint64_t i) {
    float v = s.w[i];
    if (s.piece_inputs) v += s.w[virtual_offset(s, i)];
    return v;
}

// The tile's values held by this thread: x[k][j] is cell
// base + k * kQStep + kQVec * threadIdx.x + j; cells past n are 0 (and
// counted as absent by the callers).  Full tiles of a 16-byte aligned table
// with cols % 4 == 0 take the vector path: every load is issued before any
// is used, and a float4 never straddles a row.
__device__ __forceinline__ void load_tile(const QuantSource& s, uint64_t n, uint64_t base,
                                          float (&x)[kQSteps][kQVec]) {
    const uint64_t t0 = base + (uint64_t)kQVec * threadIdx.x;
    const bool vec = base + kQTile <= n && s.cols % kQVec == 0 && ((uintptr_t)s.w & 15) == 0;
    if (vec) {
        float4 v[kQSteps];
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) v[k] = *reinterpret_cast<const float4*>(s.w + t0 + k * kQStep);
        if (s.piece_inputs) {
            float4 g[kQSteps];
#pragma unroll
            for (int k = 0; k < kQSteps; ++k)
                g[k] = *reinterpret_cast<const float4*>(s.w + virtual_offset(s, t0 + k * kQStep));
#pragma unroll
            for (int k = 0; k < kQSteps; ++k) {
                v[k].x += g[k].x;
                v[k].y += g[k].y;
                v[k].z += g[k].z;
                v[k].w += g[k].w;
            }
        }
#pragma unroll
        for (int k = 0; k < kQSteps; ++k) {
            x[k][0] = v[k].x;
            x[k][1] = v[k].y;
            x[k][2] = v[k].z;
            x[k][3] = v[k].w;
        }
        return;
    }
    for (int k = 0; k < kQSteps; ++k)
        for (int j = 0; j < kQVec; ++j) {
            const uint64_t i = t0 + k * kQStep + j;
            x[k][j] = i < n ? source_value(s, i) : 0.0f;
        }
}

// saturate_i16(round(scale * v)) with NaN -> 0.
__device__ __forceinline__ int32_t quant16(float v, double scale) {
    const double x = scale * (double)v;
    if (x != x) return 0;
    const double r = round(x);
    return r < -32768.0 ? -32768 : (r > 32767.0 ? 32767 : (int32_t)r);
}

// Signed LEB128 length of an i16 value.
__device__ __forceinline__ uint32_t leb128_len(int32_t q) {
    return (q >= -64 && q < 64) ? 1u : ((q >= -8192 && q < 8192) ? 2u : 3u);
}

__global__ __launch_bounds__(256) void quantise_i16_kernel(QuantSource s, double scale, uint64_t n,
                                                           int16_t* __restrict__ out) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = (int16_t)quant16(source_value(s, i), scale);
}

// Pass 1: bytes of each tile of kQTile values.
__global__ __launch_bounds__(kQThreads) void leb128_tile_bytes_kernel(QuantSource s, double scale, uint64_t n,
                                                                      uint32_t* __restrict__ tile_bytes) {
    const uint64_t base = (uint64_t)blockIdx.x * kQTile;
    float x[kQSteps][kQVec];
    load_tile(s, n, base, x);
    const uint64_t t0 = base + (uint64_t)kQVec * threadIdx.x;
    uint32_t sum = 0;
#pragma unroll
    for (int k = 0; k < kQSteps; ++k)
#pragma unroll
        for (int j = 0; j < kQVec; ++j)
            if (t0 + k * kQStep + j < n) sum += leb128_len(quant16(x[k][j], scale));
    using Reduce = hipcub::BlockReduce<uint32_t, kQThreads>;
    __shared__ typename Reduce::TempStorage tmp;
    const uint32_t total = Reduce(tmp).Sum(sum);
    if (threadIdx.x == 0) tile_bytes[blockIdx.x] = total;
}

// Pass 2: exclusive offsets of the tiles (one workgroup; each thread owns a
// contiguous run of tiles) and the stream's total length.
__global__ __launch_bounds__(kScanThreads) void leb128_tile_scan_kernel(const uint32_t* __restrict__ tile_bytes,
                                                                        uint64_t n_tiles,
                                                                        uint64_t* __restrict__ tile_off,
                                                                        uint64_t* __restrict__ total) {
    const uint64_t per = (n_tiles + kScanThreads - 1) / kScanThreads;
    const uint64_t a = min(n_tiles, (uint64_t)threadIdx.x * per);
    const uint64_t b = min(n_tiles, a + per);
    uint64_t run = 0;
    for (uint64_t i = a; i < b; ++i) run += tile_bytes[i];
    using Scan = hipcub::BlockScan<uint64_t, kScanThreads>;
    __shared__ typename Scan::TempStorage tmp;
    uint64_t excl, agg;
    Scan(tmp).ExclusiveSum(run, excl, agg);
    for (uint64_t i = a; i < b; ++i) {
        tile_off[i] = excl;
        excl += tile_bytes[i];
    }
    if (threadIdx.x == 0) *total = agg;
}

// Pass 3: each tile re-quantises its values and writes their LEB128 bytes in
// cell order: step by step, thread t's four cells follow threads 0..t-1's.
__global__ __launch_bounds__(kQThreads) void leb128_scatter_kernel(QuantSource s, double scale, uint64_t n,
                                                                   const uint64_t* __restrict__ tile_off,
                                                                   uint8_t* __restrict__ out) {
    using Scan = hipcub::BlockScan<uint32_t, kQThreads>;
    __shared__ typename Scan::TempStorage tmp;
    const uint64_t base = (uint64_t)blockIdx.x * kQTile;
    float x[kQSteps][kQVec];
    load_tile(s, n, base, x);
    const uint64_t t0 = base + (uint64_t)kQVec * threadIdx.x;
    uint64_t off = tile_off[blockIdx.x];
    for (int k = 0; k < kQSteps; ++k) {
        int32_t q[kQVec];
        uint32_t len = 0;
#pragma unroll
        for (int j = 0; j < kQVec; ++j) {
            q[j] = quant16(x[k][j], scale);
            if (t0 + k * kQStep + j < n) len += leb128_len(q[j]);
        }
        uint32_t excl, agg;
        Scan(tmp).ExclusiveSum(len, excl, agg);
        uint8_t* p = out + off + excl;
#pragma unroll
        for (int j = 0; j < kQVec; ++j) {
            if (t0 + k * kQStep + j >= n) break;
            const int32_t v = q[j];
            const uint32_t l = leb128_len(v);
            if (l == 1) {
                p[0] = (uint8_t)(v & 0x7f);
            } else if (l == 2) {
                p[0] = (uint8_t)((v & 0x7f) | 0x80);
                p[1] = (uint8_t)((v >> 7) & 0x7f);
            } else {
                p[0] = (uint8_t)((v & 0x7f) | 0x80);
                p[1] = (uint8_t)(((v >> 7) & 0x7f) | 0x80);
                p[2] = (uint8_t)((v >> 14) & 0x7f);
            }
            p += l;
        }
        off += agg;
        __syncthreads();  // the scan's temp storage is reused by the next step
    }
}

inline uint32_t ceil_div_u32(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// Host side: Rust numeric semantics, the byte writer, arch strings, hashes.
// ---------------------------------------------------------------------------

template <typename T>
T sat_cast(double v) {  // `f64 as T`
    if (std::isnan(v)) return 0;
    const double lo = (double)std::numeric_limits<T>::min();
    const double hi = (double)std::numeric_limits<T>::max();
    if (v <= lo) return std::numeric_limits<T>::min();
    if (v >= hi) return std::numeric_limits<T>::max();
    return (T)v;
}

int8_t ls_i8(double x) {  // clamp_i8(x.round())
    const double r = std::round(x);
    if (r < -128.0) return -128;
    if (r > 127.0) return 127;
    return sat_cast<int8_t>(r);
}

template <typename T>
T simple_q(double x) {  // clamp_round(x, T::MIN, T::MAX) as T
    const double r = std::round(x);
    const double lo = (double)std::numeric_limits<T>::min();
    const double hi = (double)std::numeric_limits<T>::max();
    return sat_cast<T>(r < lo ? lo : (r > hi ? hi : r));
}

struct Bytes {
    std::vector<uint8_t> b;
    void u8(uint8_t v) { b.push_back(v); }
    void u32(uint32_t v) {
        const uint8_t le[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
        b.insert(b.end(), le, le + 4);
    }
    void i32(int32_t v) { u32((uint32_t)v); }
    void raw(const void* p, size_t n) {
        const uint8_t* c = static_cast<const uint8_t*>(p);
        b.insert(b.end(), c, c + n);
    }
    void str(const std::string& s) {
        u32((uint32_t)s.size());
        raw(s.data(), s.size());
    }
};

// nnue-pytorch style layer hash chain: InputSlice then affine layers.
uint32_t layer_hash_chain(uint32_t slice, uint64_t out0, uint64_t out1) {
    uint32_t prev = 0xEC42E90Du ^ slice;
    const uint64_t outs[3] = {out0, out1, 1};
    for (int i = 0; i < 3; ++i) {
        uint32_t h = 0xCC03DAE4u + (uint32_t)outs[i];
        h ^= prev >> 1;
        h ^= prev << 31;
        if (i < 2) h += 0x538D24C7u;  // ClippedReLU after the hidden layers
        prev = h;
    }
    return prev;
}

std::string u(uint64_t v) { return std::to_string(v); }

struct Segment {
    const void* p;
    size_t n;
};

int32_t write_file(const char* path, std::initializer_list<Segment> parts) {
    TATARA_REQUIRE(path && *path, "export path is empty");
    FILE* f = std::fopen(path, "wb");
    if (!f) {
        set_error(std::string("export: cannot open ") + path + " for writing");
        return kErrInvalid;
    }
    bool ok = true;
    for (const Segment& g : parts)
        if (g.n && std::fwrite(g.p, 1, g.n, f) != g.n) ok = false;
    if (std::fclose(f) != 0) ok = false;
    if (!ok) {
        set_error(std::string("export: write to ") + path + " failed");
        return kErrInvalid;
    }
    return kOk;
}

}  // namespace

uint64_t leb128_tiles(uint64_t n) { return (n + kQTile - 1) / kQTile; }

int32_t launch_quantise_i16(const QuantSource& s, double scale, int16_t* out, hipStream_t stream) {
    const uint64_t n = s.rows * s.cols;
    if (n == 0) return kOk;
    const uint32_t blocks = ceil_div_u32(n, 256) < 65536u ? ceil_div_u32(n, 256) : 65536u;
    quantise_i16_kernel<<<blocks, 256, 0, stream>>>(s, scale, n, out);
    TATARA_LAUNCHED("quantise_i16");
    return kOk;
}

int32_t launch_quantise_leb128(const QuantSource& s, double scale, uint32_t* tile_bytes, uint64_t* tile_off,
                               uint64_t* d_total, uint8_t* out, hipStream_t stream) {
    const uint64_t n = s.rows * s.cols;
    const uint64_t tiles = leb128_tiles(n);
    TATARA_REQUIRE(tiles < (1ull << 31), "quantise: table too large");
    if (tiles) {
        leb128_tile_bytes_kernel<<<(uint32_t)tiles, kQThreads, 0, stream>>>(s, scale, n, tile_bytes);
        TATARA_LAUNCHED("leb128_tile_bytes");
    }
    leb128_tile_scan_kernel<<<1, kScanThreads, 0, stream>>>(tile_bytes, tiles, tile_off, d_total);
    TATARA_LAUNCHED("leb128_tile_scan");
    if (tiles && out) {
        leb128_scatter_kernel<<<(uint32_t)tiles, kQThreads, 0, stream>>>(s, scale, n, tile_off, out);
        TATARA_LAUNCHED("leb128_scatter");
    }
    return kOk;
}

HostBytes::~HostBytes() { std::free(p); }

int32_t HostBytes::alloc(size_t bytes) {
    std::free(p);
    p = nullptr;
    n = bytes;
    if (bytes && !(p = static_cast<uint8_t*>(std::malloc(bytes)))) {
        set_error("export: host allocation failed");
        return kErrOutOfMemory;
    }
    return kOk;
}

int32_t quantise_i16_to_host(const QuantSource& s, double scale, HostBytes& out, hipStream_t stream) {
    const uint64_t n = s.rows * s.cols;
    int32_t st = out.alloc(n * sizeof(int16_t));
    if (st || n == 0) return st;
    int16_t* d = nullptr;
    TATARA_HIP(hipMalloc(&d, n * sizeof(int16_t)), "hipMalloc export i16");
    st = launch_quantise_i16(s, scale, d, stream);
    hipError_t e = hipSuccess;
    if (st == kOk) e = hipMemcpyAsync(out.p, d, n * sizeof(int16_t), hipMemcpyDeviceToHost, stream);
    if (st == kOk && e == hipSuccess) e = hipStreamSynchronize(stream);
    (void)hipFree(d);
    if (st) return st;
    TATARA_HIP(e, "export i16 download");
    return kOk;
}

int32_t quantise_leb128_to_host(const QuantSource& s, double scale, HostBytes& out, hipStream_t stream) {
    const uint64_t n = s.rows * s.cols;
    const uint64_t tiles = leb128_tiles(n);
    uint32_t* tile_bytes = nullptr;
    uint64_t* tile_off = nullptr;  // tile offsets, then the total in the last slot
    uint8_t* d = nullptr;
    int32_t st = kOk;
    hipError_t e = hipMalloc(&tile_bytes, (tiles + 1) * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&tile_off, (tiles + 1) * sizeof(uint64_t));
    uint64_t bytes = 0;
    if (e == hipSuccess) st = launch_quantise_leb128(s, scale, tile_bytes, tile_off, tile_off + tiles, nullptr, stream);
    if (e == hipSuccess && st == kOk)
        e = hipMemcpyAsync(&bytes, tile_off + tiles, sizeof bytes, hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess && st == kOk) e = hipStreamSynchronize(stream);
    if (e == hipSuccess && st == kOk) st = out.alloc(bytes);
    if (e == hipSuccess && st == kOk && bytes) e = hipMalloc(&d, bytes);
    if (e == hipSuccess && st == kOk && bytes) {
        leb128_scatter_kernel<<<(uint32_t)tiles, kQThreads, 0, stream>>>(s, scale, n, tile_off, d);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(out.p, d, bytes, hipMemcpyDeviceToHost, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
    }
    (void)hipFree(d);
    (void)hipFree(tile_off);
    (void)hipFree(tile_bytes);
    if (st) return st;
    TATARA_HIP(e, "export LEB128 stream");
    return kOk;
}

int32_t export_feature_set(int32_t feature_set, ExportFeatureSet& out) {
    // FeatureSetSpec::arch_feature_name (crates/shogi-features/src/feature_set.rs:519-521,
    // names pinned by arch_feature_name_uses_pascal_case, :1204-1217)
    static const char* kNames[5] = {"HalfKP", "HalfKaSplit", "HalfKaMerged", "HalfKaHmSplit", "HalfKaHmMerged"};
    FeatureSetShape sh;
    int32_t st = feature_set_shape(feature_set, sh);
    if (st) return st;
    out.arch_name = kNames[feature_set];
    out.feature_hash = sh.feature_hash;
    out.ft_in = (uint64_t)sh.king_buckets * sh.piece_inputs;
    return kOk;
}

int32_t write_layerstack_bin(const char* path, const ExportFeatureSet& fs, const QuantSource& ft,
                             const QuantSource& ft_b, uint32_t l1_out, uint32_t l2_out, uint32_t nb,
                             const LayerStackHost& h, bool has_fv, int32_t fv, hipStream_t stream) {
    const uint64_t ft_out = ft.cols;
    const uint64_t l2_in = 2ull * (l1_out - 1);
    TATARA_REQUIRE(nb >= 1 && l1_out >= 2 && ft.rows == fs.ft_in && ft_b.rows * ft_b.cols == ft_out,
                   "LayerStack export: dimensions do not match the feature set");
    TATARA_REQUIRE(h.l1_w.size() == (uint64_t)nb * l1_out * ft_out && h.l1_b.size() == (uint64_t)nb * l1_out &&
                       h.l1s_w.size() == ft_out * l1_out && h.l1s_b.size() == l1_out &&
                       h.l2_w.size() == (uint64_t)nb * l2_out * l2_in && h.l2_b.size() == (uint64_t)nb * l2_out &&
                       h.l3_w.size() == (uint64_t)nb * l2_out && h.l3_b.size() == nb,
                   "LayerStack export: dense group sizes");
    const uint32_t ft_hash = fs.feature_hash ^ (uint32_t)(ft_out * 2);
    const uint32_t fc_hash = layer_hash_chain((uint32_t)(ft_out * 2), ft_out, l2_out);
    const std::string F2 = u(ft_out * 2);
    std::string arch = std::string("Features=") + fs.arch_name + "(Friend)[" + u(fs.ft_in) + "->" + u(ft_out) +
                       "x2],Network=AffineTransform[1<-" + u(l2_out) + "](ClippedReLU[" + u(l2_out) +
                       "](AffineTransform[" + u(l2_out) + "<-" + u(l2_in) + "](SqrClippedReLU[" + u(l2_in) +
                       "](AffineTransform[" + u(l1_out) + "<-" + F2 + "](InputSlice[" + F2 + "(0:" + F2 +
                       ")])))))";
    if (has_fv) arch += ",fv_scale=" + std::to_string(fv);

    HostBytes bias_stream, weight_stream;
    int32_t st;
    if ((st = quantise_leb128_to_host(ft_b, 127.0, bias_stream, stream))) return st;
    if ((st = quantise_leb128_to_host(ft, 127.0, weight_stream, stream))) return st;

    // head: header, FT bias block, FT weight block prefix; the weight stream
    // itself is written straight from its staging buffer
    Bytes head, w;
    head.u32(0x7AF32F21u);  // NNUE_VERSION
    head.u32(fc_hash ^ ft_hash);
    head.str(arch);
    head.u32(nb);
    head.u32(ft_hash);
    head.raw("COMPRESSED_LEB128", 17);
    head.u32((uint32_t)bias_stream.n);
    head.raw(bias_stream.p, bias_stream.n);
    head.raw("COMPRESSED_LEB128", 17);
    head.u32((uint32_t)weight_stream.n);
    w.b.reserve((size_t)nb * (l1_out * (ft_out + 64) + 4096));
    const uint64_t pin1 = (ft_out + 31) / 32 * 32, pin2 = (l2_in + 31) / 32 * 32, pin3 = (l2_out + 31) / 32 * 32;
    for (uint64_t b = 0; b < nb; ++b) {
        w.u32(fc_hash);
        for (uint64_t o = 0; o < l1_out; ++o) {
            const float merged = h.l1_b[b * l1_out + o] + h.l1s_b[o];
            w.i32(sat_cast<int32_t>(std::round(8128.0 * (double)merged)));
        }
        for (uint64_t o = 0; o < l1_out; ++o)
            for (uint64_t i = 0; i < pin1; ++i) {
                int8_t q = 0;
                if (i < ft_out) {
                    const float merged = h.l1_w[(b * l1_out + o) * ft_out + i] + h.l1s_w[i * l1_out + o];
                    q = ls_i8(64.0 * (double)merged);
                }
                w.u8((uint8_t)q);
            }
        for (uint64_t o = 0; o < l2_out; ++o)
            w.i32(sat_cast<int32_t>(std::round(8128.0 * (double)h.l2_b[b * l2_out + o])));
        for (uint64_t o = 0; o < l2_out; ++o)
            for (uint64_t i = 0; i < pin2; ++i)
                w.u8((uint8_t)(i < l2_in ? ls_i8(64.0 * (double)h.l2_w[(b * l2_out + o) * l2_in + i]) : 0));
        w.i32(sat_cast<int32_t>(std::round(8128.0 * (double)h.l3_b[b])));
        for (uint64_t i = 0; i < pin3; ++i)
            w.u8((uint8_t)(i < l2_out ? ls_i8(64.0 * (double)h.l3_w[b * l2_out + i]) : 0));
    }
    return write_file(path, {{head.b.data(), head.b.size()}, {weight_stream.p, weight_stream.n}, {w.b.data(), w.b.size()}});
}

int32_t write_simple_bin(const char* path, const ExportFeatureSet& fs, const QuantSource& ft,
                         const QuantSource& ft_b, uint32_t l1_out, uint32_t l2_out, const SimpleHost& h, int32_t fv,
                         hipStream_t stream) {
    const uint64_t ft_out = ft.cols;
    const uint64_t l1_in = 2 * ft_out;  // CReLU: both perspectives concatenated
    TATARA_REQUIRE(ft.rows == fs.ft_in && ft_b.rows * ft_b.cols == ft_out,
                   "Simple export: dimensions do not match the feature set");
    TATARA_REQUIRE(h.l1_w.size() == l1_in * l1_out && h.l1_b.size() == l1_out &&
                       h.l2_w.size() == (uint64_t)l1_out * l2_out && h.l2_b.size() == l2_out &&
                       h.l3_w.size() == l2_out && h.l3_b.size() == 1,
                   "Simple export: dense group sizes");
    const uint32_t ft_hash = fs.feature_hash ^ (uint32_t)(ft_out * 2);
    const uint32_t fc_hash = layer_hash_chain((uint32_t)l1_in, l1_out, l2_out);
    const std::string L = u(l1_in);
    const std::string arch = std::string("Features=") + fs.arch_name + "(Friend)[" + u(fs.ft_in) + "->" +
                             u(ft_out) + "x2],Network=AffineTransform[1<-" + u(l2_out) + "](ClippedReLU[" +
                             u(l2_out) + "](AffineTransform[" + u(l2_out) + "<-" + u(l1_out) + "](ClippedReLU[" +
                             u(l1_out) + "](AffineTransformSparseInput[" + u(l1_out) + "<-" + L + "](InputSlice[" +
                             L + "(0:" + L + ")])))))" + ",fv_scale=" + std::to_string(fv);

    HostBytes qb, qw;
    int32_t st;
    if ((st = quantise_i16_to_host(ft_b, 127.0, qb, stream))) return st;
    if ((st = quantise_i16_to_host(ft, 127.0, qw, stream))) return st;

    Bytes head, w;
    head.u32(0x7AF32F16u);  // NNUE_VERSION (YaneuraOu kVersion)
    head.u32(fc_hash ^ ft_hash);
    head.str(arch);
    head.u32(ft_hash);
    w.b.reserve(8192 + l1_out * (l1_in + 32));
    w.u32(fc_hash);
    const double bs = 127.0 * 64.0, ws = 64.0;
    auto pad = [](uint64_t x) { return (x + 31) / 32 * 32; };
    // L1: bias, then weights out-major from the in-major [l1_in][l1_out] table
    for (uint64_t o = 0; o < l1_out; ++o) w.i32(simple_q<int32_t>(bs * (double)h.l1_b[o]));
    for (uint64_t o = 0; o < l1_out; ++o)
        for (uint64_t i = 0; i < pad(l1_in); ++i)
            w.u8((uint8_t)(i < l1_in ? simple_q<int8_t>(ws * (double)h.l1_w[i * l1_out + o]) : 0));
    for (uint64_t o = 0; o < l2_out; ++o) w.i32(simple_q<int32_t>(bs * (double)h.l2_b[o]));
    for (uint64_t o = 0; o < l2_out; ++o)
        for (uint64_t i = 0; i < pad(l1_out); ++i)
            w.u8((uint8_t)(i < l1_out ? simple_q<int8_t>(ws * (double)h.l2_w[i * l2_out + o]) : 0));
    w.i32(simple_q<int32_t>(bs * (double)h.l3_b[0]));
    for (uint64_t i = 0; i < pad(l2_out); ++i)
        w.u8((uint8_t)(i < l2_out ? simple_q<int8_t>(ws * (double)h.l3_w[i]) : 0));
    // the i16 blocks are little-endian host order, written from the staging buffers
    return write_file(path, {{head.b.data(), head.b.size()}, {qb.p, qb.n}, {qw.p, qw.n}, {w.b.data(), w.b.size()}});
}

}  // namespace tatara
