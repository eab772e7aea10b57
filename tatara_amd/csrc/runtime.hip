// C ABI: error reporting, device runtime surface and kernel-level ops.
//
// The runtime calls mirror crates/gpu-runtime/src/lib.rs:50-126 and
// native_backend.rs:17-300 (DeviceBuffer, memset, synchronize, device
// queries); the op calls wrap one reference kernel family each so that tests
// can check them against the CPU oracle kernel by kernel, as
// bins/nnue_train/src/tests/gpu_cpu_equivalence_tests.rs does.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "../../include/tatara_hip.h"
#include "binsort.hpp"
#include "common.hpp"
#include "export.hpp"
#include "ft_kernels.hpp"
#include "psv_kernels.hpp"

namespace tatara {

namespace {
thread_local std::string g_last_error = "no error";
}

void set_error(const std::string& msg) { g_last_error = msg; }
const char* last_error() { return g_last_error.c_str(); }

int32_t hip_status(hipError_t e, const char* what) {
    std::string msg = "HIP error " + std::to_string((int)e) + ": " + hipGetErrorName(e) + ": " +
                      hipGetErrorString(e) + " [" + what + "]";
    set_error(msg);
    // The runtime keeps a failed call's error as the thread's last error
    // until it is read; the error is reported here, so it is cleared, and a
    // later launch check (hipGetLastError) sees only its own launch.
    (void)hipGetLastError();
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) return kErrOutOfMemory;
    return kErrHip;
}

// Scoped device allocation for the standalone ops.
struct DevScratch {
    void* p = nullptr;
    ~DevScratch() {
        if (p) (void)hipFree(p);
    }
    int32_t alloc(size_t bytes) {
        if (bytes == 0) bytes = 4;
        TATARA_HIP(hipMalloc(&p, bytes), "hipMalloc scratch");
        return kOk;
    }
    template <class T>
    T* as() {
        return static_cast<T*>(p);
    }
};

// row-major [rows][ft_out] -> chunk-major [ceil(ft_out/256)][rows][256]
template <typename T>
__global__ void to_chunk_major_kernel(const T* __restrict__ src, T* __restrict__ dst, uint64_t rows,
                                      uint32_t ft_out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * ft_out) return;
    const uint64_t r = i / ft_out;
    const uint32_t c = (uint32_t)(i - r * ft_out);
    dst[(uint64_t)(c / kDftChunk) * rows * kDftChunk + r * kDftChunk + c % kDftChunk] = src[i];
}

__global__ void copy_f4_kernel(const float4* __restrict__ src, float4* __restrict__ dst, uint64_t n4) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
        dst[i] = src[i];
}

}  // namespace tatara

using namespace tatara;

extern "C" {

const char* tatara_last_error(void) { return last_error(); }
const char* tatara_version(void) { return "tatara-mi355x 0.1.0 (gfx950)"; }

int32_t tatara_device_count(int32_t* count) {
    TATARA_REQUIRE(count, "count is null");
    int n = 0;
    TATARA_HIP(hipGetDeviceCount(&n), "hipGetDeviceCount");
    *count = n;
    return kOk;
}

int32_t tatara_set_device(int32_t device) {
    TATARA_HIP(hipSetDevice(device), "hipSetDevice");
    return kOk;
}

int32_t tatara_device_info(int32_t device, char* name, int32_t name_len, int32_t* cu_count) {
    hipDeviceProp_t prop;
    TATARA_HIP(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (name && name_len > 0) {
        std::strncpy(name, prop.gcnArchName, (size_t)name_len - 1);
        name[name_len - 1] = 0;
    }
    if (cu_count) *cu_count = prop.multiProcessorCount;
    return kOk;
}

int32_t tatara_malloc(void** ptr, uint64_t bytes) {
    TATARA_REQUIRE(ptr, "ptr is null");
    *ptr = nullptr;
    TATARA_HIP(hipMalloc(ptr, bytes ? bytes : 4), "hipMalloc");
    return kOk;
}

int32_t tatara_free(void* ptr) {
    if (ptr) TATARA_HIP(hipFree(ptr), "hipFree");
    return kOk;
}

int32_t tatara_memcpy_htod(void* dst, const void* src, uint64_t bytes) {
    if (bytes) TATARA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return kOk;
}

int32_t tatara_memcpy_dtoh(void* dst, const void* src, uint64_t bytes) {
    if (bytes) TATARA_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return kOk;
}

int32_t tatara_memset(void* dst, int32_t byte, uint64_t bytes) {
    if (bytes) TATARA_HIP(hipMemset(dst, byte, bytes), "hipMemset");
    return kOk;
}

int32_t tatara_synchronize(void) {
    TATARA_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return kOk;
}

int32_t tatara_op_copy(void* dst, const void* src, uint64_t bytes) {
    TATARA_REQUIRE(bytes % 16 == 0, "bytes must be a multiple of 16");
    const uint64_t n4 = bytes / 16;
    if (n4 == 0) return kOk;
    copy_f4_kernel<<<2048, 256, 0, 0>>>(static_cast<const float4*>(src), static_cast<float4*>(dst), n4);
    TATARA_LAUNCHED("copy_f4");
    TATARA_HIP(hipDeviceSynchronize(), "copy_f4");
    return kOk;
}

int32_t tatara_radam_step_size_denom(uint64_t step, float beta1, float beta2,
                                     float n_sma_threshold, float* step_size, int32_t* denom) {
    TATARA_REQUIRE(step >= 1, "step must be >= 1");
    TATARA_REQUIRE(step_size && denom, "null output");
    const float step_f = (float)step;
    const float beta2_t = std::pow(beta2, step_f);
    const float n_sma_max = 2.0f / (1.0f - beta2) - 1.0f;
    const float n_sma = n_sma_max - 2.0f * step_f * beta2_t / (1.0f - beta2_t);
    const float bc1 = 1.0f - std::pow(beta1, step_f);
    float ss;
    if (n_sma > n_sma_threshold) {
        const float p1 = (n_sma - 4.0f) / (n_sma_max - 4.0f);
        const float p2 = (n_sma - 2.0f) / n_sma;
        const float p3 = n_sma_max / (n_sma_max - 2.0f);
        ss = std::sqrt((1.0f - beta2_t) * p1 * p2 * p3) / bc1;
    } else {
        ss = 1.0f / bc1;
    }
    *step_size = ss;
    *denom = n_sma > n_sma_threshold ? 1 : 0;
    return kOk;
}

int32_t tatara_op_sparse_ft_forward(const float* weight, const int32_t* indices,
                                    const int32_t* nnz, float* out, uint32_t batch, uint32_t rows,
                                    uint32_t cols, uint32_t max_active) {
    TATARA_REQUIRE(rows % 8 == 0, "rows must be a multiple of 8");
    FtForwardArgs a{};
    a.mode = 0;
    a.W = weight;
    a.idx_stm = indices;
    a.idx_nstm = indices;
    a.nnz = nnz;
    a.out_stm = out;
    a.out_nstm = out;
    a.batch = batch;
    a.ft_out = rows;
    a.cols = cols;
    a.max_active = max_active;
    a.n_persp = 1;
    int32_t st = launch_ft_forward(a, 0);
    if (st) return st;
    TATARA_HIP(hipDeviceSynchronize(), "sparse_ft_forward");
    return kOk;
}

int32_t tatara_op_ft_forward_pairwise(const float* weight, const int32_t* stm_idx,
                                      const int32_t* nstm_idx, const int32_t* nnz,
                                      const float* bias, float* stm_out, float* nstm_out,
                                      float* combined, uint32_t batch, uint32_t ft_out,
                                      uint32_t cols, uint32_t max_active, uint32_t piece_inputs,
                                      float scale) {
    TATARA_REQUIRE(ft_out % 8 == 0, "ft_out must be a multiple of 8");
    DevScratch keys, sched, hist, bstart, bcount;
    int32_t* schedule = nullptr;
    if (piece_inputs > 0 && batch > 0) {
        uint32_t n_bins = ceil_div(cols, piece_inputs);
        if (n_bins > 128) n_bins = 128;
        int32_t st;
        if ((st = keys.alloc(2ull * batch)) || (st = sched.alloc(8ull * batch)) ||
            (st = hist.alloc(4ull * 2 * n_bins * binsort_tiles(2 * batch))) ||
            (st = bstart.alloc(4ull * (2 * n_bins + 1))) || (st = bcount.alloc(4ull * 2 * n_bins)))
            return st;
        st = launch_king_block_keys(stm_idx, nstm_idx, nnz, keys.as<uint8_t>(), batch, max_active,
                                    cols, piece_inputs, n_bins, 0);
        if (st) return st;
        BinSortArgs bs{};
        bs.keys = keys.as<uint8_t>();
        bs.n_items = 2 * batch;
        bs.n_bins = 2 * n_bins;
        bs.align = 1;
        bs.value_mod = batch;
        bs.hist = hist.as<uint32_t>();
        bs.bin_start = bstart.as<uint32_t>();
        bs.bin_count = bcount.as<uint32_t>();
        bs.out = sched.as<int32_t>();
        st = launch_binsort(bs, 0);
        if (st) return st;
        schedule = sched.as<int32_t>();
    }
    FtForwardArgs a{};
    a.mode = 1;
    a.W = weight;
    a.idx_stm = stm_idx;
    a.idx_nstm = nstm_idx;
    a.nnz = nnz;
    a.schedule = schedule;
    a.bias = bias;
    a.out_stm = stm_out;
    a.out_nstm = nstm_out;
    a.combined = combined;
    a.batch = batch;
    a.ft_out = ft_out;
    a.cols = cols;
    a.max_active = max_active;
    a.n_persp = 2;
    a.scale = scale;
    int32_t st = launch_ft_forward(a, 0);
    if (st) return st;
    TATARA_HIP(hipDeviceSynchronize(), "ft_forward_pairwise");
    return kOk;
}

int32_t tatara_op_ft_weight_grad(const float* dft, const int32_t* stm_idx,
                                 const int32_t* nstm_idx, const int32_t* nnz, float* grad,
                                 uint32_t batch, uint32_t ft_out, uint32_t cols,
                                 uint32_t max_active) {
    TATARA_REQUIRE(ft_out % 4 == 0, "ft_out must be a multiple of 4");
    TATARA_REQUIRE(max_active <= 64, "max_active must be <= 64");
    const uint64_t n_items = 2ull * batch * max_active;
    const uint32_t n_keys = 2 * cols + 1;
    DevScratch ki, vi, ko, vo, off, tmp;
    const size_t tb = occurrence_sort_temp_bytes(n_items, cols);
    int32_t st;
    if ((st = ki.alloc(4 * n_items)) || (st = vi.alloc(4 * n_items)) || (st = ko.alloc(4 * n_items)) ||
        (st = vo.alloc(4 * n_items)) || (st = off.alloc(4ull * (n_keys + 1))) || (st = tmp.alloc(tb)))
        return st;
    OccurrenceSortArgs os{};
    os.idx_stm = stm_idx;
    os.idx_nstm = nstm_idx;
    os.nnz = nnz;
    os.batch = batch;
    os.max_active = max_active;
    os.cols = cols;
    os.keys_in = ki.as<uint32_t>();
    os.vals_in = vi.as<uint32_t>();
    os.keys_out = ko.as<uint32_t>();
    os.vals_out = vo.as<uint32_t>();
    os.offsets = off.as<uint32_t>();
    os.temp = tmp.p;
    os.temp_bytes = tb;
    if ((st = launch_occurrence_sort(os, 0))) return st;
    FtGradArgs g{};
    g.dft = dft;
    g.dft_row_stride = ft_out;  // row-major [2][batch][ft_out]
    g.dft_chunk_stride = kDftChunk;
    g.occ_vals = vo.as<uint32_t>();
    g.occ_off = off.as<uint32_t>();
    g.grad = grad;
    g.ft_out = ft_out;
    g.rows = cols;
    g.apply_update = 0;
    if ((st = launch_ft_grad_update(g, 0))) return st;
    TATARA_HIP(hipDeviceSynchronize(), "ft_weight_grad");
    return kOk;
}

static int32_t ft_weight_grad_blocked(const float* dft, const uint16_t* dft16, float inv_scale,
                                      const int32_t* stm_idx, const int32_t* nstm_idx, const int32_t* nnz,
                                      float* grad, uint32_t batch, uint32_t ft_out, uint32_t cols,
                                      uint32_t max_active, uint32_t piece_inputs, uint32_t* used_block_scan,
                                      bool mfma = false) {
    TATARA_REQUIRE(ft_out % 4 == 0, "ft_out must be a multiple of 4");
    TATARA_REQUIRE(max_active <= 64, "max_active must be <= 64");
    TATARA_REQUIRE(ft_scan_mask_words(piece_inputs) > 0, "piece_inputs out of range for the block scan");
    int32_t st;
    uint32_t n_blocks = ceil_div(cols, piece_inputs);
    if (n_blocks > 128) n_blocks = 128;
    const uint64_t two_b = 2ull * batch;
    const uint32_t chunks = ceil_div(ft_out, kDftChunk);
    // king-block schedule, as the trainer builds it for the forward
    DevScratch keys, sched, hist, start, count, cm, multi, srows, smasks;
    const uint64_t stages = ft_scan_max_stages(batch, n_blocks);
    if ((st = keys.alloc(two_b)) || (st = sched.alloc(4 * two_b)) ||
        (st = hist.alloc(4ull * 2 * n_blocks * binsort_tiles((uint32_t)two_b))) ||
        (st = start.alloc(4ull * (2 * n_blocks + 1))) || (st = count.alloc(4ull * 2 * n_blocks)) ||
        (st = cm.alloc(4ull * chunks * two_b * kDftChunk)) ||
        (st = multi.alloc(4)) || (st = srows.alloc(4ull * stages * 32)) ||
        (st = smasks.alloc(4ull * stages * ft_scan_mask_words(piece_inputs) * 16)))
        return st;
    if ((st = launch_king_block_keys(stm_idx, nstm_idx, nnz, keys.as<uint8_t>(), batch, max_active, cols,
                                     piece_inputs, n_blocks, 0)))
        return st;
    BinSortArgs bs{};
    bs.keys = keys.as<uint8_t>();
    bs.n_items = (uint32_t)two_b;
    bs.n_bins = 2 * n_blocks;
    bs.align = 1;
    bs.value_mod = batch;
    bs.hist = hist.as<uint32_t>();
    bs.bin_start = start.as<uint32_t>();
    bs.bin_count = count.as<uint32_t>();
    bs.out = sched.as<int32_t>();
    if ((st = launch_binsort(bs, 0))) return st;
    if (two_b * ft_out > 0) {
        if (dft16)
            to_chunk_major_kernel<<<ceil_div(two_b * ft_out, 256), 256>>>(dft16, cm.as<uint16_t>(), two_b, ft_out);
        else
            to_chunk_major_kernel<<<ceil_div(two_b * ft_out, 256), 256>>>(dft, cm.as<float>(), two_b, ft_out);
        TATARA_LAUNCHED("to_chunk_major");
    }
    FtBlockScan sc{};
    sc.idx_stm = stm_idx;
    sc.idx_nstm = nstm_idx;
    sc.nnz = nnz;
    sc.schedule = sched.as<int32_t>();
    sc.sched_start = start.as<uint32_t>();
    sc.multi = multi.as<uint32_t>();
    sc.stage_rows = srows.as<uint32_t>();
    sc.stage_masks = smasks.as<uint32_t>();
    sc.batch = batch;
    sc.max_active = max_active;
    sc.cols = cols;
    sc.piece_inputs = piece_inputs;
    sc.n_blocks = n_blocks;
    sc.dealt = mfma ? 0u : 1u;
    if ((st = launch_ft_scan_tables(sc, 0))) return st;
    // occurrence lists for the fallback (a row with features of two blocks)
    const uint64_t n_items = two_b * max_active;
    const uint32_t n_keys = 2 * cols + 1;
    DevScratch ki, vi, ko, vo, off, tmp;
    const size_t tb = occurrence_sort_temp_bytes(n_items, cols);
    if ((st = ki.alloc(4 * n_items)) || (st = vi.alloc(4 * n_items)) || (st = ko.alloc(4 * n_items)) ||
        (st = vo.alloc(4 * n_items)) || (st = off.alloc(4ull * (n_keys + 1))) || (st = tmp.alloc(tb)))
        return st;
    OccurrenceSortArgs os{};
    os.idx_stm = stm_idx;
    os.idx_nstm = nstm_idx;
    os.nnz = nnz;
    os.batch = batch;
    os.max_active = max_active;
    os.cols = cols;
    os.keys_in = ki.as<uint32_t>();
    os.vals_in = vi.as<uint32_t>();
    os.keys_out = ko.as<uint32_t>();
    os.vals_out = vo.as<uint32_t>();
    os.offsets = off.as<uint32_t>();
    os.temp = tmp.p;
    os.temp_bytes = tb;
    if ((st = launch_occurrence_sort(os, 0))) return st;
    FtGradArgs g{};
    if (dft16) {
        g.dft16 = cm.as<uint16_t>();
        g.dft_inv_scale = inv_scale;
    } else {
        g.dft = cm.as<float>();
    }
    g.dft_row_stride = kDftChunk;
    g.dft_chunk_stride = two_b * kDftChunk;
    g.occ_vals = vo.as<uint32_t>();
    g.occ_off = off.as<uint32_t>();
    g.grad = grad;
    g.ft_out = ft_out;
    g.rows = cols;
    g.apply_update = 0;
    if ((st = mfma ? launch_ft_grad_mfma(g, sc, 0) : launch_ft_grad_scan(g, sc, 0))) return st;
    uint32_t m = 0;
    TATARA_HIP(hipMemcpy(&m, multi.p, 4, hipMemcpyDeviceToHost), "ft_weight_grad_blocked");
    if (used_block_scan) *used_block_scan = m ? 0u : 1u;
    return kOk;
}

int32_t tatara_op_ft_weight_grad_blocked(const float* dft, const int32_t* stm_idx, const int32_t* nstm_idx,
                                         const int32_t* nnz, float* grad, uint32_t batch, uint32_t ft_out,
                                         uint32_t cols, uint32_t max_active, uint32_t piece_inputs,
                                         uint32_t* used_block_scan) {
    return ft_weight_grad_blocked(dft, nullptr, 1.0f, stm_idx, nstm_idx, nnz, grad, batch, ft_out, cols,
                                  max_active, piece_inputs, used_block_scan);
}

int32_t tatara_op_ft_weight_grad_blocked_f16(const uint16_t* dft16, float dft_inv_scale, const int32_t* stm_idx,
                                             const int32_t* nstm_idx, const int32_t* nnz, float* grad,
                                             uint32_t batch, uint32_t ft_out, uint32_t cols,
                                             uint32_t max_active, uint32_t piece_inputs,
                                             uint32_t* used_block_scan) {
    return ft_weight_grad_blocked(nullptr, dft16, dft_inv_scale, stm_idx, nstm_idx, nnz, grad, batch, ft_out,
                                  cols, max_active, piece_inputs, used_block_scan);
}

int32_t tatara_op_ft_weight_grad_mfma_f16(const uint16_t* dft16, float dft_inv_scale, const int32_t* stm_idx,
                                          const int32_t* nstm_idx, const int32_t* nnz, float* grad, uint32_t batch,
                                          uint32_t ft_out, uint32_t cols, uint32_t max_active,
                                          uint32_t piece_inputs, uint32_t* used_matrix_cores) {
    return ft_weight_grad_blocked(nullptr, dft16, dft_inv_scale, stm_idx, nstm_idx, nnz, grad, batch, ft_out,
                                  cols, max_active, piece_inputs, used_matrix_cores, true);
}

int32_t tatara_op_ft_fold_virtual(const float* weight, float* comb, uint32_t ft_in,
                                  uint32_t ft_out, uint32_t piece_inputs) {
    int32_t st = launch_ft_fold(weight, comb, nullptr, ft_in, ft_out, piece_inputs, 0);
    if (st) return st;
    TATARA_HIP(hipDeviceSynchronize(), "ft_fold_virtual");
    return kOk;
}

int32_t tatara_op_ft_reduce_virtual_grad(float* grad, uint32_t ft_in, uint32_t ft_out,
                                         uint32_t piece_inputs) {
    int32_t st = launch_ft_reduce(grad, ft_in, ft_out, piece_inputs, 0);
    if (st) return st;
    TATARA_HIP(hipDeviceSynchronize(), "ft_reduce_virtual_grad");
    return kOk;
}

int32_t tatara_op_radam_step(float* weights, float* m, float* v, float* grad, float lr,
                             float step_size, int32_t denom, float decay, float beta1,
                             float beta2, float eps, float min_w, float max_w, uint64_t n) {
    OptScalars s{lr, step_size, denom, decay, beta1, beta2, eps, min_w, max_w, 0, 0.0f};
    int32_t st = launch_radam(weights, m, v, grad, nullptr, n, s, 0);
    if (st) return st;
    TATARA_HIP(hipDeviceSynchronize(), "radam_step");
    return kOk;
}

int32_t tatara_op_ranger_lookahead_lerp(float* weights, float* slow, float alpha, uint64_t n) {
    int32_t st = launch_lerp(weights, slow, n, alpha, 0);
    if (st) return st;
    TATARA_HIP(hipDeviceSynchronize(), "ranger_lookahead_lerp");
    return kOk;
}

int32_t tatara_op_expf(const float* x, float* y, uint64_t n) {
    int32_t st = launch_expf(x, y, n, 0);
    if (st) return st;
    TATARA_HIP(hipDeviceSynchronize(), "expf");
    return kOk;
}

int32_t tatara_op_quantise_ft(const float* w, uint64_t rows, uint32_t cols, uint32_t piece_inputs,
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
        TATARA_HIP(hipDeviceSynchronize(), "quantise_ft");
        *out_bytes = 2 * n;
        return kOk;
    }
    const uint64_t tiles = leb128_tiles(n);
    uint32_t* tile_bytes = nullptr;
    uint64_t* tile_off = nullptr;  // tile offsets, then the total in the last slot
    TATARA_HIP(hipMalloc(&tile_bytes, (tiles + 1) * sizeof(uint32_t)), "hipMalloc quantise_ft");
    hipError_t e = hipMalloc(&tile_off, (tiles + 1) * sizeof(uint64_t));
    int32_t st = kOk;
    uint64_t total = 0;
    if (e == hipSuccess) st = launch_quantise_leb128(src, scale, tile_bytes, tile_off, tile_off + tiles, nullptr, 0);
    if (e == hipSuccess && st == kOk)
        e = hipMemcpy(&total, tile_off + tiles, sizeof total, hipMemcpyDeviceToHost);
    if (e == hipSuccess && st == kOk && total > out_capacity) {
        set_error("invalid argument: out_capacity is smaller than the LEB128 stream");
        st = kErrInvalid;
    }
    if (e == hipSuccess && st == kOk && total)
        st = launch_quantise_leb128(src, scale, tile_bytes, tile_off, tile_off + tiles, out, 0);
    if (e == hipSuccess && st == kOk) e = hipDeviceSynchronize();
    (void)hipFree(tile_off);
    (void)hipFree(tile_bytes);
    if (st) return st;
    TATARA_HIP(e, "quantise_ft");
    *out_bytes = total;
    return kOk;
}

int32_t tatara_feature_set_info(int32_t feature_set, int32_t* king_buckets, int32_t* piece_inputs,
                                int32_t* ft_in, int32_t* max_active, uint32_t* feature_hash) {
    FeatureSetShape s;
    int32_t st = feature_set_shape(feature_set, s);
    if (st) return st;
    if (king_buckets) *king_buckets = s.king_buckets;
    if (piece_inputs) *piece_inputs = s.piece_inputs;
    if (ft_in) *ft_in = s.king_buckets * s.piece_inputs;
    if (max_active) *max_active = s.max_active;
    if (feature_hash) *feature_hash = s.feature_hash;
    return kOk;
}

int32_t tatara_psv_to_batch(const uint8_t* psv, int32_t n, int32_t feature_set, int32_t bucket_mode,
                            int32_t num_buckets, const float* progress_weights, int32_t* stm_indices,
                            int32_t* nstm_indices, int32_t* nnz, int32_t* bucket_idx, float* score,
                            float* wdl) {
    TATARA_REQUIRE(n >= 0, "n must be >= 0");
    TATARA_REQUIRE(n == 0 || (psv && stm_indices && nstm_indices && nnz && score && wdl), "null argument");
    FeatureSetShape s;
    int32_t st = feature_set_shape(feature_set, s);
    if (st) return st;
    PsvArgs a{};
    a.psv = psv;
    a.n = (uint32_t)n;
    a.piece_inputs = s.piece_inputs;
    a.max_active = s.max_active;
    a.emit_king = s.emit_king;
    a.fold_enemy = s.fold_enemy;
    a.mirror = s.mirror;
    a.bucket_mode = bucket_mode;
    a.num_buckets = num_buckets;
    a.weights = progress_weights;
    a.stm = stm_indices;
    a.nstm = nstm_indices;
    a.nnz = nnz;
    a.bucket = bucket_idx;
    a.score = score;
    a.wdl = wdl;
    a.progress = nullptr;
    if ((st = launch_psv_to_batch(a, 0))) return st;
    TATARA_HIP(hipDeviceSynchronize(), "psv_to_batch");
    return kOk;
}

}  // extern "C"
