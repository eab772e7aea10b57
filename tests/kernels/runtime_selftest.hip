// Kernels loaded by name through tatara_module_load_image /
// tatara_module_launch in tests/test_gpu_runtime.py.  Each takes its buffers
// as (device pointer, u64 length) pairs, the layout KernelArgs::push_slice
// gives them (crates/gpu-runtime/src/native_backend.rs:273-276), and checks
// every access against those lengths.
#include <hip/hip_runtime.h>

#include <cstdint>

// y[i] = a * x[i] + y[i]
extern "C" __global__ void selftest_axpy(float* y, uint64_t y_len, const float* x, uint64_t x_len, float a) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < y_len && i < x_len) y[i] = a * x[i] + y[i];
}

// out[r][c] = base + r * width + c over a 2-D grid of 2-D blocks
extern "C" __global__ void selftest_iota2d(uint32_t* out, uint64_t out_len, uint32_t width, uint32_t height,
                                           uint32_t base) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t r = blockIdx.y * blockDim.y + threadIdx.y;
    const uint64_t i = (uint64_t)r * width + c;
    if (c < width && r < height && i < out_len) out[i] = base + (uint32_t)i;
}

// Reverses each block-sized segment of `in` through dynamic LDS (one word
// per thread, so the launch passes blockDim.x * 4 shared bytes).
extern "C" __global__ void selftest_reverse_segments(uint32_t* out, uint64_t out_len, const uint32_t* in,
                                                     uint64_t in_len) {
    extern __shared__ uint32_t seg[];
    const uint32_t t = threadIdx.x, n = blockDim.x;
    const uint64_t i = (uint64_t)blockIdx.x * n + t;
    seg[t] = i < in_len ? in[i] : 0u;
    __syncthreads();
    const uint64_t j = (uint64_t)blockIdx.x * n + (n - 1 - t);
    if (j < out_len && (uint64_t)blockIdx.x * n + n <= in_len) out[j] = seg[t];
}
