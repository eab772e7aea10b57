// CPU oracle for the tatara training-step hot path.
//
// TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP product
// path (tatara_amd/) is compared against.  Only tests/, __graft_entry__.smoke()
// and bench.py's cpu_baseline leg may load it; the product never links it.
//
// Every function restates one of the reference's CPU reference kernels
// (crates/gpu-kernels/src/**) or host helpers, in the same loop order and the
// same floating-point expression order.  The file is compiled with
// -ffp-contract=off so that a*b+c is never fused, which matches Rust's default
// (no contraction), so sequential loops are bit-identical to the reference.
// Transcendentals call glibc expf/powf/sqrtf, the same routines Rust's f32
// methods lower to on linux-gnu.
//
// OpenMP is used only across outputs that are independent in the reference
// loop nest (rows of a forward, columns of a scatter, elements of an
// optimizer pass), so every output keeps its reference summation order and
// the result does not depend on the thread count.
//
// Parity pins (see tests/test_oracle_kat.py): every function below is checked
// against the known-answer tests that the reference holds for it, plus
// closed forms / brute force where the reference has none.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

extern "C" {

// ---------------------------------------------------------------------------
// threads
// ---------------------------------------------------------------------------

int orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

// ---------------------------------------------------------------------------
// sparse FT
// ---------------------------------------------------------------------------

// crates/gpu-kernels/src/sparse/sparse_ft_forward.rs:100-122
// out[bi*rows+ri] = sum over ni < nnz[bi] of weight[idx*rows+ri] (idx valid),
// summed from 0.0 in ni order.
void orc_sparse_ft_forward(const float* weight, const int32_t* indices, const int32_t* nnz_arr,
                           float* out, int64_t batch, int64_t rows, int64_t cols,
                           int64_t max_active) {
#pragma omp parallel for schedule(static)
    for (int64_t bi = 0; bi < batch; ++bi) {
        const int32_t* idx_row = indices + bi * max_active;
        const int64_t n = nnz_arr[bi];
        float* o = out + bi * rows;
        for (int64_t ri = 0; ri < rows; ++ri) o[ri] = 0.0f;
        // Same per-(bi, ri) sum order as the reference: ni ascending.  The
        // ri loop is inside so that each row of `weight` streams once.
        for (int64_t ni = 0; ni < n; ++ni) {
            const int32_t idx = idx_row[ni];
            if (idx >= 0 && (int64_t)idx < cols) {
                const float* w = weight + (int64_t)idx * rows;
                for (int64_t ri = 0; ri < rows; ++ri) o[ri] += w[ri];
            }
        }
    }
}

// crates/gpu-kernels/src/sparse/sparse_ft_backward.rs:247-267 (accumulate into
// grad_weight; every one of the `nnz` slots of a row is visited and invalid
// indices are skipped).  Order per cell: bi ascending, ni ascending.
// Parallel over column ranges only, so each cell keeps that order.
void orc_sparse_ft_backward(const float* grad_out, const int32_t* indices, float* grad_weight,
                            int64_t batch, int64_t rows, int64_t cols, int64_t nnz) {
#pragma omp parallel
    {
#ifdef _OPENMP
        const int nt = omp_get_num_threads();
        const int t = omp_get_thread_num();
#else
        const int nt = 1, t = 0;
#endif
        const int64_t r0 = rows * t / nt, r1 = rows * (t + 1) / nt;
        for (int64_t bi = 0; bi < batch; ++bi) {
            const float* g = grad_out + bi * rows;
            for (int64_t ni = 0; ni < nnz; ++ni) {
                const int32_t idx = indices[bi * nnz + ni];
                if (idx >= 0 && (int64_t)idx < cols) {
                    float* gw = grad_weight + (int64_t)idx * rows;
                    for (int64_t ri = r0; ri < r1; ++ri) gw[ri] += g[ri];
                }
            }
        }
    }
}

// gather_and_sum_per_feature_{overwrite,add}_fp16
// (crates/cuda-native-runtime/kernels/native_kernels.cu:1030-1100) on the
// per-feature position lists of the trainer's backward (slots < nnz, indices
// in [0, cols), one entry per occurrence).  The reference fills those lists
// with atomics, so their order is unspecified; ascending position order is
// used here.  dft16 holds the f16 activation gradients (scaled) as f32
// values.  Per cell: four interleaved f32 partial sums, combined as
// (s0 + s1) + (s2 + s3), times inv_scale; add = 0 overwrites every real
// feature's cell, add = 1 adds the scaled sum when the sum is nonzero.
void orc_ft_grad_fp16(const float* dft16, const int32_t* indices, const int32_t* nnz_arr,
                      float* grad_weight, int64_t batch, int64_t rows, int64_t cols, int64_t max_active,
                      float inv_scale, int32_t add) {
    std::vector<int64_t> count(cols + 1, 0);
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t ni = 0; ni < nnz_arr[bi]; ++ni) {
            const int32_t idx = indices[bi * max_active + ni];
            if (idx >= 0 && (int64_t)idx < cols) ++count[idx + 1];
        }
    for (int64_t f = 0; f < cols; ++f) count[f + 1] += count[f];
    std::vector<int64_t> fill(count.begin(), count.end() - 1);
    std::vector<int64_t> pos(count[cols]);
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t ni = 0; ni < nnz_arr[bi]; ++ni) {
            const int32_t idx = indices[bi * max_active + ni];
            if (idx >= 0 && (int64_t)idx < cols) pos[fill[idx]++] = bi;
        }
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t f = 0; f < cols; ++f) {
        const int64_t start = count[f], end = count[f + 1];
        const int64_t unroll_end = end >= start + 3 ? end - 3 : start;
        for (int64_t r = 0; r < rows; ++r) {
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
            int64_t i = start;
            while (i < unroll_end) {
                s0 += dft16[pos[i] * rows + r];
                s1 += dft16[pos[i + 1] * rows + r];
                s2 += dft16[pos[i + 2] * rows + r];
                s3 += dft16[pos[i + 3] * rows + r];
                i += 4;
            }
            while (i < end) {
                s0 += dft16[pos[i] * rows + r];
                ++i;
            }
            const float sum = (s0 + s1) + (s2 + s3);
            const float scaled = sum * inv_scale;
            float& g = grad_weight[f * rows + r];
            if (add) {
                if (sum != 0.0f) g += scaled;
            } else {
                g = scaled;
            }
        }
    }
}

// The trainer-level variant of the backward: slots at or beyond nnz[bi] are
// ignored, as build_feature_counts / scatter_positions do in the reference
// trainer (crates/cuda-native-runtime/kernels/native_kernels.cu:1630-1765).
// Same per-cell order as orc_sparse_ft_backward.
void orc_sparse_ft_backward_nnz(const float* grad_out, const int32_t* indices,
                                const int32_t* nnz_arr, float* grad_weight, int64_t batch,
                                int64_t rows, int64_t cols, int64_t max_active) {
#pragma omp parallel
    {
#ifdef _OPENMP
        const int nt = omp_get_num_threads();
        const int t = omp_get_thread_num();
#else
        const int nt = 1, t = 0;
#endif
        const int64_t r0 = rows * t / nt, r1 = rows * (t + 1) / nt;
        for (int64_t bi = 0; bi < batch; ++bi) {
            const float* g = grad_out + bi * rows;
            const int64_t n = nnz_arr[bi];
            for (int64_t ni = 0; ni < n; ++ni) {
                const int32_t idx = indices[bi * max_active + ni];
                if (idx >= 0 && (int64_t)idx < cols) {
                    float* gw = grad_weight + (int64_t)idx * rows;
                    for (int64_t ri = r0; ri < r1; ++ri) gw[ri] += g[ri];
                }
            }
        }
    }
}

// crates/gpu-kernels/src/sparse/ft_factorize.rs (ft_fold_virtual_cpu), Base
// mode, no threat rows: comb[f][c] = w[f][c] + w[ft_in + f % piece_inputs][c].
void orc_ft_fold_virtual(const float* w, float* comb, int64_t ft_in, int64_t ft_out,
                         int64_t piece_inputs) {
#pragma omp parallel for schedule(static)
    for (int64_t f = 0; f < ft_in; ++f) {
        const float* real = w + f * ft_out;
        const float* virt = w + (ft_in + f % piece_inputs) * ft_out;
        float* c = comb + f * ft_out;
        for (int64_t ri = 0; ri < ft_out; ++ri) c[ri] = real[ri] + virt[ri];
    }
}

// crates/gpu-kernels/src/sparse/ft_factorize.rs (ft_reduce_virtual_grad_cpu),
// Base mode: grad[ft_in+v][c] = sum over features f (ascending) with
// f % piece_inputs == v of grad[f][c], summed from 0.0 (overwrite).
void orc_ft_reduce_virtual_grad(float* grad, int64_t ft_in, int64_t ft_out,
                                int64_t piece_inputs) {
#pragma omp parallel for schedule(static)
    for (int64_t v = 0; v < piece_inputs; ++v) {
        float* dst = grad + (ft_in + v) * ft_out;
        std::vector<float> sum(ft_out, 0.0f);
        for (int64_t f = v; f < ft_in; f += piece_inputs) {
            const float* g = grad + f * ft_out;
            for (int64_t ri = 0; ri < ft_out; ++ri) sum[ri] += g[ri];
        }
        for (int64_t ri = 0; ri < ft_out; ++ri) dst[ri] = sum[ri];
    }
}

// ---------------------------------------------------------------------------
// FT post (pairwise CReLU product)
// ---------------------------------------------------------------------------

static inline float crelu01(float x) { return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x); }

// crates/gpu-kernels/src/layerstack/ft_post_perspective.rs (fwd)
void orc_ft_post_perspective_fwd(const float* stm, const float* nstm, const float* bias,
                                 float* combined, int64_t batch, int64_t ft_dim, float scale) {
    const int64_t half = ft_dim / 2;
#pragma omp parallel for schedule(static)
    for (int64_t bi = 0; bi < batch; ++bi) {
        const int64_t base = bi * ft_dim;
        for (int64_t ri = 0; ri < ft_dim; ++ri) {
            float val;
            if (ri < half) {
                const float xa = stm[base + ri] + bias[ri];
                const float xb = stm[base + half + ri] + bias[half + ri];
                val = crelu01(xa) * crelu01(xb) * scale;
            } else {
                const int64_t p = ri - half;
                const float xa = nstm[base + p] + bias[p];
                const float xb = nstm[base + half + p] + bias[half + p];
                val = crelu01(xa) * crelu01(xb) * scale;
            }
            combined[base + ri] = val;
        }
    }
}

// crates/gpu-kernels/src/layerstack/ft_post_perspective.rs (grad).  grad_bias
// accumulates in (bi, ii) order; the row loop is therefore serial.
void orc_ft_post_perspective_grad(const float* d_combined, const float* ft_out, const float* bias,
                                  float* grad_ft_out, float* grad_bias, int64_t batch,
                                  int64_t ft_dim, int64_t d_off, int64_t d_stride, float scale) {
    const int64_t half = ft_dim / 2;
#pragma omp parallel for schedule(static)
    for (int64_t bi = 0; bi < batch; ++bi) {
        const int64_t base = bi * ft_dim;
        for (int64_t ii = 0; ii < ft_dim; ++ii) {
            const bool first = ii < half;
            const int64_t p = first ? ii : ii - half;
            const float dy = d_combined[bi * d_stride + d_off + p];
            const float xa = ft_out[base + p] + bias[p];
            const float xb = ft_out[base + half + p] + bias[half + p];
            const float ya = crelu01(xa), yb = crelu01(xb);
            const float my_pre = first ? xa : xb;
            const float partner = first ? yb : ya;
            const float g_post = dy * partner * scale;
            grad_ft_out[base + ii] = (my_pre > 0.0f && my_pre < 1.0f) ? g_post : 0.0f;
        }
    }
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t ii = 0; ii < ft_dim; ++ii) grad_bias[ii] += grad_ft_out[bi * ft_dim + ii];
}

// ---------------------------------------------------------------------------
// dense layers (crates/gpu-kernels/src/layerstack/dense_mm.rs)
// w layout: [in_dim][out_dim]
// ---------------------------------------------------------------------------

void orc_dense_mm_fwd(const float* x, const float* w, const float* bias, float* y, int64_t batch,
                      int64_t in_dim, int64_t out_dim) {
#pragma omp parallel for schedule(static)
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t oi = 0; oi < out_dim; ++oi) {
            float sum = bias[oi];
            for (int64_t k = 0; k < in_dim; ++k) sum += x[bi * in_dim + k] * w[k * out_dim + oi];
            y[bi * out_dim + oi] = sum;
        }
}

void orc_dense_mm_bwd_input(const float* dy, const float* w, float* dx, int64_t batch,
                            int64_t in_dim, int64_t out_dim) {
#pragma omp parallel for schedule(static)
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t ii = 0; ii < in_dim; ++ii) {
            float sum = 0.0f;
            for (int64_t o = 0; o < out_dim; ++o) sum += dy[bi * out_dim + o] * w[ii * out_dim + o];
            dx[bi * in_dim + ii] = sum;
        }
}

void orc_dense_mm_bwd_weight(const float* x, const float* dy, float* grad_w, int64_t batch,
                             int64_t in_dim, int64_t out_dim) {
#pragma omp parallel for schedule(static)
    for (int64_t ii = 0; ii < in_dim; ++ii)
        for (int64_t oi = 0; oi < out_dim; ++oi) {
            float sum = 0.0f;
            for (int64_t b = 0; b < batch; ++b) sum += x[b * in_dim + ii] * dy[b * out_dim + oi];
            grad_w[ii * out_dim + oi] = sum;
        }
}

void orc_bias_grad(const float* dy, float* grad_bias, int64_t batch, int64_t out_dim) {
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t oi = 0; oi < out_dim; ++oi) grad_bias[oi] += dy[bi * out_dim + oi];
}

// ---------------------------------------------------------------------------
// per-bucket dense layers (crates/gpu-kernels/src/layerstack/dense_mm_bucket.rs)
// w layout: [num_buckets][out_dim][in_dim]
// ---------------------------------------------------------------------------

void orc_dense_mm_fwd_bucket(const float* x, const float* w, const float* bias,
                             const int32_t* bucket_idx, float* y, int64_t batch, int64_t in_dim,
                             int64_t out_dim, int64_t num_buckets) {
#pragma omp parallel for schedule(static)
    for (int64_t bi = 0; bi < batch; ++bi) {
        const int32_t buc = bucket_idx[bi];
        if (buc < 0 || (int64_t)buc >= num_buckets) {
            for (int64_t oi = 0; oi < out_dim; ++oi) y[bi * out_dim + oi] = 0.0f;
            continue;
        }
        const int64_t g = buc;
        for (int64_t oi = 0; oi < out_dim; ++oi) {
            const int64_t wb = g * out_dim * in_dim + oi * in_dim;
            float sum = bias[g * out_dim + oi];
            for (int64_t k = 0; k < in_dim; ++k) sum += x[bi * in_dim + k] * w[wb + k];
            y[bi * out_dim + oi] = sum;
        }
    }
}

void orc_dense_mm_bwd_input_bucket(const float* dy, const float* w, const int32_t* bucket_idx,
                                   float* dx, int64_t batch, int64_t in_dim, int64_t out_dim,
                                   int64_t num_buckets) {
#pragma omp parallel for schedule(static)
    for (int64_t bi = 0; bi < batch; ++bi) {
        const int32_t buc = bucket_idx[bi];
        if (buc < 0 || (int64_t)buc >= num_buckets) {
            for (int64_t ii = 0; ii < in_dim; ++ii) dx[bi * in_dim + ii] = 0.0f;
            continue;
        }
        const int64_t g = buc;
        for (int64_t ii = 0; ii < in_dim; ++ii) {
            float sum = 0.0f;
            for (int64_t o = 0; o < out_dim; ++o)
                sum += dy[bi * out_dim + o] * w[g * out_dim * in_dim + o * in_dim + ii];
            dx[bi * in_dim + ii] = sum;
        }
    }
}

void orc_dense_mm_bwd_weight_bucket(const float* x, const float* dy, const int32_t* bucket_idx,
                                    float* grad_w, int64_t batch, int64_t in_dim, int64_t out_dim,
                                    int64_t num_buckets) {
    const int64_t per_bucket = out_dim * in_dim;
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t g = 0; g < num_buckets; ++g)
        for (int64_t oi = 0; oi < out_dim; ++oi)
            for (int64_t ii = 0; ii < in_dim; ++ii) {
                float sum = 0.0f;
                for (int64_t b = 0; b < batch; ++b)
                    if (bucket_idx[b] == (int32_t)g) sum += x[b * in_dim + ii] * dy[b * out_dim + oi];
                grad_w[g * per_bucket + oi * in_dim + ii] = sum;
            }
}

void orc_bias_grad_bucket(const float* dy, const int32_t* bucket_idx, float* grad_bias,
                          int64_t batch, int64_t out_dim, int64_t num_buckets) {
    for (int64_t bi = 0; bi < batch; ++bi) {
        const int32_t buc = bucket_idx[bi];
        if (buc < 0 || (int64_t)buc >= num_buckets) continue;
        for (int64_t oi = 0; oi < out_dim; ++oi) grad_bias[buc * out_dim + oi] += dy[bi * out_dim + oi];
    }
}

// ---------------------------------------------------------------------------
// pointwise layerstack glue
// ---------------------------------------------------------------------------

// crates/gpu-kernels/src/layerstack/crelu.rs
void orc_crelu_fwd(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = crelu01(x[i]);
}
void orc_crelu_grad(const float* x, const float* dy, float* dx, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dx[i] = (x[i] > 0.0f && x[i] < 1.0f) ? dy[i] : 0.0f;
}
// crates/gpu-kernels/src/layerstack/abs_pow2_scale.rs
void orc_abs_pow2_scale_fwd(const float* x, float* y, float scale, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] * x[i] * scale;
}
void orc_abs_pow2_scale_grad(const float* x, const float* dy, float* dx, float scale, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dx[i] = 2.0f * x[i] * scale * dy[i];
}
// crates/gpu-kernels/src/layerstack/concat_l1sqr_main.rs
void orc_concat_l1sqr_main_fwd(const float* a, const float* b, float* out, int64_t batch,
                               int64_t a_dim, int64_t b_dim) {
    const int64_t od = a_dim + b_dim;
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t oi = 0; oi < od; ++oi)
            out[bi * od + oi] = oi < a_dim ? a[bi * a_dim + oi] : b[bi * b_dim + (oi - a_dim)];
}
void orc_concat_l1sqr_main_grad(const float* dout, float* da, float* db, int64_t batch,
                                int64_t dim) {
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t ii = 0; ii < dim; ++ii) {
            da[bi * dim + ii] = dout[bi * 2 * dim + ii];
            db[bi * dim + ii] = dout[bi * 2 * dim + dim + ii];
        }
}
// crates/gpu-kernels/src/layerstack/elementwise.rs
void orc_elementwise_add(const float* a, const float* b, float* c, int64_t n) {
    for (int64_t i = 0; i < n; ++i) c[i] = a[i] + b[i];
}
// crates/gpu-kernels/src/layerstack/slice2d.rs
void orc_slice_extract_2d(const float* src, float* dst, int64_t batch, int64_t src_stride,
                          int64_t src_offset, int64_t out_dim) {
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t oi = 0; oi < out_dim; ++oi)
            dst[bi * out_dim + oi] = src[bi * src_stride + src_offset + oi];
}
void orc_slice_scatter_2d(const float* src, float* dst, int64_t batch, int64_t in_dim,
                          int64_t dst_stride, int64_t dst_offset) {
    for (int64_t bi = 0; bi < batch; ++bi)
        for (int64_t ii = 0; ii < in_dim; ++ii)
            dst[bi * dst_stride + dst_offset + ii] = src[bi * in_dim + ii];
}

// ---------------------------------------------------------------------------
// losses
// ---------------------------------------------------------------------------

static inline float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// crates/gpu-kernels/src/pointwise/loss_wdl.rs (loss_wdl_cpu); per_pos_norm is
// the per-position array the reference takes (the trainer broadcasts 1/b).
void orc_loss_wdl(const float* out, const float* score, const float* wdl,
                  const float* per_pos_norm, float* dl_dout, double* loss_acc, float lambda,
                  float scale, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float p = sigmoid_f32(out[i] * scale);
        const float ys = sigmoid_f32(score[i] * scale);
        const float y = lambda * wdl[i] + (1.0f - lambda) * ys;
        const float err = p - y;
        const float norm = per_pos_norm[i];
        *loss_acc += (double)err * (double)err;
        dl_dout[i] = 2.0f * err * p * (1.0f - p) * scale * norm;
    }
}

static float wrm_weight(float score, float t_off, float t_scale, float w1, float w2) {
    const float pt = (score - t_off) / t_scale;
    const float pmt = (-score - t_off) / t_scale;
    const float pf = 0.5f * (1.0f + sigmoid_f32(pt) - sigmoid_f32(pmt));
    const float wb = (pf - 0.5f) * (pf - 0.5f) * pf * (1.0f - pf);
    return 1.0f + (powf(2.0f, w1) - 1.0f) * powf(wb, w2);
}

// crates/gpu-kernels/src/pointwise/loss_wrm.rs (loss_wrm_cpu)
void orc_loss_wrm(const float* out, const float* score, const float* wdl,
                  const float* per_pos_norm, float* dl_dout, double* loss_acc, float lambda,
                  float nnue2score, float in_scaling, float in_offset, float target_offset,
                  float target_scaling, float pow_exp, float qp_asymmetry, float w1, float w2,
                  int32_t extended, int64_t n) {
    float inv_sum_w = 0.0f;
    if (extended) {
        double sum_w = 0.0;
        for (int64_t i = 0; i < n; ++i)
            sum_w += (double)wrm_weight(score[i], target_offset, target_scaling, w1, w2);
        inv_sum_w = (float)(1.0 / sum_w);
    }
    for (int64_t i = 0; i < n; ++i) {
        const float s = score[i];
        const float pt = (s - target_offset) / target_scaling;
        const float pmt = (-s - target_offset) / target_scaling;
        const float target_wrm = 0.5f * (1.0f + sigmoid_f32(pt) - sigmoid_f32(pmt));
        const float target = lambda * wdl[i] + (1.0f - lambda) * target_wrm;
        const float scorenet = out[i] * nnue2score;
        const float q = sigmoid_f32((scorenet - in_offset) / in_scaling);
        const float qm = sigmoid_f32((-scorenet - in_offset) / in_scaling);
        const float qf = 0.5f * (1.0f + q - qm);
        const float err = qf - target;
        if (!extended) {
            const float norm = per_pos_norm[i];
            *loss_acc += (double)err * (double)err;
            dl_dout[i] = err * (nnue2score / in_scaling) * (q * (1.0f - q) + qm * (1.0f - qm)) * norm;
            continue;
        }
        const float pf = target_wrm;
        const float wb = (pf - 0.5f) * (pf - 0.5f) * pf * (1.0f - pf);
        const float weight = 1.0f + (powf(2.0f, w1) - 1.0f) * powf(wb, w2);
        const float asym = qf > target ? 1.0f + qp_asymmetry : 1.0f;
        const float abs_err = fabsf(err);
        const float pow_abs = powf(abs_err, pow_exp - 1.0f);
        const float signed_pow = err < 0.0f ? -pow_abs : pow_abs;
        const float dqf = 0.5f * (nnue2score / in_scaling) * (q * (1.0f - q) + qm * (1.0f - qm));
        dl_dout[i] = (weight * inv_sum_w) * (asym * pow_exp * signed_pow) * dqf;
        const float loss_i = asym * powf(abs_err, pow_exp) * weight * (float)n * inv_sum_w;
        *loss_acc += (double)loss_i;
    }
}

// ---------------------------------------------------------------------------
// optimizer
// ---------------------------------------------------------------------------

// crates/gpu-kernels/src/pointwise/radam_step.rs:75-97
void orc_radam_step_size_denom(uint64_t step, float beta1, float beta2, float n_sma_threshold,
                               float* step_size_out, int32_t* denom_out) {
    const float step_f = (float)step;
    const float beta2_t = powf(beta2, step_f);
    const float n_sma_max = 2.0f / (1.0f - beta2) - 1.0f;
    const float n_sma = n_sma_max - 2.0f * step_f * beta2_t / (1.0f - beta2_t);
    const float bc1 = 1.0f - powf(beta1, step_f);
    float ss;
    if (n_sma > n_sma_threshold) {
        const float p1 = (n_sma - 4.0f) / (n_sma_max - 4.0f);
        const float p2 = (n_sma - 2.0f) / n_sma;
        const float p3 = n_sma_max / (n_sma_max - 2.0f);
        ss = sqrtf((1.0f - beta2_t) * p1 * p2 * p3) / bc1;
    } else {
        ss = 1.0f / bc1;
    }
    *step_size_out = ss;
    *denom_out = n_sma > n_sma_threshold ? 1 : 0;
}

// crates/gpu-kernels/src/pointwise/radam_step.rs:116-149
void orc_radam_step(float* weights, float* m, float* v, float* grad, float lr, float step_size,
                    int32_t denom, float decay, float beta1, float beta2, float eps, float min_w,
                    float max_w, int64_t n) {
    const float rate = lr * step_size;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float g = grad[i];
        float p = weights[i];
        p *= 1.0f - decay * rate;
        const float mi = beta1 * m[i] + (1.0f - beta1) * g;
        const float vi = beta2 * v[i] + (1.0f - beta2) * g * g;
        m[i] = mi;
        v[i] = vi;
        float val = mi;
        if (denom != 0) val /= sqrtf(vi) + eps;
        p -= rate * val;
        // f32::clamp(min, max)
        p = p < min_w ? min_w : (p > max_w ? max_w : p);
        weights[i] = p;
        grad[i] = 0.0f;
    }
}

// crates/gpu-kernels/src/pointwise/ranger_step.rs:52-59
void orc_ranger_lookahead_lerp(float* weights, float* slow, float alpha, int64_t n) {
    const float oma = 1.0f - alpha;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float nw = alpha * weights[i] + oma * slow[i];
        weights[i] = nw;
        slow[i] = nw;
    }
}

// ---------------------------------------------------------------------------
// init (crates/nnue-train/src/init.rs:109-209)
// dist: 0 zeroed, 1 uniform, 2 normal.  scale_kind: 0 Abs(value), 1 FanIn(gain=value).
// ---------------------------------------------------------------------------

void orc_init_sample(int64_t n, int64_t num_buckets, int64_t fan_in, int32_t dist,
                     int32_t scale_kind, float value, int32_t per_bucket_repeat, uint64_t seed,
                     float* out) {
    if (dist == 0) {
        for (int64_t i = 0; i < n; ++i) out[i] = 0.0f;
        return;
    }
    float mag;
    if (scale_kind == 0) {
        mag = value;
    } else {
        const float f = (float)(fan_in < 1 ? 1 : fan_in);
        mag = sqrtf(value / f);
    }
    const int64_t block_len = per_bucket_repeat ? n / num_buckets : n;
    uint64_t s = seed > 1 ? seed : 1;
    auto next_unit = [&s]() -> float {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return (float)(s >> 11) / (float)(1ULL << 53);
    };
    if (dist == 1) {
        for (int64_t i = 0; i < block_len; ++i) out[i] = (next_unit() * 2.0f - 1.0f) * mag;
    } else {
        int64_t i = 0;
        const float pi = 3.14159265358979323846f;
        while (i < block_len) {
            float u1 = next_unit();
            u1 = u1 > 1.0e-12f ? u1 : 1.0e-12f;
            const float u2 = next_unit();
            const float r = sqrtf(-2.0f * logf(u1));
            const float theta = 2.0f * pi * u2;
            out[i++] = r * cosf(theta) * mag;
            if (i < block_len) out[i++] = r * sinf(theta) * mag;
        }
    }
    if (per_bucket_repeat && num_buckets > 1)
        for (int64_t b = 1; b < num_buckets; ++b)
            std::memcpy(out + b * block_len, out, sizeof(float) * block_len);
}

}  // extern "C"
