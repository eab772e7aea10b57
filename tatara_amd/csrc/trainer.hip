// LayerStack training step on one MI355X, behind the TrainerBackend-shaped
// C ABI of include/tatara_hip.h.
//
// Mirrors GpuTrainer (bins/nnue_train/src/trainer_layerstack.rs): the same
// parameter groups, initialisation (:781-1064), step order (forward
// :2038-2848, backward :2849-3936, optimizer :4034-4489), optimizer scalars
// (crates/nnue-train/src/optimizer.rs:62-87) and lagged loss
// (AsyncLossRing, trainer_common.rs:909-1035).  The launch sequence is
// re-designed for gfx950 (about a dozen fused, deterministic kernels instead
// of ~100 launches with float atomics):
//
//   prep      king-block schedule (stable bin sort), bucket sort (16-aligned),
//             occurrence sort for the FT backward (radix, stable)
//   forward   FT gather + pairwise CReLU  ->  L1 (MFMA, sorted tiles)
//             -> tail (L1 glue, L2, L3, loss) per row
//   backward  tail backward (same kernel)  ->  L1 weight grad (MFMA)
//             -> L1 input grad + FT-post grad (dft)
//   optimizer FT gradient (segmented sums) + RAdam/Ranger + fold, fused
//             -> dense gradients from partials + RAdam/Ranger
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <vector>

#include "../../include/tatara_hip.h"
#include "binsort.hpp"
#include "common.hpp"
#include "dense_kernels.hpp"
#include "ft_kernels.hpp"
#include "init.hpp"

namespace tatara {

namespace {

constexpr float kFtPostScale = 127.0f / 128.0f;  // arch.rs FT_POST_SCALE
constexpr float kL1SqrScale = 127.0f / 128.0f;   // arch.rs L1_SQR_SCALE
constexpr float kBeta2 = 0.999f;                 // RangerParams::DEFAULT
constexpr float kEps = 1e-8f;
constexpr float kAlpha = 0.5f;
constexpr uint64_t kRangerK = 6;
constexpr float kNSmaThreshold = 5.0f;
constexpr float kQuantClamp = 127.0f / 64.0f;    // i8::MAX / QB

__global__ void bucket_keys_kernel(const int32_t* __restrict__ bucket, uint8_t* __restrict__ keys,
                                   uint32_t n, uint32_t nb) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t b = bucket[i];
    keys[i] = (uint8_t)((b >= 0 && (uint32_t)b < nb) ? b : nb);
}

uint32_t padded_sort_batch(uint32_t b, uint32_t nb) {
    const uint32_t raw = b + (nb + 1) * 16;
    return (raw + 15) / 16 * 16;
}

struct DeviceArena {
    std::vector<void*> ptrs;
    ~DeviceArena() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <class T>
    int32_t alloc(T** out, uint64_t count, bool zero = true) {
        void* p = nullptr;
        const uint64_t bytes = count * sizeof(T) ? count * sizeof(T) : 4;
        TATARA_HIP(hipMalloc(&p, bytes), "hipMalloc trainer buffer");
        ptrs.push_back(p);
        if (zero) TATARA_HIP(hipMemset(p, 0, bytes), "hipMemset trainer buffer");
        *out = static_cast<T*>(p);
        return kOk;
    }
};

struct ParamGroup {
    const char* name;
    float *w = nullptr, *m = nullptr, *v = nullptr, *slow = nullptr, *grad = nullptr;
    uint64_t n = 0;
    float min_w, max_w;
    int32_t kind;  // 0 ft, 1 dense, 2 bias
};

}  // namespace

struct LayerStackTrainer {
    TataraTrainerConfig cfg{};
    hipStream_t stream = nullptr;
    DeviceArena arena;

    uint32_t ft_in = 0, train_ft_in = 0, max_active = 0, pi = 0, ft_out = 0, l1 = 0, l2 = 0, nb = 0;
    uint32_t max_b = 0, max_p = 0;
    bool factorized = false;

    ParamGroup ft;          // ft_w
    ParamGroup small[9];    // uniform_optim_group_layout order
    float* comb = nullptr;  // factorized forward table [ft_in][ft_out]

    // device copies of host batches
    int32_t *in_stm = nullptr, *in_nstm = nullptr, *in_nnz = nullptr, *in_bucket = nullptr;
    float *in_score = nullptr, *in_wdl = nullptr;
    // schedule
    uint32_t n_king_bins = 1;
    uint8_t* sched_keys = nullptr;
    int32_t* schedule = nullptr;
    uint32_t *sched_hist = nullptr, *sched_start = nullptr, *sched_count = nullptr;
    // bucket sort
    uint8_t* bkt_keys = nullptr;
    int32_t *perm = nullptr, *sorted_bin = nullptr;
    uint32_t *bkt_hist = nullptr, *bin_start = nullptr, *bin_count = nullptr;
    // occurrence sort
    uint32_t *occ_ki = nullptr, *occ_vi = nullptr, *occ_ko = nullptr, *occ_vo = nullptr;
    uint32_t* occ_off = nullptr;
    void* occ_tmp = nullptr;
    size_t occ_tmp_bytes = 0;
    // activations
    float *ft_stm = nullptr, *ft_nstm = nullptr, *combined = nullptr, *dft = nullptr;
    float *l1_sorted = nullptr, *dl1_sorted = nullptr, *net_out = nullptr;
    // partials
    float *tail_partial = nullptr, *b1s_partial = nullptr, *w1_partial = nullptr,
          *ftb_partial = nullptr;
    double* loss_partial = nullptr;
    uint32_t* chunk_info = nullptr;
    float *tail_sum = nullptr, *b1s_sum = nullptr, *ftb_sum = nullptr, *w1_seg = nullptr;
    uint32_t max_chunks = 0;
    double *loss_out = nullptr, *weight_sum = nullptr, *wrm_scratch = nullptr;
    // lagged loss ring
    double* pinned_loss = nullptr;
    hipEvent_t loss_ev[2] = {nullptr, nullptr};
    int pending = -1;  // slot holding the last queued loss
    int next_slot = 0;

    uint64_t step_count = 0;
    uint32_t last_b = 0;

    // phase profiling: events recorded between phases of each profiled step
    static constexpr int kPhases = 7;
    bool profiling = false;
    std::vector<hipEvent_t> prof_events;  // (kPhases + 1) per profiled step
    double phase_ms[kPhases] = {0, 0, 0, 0, 0, 0, 0};
    uint64_t prof_steps = 0;
    int prof_cursor = -1;  // first event of the current step

    int32_t prof_mark(int k) {
        if (!profiling) return kOk;
        hipEvent_t e = nullptr;
        TATARA_HIP(hipEventCreate(&e), "hipEventCreate (profiling)");
        TATARA_HIP(hipEventRecord(e, stream), "hipEventRecord (profiling)");
        if (k == 0) prof_cursor = (int)prof_events.size();
        prof_events.push_back(e);
        return kOk;
    }

    int32_t prof_collect() {
        TATARA_HIP(hipStreamSynchronize(stream), "profiling sync");
        const size_t per = kPhases + 1;
        for (size_t s = 0; s + per <= prof_events.size(); s += per) {
            for (int k = 0; k < kPhases; ++k) {
                float ms = 0.f;
                TATARA_HIP(hipEventElapsedTime(&ms, prof_events[s + k], prof_events[s + k + 1]),
                           "hipEventElapsedTime");
                phase_ms[k] += ms;
            }
            prof_steps += 1;
        }
        for (hipEvent_t e : prof_events) (void)hipEventDestroy(e);
        prof_events.clear();
        return kOk;
    }

    ~LayerStackTrainer() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (hipEvent_t e : prof_events) (void)hipEventDestroy(e);
        for (auto& e : loss_ev)
            if (e) (void)hipEventDestroy(e);
        if (pinned_loss) (void)hipHostFree(pinned_loss);
        if (stream) (void)hipStreamDestroy(stream);
    }

    int32_t alloc_group(ParamGroup& g, const char* name, uint64_t n, float mn, float mx, int kind,
                        bool with_grad) {
        g.name = name;
        g.n = n;
        g.min_w = mn;
        g.max_w = mx;
        g.kind = kind;
        int32_t st;
        if ((st = arena.alloc(&g.w, n)) || (st = arena.alloc(&g.m, n)) ||
            (st = arena.alloc(&g.v, n)) || (st = arena.alloc(&g.slow, n)))
            return st;
        if (with_grad && (st = arena.alloc(&g.grad, n))) return st;
        return kOk;
    }

    int32_t upload(float* dst, const std::vector<float>& src) {
        TATARA_HIP(hipMemcpy(dst, src.data(), src.size() * sizeof(float), hipMemcpyHostToDevice),
                   "upload init weights");
        return kOk;
    }

    int32_t create(const TataraTrainerConfig& c) {
        cfg = c;
        TATARA_REQUIRE(c.arch == TATARA_ARCH_LAYERSTACK, "only the LayerStack architecture is built");
        TATARA_REQUIRE(c.max_batch > 0 && c.max_batch % 16 == 0, "max_batch must be a positive multiple of 16");
        TATARA_REQUIRE(c.ft_in > 0 && c.max_active > 0 && c.max_active <= 64, "ft_in > 0, 0 < max_active <= 64");
        TATARA_REQUIRE(c.ft_out > 0 && c.ft_out % 128 == 0, "ft_out must be a positive multiple of 128");
        TATARA_REQUIRE((c.l1_out == 16 || c.l1_out == 8) && c.l2_out == 32,
                       "(l1, l2) must be (16, 32) or (8, 32)");
        TATARA_REQUIRE(c.num_buckets >= 2 && c.num_buckets <= 9, "num_buckets must be in [2, 9]");
        TATARA_REQUIRE(c.optimizer >= 0 && c.optimizer <= 2, "unknown optimizer");
        TATARA_REQUIRE(c.piece_inputs >= 0, "piece_inputs >= 0");
        if (c.piece_inputs > 0)
            TATARA_REQUIRE(c.ft_in % c.piece_inputs == 0, "ft_in must be a multiple of piece_inputs");
        TATARA_HIP(hipSetDevice(c.device), "hipSetDevice");
        TATARA_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        TATARA_HIP(hipEventCreateWithFlags(&loss_ev[0], hipEventDisableTiming), "hipEventCreate");
        TATARA_HIP(hipEventCreateWithFlags(&loss_ev[1], hipEventDisableTiming), "hipEventCreate");
        TATARA_HIP(hipHostMalloc((void**)&pinned_loss, 2 * sizeof(double), hipHostMallocDefault),
                   "hipHostMalloc loss ring");

        ft_in = c.ft_in;
        pi = c.piece_inputs;
        factorized = pi > 0;
        train_ft_in = ft_in + (factorized ? pi : 0);
        max_active = c.max_active;
        ft_out = c.ft_out;
        l1 = c.l1_out;
        l2 = c.l2_out;
        nb = c.num_buckets;
        max_b = c.max_batch;
        max_p = padded_sort_batch(max_b, nb);
        const bool keep = c.keep_grads != 0;
        const float fmin = std::numeric_limits<float>::lowest();
        const float fmax = std::numeric_limits<float>::max();
        const uint32_t l2_in = 2 * (l1 - 1);

        int32_t st;
        if ((st = alloc_group(ft, "ft_w", (uint64_t)train_ft_in * ft_out, fmin, fmax, 0,
                              keep || c.piece_inputs > 0)))
            return st;
        const struct {
            const char* name;
            uint64_t n;
            bool quant;
            int kind;
        } layout[9] = {
            {"ft_b", ft_out, false, 2},
            {"l1_w", (uint64_t)nb * l1 * ft_out, true, 1},
            {"l1_b", (uint64_t)nb * l1, true, 2},
            {"l1_shared_weight", (uint64_t)ft_out * l1, true, 1},
            {"l1_shared_bias", l1, true, 2},
            {"l2_w", (uint64_t)nb * l2 * l2_in, true, 1},
            {"l2_b", (uint64_t)nb * l2, true, 2},
            {"l3_w", (uint64_t)nb * l2, true, 1},
            {"l3_b", nb, false, 2},
        };
        for (int k = 0; k < 9; ++k) {
            const float mn = layout[k].quant ? -kQuantClamp : fmin;
            const float mx = layout[k].quant ? kQuantClamp : fmax;
            if ((st = alloc_group(small[k], layout[k].name, layout[k].n, mn, mx, layout[k].kind, true)))
                return st;
        }
        if (factorized && (st = arena.alloc(&comb, (uint64_t)ft_in * ft_out))) return st;

        // initial weights: LayerStackInit::default_uniform; FT real block sampled
        // with the base fan-in, factorizer rows appended as zeros (:844-870)
        LayerStackInitSpec spec;
        {
            std::vector<float> w = init_sample((uint64_t)ft_in * ft_out, ft_in, spec.ft_w);
            w.resize((uint64_t)train_ft_in * ft_out, 0.0f);
            if ((st = upload(ft.w, w))) return st;
        }
        const LayerInit* inits[9] = {&spec.ft_b, &spec.l1_w, &spec.l1_b, &spec.l1s_w, &spec.l1s_b,
                                     &spec.l2_w, &spec.l2_b, &spec.l3_w, &spec.l3_b};
        const uint64_t fan[9] = {ft_in, ft_out, ft_out, ft_out, ft_out, l2_in, l2_in, l2, l2};
        for (int k = 0; k < 9; ++k)
            if ((st = upload(small[k].w, init_sample(small[k].n, fan[k], *inits[k])))) return st;

        // workspace
        const uint64_t B = max_b, P = max_p;
        if ((st = arena.alloc(&in_stm, B * max_active)) || (st = arena.alloc(&in_nstm, B * max_active)) ||
            (st = arena.alloc(&in_nnz, B)) || (st = arena.alloc(&in_bucket, B)) ||
            (st = arena.alloc(&in_score, B)) || (st = arena.alloc(&in_wdl, B)))
            return st;
        n_king_bins = factorized ? ceil_div(ft_in, pi) : 1;
        if (n_king_bins > 128) n_king_bins = 128;
        if ((st = arena.alloc(&sched_keys, 2 * B)) || (st = arena.alloc(&schedule, 2 * B)) ||
            (st = arena.alloc(&sched_hist, (uint64_t)2 * n_king_bins * binsort_tiles(2 * B))) ||
            (st = arena.alloc(&sched_start, 2 * n_king_bins + 1)) ||
            (st = arena.alloc(&sched_count, 2 * n_king_bins)))
            return st;
        if ((st = arena.alloc(&bkt_keys, B)) || (st = arena.alloc(&perm, P)) ||
            (st = arena.alloc(&sorted_bin, P)) ||
            (st = arena.alloc(&bkt_hist, (uint64_t)(nb + 1) * binsort_tiles(B))) ||
            (st = arena.alloc(&bin_start, nb + 2)) || (st = arena.alloc(&bin_count, nb + 1)))
            return st;
        const uint64_t n_items = 2 * B * max_active;
        occ_tmp_bytes = occurrence_sort_temp_bytes(n_items, ft_in);
        if ((st = arena.alloc(&occ_ki, n_items, false)) || (st = arena.alloc(&occ_vi, n_items, false)) ||
            (st = arena.alloc(&occ_ko, n_items, false)) || (st = arena.alloc(&occ_vo, n_items, false)) ||
            (st = arena.alloc(&occ_off, 2ull * ft_in + 2)) ||
            (st = arena.alloc((uint8_t**)&occ_tmp, occ_tmp_bytes, false)))
            return st;
        if ((st = arena.alloc(&ft_stm, B * ft_out, false)) || (st = arena.alloc(&ft_nstm, B * ft_out, false)) ||
            (st = arena.alloc(&combined, B * ft_out, false)) || (st = arena.alloc(&dft, 2 * B * ft_out, false)) ||
            (st = arena.alloc(&l1_sorted, P * 2 * l1)) || (st = arena.alloc(&dl1_sorted, P * l1)) ||
            (st = arena.alloc(&net_out, B)))
            return st;
        const TailDims td{l1, l2, nb};
        const uint64_t n_tail = ls_tail_workgroups(max_p), n_post = ls_post_workgroups(max_p);
        max_chunks = ls_max_chunks(max_p, nb);
        if ((st = arena.alloc(&tail_partial, n_tail * nb * td.cells())) ||
            (st = arena.alloc(&b1s_partial, n_tail * l1)) || (st = arena.alloc(&loss_partial, n_tail)) ||
            (st = arena.alloc(&w1_partial, (uint64_t)max_chunks * l1 * ft_out)) ||
            (st = arena.alloc(&ftb_partial, n_post * 2 * ft_out)) ||
            (st = arena.alloc(&chunk_info, 3ull * max_chunks + 1 + nb + 2)) ||
            (st = arena.alloc(&tail_sum, (uint64_t)nb * td.cells())) || (st = arena.alloc(&b1s_sum, l1)) ||
            (st = arena.alloc(&ftb_sum, 2ull * ft_out)) ||
            (st = arena.alloc(&w1_seg, (uint64_t)(nb + 1) * l1 * ft_out)) ||
            (st = arena.alloc(&loss_out, 2)) || (st = arena.alloc(&weight_sum, 1)) ||
            (st = arena.alloc(&wrm_scratch, ceil_div(B, 256) + 1)))
            return st;
        TATARA_HIP(hipDeviceSynchronize(), "trainer init");
        return sync_forward_weights();
    }

    int32_t sync_forward_weights() {
        if (!factorized) return kOk;
        int32_t st = launch_ft_fold(ft.w, comb, ft_in, ft_out, pi, stream);
        if (st) return st;
        TATARA_HIP(hipStreamSynchronize(stream), "sync_forward_weights");
        return kOk;
    }

    ParamGroup* find(const char* name) {
        if (!std::strcmp(name, "ft_w")) return &ft;
        for (auto& g : small)
            if (!std::strcmp(name, g.name)) return &g;
        return nullptr;
    }

    OptScalars scalars(int kind, float lr, uint64_t step) const {
        OptScalars s{};
        const int opt = cfg.optimizer;
        s.beta1 = opt == TATARA_OPT_RANGER ? 0.99f : 0.9f;
        s.beta2 = kBeta2;
        s.eps = kEps;
        if (opt == TATARA_OPT_ADAMW) {
            s.step_size = 1.0f;
            s.denom = 1;
        } else {
            (void)tatara_radam_step_size_denom(step, s.beta1, kBeta2, kNSmaThreshold, &s.step_size,
                                               &s.denom);
        }
        float wd, mult;
        if (kind == 0) {
            wd = cfg.ft_weight_decay;
            mult = cfg.ft_lr_mult;
        } else if (kind == 1) {
            wd = cfg.dense_weight_decay;
            mult = cfg.dense_lr_mult;
        } else {
            wd = cfg.bias_weight_decay;
            mult = cfg.bias_lr_mult;
        }
        s.decay = wd;
        s.lr = lr * mult;
        s.lookahead = (opt == TATARA_OPT_RANGER && step % kRangerK == 0) ? 1 : 0;
        s.alpha = kAlpha;
        // the FT weight has no clamp (W_CLAMP_NONE); the dense groups get
        // their per-group bounds in the finalize kernel
        s.min_w = std::numeric_limits<float>::lowest();
        s.max_w = std::numeric_limits<float>::max();
        return s;
    }

    struct BatchPtrs {
        const int32_t *stm, *nstm, *nnz, *bucket;
        const float *score, *wdl;
        uint32_t b;
    };

    int32_t stage_batch(const TataraBatch* bt, BatchPtrs& p) {
        TATARA_REQUIRE(bt, "batch is null");
        TATARA_REQUIRE(bt->n_pos >= 0 && bt->n_pos % 16 == 0,
                       "batch.n_pos must be a multiple of 16 (tiled kernels require b % 16 == 0)");
        TATARA_REQUIRE((uint32_t)bt->n_pos <= max_b, "batch exceeds workspace capacity");
        TATARA_REQUIRE((uint32_t)bt->max_active == max_active, "batch.max_active != feature set max_active");
        p.b = bt->n_pos;
        if (p.b == 0) return kOk;
        TATARA_REQUIRE(bt->stm_indices && bt->nstm_indices && bt->nnz && bt->bucket_idx && bt->score &&
                           bt->wdl,
                       "batch array is null");
        if (bt->on_device) {
            p.stm = bt->stm_indices;
            p.nstm = bt->nstm_indices;
            p.nnz = bt->nnz;
            p.bucket = bt->bucket_idx;
            p.score = bt->score;
            p.wdl = bt->wdl;
            return kOk;
        }
        const uint64_t b = p.b;
        TATARA_HIP(hipMemcpyAsync(in_stm, bt->stm_indices, 4 * b * max_active, hipMemcpyHostToDevice, stream), "H2D stm");
        TATARA_HIP(hipMemcpyAsync(in_nstm, bt->nstm_indices, 4 * b * max_active, hipMemcpyHostToDevice, stream), "H2D nstm");
        TATARA_HIP(hipMemcpyAsync(in_nnz, bt->nnz, 4 * b, hipMemcpyHostToDevice, stream), "H2D nnz");
        TATARA_HIP(hipMemcpyAsync(in_bucket, bt->bucket_idx, 4 * b, hipMemcpyHostToDevice, stream), "H2D bucket");
        TATARA_HIP(hipMemcpyAsync(in_score, bt->score, 4 * b, hipMemcpyHostToDevice, stream), "H2D score");
        TATARA_HIP(hipMemcpyAsync(in_wdl, bt->wdl, 4 * b, hipMemcpyHostToDevice, stream), "H2D wdl");
        // pageable sources: make sure they were consumed before returning
        TATARA_HIP(hipStreamSynchronize(stream), "H2D batch");
        p.stm = in_stm;
        p.nstm = in_nstm;
        p.nnz = in_nnz;
        p.bucket = in_bucket;
        p.score = in_score;
        p.wdl = in_wdl;
        return kOk;
    }

    LossParams loss_params(const TataraLoss* l) const {
        LossParams lp{};
        lp.kind = l->kind;
        lp.scale = l->scale;
        lp.nnue2score = l->nnue2score;
        lp.in_scaling = l->in_scaling;
        lp.in_offset = l->in_offset;
        lp.target_offset = l->target_offset;
        lp.target_scaling = l->target_scaling;
        lp.pow_exp = l->pow_exp;
        lp.qp_asymmetry = l->qp_asymmetry;
        lp.w1 = l->weight_boost_w1;
        lp.w2 = l->weight_boost_w2;
        lp.extended = (l->kind == 1 &&
                       (l->pow_exp != 2.0f || l->qp_asymmetry != 0.0f || l->weight_boost_w1 != 0.0f))
                          ? 1
                          : 0;
        return lp;
    }

    int32_t check_loss(const TataraLoss* l) {
        TATARA_REQUIRE(l, "loss is null");
        if (l->kind == 0) {
            TATARA_REQUIRE(std::isfinite(l->scale) && l->scale > 0.0f, "loss scale must be finite and > 0");
        } else {
            TATARA_REQUIRE(l->kind == 1, "unknown loss kind");
            TATARA_REQUIRE(std::isfinite(l->nnue2score) && l->nnue2score > 0.0f, "wrm nnue2score must be finite and > 0");
            TATARA_REQUIRE(std::isfinite(l->in_scaling) && l->in_scaling > 0.0f, "wrm in_scaling must be finite and > 0");
            TATARA_REQUIRE(std::isfinite(l->in_offset), "wrm in_offset must be finite");
            TATARA_REQUIRE(std::isfinite(l->target_offset), "wrm target_offset must be finite");
            TATARA_REQUIRE(std::isfinite(l->target_scaling) && l->target_scaling > 0.0f, "wrm target_scaling must be finite and > 0");
            TATARA_REQUIRE(std::isfinite(l->pow_exp) && l->pow_exp >= 1.0f, "wrm pow_exp must be finite and >= 1");
            TATARA_REQUIRE(std::isfinite(l->qp_asymmetry) && l->qp_asymmetry >= 0.0f, "wrm qp_asymmetry must be finite and >= 0");
            TATARA_REQUIRE(std::isfinite(l->weight_boost_w1) && l->weight_boost_w1 >= 0.0f, "wrm weight_boost_w1 must be finite and >= 0");
            TATARA_REQUIRE(std::isfinite(l->weight_boost_w2) && l->weight_boost_w2 >= 0.0f, "wrm weight_boost_w2 must be finite and >= 0");
        }
        return kOk;
    }

    LsDenseArgs dense_args(const BatchPtrs& p, uint32_t padded, float wdl_lambda, const LossParams& lp,
                           int slot) const {
        LsDenseArgs a{};
        a.batch = p.b;
        a.padded_b = padded;
        a.ft_out = ft_out;
        a.l1 = l1;
        a.l2 = l2;
        a.nb = nb;
        a.perm = perm;
        a.sorted_bin = sorted_bin;
        a.bin_start = bin_start;
        a.bin_count = bin_count;
        a.chunk_info = chunk_info;
        a.max_chunks = max_chunks;
        a.combined = combined;
        a.ft_stm = ft_stm;
        a.ft_nstm = ft_nstm;
        a.l1_sorted = l1_sorted;
        a.dl1_sorted = dl1_sorted;
        a.net_output = net_out;
        a.dft = dft;
        a.score = p.score;
        a.wdl = p.wdl;
        a.per_pos_norm = p.b ? 1.0f / (float)p.b : 0.0f;
        a.wdl_lambda = wdl_lambda;
        a.loss = lp;
        a.weight_sum = weight_sum;
        a.ft_b = small[0].w;
        a.l1_w = small[1].w;
        a.l1_b = small[2].w;
        a.l1s_w = small[3].w;
        a.l1s_b = small[4].w;
        a.l2_w = small[5].w;
        a.l2_b = small[6].w;
        a.l3_w = small[7].w;
        a.l3_b = small[8].w;
        a.ft_post_scale = kFtPostScale;
        a.l1_sqr_scale = kL1SqrScale;
        a.tail_partial = tail_partial;
        a.b1s_partial = b1s_partial;
        a.loss_partial = loss_partial;
        a.w1_partial = w1_partial;
        a.ftb_partial = ftb_partial;
        a.tail_sum = tail_sum;
        a.b1s_sum = b1s_sum;
        a.ftb_sum = ftb_sum;
        a.w1_seg = w1_seg;
        a.loss_out = loss_out + slot;
        return a;
    }

    // prep + forward (+ loss); shared by train and validate
    int32_t forward(const BatchPtrs& p, float wdl_lambda, const LossParams& lp, int32_t train,
                    int slot, uint32_t& padded) {
        int32_t st;
        const uint32_t b = p.b;
        padded = padded_sort_batch(b, nb);
        if (train && (st = prof_mark(0))) return st;
        // king-block schedule for the gather
        const int32_t* sched = nullptr;
        if (factorized) {
            if ((st = launch_king_block_keys(p.stm, p.nstm, p.nnz, sched_keys, b, max_active, ft_in, pi,
                                             n_king_bins, stream)))
                return st;
            BinSortArgs bs{};
            bs.keys = sched_keys;
            bs.n_items = 2 * b;
            bs.n_bins = 2 * n_king_bins;
            bs.align = 1;
            bs.value_mod = b;
            bs.hist = sched_hist;
            bs.bin_start = sched_start;
            bs.bin_count = sched_count;
            bs.out = schedule;
            if ((st = launch_binsort(bs, stream))) return st;
            sched = schedule;
        }
        // bucket sort (16-aligned, invalid buckets in bin nb)
        bucket_keys_kernel<<<ceil_div(b, 256), 256, 0, stream>>>(p.bucket, bkt_keys, b, nb);
        TATARA_LAUNCHED("bucket_keys");
        {
            BinSortArgs bs{};
            bs.keys = bkt_keys;
            bs.n_items = b;
            bs.n_bins = nb + 1;
            bs.align = 16;
            bs.value_mod = 0;
            bs.hist = bkt_hist;
            bs.bin_start = bin_start;
            bs.bin_count = bin_count;
            bs.out = perm;
            bs.out_key = sorted_bin;
            bs.out_fill_len = padded;
            if ((st = launch_binsort(bs, stream))) return st;
        }
        if (train) {
            OccurrenceSortArgs os{};
            os.idx_stm = p.stm;
            os.idx_nstm = p.nstm;
            os.nnz = p.nnz;
            os.batch = b;
            os.max_active = max_active;
            os.cols = ft_in;
            os.keys_in = occ_ki;
            os.vals_in = occ_vi;
            os.keys_out = occ_ko;
            os.vals_out = occ_vo;
            os.offsets = occ_off;
            os.temp = occ_tmp;
            os.temp_bytes = occ_tmp_bytes;
            if ((st = launch_occurrence_sort(os, stream))) return st;
        }
        if (train && (st = prof_mark(1))) return st;
        // FT gather + pairwise post
        FtForwardArgs fa{};
        fa.mode = 1;
        fa.W = factorized ? comb : ft.w;
        fa.idx_stm = p.stm;
        fa.idx_nstm = p.nstm;
        fa.nnz = p.nnz;
        fa.schedule = sched;
        fa.bias = small[0].w;
        fa.out_stm = ft_stm;
        fa.out_nstm = ft_nstm;
        fa.combined = combined;
        fa.batch = b;
        fa.ft_out = ft_out;
        fa.cols = ft_in;
        fa.max_active = max_active;
        fa.n_persp = 2;
        fa.scale = kFtPostScale;
        if ((st = launch_ft_forward(fa, stream))) return st;
        if (train && (st = prof_mark(2))) return st;
        LsDenseArgs da = dense_args(p, padded, wdl_lambda, lp, slot);
        if ((st = launch_ls_l1_forward(da, stream))) return st;
        if (lp.kind == 1 && lp.extended) {
            if ((st = launch_wrm_weight_sum(p.score, b, lp, weight_sum, wrm_scratch, stream))) return st;
        }
        if ((st = launch_ls_tail(da, train, stream))) return st;
        if ((st = launch_ls_loss_reduce(da, stream))) return st;
        return kOk;
    }

    int32_t train_step(const TataraBatch* bt, float lr, float wdl_lambda, const TataraLoss* l,
                       double* lagged) {
        int32_t st;
        if ((st = check_loss(l))) return st;
        BatchPtrs p{};
        if ((st = stage_batch(bt, p))) return st;
        if (p.b == 0) {
            if (lagged) *lagged = 0.0;
            return kOk;
        }
        const LossParams lp = loss_params(l);
        const int slot = next_slot;
        uint32_t padded = 0;
        if ((st = forward(p, wdl_lambda, lp, 1, slot, padded))) return st;
        LsDenseArgs da = dense_args(p, padded, wdl_lambda, lp, slot);
        if ((st = prof_mark(3))) return st;
        if ((st = launch_ls_l1_weight_grad(da, stream))) return st;
        if ((st = launch_ls_l1_input_post(da, stream))) return st;
        if ((st = prof_mark(4))) return st;

        // optimizer
        step_count += 1;
        const OptScalars sf = scalars(0, lr, step_count);
        const OptScalars sd = scalars(1, lr, step_count);
        const OptScalars sb = scalars(2, lr, step_count);
        FtGradArgs fb{};
        fb.dft = dft;
        fb.occ_vals = occ_vo;
        fb.occ_off = occ_off;
        fb.w = ft.w;
        fb.m = ft.m;
        fb.v = ft.v;
        fb.slow = ft.slow;
        fb.grad = ft.grad;
        fb.ft_out = ft_out;
        fb.rows = ft_in;
        fb.apply_update = 1;
        fb.opt = sf;
        if ((st = launch_ft_grad_update(fb, stream))) return st;
        if ((st = prof_mark(5))) return st;
        if (factorized && (st = launch_ft_virtual_fold(fb, pi, comb, stream))) return st;
        if ((st = prof_mark(6))) return st;
        LsDenseGroup groups[9];
        for (int k = 0; k < 9; ++k) {
            groups[k].w = small[k].w;
            groups[k].m = small[k].m;
            groups[k].v = small[k].v;
            groups[k].slow = small[k].slow;
            groups[k].grad = small[k].grad;
            groups[k].n = small[k].n;
            groups[k].min_w = small[k].min_w;
            groups[k].max_w = small[k].max_w;
            groups[k].kind = small[k].kind;
        }
        if ((st = launch_ls_dense_finalize(da, groups, sd, sb, 1, cfg.keep_grads, stream))) return st;
        if ((st = prof_mark(7))) return st;

        // lagged loss (AsyncLossRing::read_and_queue_next)
        double prev = 0.0;
        if (pending >= 0) {
            TATARA_HIP(hipEventSynchronize(loss_ev[pending]), "loss ring event");
            prev = pinned_loss[pending];
        }
        TATARA_HIP(hipMemcpyAsync(pinned_loss + slot, loss_out + slot, sizeof(double),
                                  hipMemcpyDeviceToHost, stream),
                   "loss D2H");
        TATARA_HIP(hipEventRecord(loss_ev[slot], stream), "loss ring record");
        pending = slot;
        next_slot = 1 - slot;
        last_b = p.b;
        if (lagged) *lagged = prev;
        return kOk;
    }

    int32_t flush(double* out) {
        double v = 0.0;
        if (pending >= 0) {
            TATARA_HIP(hipEventSynchronize(loss_ev[pending]), "loss ring flush");
            v = pinned_loss[pending];
            pending = -1;
        }
        if (out) *out = v;
        return kOk;
    }

    int32_t validate(const TataraBatch* bt, float wdl_lambda, const TataraLoss* l, double* sse,
                     float* net_host) {
        int32_t st;
        if ((st = check_loss(l))) return st;
        TATARA_HIP(hipStreamSynchronize(stream), "validate sync");
        BatchPtrs p{};
        if ((st = stage_batch(bt, p))) return st;
        if (p.b == 0) {
            if (sse) *sse = 0.0;
            return kOk;
        }
        const LossParams lp = loss_params(l);
        const int slot = next_slot;
        uint32_t padded = 0;
        if ((st = forward(p, wdl_lambda, lp, 0, slot, padded))) return st;
        double v = 0.0;
        TATARA_HIP(hipMemcpyAsync(&v, loss_out + slot, sizeof(double), hipMemcpyDeviceToHost, stream), "validate loss");
        if (net_host)
            TATARA_HIP(hipMemcpyAsync(net_host, net_out, 4ull * p.b, hipMemcpyDeviceToHost, stream), "validate net");
        TATARA_HIP(hipStreamSynchronize(stream), "validate");
        last_b = p.b;
        if (sse) *sse = v;
        return kOk;
    }
};

}  // namespace tatara

using namespace tatara;

struct TataraTrainer {
    std::unique_ptr<LayerStackTrainer> ls;
};

extern "C" {

int32_t tatara_trainer_create(const TataraTrainerConfig* config, TataraTrainer** out) {
    TATARA_REQUIRE(config && out, "null argument");
    *out = nullptr;
    auto t = std::make_unique<TataraTrainer>();
    t->ls = std::make_unique<LayerStackTrainer>();
    const int32_t st = t->ls->create(*config);
    if (st) return st;
    *out = t.release();
    return kOk;
}

int32_t tatara_trainer_destroy(TataraTrainer* trainer) {
    delete trainer;
    return kOk;
}

int32_t tatara_trainer_train_step(TataraTrainer* trainer, const TataraBatch* batch, float lr,
                                  float wdl_lambda, const TataraLoss* loss, double* lagged_loss) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->ls->train_step(batch, lr, wdl_lambda, loss, lagged_loss);
}

int32_t tatara_trainer_flush_pending_loss(TataraTrainer* trainer, double* loss) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->ls->flush(loss);
}

int32_t tatara_trainer_validate_step(TataraTrainer* trainer, const TataraBatch* batch,
                                     float wdl_lambda, const TataraLoss* loss, double* sum_sq_err,
                                     float* net_output) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->ls->validate(batch, wdl_lambda, loss, sum_sq_err, net_output);
}

int32_t tatara_trainer_step_count(TataraTrainer* trainer, uint64_t* steps) {
    TATARA_REQUIRE(trainer && steps, "null argument");
    *steps = trainer->ls->step_count;
    return kOk;
}

int32_t tatara_trainer_tensor_size(TataraTrainer* trainer, const char* name, uint64_t* n) {
    TATARA_REQUIRE(trainer && name && n, "null argument");
    ParamGroup* g = trainer->ls->find(name);
    TATARA_REQUIRE(g, std::string("unknown tensor ") + name);
    *n = g->n;
    return kOk;
}

static float* group_ptr(ParamGroup* g, int32_t which) {
    switch (which) {
        case 0: return g->w;
        case 1: return g->m;
        case 2: return g->v;
        case 3: return g->slow;
        case 4: return g->grad;
        default: return nullptr;
    }
}

int32_t tatara_trainer_get_tensor(TataraTrainer* trainer, const char* name, int32_t which,
                                  float* host, uint64_t n) {
    TATARA_REQUIRE(trainer && name && host, "null argument");
    LayerStackTrainer& t = *trainer->ls;
    ParamGroup* g = t.find(name);
    TATARA_REQUIRE(g, std::string("unknown tensor ") + name);
    TATARA_REQUIRE(n == g->n, "element count mismatch");
    TATARA_HIP(hipStreamSynchronize(t.stream), "get_tensor sync");
    float* src = group_ptr(g, which);
    if (which == 4 && !t.cfg.keep_grads) src = nullptr;  // the optimizer leaves zero gradients
    if (!src) {
        TATARA_REQUIRE(which == 4, "which must be 0..4");
        // gradients are zeroed by the optimizer; without keep_grads none are kept
        std::memset(host, 0, n * sizeof(float));
        return kOk;
    }
    TATARA_HIP(hipMemcpy(host, src, n * sizeof(float), hipMemcpyDeviceToHost), "get_tensor");
    return kOk;
}

int32_t tatara_trainer_set_tensor(TataraTrainer* trainer, const char* name, int32_t which,
                                  const float* host, uint64_t n) {
    TATARA_REQUIRE(trainer && name && host, "null argument");
    LayerStackTrainer& t = *trainer->ls;
    ParamGroup* g = t.find(name);
    TATARA_REQUIRE(g, std::string("unknown tensor ") + name);
    TATARA_REQUIRE(n == g->n, "element count mismatch");
    float* dst = group_ptr(g, which);
    TATARA_REQUIRE(dst, "tensor not allocated (which)");
    TATARA_HIP(hipStreamSynchronize(t.stream), "set_tensor sync");
    TATARA_HIP(hipMemcpy(dst, host, n * sizeof(float), hipMemcpyHostToDevice), "set_tensor");
    if (g == &t.ft && which == 0) return t.sync_forward_weights();
    return kOk;
}

int32_t tatara_trainer_get_activation(TataraTrainer* trainer, const char* name, float* host,
                                      uint64_t n) {
    TATARA_REQUIRE(trainer && name && host, "null argument");
    LayerStackTrainer& t = *trainer->ls;
    const uint64_t bf = (uint64_t)t.last_b * t.ft_out;
    const float* src = nullptr;
    uint64_t cap = 0;
    if (!std::strcmp(name, "ft_stm_out")) { src = t.ft_stm; cap = bf; }
    else if (!std::strcmp(name, "ft_nstm_out")) { src = t.ft_nstm; cap = bf; }
    else if (!std::strcmp(name, "combined")) { src = t.combined; cap = bf; }
    else if (!std::strcmp(name, "net_output")) { src = t.net_out; cap = t.last_b; }
    else if (!std::strcmp(name, "dft_stm")) { src = t.dft; cap = bf; }
    else if (!std::strcmp(name, "dft_nstm")) { src = t.dft + bf; cap = bf; }
    TATARA_REQUIRE(src, std::string("unknown activation ") + name);
    TATARA_REQUIRE(n <= cap, "activation request exceeds the last batch");
    TATARA_HIP(hipStreamSynchronize(t.stream), "get_activation sync");
    TATARA_HIP(hipMemcpy(host, src, n * sizeof(float), hipMemcpyDeviceToHost), "get_activation");
    return kOk;
}

int32_t tatara_trainer_set_profiling(TataraTrainer* trainer, int32_t enable) {
    TATARA_REQUIRE(trainer, "trainer is null");
    LayerStackTrainer& t = *trainer->ls;
    int32_t st = t.prof_collect();
    if (st) return st;
    for (double& v : t.phase_ms) v = 0.0;
    t.prof_steps = 0;
    t.profiling = enable != 0;
    return kOk;
}

int32_t tatara_trainer_phase_times(TataraTrainer* trainer, double* ms, int32_t n_phases,
                                   uint64_t* steps) {
    TATARA_REQUIRE(trainer && ms, "null argument");
    LayerStackTrainer& t = *trainer->ls;
    int32_t st = t.prof_collect();
    if (st) return st;
    for (int k = 0; k < n_phases && k < LayerStackTrainer::kPhases; ++k) ms[k] = t.phase_ms[k];
    if (steps) *steps = t.prof_steps;
    return kOk;
}

int32_t tatara_trainer_sync_forward_weights(TataraTrainer* trainer) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->ls->sync_forward_weights();
}

}  // extern "C"
