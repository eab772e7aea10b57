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
//             hit masks of the block-scan FT backward (second stream); the
//             occurrence sort (radix, stable) only where the scan cannot run
//   forward   FT gather + pairwise CReLU  ->  L1 (MFMA, sorted tiles)
//             -> tail (L1 glue, L2, L3, loss) per row
//   backward  tail backward (same kernel)  ->  L1 weight grad (MFMA)
//             -> L1 input grad + FT-post grad (dft)
//   optimizer FT gradient (block scan; f16 dft: hit-mask x dft GEMM on the
//             matrix cores) + RAdam/Ranger + fold, fused
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
#include "export.hpp"
#include "psv_kernels.hpp"
#include "ft_kernels.hpp"
#include "init.hpp"
#include "checkpoint.hpp"
#include "trainer_base.hpp"

namespace tatara {

TrainerBase* new_simple_trainer();

namespace {

constexpr float kFtPostScale = 127.0f / 128.0f;  // arch.rs FT_POST_SCALE
constexpr float kL1SqrScale = 127.0f / 128.0f;   // arch.rs L1_SQR_SCALE
constexpr float kQuantClamp = 127.0f / 64.0f;    // i8::MAX / QB
// f16 modes (bins/nnue_train/src/trainer_common.rs:134-166): dft loss scale
// base (x batch), ft_w moment scales
constexpr float kDftF16BaseScale = 16384.0f;              // FT_DFT_FP16_BASE_SCALE = 2^14
constexpr float kMomentF16Scale = 268435456.0f;           // FT_OPT_M_SCALE = 2^28
constexpr float kVelocityF16Scale = 1099511627776.0f;     // FT_OPT_V_SCALE = 2^40

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

}  // namespace

class LayerStackTrainer final : public TrainerBase {
   public:
    uint32_t ft_in = 0, train_ft_in = 0, max_active = 0, pi = 0, ft_out = 0, l1 = 0, l2 = 0, nb = 0;
    uint32_t max_b = 0, max_p = 0;
    bool factorized = false;

    ParamGroup ft;          // ft_w
    ParamGroup small[9];    // uniform_optim_group_layout order
    float* comb = nullptr;  // factorized forward table [ft_in][ft_out]
    // mixed precision (PrecisionFlags): f16 forward table, f16 FT activations
    // and dft, f16 ft_w moments
    bool h_fwd = false, h_out = false, h_state = false;
    bool l1_lowp = false;  // tf32: TF32-class L1 products (f16 / bf16 operands, f32 sums)
    uint16_t* fwd16 = nullptr;  // [ft_in][ft_out] f16 comb (factorizer) or mirror of the real rows
    uint16_t *ft_stm16 = nullptr, *ft_nstm16 = nullptr, *dft16 = nullptr;
    uint16_t* combined16 = nullptr;  // `combined` held as f16 (tf32)
    // the tf32 L1 forward's f16 weight copies (shared weights transposed)
    uint16_t *l1_w16 = nullptr, *l1s_wt16 = nullptr;
    unsigned long long* clamp_ctr = nullptr;  // cumulative dft clamps
    uint64_t clamp_elems = 0;                 // cumulative dft values written

    // schedule
    uint32_t n_king_bins = 1;
    uint8_t* sched_keys = nullptr;
    uint32_t* fb_off = nullptr;  // LDS slot offsets of the block-resident gather, or null
    uint8_t* fb_bad = nullptr;
    // layout of the folded forward table: slice-major for the block-resident gather
    int table_layout() const { return fb_off ? kTablePairSlices : kTableRows; }
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
    uint32_t *radix_hist = nullptr, *radix_count = nullptr;  // the gated occurrence sort's scratch
    // block-scan FT backward (f32 dft, factorized feature sets)
    bool use_scan = false;
    uint32_t* scan_multi = nullptr;
    uint32_t *scan_stage_rows = nullptr, *scan_stage_masks = nullptr;  // the block scan's stage tables
    // activations
    float *ft_stm = nullptr, *ft_nstm = nullptr, *combined = nullptr, *dft = nullptr;
    float *l1_sorted = nullptr, *dl1_sorted = nullptr, *net_out = nullptr;
    // partials
    uint32_t* tail_seg = nullptr;
    float *tail_partial = nullptr, *b1s_partial = nullptr, *w1_partial = nullptr,
          *ftb_partial = nullptr;
    double* loss_partial = nullptr;
    uint32_t* chunk_info = nullptr;
    float *tail_sum = nullptr, *b1s_sum = nullptr, *ftb_sum = nullptr, *w1_seg = nullptr;
    uint32_t max_chunks = 0;
    double *loss_out = nullptr, *weight_sum = nullptr, *wrm_scratch = nullptr;

    int32_t create(const TataraTrainerConfig& c) override {
        cfg = c;
        TATARA_REQUIRE(c.arch == TATARA_ARCH_LAYERSTACK, "only the LayerStack architecture is built");
        TATARA_REQUIRE(c.max_batch > 0 && c.max_batch % 16 == 0, "max_batch must be a positive multiple of 16");
        TATARA_REQUIRE(c.ft_in > 0 && c.max_active > 0 && c.max_active <= 64, "ft_in > 0, 0 < max_active <= 64");
        TATARA_REQUIRE(c.ft_out > 0 && c.ft_out % 128 == 0, "ft_out must be a positive multiple of 128");
        TATARA_REQUIRE(ls_dense_shape_ok(c.l1_out, c.l2_out),
                       std::string(kLsDenseShapes) + " (got " + std::to_string(c.l1_out) + ", " +
                           std::to_string(c.l2_out) + ")");
        TATARA_REQUIRE(c.num_buckets >= 2 && c.num_buckets <= 9, "num_buckets must be in [2, 9]");
        TATARA_REQUIRE(c.optimizer >= 0 && c.optimizer <= 2, "unknown optimizer");
        TATARA_REQUIRE(c.piece_inputs >= 0, "piece_inputs >= 0");
        if (c.piece_inputs > 0)
            TATARA_REQUIRE(c.ft_in % c.piece_inputs == 0, "ft_in must be a multiple of piece_inputs");
        // trainer_layerstack.rs:801-805
        TATARA_REQUIRE(!c.ft_fp16_out || c.ft_fp16, "ft_fp16_out requires ft_fp16");
        int32_t st;
        if ((st = init_runtime(c.device))) return st;

        h_fwd = c.ft_fp16 != 0;
        h_out = c.ft_fp16_out != 0;
        h_state = c.fp16_opt_state != 0;
        l1_lowp = c.tf32 != 0;
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

        if ((st = alloc_group(ft, "ft_w", (uint64_t)train_ft_in * ft_out, fmin, fmax, 0,
                              keep || c.piece_inputs > 0, h_state)))
            return st;
        ft.m_scale = kMomentF16Scale;
        ft.v_scale = kVelocityF16Scale;
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
        if (h_fwd) {
            if ((st = arena.alloc(&fwd16, (uint64_t)ft_in * ft_out))) return st;
        } else if (factorized && (st = arena.alloc(&comb, (uint64_t)ft_in * ft_out))) {
            return st;
        }
        if ((st = arena.alloc(&clamp_ctr, 1))) return st;

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
        if ((st = alloc_inputs(B, max_active))) return st;
        n_king_bins = factorized ? ceil_div(ft_in, pi) : 1;
        if (n_king_bins > 128) n_king_bins = 128;
        if ((st = arena.alloc(&sched_keys, 2 * B)) || (st = arena.alloc(&schedule, 2 * B)) ||
            (st = arena.alloc(&sched_hist, (uint64_t)2 * n_king_bins * binsort_tiles(2 * B))) ||
            (st = arena.alloc(&sched_start, 2 * n_king_bins + 1)) ||
            (st = arena.alloc(&sched_count, 2 * n_king_bins)))
            return st;
        if (factorized && n_king_bins == ceil_div(ft_in, pi) &&
            ft_forward_block_ok(1, h_fwd, ft_out, pi, max_active)) {
            if ((st = arena.alloc(&fb_off, 2 * B * ft_block_slot_stride(max_active), false)) || (st = arena.alloc(&fb_bad, 2 * B, false)))
                return st;
        }
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
        // the block scan (f32 dft) or its matrix-core form (f16 dft)
        use_scan = factorized && ft_out >= 2 * kDftChunk && ft_scan_mask_words(pi) > 0;
        if (use_scan && ((st = arena.alloc(&scan_multi, 1)) ||
                         (st = arena.alloc(&scan_stage_rows, ft_scan_max_stages(B, n_king_bins) * 32, false)) ||
                         (st = arena.alloc(&scan_stage_masks,
                                           ft_scan_max_stages(B, n_king_bins) * ft_scan_mask_words(pi) * 16, false)) ||
                         (st = arena.alloc(&radix_hist, 256ull * binsort_tiles((uint32_t)n_items), false)) ||
                         (st = arena.alloc(&radix_count, 256))))
            return st;
        const uint64_t dft_n = 2 * B * dft_chunks() * kDftChunk;
        if (h_out) {
            if ((st = arena.alloc(&ft_stm16, B * ft_out, false)) || (st = arena.alloc(&ft_nstm16, B * ft_out, false)) ||
                (st = arena.alloc(&dft16, dft_n, false)))
                return st;
        } else if ((st = arena.alloc(&ft_stm, B * ft_out, false)) ||
                   (st = arena.alloc(&ft_nstm, B * ft_out, false)) || (st = arena.alloc(&dft, dft_n, false))) {
            return st;
        }
        if ((l1_lowp ? ((st = arena.alloc(&combined16, B * ft_out, false)) ||
                        (st = arena.alloc(&l1_w16, (uint64_t)nb * l1 * ft_out, false)) ||
                        (st = arena.alloc(&l1s_wt16, (uint64_t)l1 * ft_out, false)))
                     : (st = arena.alloc(&combined, B * ft_out, false))) ||
            (st = arena.alloc(&l1_sorted, P * 2 * l1)) ||
            (st = arena.alloc(&dl1_sorted, P * l1)) || (st = arena.alloc(&net_out, B)))
            return st;
        const TailDims td{l1, l2, nb};
        const uint64_t n_tail = ls_tail_workgroups(max_p), n_post = ls_post_workgroups(max_p);
        max_chunks = ls_max_chunks(max_p, nb);
        if ((st = arena.alloc(&tail_partial, n_tail * td.cells())) || (st = arena.alloc(&tail_seg, nb + 1)) ||
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

    // LayerStackWeights::save_quantised of to_layerstack_weights()
    // (trainer_layerstack.rs:1351-1420): the factorizer is folded into the
    // exported rows, L1 bucket + shared terms are merged per bucket.
    int32_t export_quantised(const char* path, int32_t feature_set, int32_t has_fv, int32_t fv) override {
        ExportFeatureSet fs;
        int32_t st = export_feature_set(feature_set, fs);
        if (st) return st;
        TATARA_REQUIRE(fs.ft_in == ft_in, "export: the feature set's ft_in differs from the trainer's");
        if (factorized) {
            FeatureSetShape sh;
            if ((st = feature_set_shape(feature_set, sh))) return st;
            TATARA_REQUIRE((uint32_t)sh.piece_inputs == pi,
                           "export: the trainer's piece_inputs differ from the feature set's");
        }
        LayerStackHost h;
        std::vector<float>* dst[8] = {&h.l1_w, &h.l1_b, &h.l1s_w, &h.l1s_b, &h.l2_w, &h.l2_b, &h.l3_w, &h.l3_b};
        for (int k = 0; k < 8; ++k)
            if ((st = download(small[k + 1], *dst[k]))) return st;
        QuantSource src{ft.w, ft_in, ft_out, factorized ? pi : 0u};
        QuantSource bias{small[0].w, 1, ft_out, 0};
        return write_layerstack_bin(path, fs, src, bias, l1, l2, nb, h, has_fv != 0, fv, stream);
    }

    int32_t fp16_clamp_count(uint64_t* clamps, uint64_t* elems) override {
        unsigned long long c = 0;
        TATARA_HIP(hipMemcpyAsync(&c, clamp_ctr, sizeof c, hipMemcpyDeviceToHost, stream), "clamp count");
        TATARA_HIP(hipStreamSynchronize(stream), "clamp count");
        *clamps = c;
        *elems = clamp_elems;
        return kOk;
    }

    // Rebuilds the forward table from the master weights: f32 comb, f16 comb
    // (ft_fold_virtual_f16) or the f16 mirror (cast_f32_to_f16,
    // trainer_layerstack.rs:1782-1835).
    int32_t sync_forward_weights() override {
        int32_t st = kOk;
        if (h_fwd && factorized)
            st = launch_ft_fold(ft.w, nullptr, fwd16, ft_in, ft_out, pi, stream, table_layout());
        else if (h_fwd)
            st = launch_cast_f16(ft.w, fwd16, (uint64_t)ft_in * ft_out, stream);
        else if (factorized)
            st = launch_ft_fold(ft.w, comb, nullptr, ft_in, ft_out, pi, stream, table_layout());
        else
            return kOk;
        if (st) return st;
        TATARA_HIP(hipStreamSynchronize(stream), "sync_forward_weights");
        return kOk;
    }

    std::vector<const char*> group_names() const override {
        std::vector<const char*> names{"ft_w"};
        for (const auto& g : small) names.push_back(g.name);
        return names;
    }

    ParamGroup* find(const char* name) override {
        if (!std::strcmp(name, "ft_w")) return &ft;
        for (auto& g : small)
            if (!std::strcmp(name, g.name)) return &g;
        return nullptr;
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
        a.combined16 = combined16;
        a.ft_stm = ft_stm;
        a.ft_nstm = ft_nstm;
        a.l1_sorted = l1_sorted;
        a.dl1_sorted = dl1_sorted;
        a.net_output = net_out;
        a.dft = dft;
        a.ft_stm16 = ft_stm16;
        a.ft_nstm16 = ft_nstm16;
        a.dft16 = dft16;
        a.dft_scale = kDftF16BaseScale * (float)p.b;
        a.clamp_counter = clamp_ctr;
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
        a.l1_w16 = l1_w16;
        a.l1s_wt16 = l1s_wt16;
        a.l1s_b = small[4].w;
        a.l2_w = small[5].w;
        a.l2_b = small[6].w;
        a.l3_w = small[7].w;
        a.l3_b = small[8].w;
        a.ft_post_scale = kFtPostScale;
        a.l1_sqr_scale = kL1SqrScale;
        a.tail_partial = tail_partial;
        a.tail_seg = tail_seg;
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

    // Occurrence lists of the batch (key 2*feature + perspective).
    // gated: the sort runs only if the hit-mask pass set scan_multi
    int32_t sort_occurrences(const BatchPtrs& p, hipStream_t s, bool gated = false) {
        OccurrenceSortArgs os{};
        os.idx_stm = p.stm;
        os.idx_nstm = p.nstm;
        os.nnz = p.nnz;
        os.batch = p.b;
        os.max_active = max_active;
        os.cols = ft_in;
        os.keys_in = occ_ki;
        os.vals_in = occ_vi;
        os.keys_out = occ_ko;
        os.vals_out = occ_vo;
        os.offsets = occ_off;
        os.temp = occ_tmp;
        os.temp_bytes = occ_tmp_bytes;
        if (gated) {
            os.run_if = scan_multi;
            os.radix_hist = radix_hist;
            os.radix_count = radix_count;
        }
        return launch_occurrence_sort(os, s);
    }

    // FT gradient + update: the block scan (its matrix-core form for an f16
    // dft) and, gated on the device by the flag of the hit-mask pass, the
    // occurrence-list kernel for a batch with a row the scan cannot take; or
    // occurrence lists every step when the trainer does not scan.
    int32_t ft_gradient(const BatchPtrs& p, const FtGradArgs& fb) {
        if (use_scan)
            return h_out ? launch_ft_grad_mfma(fb, block_scan(p), stream, !batch_king_blocked)
                         : launch_ft_grad_scan(fb, block_scan(p), stream, !batch_king_blocked);
        return launch_ft_grad_update(fb, stream);
    }

    FtBlockScan block_scan(const BatchPtrs& p) const {
        FtBlockScan sc{};
        sc.idx_stm = p.stm;
        sc.idx_nstm = p.nstm;
        sc.nnz = p.nnz;
        sc.schedule = schedule;
        sc.sched_start = sched_start;
        sc.multi = scan_multi;
        sc.stage_rows = scan_stage_rows;
        sc.stage_masks = scan_stage_masks;
        sc.batch = p.b;
        sc.max_active = max_active;
        sc.cols = ft_in;
        sc.piece_inputs = pi;
        sc.n_blocks = n_king_bins;
        sc.multi_sticky = batch_king_blocked ? kb_broken_dev : nullptr;
        sc.dealt = h_out ? 0u : 1u;  // the matrix-core form reads runs of 16
        return sc;
    }

    // prep + forward (+ loss); shared by train and validate
    int32_t forward(const BatchPtrs& p, float wdl_lambda, const LossParams& lp, int32_t train,
                    int slot, uint32_t& padded) {
        int32_t st;
        const uint32_t b = p.b;
        padded = padded_sort_batch(b, nb);
        if (train && (st = prof_mark(0))) return st;
        if (train && !use_scan) {
            // occurrence lists for the FT backward, on the side stream: they
            // depend only on the indices and are first needed by the FT
            // gradient, so the sort overlaps the forward
            if ((st = fork_side())) return st;
            if ((st = sort_occurrences(p, side))) return st;
        }
        // king-block schedule for the gather
        const int32_t* sched = nullptr;
        if (factorized) {
            if ((st = launch_king_block_keys(p.stm, p.nstm, p.nnz, sched_keys, b, max_active, ft_in, pi,
                                             n_king_bins, stream, fb_off, fb_bad)))
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
            if (train && use_scan) {
                // hit masks of the block-scan backward, beside the forward,
                // then the occurrence sort, which runs only when a row has
                // features of two king blocks or one feature twice (the
                // mask pass sets scan_multi); no host wait.  A batch passed
                // as king-blocked (on_device = 2) queues no sort.
                if ((st = fork_side())) return st;
                if ((st = launch_ft_scan_tables(block_scan(p), side))) return st;
                if ((st = batch_king_blocked ? note_king_blocked_tables() : sort_occurrences(p, side, true)))
                    return st;
            }
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
        if (train && (st = prof_mark(1))) return st;
        // FT gather + pairwise post
        FtForwardArgs fa{};
        fa.mode = 1;
        fa.W = factorized ? comb : ft.w;
        fa.W16 = h_fwd ? fwd16 : nullptr;
        fa.out_stm16 = ft_stm16;
        fa.out_nstm16 = ft_nstm16;
        fa.idx_stm = p.stm;
        fa.idx_nstm = p.nstm;
        fa.nnz = p.nnz;
        fa.schedule = sched;
        if (sched && fb_off) {
            // the schedule's bins: the gather holds each king block's slice in LDS
            fa.sched_start = sched_start;
            fa.n_blocks = n_king_bins;
            fa.piece_inputs = pi;
            fa.slot_off = fb_off;
            fa.row_bad = fb_bad;
            fa.w_layout = factorized ? table_layout() : kTableRows;
        }
        fa.bias = small[0].w;
        fa.out_stm = ft_stm;
        fa.out_nstm = ft_nstm;
        fa.combined = combined;
        fa.combined16 = combined16;
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
                       double* lagged) override {
        int32_t st;
        if ((st = check_loss(l))) return st;
        BatchPtrs p{};
        if ((st = stage_batch(bt, p, true, 16, max_b))) return st;
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
        fb.dft16 = dft16;
        fb.dft_inv_scale = 1.0f / da.dft_scale;
        fb.dft_row_stride = kDftChunk;  // chunk-major [chunk][2*b][256]
        fb.dft_chunk_stride = 2ull * p.b * kDftChunk;
        fb.occ_vals = occ_vo;
        fb.occ_off = occ_off;
        fb.w = ft.w;
        fb.m = ft.m;
        fb.v = ft.v;
        fb.m16 = ft.m16;
        fb.v16 = ft.v16;
        fb.m_scale = ft.m_scale;
        fb.v_scale = ft.v_scale;
        fb.mirror16 = (h_fwd && !factorized) ? fwd16 : nullptr;
        fb.slow = ft.slow;
        fb.grad = ft.grad;
        fb.ft_out = ft_out;
        fb.rows = ft_in;
        fb.apply_update = 1;
        fb.opt = sf;
        if ((st = join_side())) return st;
        if ((st = ft_gradient(p, fb))) return st;
        if ((st = prof_mark(5))) return st;
        if (factorized &&
            (st = launch_ft_virtual_fold(fb, pi, comb, h_fwd ? fwd16 : nullptr, stream, table_layout())))
            return st;
        if (h_out) clamp_elems += 2ull * p.b * ft_out;
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
        last_b = p.b;
        if ((st = release_batch())) return st;
        return queue_loss(loss_out, slot, lagged);
    }

    int32_t validate(const TataraBatch* bt, float wdl_lambda, const TataraLoss* l, double* sse,
                     float* net_host) override {
        int32_t st;
        if ((st = check_loss(l))) return st;
        TATARA_HIP(hipStreamSynchronize(stream), "validate sync");
        BatchPtrs p{};
        if ((st = stage_batch(bt, p, true, 16, max_b))) return st;
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
        if ((st = release_batch())) return st;
        if (sse) *sse = v;
        return kOk;
    }

    uint32_t dft_chunks() const { return ceil_div(ft_out, kDftChunk); }

    int32_t copy_activation(const char* name, float* host, uint64_t n) override {
        // f16 activations are returned as the f32 values of what is stored
        // (the dft scaled by 2^14 * batch)
        const bool s = !std::strcmp(name, "dft_stm"), ns = !std::strcmp(name, "dft_nstm");
        if (s || ns)
            return copy_chunk_major(h_out ? (const void*)dft16 : (const void*)dft, h_out, last_b, ft_out, ns ? 1 : 0,
                                    host, n);
        if (!std::strcmp(name, "l1_total")) {
            // bucket + shared L1 output of each position (original order), the
            // f32 sum the tail takes (elementwise_add)
            TATARA_REQUIRE(n <= (uint64_t)last_b * l1, "activation request exceeds the last batch");
            const uint64_t P = padded_sort_batch(last_b, nb);
            std::vector<float> ls(P * 2 * l1);
            std::vector<int32_t> pm(P);
            TATARA_HIP(hipStreamSynchronize(stream), "get_activation sync");
            TATARA_HIP(hipMemcpy(ls.data(), l1_sorted, ls.size() * sizeof(float), hipMemcpyDeviceToHost),
                       "get_activation l1_total");
            TATARA_HIP(hipMemcpy(pm.data(), perm, P * sizeof(int32_t), hipMemcpyDeviceToHost), "get_activation perm");
            for (uint64_t r = 0; r < P; ++r) {
                if (pm[r] < 0) continue;
                for (uint32_t j = 0; j < l1; ++j) {
                    const uint64_t i = (uint64_t)pm[r] * l1 + j;
                    if (i < n) host[i] = ls[r * 2 * l1 + j] + ls[r * 2 * l1 + l1 + j];
                }
            }
            return kOk;
        }
        if (h_out && (!std::strcmp(name, "ft_stm_out") || !std::strcmp(name, "ft_nstm_out"))) {
            TATARA_REQUIRE(n <= (uint64_t)last_b * ft_out, "activation request exceeds the last batch");
            return copy_f16(!std::strcmp(name, "ft_stm_out") ? ft_stm16 : ft_nstm16, host, n);
        }
        if (l1_lowp && !std::strcmp(name, "combined")) {
            TATARA_REQUIRE(n <= (uint64_t)last_b * ft_out, "activation request exceeds the last batch");
            return copy_f16(combined16, host, n);
        }
        return TrainerBase::copy_activation(name, host, n);
    }

    const float* activation(const char* name, uint64_t& cap) override {
        const uint64_t bf = (uint64_t)last_b * ft_out;
        cap = bf;
        if (!std::strcmp(name, "ft_stm_out")) return ft_stm;
        if (!std::strcmp(name, "ft_nstm_out")) return ft_nstm;
        if (!std::strcmp(name, "combined")) return combined;
        cap = last_b;
        if (!std::strcmp(name, "net_output")) return net_out;
        return nullptr;
    }
};

}  // namespace tatara

using namespace tatara;

struct TataraTrainer {
    std::unique_ptr<TrainerBase> t;
};

namespace tatara {
hipStream_t trainer_stream(const TataraTrainer* h) { return h->t->stream; }
}  // namespace tatara

extern "C" {

int32_t tatara_trainer_create(const TataraTrainerConfig* config, TataraTrainer** out) {
    TATARA_REQUIRE(config && out, "null argument");
    *out = nullptr;
    auto h = std::make_unique<TataraTrainer>();
    if (config->arch == TATARA_ARCH_LAYERSTACK) {
        h->t = std::make_unique<LayerStackTrainer>();
    } else {
        TATARA_REQUIRE(config->arch == TATARA_ARCH_SIMPLE, "unknown architecture");
        h->t.reset(new_simple_trainer());
    }
    const int32_t st = h->t->create(*config);
    if (st) return st;
    *out = h.release();
    return kOk;
}

int32_t tatara_trainer_destroy(TataraTrainer* trainer) {
    delete trainer;
    return kOk;
}

int32_t tatara_trainer_train_step(TataraTrainer* trainer, const TataraBatch* batch, float lr,
                                  float wdl_lambda, const TataraLoss* loss, double* lagged_loss) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->t->train_step(batch, lr, wdl_lambda, loss, lagged_loss);
}

int32_t tatara_trainer_flush_pending_loss(TataraTrainer* trainer, double* loss) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->t->flush(loss);
}

int32_t tatara_trainer_validate_step(TataraTrainer* trainer, const TataraBatch* batch,
                                     float wdl_lambda, const TataraLoss* loss, double* sum_sq_err,
                                     float* net_output) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->t->validate(batch, wdl_lambda, loss, sum_sq_err, net_output);
}

int32_t tatara_trainer_step_count(TataraTrainer* trainer, uint64_t* steps) {
    TATARA_REQUIRE(trainer && steps, "null argument");
    *steps = trainer->t->step_count;
    return kOk;
}

int32_t tatara_trainer_tensor_size(TataraTrainer* trainer, const char* name, uint64_t* n) {
    TATARA_REQUIRE(trainer && name && n, "null argument");
    ParamGroup* g = trainer->t->find(name);
    TATARA_REQUIRE(g, std::string("unknown tensor ") + name);
    *n = g->n;
    return kOk;
}

int32_t tatara_trainer_get_tensor(TataraTrainer* trainer, const char* name, int32_t which,
                                  float* host, uint64_t n) {
    TATARA_REQUIRE(trainer && name && host, "null argument");
    TrainerBase& t = *trainer->t;
    ParamGroup* g = t.find(name);
    TATARA_REQUIRE(g, std::string("unknown tensor ") + name);
    TATARA_REQUIRE(which >= 0 && which <= 4, "which must be 0..4");
    TATARA_REQUIRE(n == g->n, "element count mismatch");
    return t.read_group(*g, which, host);
}

int32_t tatara_trainer_set_tensor(TataraTrainer* trainer, const char* name, int32_t which,
                                  const float* host, uint64_t n) {
    TATARA_REQUIRE(trainer && name && host, "null argument");
    TrainerBase& t = *trainer->t;
    ParamGroup* g = t.find(name);
    TATARA_REQUIRE(g, std::string("unknown tensor ") + name);
    TATARA_REQUIRE(n == g->n, "element count mismatch");
    int32_t st = t.write_group(*g, which, host);
    if (st) return st;
    if (!std::strcmp(name, "ft_w") && which == 0) return t.sync_forward_weights();
    return kOk;
}

int32_t tatara_trainer_fp16_clamp_count(TataraTrainer* trainer, uint64_t* clamps, uint64_t* elems) {
    TATARA_REQUIRE(trainer && clamps && elems, "null argument");
    return trainer->t->fp16_clamp_count(clamps, elems);
}

int32_t tatara_trainer_get_activation(TataraTrainer* trainer, const char* name, float* host,
                                      uint64_t n) {
    TATARA_REQUIRE(trainer && name && host, "null argument");
    return trainer->t->copy_activation(name, host, n);
}

int32_t tatara_trainer_set_profiling(TataraTrainer* trainer, int32_t enable) {
    TATARA_REQUIRE(trainer, "trainer is null");
    TrainerBase& t = *trainer->t;
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
    TrainerBase& t = *trainer->t;
    int32_t st = t.prof_collect();
    if (st) return st;
    for (int k = 0; k < n_phases && k < TrainerBase::kPhases; ++k) ms[k] = t.phase_ms[k];
    if (steps) *steps = t.prof_steps;
    return kOk;
}

int32_t tatara_trainer_sync_forward_weights(TataraTrainer* trainer) {
    TATARA_REQUIRE(trainer, "trainer is null");
    return trainer->t->sync_forward_weights();
}

// The checkpoint identity of a trainer: the feature set (TATARA_FS_*) must
// have the trainer's base ft_in and, with a factorizer, its piece inputs.
static int32_t trainer_ckpt_arch(const TrainerBase& t, int32_t feature_set, int32_t bucket_mode, CkptArch& a) {
    FeatureSetShape s{};
    int32_t st = feature_set_shape(feature_set, s);
    if (st) return st;
    const TataraTrainerConfig& c = t.cfg;
    TATARA_REQUIRE((int64_t)s.king_buckets * s.piece_inputs == c.ft_in,
                   "the feature set's ft_in differs from the trainer's");
    TATARA_REQUIRE(c.piece_inputs == 0 || c.piece_inputs == s.piece_inputs,
                   "the feature set's piece inputs differ from the trainer's factorizer");
    TataraCkptArch ca{};
    ca.feature_set = feature_set;
    ca.ft_factorize = c.piece_inputs > 0;
    ca.arch = c.arch;
    ca.bucket_mode = bucket_mode;
    ca.ft_out = (uint64_t)c.ft_out;
    ca.l1_out = (uint64_t)c.l1_out;
    ca.l2_out = (uint64_t)c.l2_out;
    ca.num_buckets = c.arch == TATARA_ARCH_LAYERSTACK ? (uint64_t)c.num_buckets : 0;
    return ckpt_arch_from_c(ca, a);
}

int32_t tatara_trainer_save_resume(TataraTrainer* trainer, const char* path, int32_t feature_set,
                                   int32_t bucket_mode, uint64_t superbatch, const char* run_id,
                                   uint64_t lr_horizon) {
    TATARA_REQUIRE(trainer && path, "null argument");
    TrainerBase& t = *trainer->t;
    CkptArch a;
    int32_t st = trainer_ckpt_arch(t, feature_set, bucket_mode, a);
    if (st) return st;
    return save_resume_checkpoint(t, path, a, t.group_names(), superbatch, run_id, lr_horizon);
}

int32_t tatara_trainer_load_resume(TataraTrainer* trainer, const char* path, int32_t feature_set,
                                   int32_t bucket_mode, TataraCkptHeader* header) {
    TATARA_REQUIRE(trainer && path, "null argument");
    TrainerBase& t = *trainer->t;
    CkptArch a;
    int32_t st = trainer_ckpt_arch(t, feature_set, bucket_mode, a);
    if (st) return st;
    return load_resume_checkpoint(t, path, a, t.group_names(), header);
}

int32_t tatara_trainer_export_quantised(TataraTrainer* trainer, const char* path, int32_t feature_set,
                                        int32_t has_fv_scale, int32_t fv_scale) {
    TATARA_REQUIRE(trainer && path, "null argument");
    return trainer->t->export_quantised(path, feature_set, has_fv_scale, fv_scale);
}

}  // extern "C"
