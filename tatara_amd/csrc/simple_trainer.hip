// Simple-architecture (FT -> L1 -> L2 -> L3, CReLU) training step on one
// MI355X, behind the same C ABI as the LayerStack trainer.
//
// Mirrors SimpleGpuTrainer (bins/nnue_train/src/trainer_simple.rs): groups
// and initialisation (:392-600: SimpleInit::default_uniform, FT factorizer
// rows appended as zeros, slow weights equal to the initial weights), step
// order (step :742-856, forward :857-1506, backward :1509-2347, optimizer
// :2359-2690) and the lagged loss.  Launch sequence on gfx950:
//
//   prep      king-block schedule of the gather (factorized feature sets),
//             occurrence sort for the FT backward
//   forward   FT gather + bias + CReLU into combined [b][2*ft_out]
//             -> L1 (MFMA) -> L2, L3, loss per row
//   backward  L2/L3 backward in the same kernel -> L1 weight grad (MFMA)
//             -> L1 input grad + CReLU grad (dft) + ft_b partials
//   optimizer FT gradient (segmented sums) + RAdam/Ranger/AdamW + fold,
//             then the seven dense groups from their partials
#include <hip/hip_runtime.h>

#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "binsort.hpp"
#include "dense_kernels.hpp"
#include "export.hpp"
#include "psv_kernels.hpp"
#include "ft_kernels.hpp"
#include "init.hpp"
#include "simple_kernels.hpp"
#include "trainer_base.hpp"

namespace tatara {

namespace {

constexpr float kQuantClamp = 127.0f / 64.0f;  // W_CLAMP_QUANT (i8::MAX / QB)

class SimpleTrainer final : public TrainerBase {
   public:
    uint32_t ft_in = 0, train_ft_in = 0, max_active = 0, pi = 0, ft_out = 0, l1 = 0, l2 = 0;
    uint32_t max_b = 0;
    bool factorized = false;

    ParamGroup ft;          // ft_w
    ParamGroup small[7];    // ft_b, l1_w, l1_b, l2_w, l2_b, l3_w, l3_b
    float* comb = nullptr;  // factorized forward table [ft_in][ft_out]

    // gather schedule
    uint32_t n_king_bins = 1;
    uint8_t* sched_keys = nullptr;
    uint32_t* fb_off = nullptr;  // LDS slot offsets of the block-resident gather, or null
    uint8_t* fb_bad = nullptr;
    // layout of the folded forward table: row-major also for the block-resident
    // gather (the 256-column table stays in the Infinity Cache, where the
    // slice-major form saved the forward less than it cost the fold)
    int table_layout() const { return kTableRows; }
    int32_t* schedule = nullptr;
    uint32_t *sched_hist = nullptr, *sched_start = nullptr, *sched_count = nullptr;
    // occurrence sort
    uint32_t *occ_ki = nullptr, *occ_vi = nullptr, *occ_ko = nullptr, *occ_vo = nullptr;
    uint32_t* occ_off = nullptr;
    void* occ_tmp = nullptr;
    size_t occ_tmp_bytes = 0;
    uint32_t *radix_hist = nullptr, *radix_count = nullptr;  // the gated occurrence sort's scratch
    // block-scan FT backward (factorized feature sets)
    bool use_scan = false;
    uint32_t* scan_multi = nullptr;
    uint32_t *scan_stage_rows = nullptr, *scan_stage_masks = nullptr;  // the block scan's stage tables
    // activations
    float *ft_stm = nullptr, *ft_nstm = nullptr, *combined = nullptr, *dft = nullptr;
    float *l1_pre = nullptr, *dl1 = nullptr, *net_out = nullptr;
    // partials and their sums
    float *tail_partial = nullptr, *w1_partial = nullptr, *ftb_partial = nullptr;
    float *tail_sum = nullptr, *w1_sum = nullptr, *ftb_sum = nullptr;
    double *loss_partial = nullptr, *loss_out = nullptr, *weight_sum = nullptr, *wrm_scratch = nullptr;

    int32_t create(const TataraTrainerConfig& c) override {
        cfg = c;
        TATARA_REQUIRE(c.max_batch > 0, "max_batch must be positive");
        TATARA_REQUIRE(c.ft_in > 0 && c.max_active > 0 && c.max_active <= 64, "ft_in > 0, 0 < max_active <= 64");
        TATARA_REQUIRE(c.ft_out > 0 && c.ft_out % 32 == 0, "ft_out must be a positive multiple of 32");
        TATARA_REQUIRE(simple_dense_shape_ok(c.l1_out, c.l2_out),
                       std::string(kSimpleDenseShapes) + " (got " + std::to_string(c.l1_out) + ", " +
                           std::to_string(c.l2_out) + ")");
        TATARA_REQUIRE(c.optimizer >= 0 && c.optimizer <= 2, "unknown optimizer");
        TATARA_REQUIRE(c.piece_inputs >= 0, "piece_inputs >= 0");
        TATARA_REQUIRE(!c.ft_fp16 && !c.ft_fp16_out && !c.fp16_opt_state && !c.tf32,
                       "the f16 modes are built for the LayerStack architecture only");
        if (c.piece_inputs > 0)
            TATARA_REQUIRE(c.ft_in % c.piece_inputs == 0, "ft_in must be a multiple of piece_inputs");
        int32_t st;
        if ((st = init_runtime(c.device))) return st;

        ft_in = c.ft_in;
        pi = c.piece_inputs;
        factorized = pi > 0;
        train_ft_in = ft_in + (factorized ? pi : 0);
        max_active = c.max_active;
        ft_out = c.ft_out;
        l1 = c.l1_out;
        l2 = c.l2_out;
        max_b = c.max_batch;
        const uint32_t K = 2 * ft_out;
        const bool keep = c.keep_grads != 0;
        const float fmin = std::numeric_limits<float>::lowest();
        const float fmax = std::numeric_limits<float>::max();

        if ((st = alloc_group(ft, "ft_w", (uint64_t)train_ft_in * ft_out, fmin, fmax, 0, keep || factorized)))
            return st;
        // run_optimizer_step group order and clamps (trainer_simple.rs:2443-2520)
        const struct {
            const char* name;
            uint64_t n;
            bool quant;
            int kind;
        } layout[7] = {
            {"ft_b", ft_out, false, 2},
            {"l1_w", (uint64_t)K * l1, true, 1},
            {"l1_b", l1, true, 2},
            {"l2_w", (uint64_t)l1 * l2, true, 1},
            {"l2_b", l2, true, 2},
            {"l3_w", l2, true, 1},
            {"l3_b", 1, false, 2},
        };
        for (int k = 0; k < 7; ++k) {
            const float mn = layout[k].quant ? -kQuantClamp : fmin;
            const float mx = layout[k].quant ? kQuantClamp : fmax;
            if ((st = alloc_group(small[k], layout[k].name, layout[k].n, mn, mx, layout[k].kind, true)))
                return st;
        }
        if (factorized && (st = arena.alloc(&comb, (uint64_t)ft_in * ft_out))) return st;

        // SimpleInit::default_uniform with the fan-ins of trainer_simple.rs:454-463
        SimpleInitSpec spec;
        {
            std::vector<float> w = init_sample((uint64_t)ft_in * ft_out, ft_in, spec.ft_w);
            w.resize((uint64_t)train_ft_in * ft_out, 0.0f);
            if ((st = upload(ft.w, w)) || (st = upload(ft.slow, w))) return st;
        }
        const LayerInit* inits[7] = {&spec.ft_b, &spec.l1_w, &spec.l1_b, &spec.l2_w,
                                     &spec.l2_b, &spec.l3_w, &spec.l3_b};
        const uint64_t fan[7] = {ft_in, K, K, l1, l1, l2, l2};
        for (int k = 0; k < 7; ++k) {
            const std::vector<float> w = init_sample(small[k].n, fan[k], *inits[k]);
            if ((st = upload(small[k].w, w)) || (st = upload(small[k].slow, w))) return st;
        }

        // workspace
        const uint64_t B = max_b;
        if ((st = alloc_inputs(B, max_active))) return st;
        n_king_bins = factorized ? ceil_div(ft_in, pi) : 1;
        if (n_king_bins > 128) n_king_bins = 128;
        if ((st = arena.alloc(&sched_keys, 2 * B)) || (st = arena.alloc(&schedule, 2 * B)) ||
            (st = arena.alloc(&sched_hist, (uint64_t)2 * n_king_bins * binsort_tiles(2 * B))) ||
            (st = arena.alloc(&sched_start, 2 * n_king_bins + 1)) ||
            (st = arena.alloc(&sched_count, 2 * n_king_bins)))
            return st;
        if (factorized && n_king_bins == ceil_div(ft_in, pi) &&
            ft_forward_block_ok(2, false, ft_out, pi, max_active)) {
            if ((st = arena.alloc(&fb_off, 2 * B * ft_block_slot_stride(max_active), false)) || (st = arena.alloc(&fb_bad, 2 * B, false)))
                return st;
        }
        const uint64_t n_items = 2 * B * max_active;
        occ_tmp_bytes = occurrence_sort_temp_bytes(n_items, ft_in);
        if ((st = arena.alloc(&occ_ki, n_items, false)) || (st = arena.alloc(&occ_vi, n_items, false)) ||
            (st = arena.alloc(&occ_ko, n_items, false)) || (st = arena.alloc(&occ_vo, n_items, false)) ||
            (st = arena.alloc(&occ_off, 2ull * ft_in + 2)) ||
            (st = arena.alloc((uint8_t**)&occ_tmp, occ_tmp_bytes, false)))
            return st;
        use_scan = factorized && ft_out >= kDftChunk && ft_scan_mask_words(pi) > 0;
        if (use_scan && ((st = arena.alloc(&scan_multi, 1)) ||
                         (st = arena.alloc(&scan_stage_rows, ft_scan_max_stages(B, n_king_bins) * 32, false)) ||
                         (st = arena.alloc(&scan_stage_masks,
                                           ft_scan_max_stages(B, n_king_bins) * ft_scan_mask_words(pi) * 16, false)) ||
                         (st = arena.alloc(&radix_hist, 256ull * binsort_tiles((uint32_t)n_items), false)) ||
                         (st = arena.alloc(&radix_count, 256))))
            return st;
        if ((st = arena.alloc(&ft_stm, B * ft_out, false)) || (st = arena.alloc(&ft_nstm, B * ft_out, false)) ||
            (st = arena.alloc(&combined, B * K, false)) || (st = arena.alloc(&dft, 2 * B * dft_chunks() * kDftChunk, false)) ||
            (st = arena.alloc(&l1_pre, B * l1)) || (st = arena.alloc(&dl1, B * l1)) ||
            (st = arena.alloc(&net_out, B)))
            return st;
        const SimpleTailDims td{l1, l2};
        const uint64_t n_tail = simple_tail_workgroups(max_b), n_chunks = simple_chunks(max_b),
                       n_post = simple_post_workgroups(max_b);
        if ((st = arena.alloc(&tail_partial, n_tail * td.cells())) ||
            (st = arena.alloc(&w1_partial, n_chunks * K * l1)) ||
            (st = arena.alloc(&ftb_partial, n_post * ft_out)) || (st = arena.alloc(&tail_sum, td.cells())) ||
            (st = arena.alloc(&w1_sum, (uint64_t)K * l1)) || (st = arena.alloc(&ftb_sum, ft_out)) ||
            (st = arena.alloc(&loss_partial, n_tail)) || (st = arena.alloc(&loss_out, 2)) ||
            (st = arena.alloc(&weight_sum, 1)) || (st = arena.alloc(&wrm_scratch, ceil_div(B, 256) + 1)))
            return st;
        TATARA_HIP(hipDeviceSynchronize(), "trainer init");
        return sync_forward_weights();
    }

    // SimpleWeights::save_quantised of to_simple_weights() (trainer_simple.rs:
    // 2680-2745): CReLU activation, the factorizer folded into the exported
    // rows, dense weights transposed to out-major while writing.
    int32_t export_quantised(const char* path, int32_t feature_set, int32_t has_fv, int32_t fv) override {
        TATARA_REQUIRE(has_fv, "Simple export: the arch string always carries fv_scale");
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
        SimpleHost h;
        std::vector<float>* dst[6] = {&h.l1_w, &h.l1_b, &h.l2_w, &h.l2_b, &h.l3_w, &h.l3_b};
        for (int k = 0; k < 6; ++k)
            if ((st = download(small[k + 1], *dst[k]))) return st;
        QuantSource src{ft.w, ft_in, ft_out, factorized ? pi : 0u};
        QuantSource bias{small[0].w, 1, ft_out, 0};
        return write_simple_bin(path, fs, src, bias, l1, l2, h, fv, stream);
    }

    int32_t sync_forward_weights() override {
        if (!factorized) return kOk;
        int32_t st = launch_ft_fold(ft.w, comb, nullptr, ft_in, ft_out, pi, stream, table_layout());
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

    uint32_t dft_chunks() const { return ceil_div(ft_out, kDftChunk); }

    int32_t copy_activation(const char* name, float* host, uint64_t n) override {
        const bool s = !std::strcmp(name, "dft_stm"), ns = !std::strcmp(name, "dft_nstm");
        if (!s && !ns) return TrainerBase::copy_activation(name, host, n);
        return copy_chunk_major(dft, false, last_b, ft_out, ns ? 1 : 0, host, n);
    }

    const float* activation(const char* name, uint64_t& cap) override {
        const uint64_t bf = (uint64_t)last_b * ft_out;
        cap = bf;
        if (!std::strcmp(name, "ft_stm_out")) return ft_stm;
        if (!std::strcmp(name, "ft_nstm_out")) return ft_nstm;
        cap = 2 * bf;
        if (!std::strcmp(name, "combined")) return combined;
        cap = (uint64_t)last_b * l1;
        if (!std::strcmp(name, "l1_pre")) return l1_pre;
        if (!std::strcmp(name, "dl1_pre")) return dl1;
        cap = last_b;
        if (!std::strcmp(name, "net_output")) return net_out;
        return nullptr;
    }

    SimpleDenseArgs dense_args(const BatchPtrs& p, float wdl_lambda, const LossParams& lp, int slot) const {
        SimpleDenseArgs a{};
        a.batch = p.b;
        a.ft_out = ft_out;
        a.l1 = l1;
        a.l2 = l2;
        a.combined = combined;
        a.ft_stm = ft_stm;
        a.ft_nstm = ft_nstm;
        a.l1_pre = l1_pre;
        a.dl1 = dl1;
        a.net_output = net_out;
        a.dft = dft;
        a.score = p.score;
        a.wdl = p.wdl;
        a.per_pos_norm = p.b ? 1.0f / (float)p.b : 0.0f;
        a.wdl_lambda = wdl_lambda;
        a.loss = lp;
        a.weight_sum = weight_sum;
        a.l1_w = small[1].w;
        a.l1_b = small[2].w;
        a.l2_w = small[3].w;
        a.l2_b = small[4].w;
        a.l3_w = small[5].w;
        a.l3_b = small[6].w;
        a.tail_partial = tail_partial;
        a.loss_partial = loss_partial;
        a.w1_partial = w1_partial;
        a.ftb_partial = ftb_partial;
        a.tail_sum = tail_sum;
        a.w1_sum = w1_sum;
        a.ftb_sum = ftb_sum;
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

    // FT gradient + update: the block scan and, gated on the device by the
    // flag of the hit-mask pass, the occurrence-list kernel for a batch with
    // a row the scan cannot take; or occurrence lists every step when the
    // trainer does not scan.
    int32_t ft_gradient(const BatchPtrs& p, const FtGradArgs& fb) {
        if (use_scan) return launch_ft_grad_scan(fb, block_scan(p), stream, !batch_king_blocked);
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
        sc.dealt = 1;
        return sc;
    }

    int32_t forward(const BatchPtrs& p, float wdl_lambda, const LossParams& lp, int32_t train, int slot) {
        int32_t st;
        const uint32_t b = p.b;
        if (train && (st = prof_mark(0))) return st;
        if (train && !use_scan) {
            // occurrence lists for the FT backward, on the side stream: they
            // depend only on the indices and are first needed by the FT
            // gradient, so the sort overlaps the forward
            if ((st = fork_side())) return st;
            if ((st = sort_occurrences(p, side))) return st;
        }
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
        if (train && (st = prof_mark(1))) return st;
        FtForwardArgs fa{};
        fa.mode = 2;  // Simple: x = sum + bias in place, combined = [crelu(stm) | crelu(nstm)]
        fa.W = factorized ? comb : ft.w;
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
        fa.batch = b;
        fa.ft_out = ft_out;
        fa.cols = ft_in;
        fa.max_active = max_active;
        fa.n_persp = 2;
        fa.scale = 1.0f;
        if ((st = launch_ft_forward(fa, stream))) return st;
        if (train && (st = prof_mark(2))) return st;
        const SimpleDenseArgs da = dense_args(p, wdl_lambda, lp, slot);
        if ((st = launch_simple_l1_forward(da, stream))) return st;
        if (lp.kind == 1 && lp.extended) {
            if ((st = launch_wrm_weight_sum(p.score, b, lp, weight_sum, wrm_scratch, stream))) return st;
        }
        if ((st = launch_simple_tail(da, train, stream))) return st;
        return launch_sum_f64(loss_partial, simple_tail_workgroups(b), loss_out + slot, stream);
    }

    int32_t train_step(const TataraBatch* bt, float lr, float wdl_lambda, const TataraLoss* l,
                       double* lagged) override {
        int32_t st;
        if ((st = check_loss(l))) return st;
        BatchPtrs p{};
        if ((st = stage_batch(bt, p, false, 1, max_b))) return st;
        if (p.b == 0) {
            if (lagged) *lagged = 0.0;
            return kOk;
        }
        const LossParams lp = loss_params(l);
        const int slot = next_slot;
        if ((st = forward(p, wdl_lambda, lp, 1, slot))) return st;
        const SimpleDenseArgs da = dense_args(p, wdl_lambda, lp, slot);
        if ((st = prof_mark(3))) return st;
        if ((st = launch_simple_l1_weight_grad(da, stream))) return st;
        if ((st = launch_simple_l1_input_post(da, stream))) return st;
        if ((st = prof_mark(4))) return st;

        step_count += 1;
        FtGradArgs fb{};
        fb.dft = dft;
        fb.dft_row_stride = kDftChunk;  // chunk-major [chunk][2*b][256]
        fb.dft_chunk_stride = 2ull * p.b * kDftChunk;
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
        fb.opt = scalars(0, lr, step_count);
        if ((st = join_side())) return st;
        if ((st = ft_gradient(p, fb))) return st;
        if ((st = prof_mark(5))) return st;
        if (factorized && (st = launch_ft_virtual_fold(fb, pi, comb, nullptr, stream, table_layout()))) return st;
        if ((st = prof_mark(6))) return st;
        SimpleDenseGroup groups[7];
        for (int k = 0; k < 7; ++k) {
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
        if ((st = launch_simple_dense_finalize(da, groups, scalars(1, lr, step_count),
                                               scalars(2, lr, step_count), cfg.keep_grads, stream)))
            return st;
        if ((st = prof_mark(7))) return st;
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
        if ((st = stage_batch(bt, p, false, 1, max_b))) return st;
        if (p.b == 0) {
            if (sse) *sse = 0.0;
            return kOk;
        }
        const LossParams lp = loss_params(l);
        const int slot = next_slot;
        if ((st = forward(p, wdl_lambda, lp, 0, slot))) return st;
        double v = 0.0;
        TATARA_HIP(hipMemcpyAsync(&v, loss_out + slot, sizeof(double), hipMemcpyDeviceToHost, stream),
                   "validate loss");
        if (net_host)
            TATARA_HIP(hipMemcpyAsync(net_host, net_out, 4ull * p.b, hipMemcpyDeviceToHost, stream),
                       "validate net");
        TATARA_HIP(hipStreamSynchronize(stream), "validate");
        last_b = p.b;
        if ((st = release_batch())) return st;
        if (sse) *sse = v;
        return kOk;
    }
};

}  // namespace

TrainerBase* new_simple_trainer() { return new SimpleTrainer(); }

}  // namespace tatara
