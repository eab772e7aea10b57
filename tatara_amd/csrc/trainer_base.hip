// Shared trainer services (see trainer_base.hpp).
#include "trainer_base.hpp"

#include "binsort.hpp"

#include <cstring>

#include <cmath>
#include <limits>
#include <string>

namespace tatara {

namespace {
constexpr float kBeta2 = 0.999f;  // RangerParams::DEFAULT (crates/nnue-train/src/optimizer.rs)
constexpr float kEps = 1e-8f;
constexpr float kAlpha = 0.5f;
constexpr uint64_t kRangerK = 6;
constexpr float kNSmaThreshold = 5.0f;
}  // namespace

TrainerBase::~TrainerBase() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (copy_stream) (void)hipStreamSynchronize(copy_stream);
    for (int s = 0; s < kRingSlots; ++s) {
        if (ring_host[s]) (void)hipHostFree(ring_host[s]);
        if (ring_copied[s]) (void)hipEventDestroy(ring_copied[s]);
        if (ring_consumed[s]) (void)hipEventDestroy(ring_consumed[s]);
    }
    if (copy_stream) (void)hipStreamDestroy(copy_stream);
    for (hipEvent_t e : prof_events) (void)hipEventDestroy(e);
    for (auto& e : loss_ev)
        if (e) (void)hipEventDestroy(e);
    if (side) (void)hipStreamSynchronize(side);
    if (ev_fork) (void)hipEventDestroy(ev_fork);
    if (ev_join) (void)hipEventDestroy(ev_join);
    if (pinned_loss) (void)hipHostFree(pinned_loss);
    if (kb_ev) (void)hipEventDestroy(kb_ev);
    if (kb_broken_host) (void)hipHostFree(kb_broken_host);
    if (side) (void)hipStreamDestroy(side);
    if (stream) (void)hipStreamDestroy(stream);
}

int32_t TrainerBase::init_runtime(int device) {
    TATARA_HIP(hipSetDevice(device), "hipSetDevice");
    TATARA_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
    TATARA_HIP(hipStreamCreateWithFlags(&side, hipStreamNonBlocking), "hipStreamCreate (side)");
    TATARA_HIP(hipEventCreateWithFlags(&ev_fork, hipEventDisableTiming), "hipEventCreate");
    TATARA_HIP(hipEventCreateWithFlags(&ev_join, hipEventDisableTiming), "hipEventCreate");
    TATARA_HIP(hipEventCreateWithFlags(&loss_ev[0], hipEventDisableTiming), "hipEventCreate");
    TATARA_HIP(hipEventCreateWithFlags(&loss_ev[1], hipEventDisableTiming), "hipEventCreate");
    TATARA_HIP(hipHostMalloc((void**)&pinned_loss, 2 * sizeof(double), hipHostMallocDefault),
               "hipHostMalloc loss ring");
    TATARA_HIP(hipStreamCreateWithFlags(&copy_stream, hipStreamNonBlocking), "hipStreamCreate (copy)");
    TATARA_HIP(hipEventCreateWithFlags(&kb_ev, hipEventDisableTiming), "hipEventCreate");
    TATARA_HIP(hipHostMalloc((void**)&kb_broken_host, sizeof(uint32_t), hipHostMallocDefault),
               "hipHostMalloc king-block check");
    *kb_broken_host = 0;
    int32_t st = arena.alloc(&kb_broken_dev, 1);
    if (st) return st;
    for (int s = 0; s < kRingSlots; ++s) {
        TATARA_HIP(hipEventCreateWithFlags(&ring_copied[s], hipEventDisableTiming), "hipEventCreate");
        TATARA_HIP(hipEventCreateWithFlags(&ring_consumed[s], hipEventDisableTiming), "hipEventCreate");
    }
    return kOk;
}

namespace {

// Byte offsets of the arrays in an upload-ring slot of capacity B.
struct SlotLayout {
    uint64_t stm, nstm, nnz, bucket, score, wdl, bytes;
    SlotLayout(uint64_t B, uint64_t ma) {
        stm = 0;
        nstm = stm + 4 * B * ma;
        nnz = nstm + 4 * B * ma;
        bucket = nnz + 4 * B;
        score = bucket + 4 * B;
        wdl = score + 4 * B;
        bytes = wdl + 4 * B;
    }
};

}  // namespace

int32_t TrainerBase::alloc_inputs(uint64_t B, uint32_t max_active) {
    in_max_active = max_active;
    ring_cap = B;
    const SlotLayout L(B, max_active);
    int32_t st;
    for (int s = 0; s < kRingSlots; ++s)
        if ((st = arena.alloc(&ring_dev[s], L.bytes))) return st;
    return kOk;
}

int32_t TrainerBase::alloc_group(ParamGroup& g, const char* name, uint64_t n, float mn, float mx,
                                 int kind, bool with_grad, bool f16_moments) {
    g.name = name;
    g.n = n;
    g.min_w = mn;
    g.max_w = mx;
    g.kind = kind;
    int32_t st;
    if ((st = arena.alloc(&g.w, n)) || (st = arena.alloc(&g.slow, n))) return st;
    if (f16_moments) {
        if ((st = arena.alloc(&g.m16, n)) || (st = arena.alloc(&g.v16, n))) return st;
    } else if ((st = arena.alloc(&g.m, n)) || (st = arena.alloc(&g.v, n))) {
        return st;
    }
    if (with_grad && (st = arena.alloc(&g.grad, n))) return st;
    return kOk;
}

int32_t TrainerBase::upload(float* dst, const std::vector<float>& src) {
    TATARA_HIP(hipMemcpy(dst, src.data(), src.size() * sizeof(float), hipMemcpyHostToDevice),
               "upload init weights");
    return kOk;
}

int32_t TrainerBase::download(const ParamGroup& g, std::vector<float>& out) {
    out.resize(g.n);
    if (g.n == 0) return kOk;
    TATARA_HIP(hipMemcpyAsync(out.data(), g.w, g.n * sizeof(float), hipMemcpyDeviceToHost, stream),
               "download weights");
    TATARA_HIP(hipStreamSynchronize(stream), "download weights");
    return kOk;
}

int32_t TrainerBase::stage_batch(const TataraBatch* bt, BatchPtrs& p, bool need_bucket,
                                 uint32_t multiple, uint32_t max_b) {
    TATARA_REQUIRE(bt, "batch is null");
    TATARA_REQUIRE(bt->n_pos >= 0, "batch.n_pos must be >= 0");
    if (multiple > 1)
        TATARA_REQUIRE(bt->n_pos % multiple == 0,
                       "batch.n_pos must be a multiple of 16 (tiled kernels require b % 16 == 0)");
    TATARA_REQUIRE((uint32_t)bt->n_pos <= max_b, "batch exceeds workspace capacity");
    TATARA_REQUIRE((uint32_t)bt->max_active == in_max_active, "batch.max_active != feature set max_active");
    p.b = bt->n_pos;
    if (p.b == 0) return kOk;
    TATARA_REQUIRE(bt->stm_indices && bt->nstm_indices && bt->nnz && bt->score && bt->wdl,
                   "batch array is null");
    if (need_bucket) TATARA_REQUIRE(bt->bucket_idx, "batch.bucket_idx is null");
    if (ring_staged >= 0) {
        // a step that staged a batch ended early (an error): the work it
        // queued is ordered before everything that follows
        int32_t st = release_batch();
        if (st) return st;
    }
    TATARA_REQUIRE(bt->on_device >= 0 && bt->on_device <= 2, "batch.on_device must be 0, 1 or 2");
    batch_king_blocked = bt->on_device == 2;
    if (bt->on_device) {
        p.stm = bt->stm_indices;
        p.nstm = bt->nstm_indices;
        p.nnz = bt->nnz;
        p.bucket = bt->bucket_idx;
        p.score = bt->score;
        p.wdl = bt->wdl;
        return kOk;
    }
    // host arrays: copy into a pinned ring slot, upload it on the copy stream
    const uint64_t b = p.b, ma = in_max_active;
    const SlotLayout L(b, ma);  // packed for this batch: one copy moves it
    const int s = ring_next;
    if (!ring_host[s])
        TATARA_HIP(hipHostMalloc((void**)&ring_host[s], SlotLayout(ring_cap, ma).bytes, hipHostMallocDefault),
                   "hipHostMalloc upload ring");
    if (ring_busy[s]) {
        // the slot's previous upload (two steps ago) has left the pinned buffer
        TATARA_HIP(hipEventSynchronize(ring_copied[s]), "upload ring (pinned slot free)");
        // and the step that read the device slot has finished with it
        TATARA_HIP(hipStreamWaitEvent(copy_stream, ring_consumed[s], 0), "upload ring (device slot free)");
    }
    uint8_t* h = ring_host[s];
    std::memcpy(h + L.stm, bt->stm_indices, 4 * b * ma);
    std::memcpy(h + L.nstm, bt->nstm_indices, 4 * b * ma);
    std::memcpy(h + L.nnz, bt->nnz, 4 * b);
    if (need_bucket) std::memcpy(h + L.bucket, bt->bucket_idx, 4 * b);
    std::memcpy(h + L.score, bt->score, 4 * b);
    std::memcpy(h + L.wdl, bt->wdl, 4 * b);
    uint8_t* d = ring_dev[s];
    TATARA_HIP(hipMemcpyAsync(d, h, L.bytes, hipMemcpyHostToDevice, copy_stream), "H2D batch");
    TATARA_HIP(hipEventRecord(ring_copied[s], copy_stream), "upload ring record");
    TATARA_HIP(hipStreamWaitEvent(stream, ring_copied[s], 0), "upload ring wait");
    ring_busy[s] = true;
    ring_staged = s;
    ring_next = (s + 1) % kRingSlots;
    p.stm = reinterpret_cast<const int32_t*>(d + L.stm);
    p.nstm = reinterpret_cast<const int32_t*>(d + L.nstm);
    p.nnz = reinterpret_cast<const int32_t*>(d + L.nnz);
    p.bucket = need_bucket ? reinterpret_cast<const int32_t*>(d + L.bucket) : nullptr;
    p.score = reinterpret_cast<const float*>(d + L.score);
    p.wdl = reinterpret_cast<const float*>(d + L.wdl);
    return kOk;
}

int32_t TrainerBase::release_batch() {
    if (ring_staged < 0) return kOk;
    TATARA_HIP(hipEventRecord(ring_consumed[ring_staged], stream), "upload ring release");
    ring_staged = -1;
    return kOk;
}

OptScalars TrainerBase::scalars(int kind, float lr, uint64_t step) const {
    OptScalars s{};
    const int opt = cfg.optimizer;
    s.beta1 = opt == TATARA_OPT_RANGER ? 0.99f : 0.9f;
    s.beta2 = kBeta2;
    s.eps = kEps;
    if (opt == TATARA_OPT_ADAMW) {
        s.step_size = 1.0f;
        s.denom = 1;
    } else {
        (void)tatara_radam_step_size_denom(step, s.beta1, kBeta2, kNSmaThreshold, &s.step_size, &s.denom);
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
    // no clamp by default (W_CLAMP_NONE); groups with a quantised clamp set
    // their bounds where they are updated
    s.min_w = std::numeric_limits<float>::lowest();
    s.max_w = std::numeric_limits<float>::max();
    return s;
}

LossParams TrainerBase::loss_params(const TataraLoss* l) const {
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
    lp.extended =
        (l->kind == 1 && (l->pow_exp != 2.0f || l->qp_asymmetry != 0.0f || l->weight_boost_w1 != 0.0f))
            ? 1
            : 0;
    return lp;
}

int32_t TrainerBase::check_loss(const TataraLoss* l) const {
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

int32_t TrainerBase::queue_loss(const double* loss_dev, int slot, double* lagged) {
    double prev = 0.0;
    if (pending >= 0) {
        TATARA_HIP(hipEventSynchronize(loss_ev[pending]), "loss ring event");
        prev = pinned_loss[pending];
    }
    TATARA_HIP(hipMemcpyAsync(pinned_loss + slot, loss_dev + slot, sizeof(double), hipMemcpyDeviceToHost,
                              stream),
               "loss D2H");
    TATARA_HIP(hipEventRecord(loss_ev[slot], stream), "loss ring record");
    pending = slot;
    next_slot = 1 - slot;
    if (lagged) *lagged = prev;
    return kOk;
}

int32_t TrainerBase::flush(double* out) {
    double v = 0.0;
    if (pending >= 0) {
        TATARA_HIP(hipEventSynchronize(loss_ev[pending]), "loss ring flush");
        v = pinned_loss[pending];
        pending = -1;
    }
    if (out) *out = v;
    if (kb_pending) {
        TATARA_HIP(hipEventSynchronize(kb_ev), "king-block check");
        kb_pending = false;
        if (*kb_broken_host) {
            *kb_broken_host = 0;
            const int32_t st = launch_fill_i32(reinterpret_cast<int32_t*>(kb_broken_dev), 1, 0, side);
            if (st) return st;
            set_error("a batch passed with on_device = 2 had a row with features of two king blocks or one "
                      "feature twice, so its FT weight gradient was left out; pass such batches with "
                      "on_device = 1");
            return kErrState;
        }
    }
    return kOk;
}

int32_t TrainerBase::note_king_blocked_tables() {
    TATARA_HIP(hipMemcpyAsync(kb_broken_host, kb_broken_dev, sizeof(uint32_t), hipMemcpyDeviceToHost, side),
               "king-block check copy");
    TATARA_HIP(hipEventRecord(kb_ev, side), "king-block check record");
    kb_pending = true;
    return kOk;
}

int32_t TrainerBase::fork_side() {
    TATARA_HIP(hipEventRecord(ev_fork, stream), "hipEventRecord (fork)");
    TATARA_HIP(hipStreamWaitEvent(side, ev_fork, 0), "hipStreamWaitEvent (fork)");
    return kOk;
}

int32_t TrainerBase::join_side() {
    TATARA_HIP(hipEventRecord(ev_join, side), "hipEventRecord (join)");
    TATARA_HIP(hipStreamWaitEvent(stream, ev_join, 0), "hipStreamWaitEvent (join)");
    return kOk;
}

int32_t TrainerBase::copy_activation(const char* name, float* host, uint64_t n) {
    uint64_t cap = 0;
    const float* src = activation(name, cap);
    TATARA_REQUIRE(src, std::string("unknown activation ") + name);
    TATARA_REQUIRE(n <= cap, "activation request exceeds the last batch");
    TATARA_HIP(hipStreamSynchronize(stream), "get_activation sync");
    TATARA_HIP(hipMemcpy(host, src, n * sizeof(float), hipMemcpyDeviceToHost), "get_activation");
    return kOk;
}

int32_t TrainerBase::copy_chunk_major(const void* dev, bool f16, uint32_t b, uint32_t width, int persp,
                                      float* host, uint64_t n) {
    constexpr uint32_t kChunk = 256;
    TATARA_REQUIRE(n <= (uint64_t)b * width, "activation request exceeds the last batch");
    TATARA_HIP(hipStreamSynchronize(stream), "get_activation sync");
    const uint32_t chunks = (width + kChunk - 1) / kChunk;
    const uint64_t total = (uint64_t)chunks * 2 * b * kChunk;
    std::vector<float> all(total);
    if (f16) {
        std::vector<_Float16> h(total);
        TATARA_HIP(hipMemcpy(h.data(), dev, total * 2, hipMemcpyDeviceToHost), "get_activation");
        for (uint64_t i = 0; i < total; ++i) all[i] = (float)h[i];
    } else {
        TATARA_HIP(hipMemcpy(all.data(), dev, total * sizeof(float), hipMemcpyDeviceToHost), "get_activation");
    }
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t r = i / width, c = i % width;
        host[i] = all[((c / kChunk) * 2 * b + (uint64_t)persp * b + r) * kChunk + c % kChunk];
    }
    return kOk;
}

namespace {

float* group_ptr(const ParamGroup& g, int32_t which) {
    switch (which) {
        case 0: return g.w;
        case 1: return g.m;
        case 2: return g.v;
        case 3: return g.slow;
        case 4: return g.grad;
        default: return nullptr;
    }
}

// The f16 array and scale of an f16 moment (MomentBuf::F16), or false.
bool f16_moment(const ParamGroup& g, int32_t which, uint16_t*& dev, float& scale) {
    if (which == 1 && g.m16) {
        dev = g.m16;
        scale = g.m_scale;
        return true;
    }
    if (which == 2 && g.v16) {
        dev = g.v16;
        scale = g.v_scale;
        return true;
    }
    return false;
}

}  // namespace

int32_t TrainerBase::read_group(const ParamGroup& g, int32_t which, float* host) {
    TATARA_REQUIRE(which >= 0 && which <= 4, "which must be 0..4");
    const uint64_t n = g.n;
    TATARA_HIP(hipStreamSynchronize(stream), "read_group sync");
    uint16_t* dev16 = nullptr;
    float scale = 1.0f;
    if (f16_moment(g, which, dev16, scale)) {
        std::vector<_Float16> h(n);
        TATARA_HIP(hipMemcpy(h.data(), dev16, n * 2, hipMemcpyDeviceToHost), "read_group");
        const float inv = 1.0f / scale;
        for (uint64_t i = 0; i < n; ++i) host[i] = (float)h[i] * inv;
        return kOk;
    }
    const float* src = group_ptr(g, which);
    if (which == 4 && !cfg.keep_grads) src = nullptr;
    if (!src) {
        // the optimizer leaves zero gradients; without keep_grads none are kept
        std::memset(host, 0, n * sizeof(float));
        return kOk;
    }
    TATARA_HIP(hipMemcpy(host, src, n * sizeof(float), hipMemcpyDeviceToHost), "read_group");
    return kOk;
}

int32_t TrainerBase::write_group(ParamGroup& g, int32_t which, const float* host) {
    TATARA_REQUIRE(which >= 0 && which <= 4, "which must be 0..4");
    const uint64_t n = g.n;
    TATARA_HIP(hipStreamSynchronize(stream), "write_group sync");
    uint16_t* dev16 = nullptr;
    float scale = 1.0f;
    if (f16_moment(g, which, dev16, scale)) {
        std::vector<_Float16> h(n);
        for (uint64_t i = 0; i < n; ++i) {
            float x = host[i] * scale;
            x = x < -65504.0f ? -65504.0f : (x > 65504.0f ? 65504.0f : x);
            h[i] = (_Float16)x;
        }
        TATARA_HIP(hipMemcpy(dev16, h.data(), n * 2, hipMemcpyHostToDevice), "write_group");
        return kOk;
    }
    float* dst = group_ptr(g, which);
    TATARA_REQUIRE(dst, "tensor not allocated (which)");
    TATARA_HIP(hipMemcpy(dst, host, n * sizeof(float), hipMemcpyHostToDevice), "write_group");
    return kOk;
}

int32_t TrainerBase::copy_f16(const uint16_t* dev, float* host, uint64_t n) {
    TATARA_HIP(hipStreamSynchronize(stream), "get_activation sync");
    std::vector<_Float16> h(n);
    TATARA_HIP(hipMemcpy(h.data(), dev, n * 2, hipMemcpyDeviceToHost), "get_activation");
    for (uint64_t i = 0; i < n; ++i) host[i] = (float)h[i];
    return kOk;
}

int32_t TrainerBase::prof_mark(int k) {
    if (!profiling) return kOk;
    hipEvent_t e = nullptr;
    TATARA_HIP(hipEventCreate(&e), "hipEventCreate (profiling)");
    TATARA_HIP(hipEventRecord(e, stream), "hipEventRecord (profiling)");
    prof_events.push_back(e);
    (void)k;
    return kOk;
}

int32_t TrainerBase::prof_collect() {
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

}  // namespace tatara
