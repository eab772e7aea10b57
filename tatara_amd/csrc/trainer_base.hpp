// State and services shared by the LayerStack and Simple trainers: the
// stream, parameter groups, batch staging, optimizer scalars, the lagged loss
// ring (AsyncLossRing, bins/nnue_train/src/trainer_common.rs:909-1035) and
// phase profiling.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "../../include/tatara_hip.h"
#include "common.hpp"
#include "loss.hpp"
#include "optim.hpp"

namespace tatara {

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
    const char* name = "";
    float *w = nullptr, *m = nullptr, *v = nullptr, *slow = nullptr, *grad = nullptr;
    // f16 moments stored x m_scale / x v_scale, allocated instead of m / v
    // (MomentBuf::F16, bins/nnue_train/src/trainer_common.rs:63-132)
    uint16_t *m16 = nullptr, *v16 = nullptr;
    float m_scale = 1.0f, v_scale = 1.0f;
    uint64_t n = 0;
    float min_w = 0.f, max_w = 0.f;
    int32_t kind = 0;  // 0 ft, 1 dense, 2 bias
};

struct BatchPtrs {
    const int32_t *stm = nullptr, *nstm = nullptr, *nnz = nullptr, *bucket = nullptr;
    const float *score = nullptr, *wdl = nullptr;
    uint32_t b = 0;
};

class TrainerBase {
   public:
    static constexpr int kPhases = 7;  // prep, ft_forward, dense_forward, dense_backward,
                                       // ft_grad_update, ft_virtual_fold, dense_opt

    TataraTrainerConfig cfg{};
    hipStream_t stream = nullptr;
    // second stream for work that only depends on the batch indices (the
    // occurrence sort of the FT backward), overlapped with the forward
    hipStream_t side = nullptr;
    DeviceArena arena;
    uint64_t step_count = 0;
    uint32_t last_b = 0;
    bool profiling = false;
    double phase_ms[kPhases] = {0, 0, 0, 0, 0, 0, 0};
    uint64_t prof_steps = 0;

    virtual ~TrainerBase();
    virtual int32_t create(const TataraTrainerConfig& c) = 0;
    virtual ParamGroup* find(const char* name) = 0;
    virtual int32_t train_step(const TataraBatch* bt, float lr, float wdl_lambda, const TataraLoss* l,
                               double* lagged) = 0;
    virtual int32_t validate(const TataraBatch* bt, float wdl_lambda, const TataraLoss* l, double* sse,
                             float* net_host) = 0;
    virtual int32_t sync_forward_weights() = 0;
    // Device activation of the last batch and its element capacity, or null.
    virtual const float* activation(const char* name, uint64_t& cap) = 0;
    // Copies the first n elements of an activation to the host (row-major).
    virtual int32_t copy_activation(const char* name, float* host, uint64_t n);
    // Writes the quantised network of the current weights to `path`
    // (feature_set: TATARA_FS_*).
    virtual int32_t export_quantised(const char* path, int32_t feature_set, int32_t has_fv_scale,
                                     int32_t fv_scale) = 0;
    // Cumulative dft clamps and dft values written in the f16 activation path.
    virtual int32_t fp16_clamp_count(uint64_t* clamps, uint64_t* elems) {
        *clamps = 0;
        *elems = 0;
        return kOk;
    }

    // Returns the pending loss; also reports (kErrState) a step whose batch
    // was passed as king-blocked (on_device = 2) but had a row the block
    // scan cannot take.
    int32_t flush(double* out);
    int32_t prof_collect();

    // Host copies of one array of a group (which: 0 w, 1 m, 2 v, 3 slow,
    // 4 grad), n = g.n values.  f16 moments are read as f16 * (1 / scale)
    // and written as f16(clamp(x * scale, +-65504)) (MomentBuf::to_host_f32 /
    // from_host_f32, bins/nnue_train/src/trainer_common.rs:89-126).  An
    // unallocated gradient reads as zeros.  Synchronous; write_group does not
    // rebuild the forward table.
    int32_t read_group(const ParamGroup& g, int32_t which, float* host);
    int32_t write_group(ParamGroup& g, int32_t which, const float* host);
    // Reference names of the parameter groups in checkpoint order.
    virtual std::vector<const char*> group_names() const = 0;

   protected:
    // Host batches (on_device = 0) go through a two-slot upload ring
    // (InputUploadRing, bins/nnue_train/src/trainer_common.rs:1041-1370): the
    // caller's arrays are copied into a pinned slot before train_step returns,
    // the slot is uploaded on the copy stream into the matching device slot, and
    // the step waits for that upload with an event; a slot is refilled only
    // after the step that used it has finished reading it.  A batch of b
    // positions is packed the same way in the pinned and the device slot (stm,
    // nstm [b][ma] i32, nnz, bucket [b] i32, score, wdl [b] f32), so one copy
    // moves it.
    static constexpr int kRingSlots = 2;
    hipStream_t copy_stream = nullptr;
    uint8_t* ring_dev[kRingSlots] = {nullptr, nullptr};
    uint8_t* ring_host[kRingSlots] = {nullptr, nullptr};  // pinned, allocated at the first host batch
    hipEvent_t ring_copied[kRingSlots] = {nullptr, nullptr};   // upload of the slot done (copy stream)
    hipEvent_t ring_consumed[kRingSlots] = {nullptr, nullptr}; // last step using the slot done (compute stream)
    bool ring_busy[kRingSlots] = {false, false};
    int ring_next = 0;
    int ring_staged = -1;  // slot staged for the current step, released by release_batch
    uint64_t ring_cap = 0;
    uint32_t in_max_active = 0;
    // lagged loss ring
    double* pinned_loss = nullptr;
    hipEvent_t loss_ev[2] = {nullptr, nullptr};
    int pending = -1;  // slot holding the last queued loss
    int next_slot = 0;
    // A batch passed with on_device = 2: its rows are king-blocked, so the
    // step queues no occurrence-list fallback.  The stage-table pass latches
    // a violation into kb_broken_dev; a copy of it into kb_broken_host on the
    // side stream (event kb_ev) is read by the next flush.
    bool batch_king_blocked = false;
    uint32_t* kb_broken_dev = nullptr;
    uint32_t* kb_broken_host = nullptr;
    hipEvent_t kb_ev = nullptr;
    bool kb_pending = false;
    // after the stage tables of a king-blocked batch (queued on side)
    int32_t note_king_blocked_tables();
    // phase profiling: kPhases + 1 events per profiled step
    std::vector<hipEvent_t> prof_events;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;

    int32_t init_runtime(int device);
    int32_t alloc_inputs(uint64_t max_b, uint32_t max_active);
    int32_t alloc_group(ParamGroup& g, const char* name, uint64_t n, float mn, float mx, int kind,
                        bool with_grad, bool f16_moments = false);
    int32_t upload(float* dst, const std::vector<float>& src);
    // Synchronous copy of a group's weights to the host.
    int32_t download(const ParamGroup& g, std::vector<float>& out);
    // need_bucket: bucket_idx is required; multiple: n_pos must be a multiple of it
    int32_t stage_batch(const TataraBatch* bt, BatchPtrs& p, bool need_bucket, uint32_t multiple,
                        uint32_t max_b);
    // Marks the end of the current step's reads of a staged host batch (call
    // after the step's last kernel is queued).
    int32_t release_batch();
    OptScalars scalars(int kind, float lr, uint64_t step) const;
    LossParams loss_params(const TataraLoss* l) const;
    int32_t check_loss(const TataraLoss* l) const;
    // Queues this step's loss (device f64 at loss_dev[slot]) and returns the previous one.
    int32_t queue_loss(const double* loss_dev, int slot, double* lagged);
    int32_t prof_mark(int k);
    // Row-major copy of perspective persp of a chunk-major [chunk][2*b][256]
    // buffer of f32, or (f16 = true) of f16 values returned as f32.
    int32_t copy_chunk_major(const void* dev, bool f16, uint32_t b, uint32_t width, int persp, float* host,
                             uint64_t n);
    // The first n f16 values of a device buffer, as f32.
    int32_t copy_f16(const uint16_t* dev, float* host, uint64_t n);
    // side waits for everything enqueued on stream so far
    int32_t fork_side();
    // stream waits for everything enqueued on side so far
    int32_t join_side();
};

// The stream a trainer handle's steps run on (work enqueued there before a
// step is ordered before it).
hipStream_t trainer_stream(const TataraTrainer* h);

}  // namespace tatara
