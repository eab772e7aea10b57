/*
 * tatara_hip.h - C ABI of the MI355X (gfx950) training backend for tatara's
 * GPU hot path (one training step: sparse FT gather, LayerStack dense layers
 * and loss, FT backward, optimizer).
 *
 * The ABI replaces the reference's device backend below its step API:
 *   - the trainer calls re-export `trait TrainerBackend`
 *     (crates/nnue-train/src/trainer.rs:273-375) as implemented by GpuTrainer
 *     (bins/nnue_train/src/trainer_layerstack.rs:1885-2010, via the macro at
 *     bins/nnue_train/src/trainer_common.rs:276-411);
 *   - the runtime calls replace the device-runtime surface of
 *     crates/gpu-runtime/src/lib.rs:50-126 / native_backend.rs:17-300
 *     (DeviceBuffer::from_host / zeroed / to_host_vec, memset, streams) and
 *     the driver FFI of crates/cuda-native-runtime/src/runtime.rs:16-78;
 *   - the op calls are the hot kernels of
 *     crates/cuda-native-runtime/kernels/native_kernels.cu, one entry point
 *     per reference kernel family, for kernel-level parity checks.
 *
 * Conventions: every function returns int32 status (0 = ok, <0 = error; see
 * TATARA_* codes); tatara_last_error() returns the thread's last message
 * ("HIP error {code}: {name}: {msg} [{call}]").  Out-of-memory is reported as
 * TATARA_ERR_OOM so callers can classify it (native_backend.rs:294-300).
 * Device pointers are plain void* from tatara_malloc.  Nothing in this header
 * uses a torch or HIP type.
 */
#ifndef TATARA_HIP_H
#define TATARA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define TATARA_API __attribute__((visibility("default")))
#else
#define TATARA_API
#endif

#define TATARA_OK 0
#define TATARA_ERR_HIP (-1)
#define TATARA_ERR_OOM (-2)
#define TATARA_ERR_INVALID (-3)
#define TATARA_ERR_STATE (-4)

/* ------------------------------------------------------------------------ */
/* Runtime (crates/gpu-runtime/src/lib.rs:50-126, :190-400)                 */
/* ------------------------------------------------------------------------ */

/* Thread-local message of the last failing call (never NULL). */
TATARA_API const char* tatara_last_error(void);
/* Library version string. */
TATARA_API const char* tatara_version(void);
/* Number of visible GPUs (CudaContext::new ordinal range). */
TATARA_API int32_t tatara_device_count(int32_t* count);
/* Selects the device for subsequent calls on this thread. */
TATARA_API int32_t tatara_set_device(int32_t device);
/* Device name and compute-unit count (DeviceOccupancy::query). */
TATARA_API int32_t tatara_device_info(int32_t device, char* name, int32_t name_len, int32_t* cu_count);
/* DeviceBuffer::zeroed / from_host / to_host_vec / memset_d8_async. */
TATARA_API int32_t tatara_malloc(void** ptr, uint64_t bytes);
TATARA_API int32_t tatara_free(void* ptr);
TATARA_API int32_t tatara_memcpy_htod(void* dst, const void* src, uint64_t bytes);
TATARA_API int32_t tatara_memcpy_dtoh(void* dst, const void* src, uint64_t bytes);
TATARA_API int32_t tatara_memset(void* dst, int32_t byte, uint64_t bytes);
/* Waits for all work on the device (CudaStream::synchronize). */
TATARA_API int32_t tatara_synchronize(void);

/* Streams, events, asynchronous copies, pinned host memory and code-object
 * modules: the rest of the runtime surface (native_backend.rs:33-300,
 * lib.rs:186-390).  Handles are opaque.  Every stream is created at the
 * default priority and does not synchronise with the null stream; a NULL
 * stream argument is the device's null stream.  The calls that take a device
 * make it current on the calling thread (CudaContext::bind_to_thread). */
typedef struct TataraStream TataraStream;
typedef struct TataraEvent TataraEvent;
typedef struct TataraModule TataraModule;

/* (multiprocessor count, max threads per multiprocessor) as
 * device_occupancy_attributes (lib.rs:364-390, native_backend.rs:81-88);
 * here compute units and their thread capacity. */
TATARA_API int32_t tatara_device_occupancy_attributes(int32_t device, int32_t* cu_count,
                                                      int32_t* max_threads_per_cu);
/* CudaContext::compute_capability (native_backend.rs:72-79): the HIP
 * (major, minor) of the device, 9.5 for gfx950. */
TATARA_API int32_t tatara_device_compute_capability(int32_t device, int32_t* major, int32_t* minor);
/* CudaContext::new_stream / CudaStream::synchronize / CudaStream::wait
 * (native_backend.rs:54-60, :105-112). */
TATARA_API int32_t tatara_stream_create(int32_t device, TataraStream** out);
TATARA_API int32_t tatara_stream_destroy(TataraStream* stream);
TATARA_API int32_t tatara_stream_synchronize(TataraStream* stream);
TATARA_API int32_t tatara_stream_wait_event(TataraStream* stream, TataraEvent* event);
/* CudaContext::new_event / CudaEvent::record / CudaEvent::synchronize
 * (native_backend.rs:61-67, :129-136).  flags: a combination of the two
 * below (0: timing enabled, spin wait). */
#define TATARA_EVENT_BLOCKING_SYNC 1
#define TATARA_EVENT_DISABLE_TIMING 2
TATARA_API int32_t tatara_event_create(int32_t device, uint32_t flags, TataraEvent** out);
TATARA_API int32_t tatara_event_destroy(TataraEvent* event);
TATARA_API int32_t tatara_event_record(TataraEvent* event, TataraStream* stream);
TATARA_API int32_t tatara_event_synchronize(TataraEvent* event);
/* 1 when the event's recorded work has finished, 0 while it is pending. */
TATARA_API int32_t tatara_event_query(TataraEvent* event, int32_t* done);
/* Milliseconds between two completed events (both created with timing). */
TATARA_API int32_t tatara_event_elapsed_ms(TataraEvent* start, TataraEvent* end, float* ms);
/* memset_d8_async / memcpy_htod_async / memcpy_dtoh_async (lib.rs:232-310):
 * ordered on `stream`; the host buffer must stay alive (and, for dtoh,
 * untouched) until the stream has passed the copy, and overlaps other work
 * only when it is pinned (tatara_host_alloc_pinned). */
TATARA_API int32_t tatara_memset_d8_async(void* dst, uint8_t value, uint64_t bytes, TataraStream* stream);
TATARA_API int32_t tatara_memcpy_htod_async(void* dst, const void* src, uint64_t bytes, TataraStream* stream);
TATARA_API int32_t tatara_memcpy_dtoh_async(void* dst, const void* src, uint64_t bytes, TataraStream* stream);
/* alloc_pinned_host / free_pinned_host (lib.rs:318-360): page-locked host
 * memory, freed only after every copy that uses it has completed. */
TATARA_API int32_t tatara_host_alloc_pinned(uint64_t bytes, void** out);
TATARA_API int32_t tatara_host_free_pinned(void* ptr);
/* CudaContext::load_module_from_image (native_backend.rs:90-97): loads a
 * gfx950 code object (hipcc --genco) from memory; the image may be freed
 * after the call. */
TATARA_API int32_t tatara_module_load_image(int32_t device, const void* image, uint64_t bytes,
                                            TataraModule** out);
TATARA_API int32_t tatara_module_destroy(TataraModule* module);
/* CudaModule::launch (native_backend.rs:149-184): looks the kernel up by name
 * (cached per module) and launches it on `stream`.  args[i] points at the
 * i-th kernel argument's value, as KernelArgs holds them (push_slice is two
 * arguments: the device pointer and a u64 length); the caller guarantees
 * they match the kernel's parameters.  An unknown name fails with
 * TATARA_ERR_HIP before anything is launched. */
TATARA_API int32_t tatara_module_launch(TataraModule* module, const char* kernel, TataraStream* stream,
                                        const uint32_t grid[3], const uint32_t block[3], uint32_t shared_bytes,
                                        void** args);

/* ------------------------------------------------------------------------ */
/* Kernel-level ops (device pointers, default stream, synchronous errors)   */
/* ------------------------------------------------------------------------ */

/* sparse_ft_forward (native_kernels.cu:162-202; CPU ref
 * crates/gpu-kernels/src/sparse/sparse_ft_forward.rs:100-122):
 * out[b][r] = sum_{n<nnz[b]} W[idx[b][n]][r] for valid idx, in n order. */
TATARA_API int32_t tatara_op_sparse_ft_forward(const float* weight, const int32_t* indices,
                                    const int32_t* nnz, float* out, uint32_t batch,
                                    uint32_t rows, uint32_t cols, uint32_t max_active);
/* sparse_ft_forward x2 + ft_post_perspective_fwd (native_kernels.cu:1499-1527):
 * raw sums of both perspectives and the pairwise CReLU product `combined`. */
TATARA_API int32_t tatara_op_ft_forward_pairwise(const float* weight, const int32_t* stm_idx,
                                      const int32_t* nstm_idx, const int32_t* nnz,
                                      const float* bias, float* stm_out, float* nstm_out,
                                      float* combined, uint32_t batch, uint32_t ft_out,
                                      uint32_t cols, uint32_t max_active, uint32_t piece_inputs,
                                      float scale);
/* FT weight gradient of both perspectives (the inverse-index pipeline of
 * trainer_layerstack.rs:3723-3936; CPU ref sparse_ft_backward.rs:247-267,
 * stm then nstm): grad[f][c] = sum of dft rows that index f, summed in
 * (perspective, position) order.  dft is [2][batch][ft_out].  Overwrites
 * grad rows [0, cols).  Deterministic. */
TATARA_API int32_t tatara_op_ft_weight_grad(const float* dft, const int32_t* stm_idx,
                                 const int32_t* nstm_idx, const int32_t* nnz, float* grad,
                                 uint32_t batch, uint32_t ft_out, uint32_t cols,
                                 uint32_t max_active);
/* The same gradient computed the way the trainers compute it for a
 * factorized (king-bucketed) feature set: the rows of each king block are
 * walked once in (perspective, position) order and added to the features of
 * the block that occur in them, so every cell is the same sequential sum as
 * sparse_ft_backward.rs:247-267 (stm then nstm).  A batch with a row whose
 * features lie in two king blocks (piece_inputs rows each) is computed from
 * occurrence lists instead; *used_block_scan (optional) reports which path
 * ran.  Overwrites grad rows [0, cols).  Synchronises. */
TATARA_API int32_t tatara_op_ft_weight_grad_blocked(const float* dft, const int32_t* stm_idx,
                                         const int32_t* nstm_idx, const int32_t* nnz, float* grad,
                                         uint32_t batch, uint32_t ft_out, uint32_t cols,
                                         uint32_t max_active, uint32_t piece_inputs,
                                         uint32_t* used_block_scan);
/* The same from an f16 dft (the --ft-fp16-out mode,
 * gather_and_sum_per_feature_*_fp16, native_kernels.cu:1030-1100): each
 * cell is the sequential f32 sum of the f16 values (converted exactly), in
 * the same order, times dft_inv_scale. */
TATARA_API int32_t tatara_op_ft_weight_grad_blocked_f16(const uint16_t* dft16, float dft_inv_scale,
                                             const int32_t* stm_idx, const int32_t* nstm_idx,
                                             const int32_t* nnz, float* grad, uint32_t batch,
                                             uint32_t ft_out, uint32_t cols, uint32_t max_active,
                                             uint32_t piece_inputs, uint32_t* used_block_scan);
/* The same gradient from an f16 dft on the matrix cores (the mixed-precision
 * trainer's FT backward, replacing gather_and_sum_per_feature_*_fp16,
 * native_kernels.cu:1030-1100): per king block, the 0/1 hit matrix of
 * features x rows times the block's f16 dft rows, as f16 MFMA with f32
 * sums.  Each cell is the f32 sum of the same values as the sequential sum,
 * in another order, times dft_inv_scale (equal to within f32 summation
 * error, not bit for bit).  A batch with a row whose features lie in two
 * king blocks is computed from occurrence lists (sequential sums) instead;
 * *used_matrix_cores (optional) reports which path ran.  Synchronises. */
TATARA_API int32_t tatara_op_ft_weight_grad_mfma_f16(const uint16_t* dft16, float dft_inv_scale,
                                          const int32_t* stm_idx, const int32_t* nstm_idx,
                                          const int32_t* nnz, float* grad, uint32_t batch,
                                          uint32_t ft_out, uint32_t cols, uint32_t max_active,
                                          uint32_t piece_inputs, uint32_t* used_matrix_cores);
/* ft_fold_virtual / ft_reduce_virtual_grad, Base mode (native_kernels.cu:204-406). */
TATARA_API int32_t tatara_op_ft_fold_virtual(const float* weight, float* comb, uint32_t ft_in,
                                  uint32_t ft_out, uint32_t piece_inputs);
TATARA_API int32_t tatara_op_ft_reduce_virtual_grad(float* grad, uint32_t ft_in, uint32_t ft_out,
                                         uint32_t piece_inputs);
/* radam_step (native_kernels.cu:1291-1327) and ranger_lookahead_lerp (:1842). */
TATARA_API int32_t tatara_op_radam_step(float* weights, float* m, float* v, float* grad, float lr,
                             float step_size, int32_t denom, float decay, float beta1,
                             float beta2, float eps, float min_w, float max_w, uint64_t n);
TATARA_API int32_t tatara_op_ranger_lookahead_lerp(float* weights, float* slow, float alpha, uint64_t n);
/* Plain device-to-device copy (float4 grid-stride loop): the known-size
 * reference kernel used to calibrate HBM byte counters (FETCH_SIZE,
 * WRITE_SIZE).  bytes must be a multiple of 16.  No reference counterpart. */
TATARA_API int32_t tatara_op_copy(void* dst, const void* src, uint64_t bytes);
/* exp as the reference's CPU path evaluates it (Rust f32::exp = glibc expf on
 * linux-gnu; used by ShogiProgressKPAbs::progress_board,
 * crates/shogi-features/src/progress_kpabs.rs:140-150), elementwise on device
 * arrays.  Equal to glibc's result for every non-NaN float. */
TATARA_API int32_t tatara_op_expf(const float* x, float* y, uint64_t n);
/* FT-table quantisation of the quantised export.  Value i of the export-shape
 * table [rows][cols] is v = w[i], plus, with piece_inputs > 0, the virtual row
 * w[(rows + (i / cols) % piece_inputs) * cols + i % cols] added in f32
 * (coalesce_ft_factorized, crates/nnue-format/src/layerstack_weights.rs:412-491);
 * it is stored as saturate_i16(round(scale * (double)v)), rounding half away
 * from zero, NaN -> 0 (layerstack_weights.rs:639-676,
 * simple_weights.rs:596-603).  leb128 = 0: out receives rows*cols little-endian
 * i16 (the SimpleWeights FT block); leb128 = 1: out receives the values'
 * signed LEB128 bytes in order (encode_signed_leb128, layerstack_weights.rs:
 * 120-138), without the magic and size prefix.  w and out are device memory;
 * *out_bytes (host) receives the byte count, and out_capacity smaller than it
 * is an error.  Synchronous. */
TATARA_API int32_t tatara_op_quantise_ft(const float* w, uint64_t rows, uint32_t cols, uint32_t piece_inputs,
                                         double scale, int32_t leb128, uint8_t* out, uint64_t out_capacity,
                                         uint64_t* out_bytes);
/* tatara_op_quantise_ft without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results, byte for byte; the LEB128 path's per-tile
 * counts and offsets live in a static device array of 0.8 MB per GPU (held
 * until the process ends), so rows * cols is limited to 2^28 values (65536
 * tiles of 4096), larger tables are rejected with TATARA_ERR_INVALID.  Calls
 * on one GPU share that array: calls that overlap on one GPU race.
 * Synchronous. */
TATARA_API int32_t tatara_op_quantise_ft_noalloc(const float* w, uint64_t rows, uint32_t cols,
                                                 uint32_t piece_inputs, double scale, int32_t leb128, uint8_t* out,
                                                 uint64_t out_capacity, uint64_t* out_bytes);

/* ------------------------------------------------------------------------ */
/* Dataloader: PSV records -> batch (Batch::push_decoded + BucketMode)       */
/* ------------------------------------------------------------------------ */

/* FeatureSet (crates/shogi-features/src/feature_set.rs:55-185). */
#define TATARA_FS_HALFKP 0
#define TATARA_FS_HALFKA_SPLIT 1
#define TATARA_FS_HALFKA_MERGED 2
#define TATARA_FS_HALFKA_HM_SPLIT 3
#define TATARA_FS_HALFKA_HM_MERGED 4
/* BucketMode (crates/nnue-train/src/dataloader.rs:303-328); NONE gives bucket 0. */
#define TATARA_BUCKET_NONE 0
#define TATARA_BUCKET_KINGRANK9 1
#define TATARA_BUCKET_PROGRESS_KPABS 2

/* FeatureSetSpec::{king_buckets, piece_inputs, ft_in, max_active,
 * feature_hash} (feature_set.rs:262-520).  Outputs may be NULL. */
TATARA_API int32_t tatara_feature_set_info(int32_t feature_set, int32_t* king_buckets,
                                           int32_t* piece_inputs, int32_t* ft_in,
                                           int32_t* max_active, uint32_t* feature_hash);
/* n PackedSfenValue records (40 bytes each, packed_sfen.rs:255-268) -> the
 * arrays of Batch::push_decoded (dataloader.rs:444-497): index rows
 * [n][max_active] in FeatureSetSpec::extract_active_features order
 * (feature_set.rs:655-810), -1 past nnz; score = (float)i16 score; wdl 1 / 0.5 / 0
 * for win / draw / loss; bucket_idx by BucketMode::bucket_board (kingrank9,
 * kingrank9.rs:11-23, or KP-absolute progress with num_buckets in [1, 256] and
 * the 81*1548 progress weights as f32, progress_kpabs.rs:106-170; f64 file
 * values are rounded to nearest f32 as load_from_bin does).  All pointers are
 * device memory; bucket_idx may be NULL.  Decoded on the GPU, one thread per
 * record; synchronous. */
TATARA_API int32_t tatara_psv_to_batch(const uint8_t* psv, int32_t n, int32_t feature_set,
                                       int32_t bucket_mode, int32_t num_buckets,
                                       const float* progress_weights, int32_t* stm_indices,
                                       int32_t* nstm_indices, int32_t* nnz, int32_t* bucket_idx,
                                       float* score, float* wdl);

/* Host pre-compute of RAdam (crates/gpu-kernels/src/pointwise/radam_step.rs:75-97). */
TATARA_API int32_t tatara_radam_step_size_denom(uint64_t step, float beta1, float beta2,
                                     float n_sma_threshold, float* step_size, int32_t* denom);

/* ------------------------------------------------------------------------ */
/* Trainer (trait TrainerBackend, crates/nnue-train/src/trainer.rs:273-375)  */
/* ------------------------------------------------------------------------ */

typedef struct TataraTrainer TataraTrainer;

/* ------------------------------------------------------------------------ */
/* Schedules (crates/nnue-train/src/schedule.rs)                             */
/* ------------------------------------------------------------------------ */

/* LrSchedulerEnum (schedule.rs:365-420): kind and its fields.
 *   CONSTANT     ConstantLR { value = start }
 *   STEP         StepLR { start, gamma, step = period }: start * gamma^((sb-1)/step)
 *   DROP         DropLR { start, gamma, drop = period }
 *   LINEAR / COSINE / EXPONENTIAL  *DecayLR { initial_lr = start, final_lr = gamma,
 *                final_superbatch = period }
 *   ONE_CYCLE    OneCycleLR { initial_lr = start, max_lr, final_lr = gamma,
 *                warmup_superbatch = period, total_superbatch = total }
 *                (tatara_lr_schedule_one_cycle builds it as OneCycleLR::new)
 * warmup_batches > 0 wraps it in WarmupLR (LrSchedulerEnum::with_warmup).
 * next != NULL: SequenceLR { first = this, second = *next,
 * first_scheduler_final_superbatch = next_after } (schedule.rs:330-348). */
#define TATARA_LR_CONSTANT 0
#define TATARA_LR_STEP 1
#define TATARA_LR_DROP 2
#define TATARA_LR_LINEAR 3
#define TATARA_LR_COSINE 4
#define TATARA_LR_EXPONENTIAL 5
#define TATARA_LR_ONE_CYCLE 6
typedef struct TataraLrSchedule {
    int32_t kind;
    float start, gamma, max_lr;
    uint64_t period, total, warmup_batches;
    const struct TataraLrSchedule* next;
    uint64_t next_after;
} TataraLrSchedule;

/* WdlSchedulerEnum (schedule.rs:539-570): CONSTANT { value = start },
 * LINEAR { start, end }; warmup_batches > 0 wraps it in WarmupWDL; next !=
 * NULL: SequenceWDL { first = this, second = *next, midpoint = next_after }. */
#define TATARA_WDL_CONSTANT 0
#define TATARA_WDL_LINEAR 1
typedef struct TataraWdlSchedule {
    int32_t kind;
    float start, end;
    uint64_t warmup_batches;
    const struct TataraWdlSchedule* next;
    uint64_t next_after;
} TataraWdlSchedule;

/* OneCycleLR::new (schedule.rs:233-253). */
TATARA_API int32_t tatara_lr_schedule_one_cycle(float max_lr, float warmup_pct, float div_factor,
                                                float final_div_factor, uint64_t total_superbatch,
                                                TataraLrSchedule* out);
/* LrScheduler::lr(batch, superbatch) (schedule.rs:26). */
TATARA_API int32_t tatara_lr_at(const TataraLrSchedule* schedule, uint64_t batch, uint64_t superbatch, float* lr);
/* LrScheduler::horizon (schedule.rs:32-35): *has_horizon = 0 for none. */
TATARA_API int32_t tatara_lr_horizon(const TataraLrSchedule* schedule, uint64_t* horizon, int32_t* has_horizon);
/* WdlScheduler::blend(batch, superbatch, max) (schedule.rs:436); superbatch >= 1. */
TATARA_API int32_t tatara_wdl_at(const TataraWdlSchedule* schedule, uint64_t batch, uint64_t superbatch,
                                 uint64_t max, float* wdl);

#define TATARA_ARCH_LAYERSTACK 0
#define TATARA_ARCH_SIMPLE 1

#define TATARA_OPT_RANGER 0
#define TATARA_OPT_RADAM 1
#define TATARA_OPT_ADAMW 2

/* GpuTrainer::new arguments (trainer_layerstack.rs:781-1064) and the feature
 * set shape (crates/shogi-features/src/feature_set.rs:103-185). */
typedef struct TataraTrainerConfig {
    int32_t arch;          /* TATARA_ARCH_* */
    int32_t device;
    int32_t max_batch;     /* workspace capacity in positions (multiple of 16) */
    int32_t ft_in;         /* base FT input rows of the feature set */
    int32_t max_active;    /* active-feature slots per perspective (<= 64) */
    int32_t piece_inputs;  /* factorizer piece inputs; 0 = factorizer off */
    int32_t ft_out;        /* --ft-out */
    int32_t l1_out;        /* --l1 */
    int32_t l2_out;        /* --l2 */
    int32_t num_buckets;   /* --num-buckets (LayerStack) */
    int32_t optimizer;     /* TATARA_OPT_* */
    float ft_weight_decay, dense_weight_decay, bias_weight_decay;
    float ft_lr_mult, dense_lr_mult, bias_lr_mult;
    int32_t keep_grads;    /* debug: keep every gradient after the step */
    /* Mixed precision, PrecisionFlags (bins/nnue_train/src/trainer_common.rs:
     * 49-61; --all-optim sets all three).  LayerStack only; all 0 is the fp32
     * path.  ft_fp16: the FT forward reads an f16 table (the factorized comb,
     * or an f16 mirror of the weights), f32 accumulation.  ft_fp16_out (needs
     * ft_fp16): FT raw sums stored f16, the FT activation gradient stored f16
     * scaled by 2^14 * batch and clamped to +-65504 (clamps counted).
     * fp16_opt_state: the ft_w moments stored f16, scaled by 2^28 (m) and
     * 2^40 (v).  Master weights stay f32. */
    int32_t ft_fp16, ft_fp16_out, fp16_opt_state;
    /* PrecisionFlags.tf32 (--tf32, the fourth --all-optim flag): the L1
     * products (bucket and shared forward, weight and input gradients;
     * trainer_layerstack.rs:2388-2510, 3335-3540) with TF32-class operands.
     * gfx950 has no TF32 matrix instructions: `combined` is held as f16 and
     * the forward multiplies it by f16-rounded weights (10 fraction bits, as
     * TF32) on the f16 matrix cores; the weight gradients take that f16
     * `combined` with f32 dl1, and the input gradient stays f32; every sum
     * is f32.  LayerStack only. */
    int32_t tf32;
} TataraTrainerConfig;

/* LossKind (crates/nnue-train/src/trainer.rs:89-135). */
typedef struct TataraLoss {
    int32_t kind;  /* 0 Sigmoid{scale}, 1 Wrm{...} */
    float scale;
    float nnue2score, in_scaling, in_offset, target_offset, target_scaling;
    float pow_exp, qp_asymmetry, weight_boost_w1, weight_boost_w2;
} TataraLoss;

/* BatchData (bins/nnue_train/src/trainer_common.rs:142-153).  Index rows are
 * [n_pos][max_active], -1 padding; valid slots are [0, nnz[b]).  With
 * on_device = 0 the arrays are host memory and are copied before the call
 * returns; with on_device = 1 they are device pointers (tatara_malloc) that
 * must stay valid until the next train_step/validate_step/flush returns.
 * on_device = TATARA_BATCH_KING_BLOCKED (2) is on_device = 1 plus the
 * caller's statement that every row's active features lie in the king block
 * of its perspective and none repeats (true for tatara_psv_to_batch output of
 * a king-bucketed feature set from records whose two king squares differ):
 * the step then queues no occurrence-list fallback for its FT backward.  A
 * batch for which the statement is false trains without its FT weight
 * gradient, and the next tatara_trainer_flush_pending_loss returns
 * TATARA_ERR_STATE (no counterpart in the reference, whose host batches
 * carry no such statement). */
#define TATARA_BATCH_KING_BLOCKED 2
typedef struct TataraBatch {
    int32_t n_pos;
    int32_t max_active;
    const int32_t* stm_indices;
    const int32_t* nstm_indices;
    const int32_t* nnz;
    const int32_t* bucket_idx; /* LayerStack: bucket per position */
    const float* score;
    const float* wdl;
    int32_t on_device;
} TataraBatch;

/* GpuTrainer::new with LayerStackInit::default_uniform / SimpleInit (init.rs:252-310). */
TATARA_API int32_t tatara_trainer_create(const TataraTrainerConfig* config, TataraTrainer** out);
/* Drop for GpuTrainer: synchronises, then frees. */
TATARA_API int32_t tatara_trainer_destroy(TataraTrainer* trainer);
/* TrainerBackend::train_step: one forward+backward+optimizer step.  Returns in
 * *lagged_loss the sum of squared errors of the PREVIOUS step (0.0 on the
 * first), as AsyncLossRing does (trainer_common.rs:909-1035). */
TATARA_API int32_t tatara_trainer_train_step(TataraTrainer* trainer, const TataraBatch* batch, float lr,
                                  float wdl_lambda, const TataraLoss* loss, double* lagged_loss);
/* TrainerBackend::flush_pending_loss. */
TATARA_API int32_t tatara_trainer_flush_pending_loss(TataraTrainer* trainer, double* loss);
/* TrainerBackend::validate_step: forward + loss only; net_output may be NULL. */
TATARA_API int32_t tatara_trainer_validate_step(TataraTrainer* trainer, const TataraBatch* batch,
                                     float wdl_lambda, const TataraLoss* loss, double* sum_sq_err,
                                     float* net_output);
/* Quantised network export of the trainer's current weights to the file at
 * `path` (GpuTrainer::save_checkpoint with OutputFormat::Tatara).
 * LayerStack: LayerStackWeights::save_quantised (crates/nnue-format/src/
 * layerstack_weights.rs:568-829) of to_layerstack_weights
 * (bins/nnue_train/src/trainer_layerstack.rs:1351-1420): FT i16 = round(127 w)
 * as signed LEB128, L1 bucket + shared merged to i8 = round(64 w) with i32
 * biases = round(8128 b), L2 / L3 likewise, inputs padded to 32;
 * has_fv_scale = 0 omits ",fv_scale=N" (fv_scale: Option<i32>; training.rs:
 * 72-86 derives it).  Simple: SimpleWeights::save_quantised (simple_weights.rs:
 * 374-429) of to_simple_weights (trainer_simple.rs:2680-2745) with the CReLU
 * activation: raw i16 FT, fv_scale always written (has_fv_scale must be 1;
 * simple_fv_scale, simple_weights.rs:90-95).  The factorizer's virtual rows
 * are folded into the real rows (coalesce_ft_factorized).  feature_set
 * (TATARA_FS_*) names the arch string and hashes and must match the trainer's
 * ft_in (and piece_inputs with a factorizer).  Synchronous. */
TATARA_API int32_t tatara_trainer_export_quantised(TataraTrainer* trainer, const char* path, int32_t feature_set,
                                                   int32_t has_fv_scale, int32_t fv_scale);
/* TrainerBackend::read_fp16_clamp_count (crates/nnue-train/src/trainer.rs:
 * 362-373): cumulative count of dft values clamped to +-65504 and of dft
 * values written in the ft_fp16_out path (both 0 without it). */
TATARA_API int32_t tatara_trainer_fp16_clamp_count(TataraTrainer* trainer, uint64_t* clamps, uint64_t* elems);
/* Number of optimizer steps taken. */
TATARA_API int32_t tatara_trainer_step_count(TataraTrainer* trainer, uint64_t* steps);
/* Parameter groups by reference name ("ft_w", "ft_b", "l1_w", "l1_b",
 * "l1_shared_weight", "l1_shared_bias", "l2_w", "l2_b", "l3_w", "l3_b");
 * which: 0 weight, 1 m, 2 v, 3 slow, 4 grad.  n is the element count. */
TATARA_API int32_t tatara_trainer_tensor_size(TataraTrainer* trainer, const char* name, uint64_t* n);
TATARA_API int32_t tatara_trainer_get_tensor(TataraTrainer* trainer, const char* name, int32_t which,
                                  float* host, uint64_t n);
TATARA_API int32_t tatara_trainer_set_tensor(TataraTrainer* trainer, const char* name, int32_t which,
                                  const float* host, uint64_t n);
/* Activations of the last step, for parity checks: "ft_stm_out", "ft_nstm_out",
 * "combined", "net_output", "dft_stm", "dft_nstm"; LayerStack "l1_total"
 * ([b][l1], bucket + shared L1 output); Simple "l1_pre", "dl1_pre".
 * n = elements to copy. */
TATARA_API int32_t tatara_trainer_get_activation(TataraTrainer* trainer, const char* name, float* host,
                                      uint64_t n);
/* Phase timing (the NNUE_TRAIN_STEP_PROFILE breakdown, trainer_layerstack.rs:
 * 1885-1921, measured with HIP events on the trainer's stream instead of host
 * syncs).  While enabled, each step records events between its phases:
 *   0 prep (sorts)  1 FT gather + post  2 dense forward + loss
 *   3 dense backward (L1 weight grad, L1 input + FT post grad)
 *   4 FT gradient + optimizer (real rows)  5 factorizer virtual rows + fold
 *   6 dense optimizer
 * phase_times sums the elapsed milliseconds of every phase over the steps
 * run since profiling was enabled (it synchronises). */
TATARA_API int32_t tatara_trainer_set_profiling(TataraTrainer* trainer, int32_t enable);
TATARA_API int32_t tatara_trainer_phase_times(TataraTrainer* trainer, double* ms, int32_t n_phases,
                                   uint64_t* steps);
/* Rebuilds the forward weight table (factorizer fold) after set_tensor of
 * ft_w (sync_ft_forward_weights, trainer_layerstack.rs:1787). */
TATARA_API int32_t tatara_trainer_sync_forward_weights(TataraTrainer* trainer);

/* ------------------------------------------------------------------------ */
/* Raw resume checkpoints (RNRC version 8, bins/nnue_train/src/ckpt.rs)      */
/* ------------------------------------------------------------------------ */

/* RawCkptArch (ckpt.rs:213-226): the identity a header records.  The feature
 * set gives the canonical name, feature hash, train ft_in (+ its piece inputs
 * with ft_factorize) and max_active; LayerStack records bucket_mode
 * (TATARA_BUCKET_KINGRANK9 "kingrank9" or TATARA_BUCKET_PROGRESS_KPABS
 * "progress8kpabs") and topology [ft_out, l1_out, l2_out, num_buckets]
 * (layerstack_topology, ckpt.rs:186-199); Simple records no bucket mode
 * (TATARA_BUCKET_NONE) and [ft_out, l1_out, l2_out]. */
typedef struct TataraCkptArch {
    int32_t feature_set;   /* TATARA_FS_* */
    int32_t ft_factorize;
    int32_t arch;          /* TATARA_ARCH_* */
    int32_t bucket_mode;   /* TATARA_BUCKET_* */
    uint64_t ft_out, l1_out, l2_out, num_buckets;
} TataraCkptArch;

/* RawCkptHeader (ckpt.rs:247-265).  lr_horizon 0 and run_id "" mean none;
 * header_bytes is the offset of the first group. */
typedef struct TataraCkptHeader {
    uint32_t version;
    uint64_t superbatch, step_count, lr_horizon, num_groups, header_bytes;
    char run_id[257];
} TataraCkptHeader;

/* write_raw_ckpt_header (ckpt.rs:269-312): the version-8 header into out
 * (*out_bytes receives its size; capacity smaller than it is an error).  A
 * run id longer than 256 bytes is omitted.  Host only. */
TATARA_API int32_t tatara_ckpt_write_header(const TataraCkptArch* arch, const char* run_id, uint64_t superbatch,
                                            uint64_t step_count, uint64_t lr_horizon, uint64_t num_groups,
                                            uint8_t* out, uint64_t capacity, uint64_t* out_bytes);
/* read_raw_ckpt_header (ckpt.rs:322-612): parses a version 1..8 header from
 * memory and checks it against expected with the reference's rules (feature
 * set, factorizer flag, feature hash, ft_in, ft_out, max_active - twice the
 * base accepted when factorized -, arch kind, bucket mode - progress8kpabs
 * for LayerStack files before version 8 -, topology).  Malformed or
 * mismatching input returns TATARA_ERR_INVALID with the reference's message
 * ("... truncated while reading ...", "... arch kind mismatch ...").  Host
 * only. */
TATARA_API int32_t tatara_ckpt_read_header(const uint8_t* data, uint64_t n, const TataraCkptArch* expected,
                                           TataraCkptHeader* out);
/* GpuTrainer / SimpleGpuTrainer::save_raw_checkpoint (trainer_layerstack.rs:
 * 1577-1610, trainer_simple.rs:2870-2905; file by save_raw_checkpoint_file,
 * ckpt.rs:614-699): header, then per parameter group in the reference order
 * (LayerStack ft_w, ft_b, l1_w, l1_b, l1_shared_weight, l1_shared_bias, l2_w,
 * l2_b, l3_w, l3_b; Simple ft_w, ft_b, l1_w, l1_b, l2_w, l2_b, l3_w, l3_b) u64
 * len and f32 w, m, v, slow (f16 moments as their true f32 values).  Written
 * to "<path>.tmp" and renamed over path.  feature_set must match the
 * trainer's ft_in (and piece inputs with a factorizer).  Synchronous. */
TATARA_API int32_t tatara_trainer_save_resume(TataraTrainer* trainer, const char* path, int32_t feature_set,
                                              int32_t bucket_mode, uint64_t superbatch, const char* run_id,
                                              uint64_t lr_horizon);
/* load_raw_checkpoint (trainer_layerstack.rs:1631-1726, trainer_simple.rs:
 * 2907-2970; load_raw_checkpoint_file, ckpt.rs:705-754): checks the header,
 * the group count and every group length against the trainer and that the
 * file holds all group data, before changing any state; then uploads every
 * group (f16 moments re-quantised: f16(clamp(x * scale, +-65504))), restores
 * the step counter and rebuilds the forward table.  header may be NULL.
 * Synchronous. */
TATARA_API int32_t tatara_trainer_load_resume(TataraTrainer* trainer, const char* path, int32_t feature_set,
                                              int32_t bucket_mode, TataraCkptHeader* header);

/* ------------------------------------------------------------------------ */
/* Structured run log (crates/nnue-train/src/experiment.rs): one             */
/* experiment.json per run.  Host only.                                      */
/* ------------------------------------------------------------------------ */

/* ExperimentLogger (experiment.rs:356-540) with its document. */
typedef struct TataraExperiment TataraExperiment;

/* ExperimentDoc::new (experiment.rs:293-340): the document at the start of a
 * run (status "running", empty history, zeroed results; date and
 * last_updated_at from start_epoch_secs).  params_json is the "params" object
 * (experiment.rs:80-232), serialised by the caller that holds the run's
 * options; it is written as given.  NULL commit / lineage_parent_id omit
 * those fields; has_lineage = 0 omits "lineage"; has_fv_scale = 0 writes
 * "fv_scale": null. */
typedef struct TataraExperimentInit {
    const char* path;
    const char* id;
    const char* name;
    uint64_t start_epoch_secs;
    const char* commit;
    const char* command;
    const char* generator_version;
    int32_t has_lineage;
    const char* lineage_parent_id;
    const char* lineage_checkpoint;
    uint64_t lineage_superbatch;
    const char* params_json;
    const char* data_name;
    uint64_t data_positions;
    int32_t has_fv_scale, fv_scale;
} TataraExperimentInit;

TATARA_API int32_t tatara_experiment_create(const TataraExperimentInit* init, TataraExperiment** out);
TATARA_API int32_t tatara_experiment_destroy(TataraExperiment* e);
/* set_target_superbatches (experiment.rs:392-396) */
TATARA_API int32_t tatara_experiment_set_target_superbatches(TataraExperiment* e, uint64_t target);
/* record_superbatch (experiment.rs:398-487): one history entry; best loss and
 * best held-out loss (finite values only; a non-finite loss is recorded as
 * 0.0 with a warning on stderr, a non-finite held-out metric is omitted);
 * training_time_seconds = round(elapsed), mean_pos_per_sec =
 * round(positions so far / elapsed), total_positions and dataset_passes.
 * test_loss / test_accuracy may be NULL (no held-out validation). */
TATARA_API int32_t tatara_experiment_record_superbatch(TataraExperiment* e, uint64_t superbatch, double mean_loss,
                                                       uint64_t sb_positions, double elapsed_seconds,
                                                       const double* test_loss, const double* test_accuracy);
/* note_checkpoint, mark_finished, mark_interrupted (experiment.rs:489-507) */
TATARA_API int32_t tatara_experiment_note_checkpoint(TataraExperiment* e, const char* file_name);
TATARA_API int32_t tatara_experiment_mark_finished(TataraExperiment* e, double elapsed_seconds);
TATARA_API int32_t tatara_experiment_mark_interrupted(TataraExperiment* e);
/* write (experiment.rs:509-540): the pretty-printed document to <path>.tmp
 * (parent directories created), then renamed over <path>. */
TATARA_API int32_t tatara_experiment_write(TataraExperiment* e);
/* format_utc_iso / format_utc_compact (experiment.rs:562-576):
 * "YYYY-MM-DDTHH:MM:SSZ" (out: 21 bytes) and "YYYYMMDDtHHMMSSz" (17 bytes). */
TATARA_API int32_t tatara_format_utc_iso(uint64_t epoch_secs, char* out);
TATARA_API int32_t tatara_format_utc_compact(uint64_t epoch_secs, char* out);

/* ------------------------------------------------------------------------ */
/* Superbatch driver (crates/nnue-train/src/trainer.rs:759-1211, run)        */
/* ------------------------------------------------------------------------ */

/* TrainingConfig (trainer.rs:395-490), the fields the driver uses.  The
 * PSV records of data_path are read in file order and the file starts over
 * at its end (PsvEpochReader, dataloader.rs:724-760, one worker); each batch
 * is decoded on the GPU (tatara_psv_to_batch).  Checkpoints go to
 * "<output_dir>/<net_id>-<sb>.bin" (quantised, fv_scale when has_fv_scale)
 * and ".ckpt" (resume, with run_id and the LR horizon) when sb % save_rate
 * == 0 or sb == end_superbatch; has_keep_raw keeps only the newest
 * keep_raw_checkpoints ".ckpt" files (0 is ignored with a warning). */
typedef struct TataraRunConfig {
    const char* data_path;
    const char* output_dir;
    const char* net_id;
    const char* run_id;
    uint64_t start_superbatch, end_superbatch, batches_per_superbatch, batch_size, save_rate;
    int32_t has_fv_scale, fv_scale;
    int32_t has_keep_raw;
    uint64_t keep_raw_checkpoints;
    int32_t feature_set, bucket_mode, num_buckets;
    const float* progress_weights; /* device, 81*1548 f32, for the progress bucket mode */
    int32_t print_progress;         /* 1: the reference's per-superbatch line on stdout */
    /* The run's experiment.json, or NULL (run's `experiment`, trainer.rs:747-766):
     * written at the start, when control.json sets a new target, after every
     * superbatch (with the checkpoint names it saved) and, marked completed,
     * at the end; a failed write is reported on stderr and the run goes on.
     * Its id is the run id written into resume checkpoints (run_id is then
     * not used).  An error return leaves marking it interrupted to the
     * caller, as the reference's CLI does. */
    TataraExperiment* experiment;
} TataraRunConfig;

/* ControlState (crates/nnue-train/src/trainer.rs:640-656): the run's
 * effective last superbatch and the stale target last warned about. */
typedef struct TataraControlState {
    uint64_t effective_target;
    uint64_t ignored_stale_target;
    int32_t has_ignored_stale;
} TataraControlState;

/* apply_control (trainer.rs:670-731), what tatara_train_run does at the start
 * of every superbatch: reads control_path ({"target_superbatches": N}; other
 * fields ignored, null or absent = no request); a missing file is silent, an
 * unreadable or malformed one is reported on stderr and ignored; N below
 * start_superbatch is ignored with one warning per value; otherwise the
 * target is N clamped to [current_superbatch, configured_end] and, when it
 * differs from state->effective_target, becomes it, is printed and appended
 * to history_path as {"type":"control","timestamp":"<UTC ISO 8601>",
 * "target_superbatches":T,"superbatch":S} (a failed append is reported and
 * ignored).  *applied = 1 and *target = T when a new target was applied.
 * Host only. */
TATARA_API int32_t tatara_control_apply(const char* control_path, const char* history_path,
                                        TataraControlState* state, uint64_t current_superbatch,
                                        uint64_t start_superbatch, uint64_t configured_end, int32_t* applied,
                                        uint64_t* target);

/* One superbatch of a run: the summed (lagged + flushed) loss, positions,
 * mean loss, lr / wdl at batch 0, wall time, whether checkpoints were written. */
typedef struct TataraRunSuperbatch {
    uint64_t superbatch, positions;
    double loss_sum, mean_loss, seconds;
    float lr, wdl;
    int32_t saved;
} TataraRunSuperbatch;

/* run (trainer.rs:759-1211) over superbatches start..=end: per batch
 * lr = lr_scheduler.lr(batch_idx, sb), wdl = wdl_scheduler.blend(batch_idx,
 * sb, end_superbatch), train_step; per superbatch flush_pending_loss, report,
 * checkpoints.  report (capacity report_cap) receives one record per
 * superbatch; lr_seen / wdl_seen (capacity seen_cap, may be NULL) every
 * step's values.  <output_dir>/control.json is read at the start of every
 * superbatch (tatara_control_apply) and can end the run early.  Not covered:
 * held-out validation, score drop/clamp, shuffle windows, monitors. */
TATARA_API int32_t tatara_train_run(TataraTrainer* trainer, const TataraRunConfig* config,
                                    const TataraLrSchedule* lr, const TataraWdlSchedule* wdl,
                                    const TataraLoss* loss, TataraRunSuperbatch* report, uint64_t report_cap,
                                    uint64_t* n_report, float* lr_seen, float* wdl_seen, uint64_t seen_cap);

#ifdef __cplusplus
}
#endif

#endif /* TATARA_HIP_H */
