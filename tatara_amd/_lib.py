"""ctypes binding of libtatara_hip.so (the C ABI declared in include/tatara_hip.h).

The library is built in-tree by tatara_amd/build.py.  Loading fails loudly
when it is missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtatara_hip.so"

c_f32p = C.POINTER(C.c_float)
c_i32p = C.POINTER(C.c_int32)
c_u64p = C.POINTER(C.c_uint64)
c_f64p = C.POINTER(C.c_double)


class TataraTrainerConfig(C.Structure):
    _fields_ = [
        ("arch", C.c_int32),
        ("device", C.c_int32),
        ("max_batch", C.c_int32),
        ("ft_in", C.c_int32),
        ("max_active", C.c_int32),
        ("piece_inputs", C.c_int32),
        ("ft_out", C.c_int32),
        ("l1_out", C.c_int32),
        ("l2_out", C.c_int32),
        ("num_buckets", C.c_int32),
        ("optimizer", C.c_int32),
        ("ft_weight_decay", C.c_float),
        ("dense_weight_decay", C.c_float),
        ("bias_weight_decay", C.c_float),
        ("ft_lr_mult", C.c_float),
        ("dense_lr_mult", C.c_float),
        ("bias_lr_mult", C.c_float),
        ("keep_grads", C.c_int32),
        ("ft_fp16", C.c_int32),
        ("ft_fp16_out", C.c_int32),
        ("fp16_opt_state", C.c_int32),
        ("tf32", C.c_int32),
    ]


class TataraLoss(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("scale", C.c_float),
        ("nnue2score", C.c_float),
        ("in_scaling", C.c_float),
        ("in_offset", C.c_float),
        ("target_offset", C.c_float),
        ("target_scaling", C.c_float),
        ("pow_exp", C.c_float),
        ("qp_asymmetry", C.c_float),
        ("weight_boost_w1", C.c_float),
        ("weight_boost_w2", C.c_float),
    ]


class TataraBatch(C.Structure):
    _fields_ = [
        ("n_pos", C.c_int32),
        ("max_active", C.c_int32),
        ("stm_indices", C.c_void_p),
        ("nstm_indices", C.c_void_p),
        ("nnz", C.c_void_p),
        ("bucket_idx", C.c_void_p),
        ("score", C.c_void_p),
        ("wdl", C.c_void_p),
        ("on_device", C.c_int32),
    ]


class TataraCkptArch(C.Structure):
    _fields_ = [
        ("feature_set", C.c_int32),
        ("ft_factorize", C.c_int32),
        ("arch", C.c_int32),
        ("bucket_mode", C.c_int32),
        ("ft_out", C.c_uint64),
        ("l1_out", C.c_uint64),
        ("l2_out", C.c_uint64),
        ("num_buckets", C.c_uint64),
    ]


class TataraCkptHeader(C.Structure):
    _fields_ = [
        ("version", C.c_uint32),
        ("superbatch", C.c_uint64),
        ("step_count", C.c_uint64),
        ("lr_horizon", C.c_uint64),
        ("num_groups", C.c_uint64),
        ("header_bytes", C.c_uint64),
        ("run_id", C.c_char * 257),
    ]


class TataraLrSchedule(C.Structure):
    pass


TataraLrSchedule._fields_ = [
    ("kind", C.c_int32),
    ("start", C.c_float),
    ("gamma", C.c_float),
    ("max_lr", C.c_float),
    ("period", C.c_uint64),
    ("total", C.c_uint64),
    ("warmup_batches", C.c_uint64),
    ("next", C.POINTER(TataraLrSchedule)),
    ("next_after", C.c_uint64),
]


class TataraWdlSchedule(C.Structure):
    pass


TataraWdlSchedule._fields_ = [
    ("kind", C.c_int32),
    ("start", C.c_float),
    ("end", C.c_float),
    ("warmup_batches", C.c_uint64),
    ("next", C.POINTER(TataraWdlSchedule)),
    ("next_after", C.c_uint64),
]


class TataraRunConfig(C.Structure):
    _fields_ = [
        ("data_path", C.c_char_p),
        ("output_dir", C.c_char_p),
        ("net_id", C.c_char_p),
        ("run_id", C.c_char_p),
        ("start_superbatch", C.c_uint64),
        ("end_superbatch", C.c_uint64),
        ("batches_per_superbatch", C.c_uint64),
        ("batch_size", C.c_uint64),
        ("save_rate", C.c_uint64),
        ("has_fv_scale", C.c_int32),
        ("fv_scale", C.c_int32),
        ("has_keep_raw", C.c_int32),
        ("keep_raw_checkpoints", C.c_uint64),
        ("feature_set", C.c_int32),
        ("bucket_mode", C.c_int32),
        ("num_buckets", C.c_int32),
        ("progress_weights", C.c_void_p),
        ("print_progress", C.c_int32),
        ("experiment", C.c_void_p),
    ]


class TataraExperimentInit(C.Structure):
    _fields_ = [
        ("path", C.c_char_p),
        ("id", C.c_char_p),
        ("name", C.c_char_p),
        ("start_epoch_secs", C.c_uint64),
        ("commit", C.c_char_p),
        ("command", C.c_char_p),
        ("generator_version", C.c_char_p),
        ("has_lineage", C.c_int32),
        ("lineage_parent_id", C.c_char_p),
        ("lineage_checkpoint", C.c_char_p),
        ("lineage_superbatch", C.c_uint64),
        ("params_json", C.c_char_p),
        ("data_name", C.c_char_p),
        ("data_positions", C.c_uint64),
        ("has_fv_scale", C.c_int32),
        ("fv_scale", C.c_int32),
    ]


class TataraControlState(C.Structure):
    _fields_ = [
        ("effective_target", C.c_uint64),
        ("ignored_stale_target", C.c_uint64),
        ("has_ignored_stale", C.c_int32),
    ]


class TataraRunSuperbatch(C.Structure):
    _fields_ = [
        ("superbatch", C.c_uint64),
        ("positions", C.c_uint64),
        ("loss_sum", C.c_double),
        ("mean_loss", C.c_double),
        ("seconds", C.c_double),
        ("lr", C.c_float),
        ("wdl", C.c_float),
        ("saved", C.c_int32),
    ]


# name -> (restype, argtypes); every entry point returns an int32 status
# except the two string getters.
SIGNATURES = {
    "tatara_last_error": (C.c_char_p, []),
    "tatara_version": (C.c_char_p, []),
    "tatara_device_count": (C.c_int32, [c_i32p]),
    "tatara_set_device": (C.c_int32, [C.c_int32]),
    "tatara_device_info": (C.c_int32, [C.c_int32, C.c_char_p, C.c_int32, c_i32p]),
    "tatara_malloc": (C.c_int32, [C.POINTER(C.c_void_p), C.c_uint64]),
    "tatara_free": (C.c_int32, [C.c_void_p]),
    "tatara_memcpy_htod": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "tatara_memcpy_dtoh": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "tatara_memset": (C.c_int32, [C.c_void_p, C.c_int32, C.c_uint64]),
    "tatara_synchronize": (C.c_int32, []),
    "tatara_device_occupancy_attributes": (C.c_int32, [C.c_int32, c_i32p, c_i32p]),
    "tatara_device_compute_capability": (C.c_int32, [C.c_int32, c_i32p, c_i32p]),
    "tatara_stream_create": (C.c_int32, [C.c_int32, C.POINTER(C.c_void_p)]),
    "tatara_stream_destroy": (C.c_int32, [C.c_void_p]),
    "tatara_stream_synchronize": (C.c_int32, [C.c_void_p]),
    "tatara_stream_wait_event": (C.c_int32, [C.c_void_p, C.c_void_p]),
    "tatara_event_create": (C.c_int32, [C.c_int32, C.c_uint32, C.POINTER(C.c_void_p)]),
    "tatara_event_destroy": (C.c_int32, [C.c_void_p]),
    "tatara_event_record": (C.c_int32, [C.c_void_p, C.c_void_p]),
    "tatara_event_synchronize": (C.c_int32, [C.c_void_p]),
    "tatara_event_query": (C.c_int32, [C.c_void_p, c_i32p]),
    "tatara_event_elapsed_ms": (C.c_int32, [C.c_void_p, C.c_void_p, C.POINTER(C.c_float)]),
    "tatara_memset_d8_async": (C.c_int32, [C.c_void_p, C.c_uint8, C.c_uint64, C.c_void_p]),
    "tatara_memcpy_htod_async": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "tatara_memcpy_dtoh_async": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "tatara_host_alloc_pinned": (C.c_int32, [C.c_uint64, C.POINTER(C.c_void_p)]),
    "tatara_host_free_pinned": (C.c_int32, [C.c_void_p]),
    "tatara_module_load_image": (C.c_int32, [C.c_int32, C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p)]),
    "tatara_module_destroy": (C.c_int32, [C.c_void_p]),
    "tatara_module_launch": (
        C.c_int32,
        [C.c_void_p, C.c_char_p, C.c_void_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_uint32,
         C.POINTER(C.c_void_p)],
    ),
    "tatara_op_sparse_ft_forward": (C.c_int32, [C.c_void_p] * 4 + [C.c_uint32] * 4),
    "tatara_op_ft_forward_pairwise": (
        C.c_int32,
        [C.c_void_p] * 8 + [C.c_uint32] * 5 + [C.c_float],
    ),
    "tatara_op_ft_weight_grad": (C.c_int32, [C.c_void_p] * 5 + [C.c_uint32] * 4),
    "tatara_op_ft_weight_grad_blocked": (C.c_int32, [C.c_void_p] * 5 + [C.c_uint32] * 5 + [C.c_void_p]),
    "tatara_op_ft_weight_grad_blocked_f16": (
        C.c_int32,
        [C.c_void_p, C.c_float] + [C.c_void_p] * 4 + [C.c_uint32] * 5 + [C.c_void_p],
    ),
    "tatara_op_ft_weight_grad_mfma_f16": (
        C.c_int32,
        [C.c_void_p, C.c_float] + [C.c_void_p] * 4 + [C.c_uint32] * 5 + [C.c_void_p],
    ),
    "tatara_op_ft_fold_virtual": (C.c_int32, [C.c_void_p, C.c_void_p] + [C.c_uint32] * 3),
    "tatara_op_ft_reduce_virtual_grad": (C.c_int32, [C.c_void_p] + [C.c_uint32] * 3),
    "tatara_op_radam_step": (
        C.c_int32,
        [C.c_void_p] * 4
        + [C.c_float, C.c_float, C.c_int32]
        + [C.c_float] * 6
        + [C.c_uint64],
    ),
    "tatara_op_ranger_lookahead_lerp": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_float, C.c_uint64]),
    "tatara_op_copy": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "tatara_op_expf": (C.c_int32, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "tatara_op_quantise_ft": (
        C.c_int32,
        [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_double, C.c_int32, C.c_void_p, C.c_uint64, c_u64p],
    ),
    "tatara_op_quantise_ft_noalloc": (
        C.c_int32,
        [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_double, C.c_int32, C.c_void_p, C.c_uint64, c_u64p],
    ),
    "tatara_feature_set_info": (C.c_int32, [C.c_int32, c_i32p, c_i32p, c_i32p, c_i32p, C.POINTER(C.c_uint32)]),
    "tatara_psv_to_batch": (
        C.c_int32,
        [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32] + [C.c_void_p] * 7,
    ),
    "tatara_radam_step_size_denom": (
        C.c_int32,
        [C.c_uint64, C.c_float, C.c_float, C.c_float, c_f32p, c_i32p],
    ),
    "tatara_trainer_create": (C.c_int32, [C.POINTER(TataraTrainerConfig), C.POINTER(C.c_void_p)]),
    "tatara_trainer_destroy": (C.c_int32, [C.c_void_p]),
    "tatara_trainer_train_step": (
        C.c_int32,
        [C.c_void_p, C.POINTER(TataraBatch), C.c_float, C.c_float, C.POINTER(TataraLoss), c_f64p],
    ),
    "tatara_trainer_flush_pending_loss": (C.c_int32, [C.c_void_p, c_f64p]),
    "tatara_trainer_validate_step": (
        C.c_int32,
        [C.c_void_p, C.POINTER(TataraBatch), C.c_float, C.POINTER(TataraLoss), c_f64p, c_f32p],
    ),
    "tatara_trainer_step_count": (C.c_int32, [C.c_void_p, c_u64p]),
    "tatara_trainer_tensor_size": (C.c_int32, [C.c_void_p, C.c_char_p, c_u64p]),
    "tatara_trainer_get_tensor": (C.c_int32, [C.c_void_p, C.c_char_p, C.c_int32, c_f32p, C.c_uint64]),
    "tatara_trainer_set_tensor": (C.c_int32, [C.c_void_p, C.c_char_p, C.c_int32, c_f32p, C.c_uint64]),
    "tatara_trainer_get_activation": (C.c_int32, [C.c_void_p, C.c_char_p, c_f32p, C.c_uint64]),
    "tatara_trainer_sync_forward_weights": (C.c_int32, [C.c_void_p]),
    "tatara_trainer_fp16_clamp_count": (C.c_int32, [C.c_void_p, c_u64p, c_u64p]),
    "tatara_trainer_export_quantised": (C.c_int32, [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.c_int32]),
    "tatara_trainer_set_profiling": (C.c_int32, [C.c_void_p, C.c_int32]),
    "tatara_ckpt_write_header": (
        C.c_int32,
        [C.POINTER(TataraCkptArch), C.c_char_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p,
         C.c_uint64, c_u64p],
    ),
    "tatara_ckpt_read_header": (
        C.c_int32,
        [C.c_void_p, C.c_uint64, C.POINTER(TataraCkptArch), C.POINTER(TataraCkptHeader)],
    ),
    "tatara_trainer_save_resume": (
        C.c_int32,
        [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.c_uint64, C.c_char_p, C.c_uint64],
    ),
    "tatara_trainer_load_resume": (
        C.c_int32,
        [C.c_void_p, C.c_char_p, C.c_int32, C.c_int32, C.POINTER(TataraCkptHeader)],
    ),
    "tatara_trainer_phase_times": (C.c_int32, [C.c_void_p, c_f64p, C.c_int32, c_u64p]),
    "tatara_lr_schedule_one_cycle": (
        C.c_int32,
        [C.c_float, C.c_float, C.c_float, C.c_float, C.c_uint64, C.POINTER(TataraLrSchedule)],
    ),
    "tatara_lr_at": (C.c_int32, [C.POINTER(TataraLrSchedule), C.c_uint64, C.c_uint64, c_f32p]),
    "tatara_lr_horizon": (C.c_int32, [C.POINTER(TataraLrSchedule), c_u64p, c_i32p]),
    "tatara_wdl_at": (C.c_int32, [C.POINTER(TataraWdlSchedule), C.c_uint64, C.c_uint64, C.c_uint64, c_f32p]),
    "tatara_control_apply": (
        C.c_int32,
        [C.c_char_p, C.c_char_p, C.POINTER(TataraControlState), C.c_uint64, C.c_uint64, C.c_uint64, c_i32p,
         c_u64p],
    ),
    "tatara_experiment_create": (C.c_int32, [C.POINTER(TataraExperimentInit), C.POINTER(C.c_void_p)]),
    "tatara_experiment_destroy": (C.c_int32, [C.c_void_p]),
    "tatara_experiment_set_target_superbatches": (C.c_int32, [C.c_void_p, C.c_uint64]),
    "tatara_experiment_record_superbatch": (
        C.c_int32,
        [C.c_void_p, C.c_uint64, C.c_double, C.c_uint64, C.c_double, c_f64p, c_f64p],
    ),
    "tatara_experiment_note_checkpoint": (C.c_int32, [C.c_void_p, C.c_char_p]),
    "tatara_experiment_mark_finished": (C.c_int32, [C.c_void_p, C.c_double]),
    "tatara_experiment_mark_interrupted": (C.c_int32, [C.c_void_p]),
    "tatara_experiment_write": (C.c_int32, [C.c_void_p]),
    "tatara_format_utc_iso": (C.c_int32, [C.c_uint64, C.c_char_p]),
    "tatara_format_utc_compact": (C.c_int32, [C.c_uint64, C.c_char_p]),
    "tatara_train_run": (
        C.c_int32,
        [C.c_void_p, C.POINTER(TataraRunConfig), C.POINTER(TataraLrSchedule), C.POINTER(TataraWdlSchedule),
         C.POINTER(TataraLoss), C.POINTER(TataraRunSuperbatch), C.c_uint64, c_u64p, c_f32p, c_f32p,
         C.c_uint64],
    ),
}


class TataraError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status
        self.message = message


class OutOfMemory(TataraError):
    pass


_LIB: C.CDLL | None = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Loads (once) and returns the HIP library with typed entry points."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build it with `python -m tatara_amd.build` "
            "(the HIP library is the only implementation of this path)"
        )
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(status: int) -> None:
    """Raises TataraError (OutOfMemory for -2) when status is non-zero."""
    if status == 0:
        return
    msg = load().tatara_last_error().decode(errors="replace")
    if status == -2:
        raise OutOfMemory(status, msg)
    raise TataraError(status, msg)
