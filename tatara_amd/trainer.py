"""Host-side mirror of tatara's step API over the HIP C ABI.

`LayerStackTrainer` and `SimpleTrainer` follow `trait TrainerBackend`
(crates/nnue-train/src/trainer.rs:273-375) as GpuTrainer
(bins/nnue_train/src/trainer_layerstack.rs:1885-2010) and SimpleGpuTrainer
(bins/nnue_train/src/trainer_simple.rs:742-856) implement it: `train_step` returns
the previous step's sum of squared errors (0.0 on the first call),
`flush_pending_loss` drains the last one, `validate_step` runs forward + loss
only.  `Batch` mirrors crates/nnue-train/src/dataloader.rs:355-369 and
`Sigmoid` / `Wrm` mirror `LossKind` (trainer.rs:89-135).
"""
from __future__ import annotations

import ctypes as C
import math
import os
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from . import _lib
from ._lib import OutOfMemory, TataraBatch, TataraLoss, TataraTrainerConfig, check

OPTIMIZERS = {"ranger": 0, "radam": 1, "adamw": 2}
GROUPS = (
    "ft_w",
    "ft_b",
    "l1_w",
    "l1_b",
    "l1_shared_weight",
    "l1_shared_bias",
    "l2_w",
    "l2_b",
    "l3_w",
    "l3_b",
)
SIMPLE_GROUPS = ("ft_w", "ft_b", "l1_w", "l1_b", "l2_w", "l2_b", "l3_w", "l3_b")
WHICH = {"w": 0, "m": 1, "v": 2, "slow": 3, "grad": 4}


@dataclass(frozen=True)
class Sigmoid:
    """LossKind::Sigmoid (sigmoid-MSE); LayerStack default scale 1/290."""

    scale: float = 1.0 / 290.0

    def to_c(self) -> TataraLoss:
        return TataraLoss(kind=0, scale=self.scale)


@dataclass(frozen=True)
class Wrm:
    """LossKind::Wrm (win-rate-model loss)."""

    nnue2score: float = 600.0
    in_scaling: float = 340.0
    in_offset: float = 270.0
    target_offset: float = 270.0
    target_scaling: float = 380.0
    pow_exp: float = 2.0
    qp_asymmetry: float = 0.0
    weight_boost_w1: float = 0.0
    weight_boost_w2: float = 0.5

    @property
    def extended(self) -> bool:
        return self.pow_exp != 2.0 or self.qp_asymmetry != 0.0 or self.weight_boost_w1 != 0.0

    def to_c(self) -> TataraLoss:
        return TataraLoss(
            kind=1,
            scale=0.0,
            nnue2score=self.nnue2score,
            in_scaling=self.in_scaling,
            in_offset=self.in_offset,
            target_offset=self.target_offset,
            target_scaling=self.target_scaling,
            pow_exp=self.pow_exp,
            qp_asymmetry=self.qp_asymmetry,
            weight_boost_w1=self.weight_boost_w1,
            weight_boost_w2=self.weight_boost_w2,
        )


@dataclass
class Batch:
    """One training batch: [n_pos, max_active] index rows (-1 padding)."""

    stm_indices: np.ndarray
    nstm_indices: np.ndarray
    nnz: np.ndarray
    score: np.ndarray
    wdl: np.ndarray

    def __post_init__(self):
        self.stm_indices = np.ascontiguousarray(self.stm_indices, dtype=np.int32)
        self.nstm_indices = np.ascontiguousarray(self.nstm_indices, dtype=np.int32)
        self.nnz = np.ascontiguousarray(self.nnz, dtype=np.int32)
        self.score = np.ascontiguousarray(self.score, dtype=np.float32)
        self.wdl = np.ascontiguousarray(self.wdl, dtype=np.float32)
        if self.stm_indices.ndim != 2 or self.stm_indices.shape != self.nstm_indices.shape:
            raise ValueError("index arrays must both be [n_pos, max_active]")

    @property
    def n_positions(self) -> int:
        return int(self.stm_indices.shape[0])

    @property
    def max_active(self) -> int:
        return int(self.stm_indices.shape[1])


class DeviceArray:
    """A device allocation owned by the library (DeviceBuffer::from_host)."""

    def __init__(self, host: np.ndarray):
        host = np.ascontiguousarray(host)
        self.dtype = host.dtype
        self.shape = host.shape
        self.nbytes = host.nbytes
        lib = _lib.load()
        ptr = C.c_void_p()
        check(lib.tatara_malloc(C.byref(ptr), self.nbytes))
        self.ptr = ptr.value
        check(lib.tatara_memcpy_htod(self.ptr, host.ctypes.data, self.nbytes))

    @classmethod
    def empty(cls, shape, dtype) -> "DeviceArray":
        return cls(np.zeros(shape, dtype=dtype))

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(_lib.load().tatara_memcpy_dtoh(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            _lib.load().tatara_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class DeviceBatch:
    """A batch resident in device memory (inputs already in HBM).

    king_blocked: every row's features lie in its perspective's king block
    and none repeats (set by psv_to_device_batch when the records guarantee
    it); the trainer then queues no occurrence-list fallback for the step
    (on_device = TATARA_BATCH_KING_BLOCKED)."""

    n_pos: int
    max_active: int
    arrays: dict = field(default_factory=dict)
    king_blocked: bool = False

    @classmethod
    def upload(cls, batch: Batch, bucket_idx: Optional[np.ndarray] = None) -> "DeviceBatch":
        """bucket_idx: LayerStack bucket per position; None for Simple."""
        db = cls(batch.n_positions, batch.max_active)
        db.arrays = {
            "stm": DeviceArray(batch.stm_indices),
            "nstm": DeviceArray(batch.nstm_indices),
            "nnz": DeviceArray(batch.nnz),
            "score": DeviceArray(batch.score),
            "wdl": DeviceArray(batch.wdl),
        }
        if bucket_idx is not None:
            db.arrays["bucket"] = DeviceArray(np.ascontiguousarray(bucket_idx, dtype=np.int32))
        return db

    def to_c(self) -> TataraBatch:
        a = self.arrays
        return TataraBatch(
            n_pos=self.n_pos,
            max_active=self.max_active,
            stm_indices=a["stm"].ptr,
            nstm_indices=a["nstm"].ptr,
            nnz=a["nnz"].ptr,
            bucket_idx=a["bucket"].ptr if "bucket" in a else None,
            score=a["score"].ptr,
            wdl=a["wdl"].ptr,
            on_device=2 if self.king_blocked else 1,
        )


def _host_batch(batch: Batch, bucket_idx: Optional[np.ndarray]) -> tuple[TataraBatch, tuple]:
    bucket = None
    if bucket_idx is not None:
        if len(bucket_idx) != batch.n_positions:
            raise ValueError(
                f"bucket_idx len ({len(bucket_idx)}) must equal batch.n_positions ({batch.n_positions})"
            )
        bucket = np.ascontiguousarray(bucket_idx, dtype=np.int32)
    keep = (batch.stm_indices, batch.nstm_indices, batch.nnz, bucket, batch.score, batch.wdl)
    cb = TataraBatch(
        n_pos=batch.n_positions,
        max_active=batch.max_active,
        stm_indices=batch.stm_indices.ctypes.data,
        nstm_indices=batch.nstm_indices.ctypes.data,
        nnz=batch.nnz.ctypes.data,
        bucket_idx=bucket.ctypes.data if bucket is not None else None,
        score=batch.score.ctypes.data,
        wdl=batch.wdl.ctypes.data,
        on_device=0,
    )
    return cb, keep


@dataclass
class LayerStackConfig:
    """GpuTrainer::new arguments for the LayerStack architecture."""

    ft_in: int
    max_active: int
    piece_inputs: int = 0  # factorizer piece inputs (0: off)
    ft_out: int = 1536
    l1_out: int = 16
    l2_out: int = 32
    num_buckets: int = 9
    max_batch: int = 16384
    optimizer: str = "ranger"
    weight_decay: float = 0.01
    ft_weight_decay: Optional[float] = None
    dense_weight_decay: Optional[float] = None
    bias_weight_decay: Optional[float] = None
    ft_lr_mult: float = 1.0
    dense_lr_mult: float = 1.0
    bias_lr_mult: float = 1.0
    device: int = 0
    keep_grads: bool = False
    # PrecisionFlags (trainer_common.rs:49-61); all_optim() sets the four
    ft_fp16: bool = False
    ft_fp16_out: bool = False
    fp16_opt_state: bool = False
    tf32: bool = False

    def all_optim(self) -> "LayerStackConfig":
        """The --all-optim precision flags (cli.rs:627-638) on a copy of this config."""
        import dataclasses

        return dataclasses.replace(self, ft_fp16=True, ft_fp16_out=True, fp16_opt_state=True, tf32=True)

    def to_c(self) -> TataraTrainerConfig:
        wd = self.weight_decay
        return TataraTrainerConfig(
            arch=0,
            device=self.device,
            max_batch=self.max_batch,
            ft_in=self.ft_in,
            max_active=self.max_active,
            piece_inputs=self.piece_inputs,
            ft_out=self.ft_out,
            l1_out=self.l1_out,
            l2_out=self.l2_out,
            num_buckets=self.num_buckets,
            optimizer=OPTIMIZERS[self.optimizer],
            ft_weight_decay=wd if self.ft_weight_decay is None else self.ft_weight_decay,
            dense_weight_decay=wd if self.dense_weight_decay is None else self.dense_weight_decay,
            bias_weight_decay=wd if self.bias_weight_decay is None else self.bias_weight_decay,
            ft_lr_mult=self.ft_lr_mult,
            dense_lr_mult=self.dense_lr_mult,
            bias_lr_mult=self.bias_lr_mult,
            keep_grads=1 if self.keep_grads else 0,
            ft_fp16=int(self.ft_fp16),
            ft_fp16_out=int(self.ft_fp16_out),
            fp16_opt_state=int(self.fp16_opt_state),
            tf32=int(self.tf32),
        )

    @property
    def train_ft_in(self) -> int:
        return self.ft_in + self.piece_inputs


@dataclass
class SimpleConfig:
    """SimpleGpuTrainer::new arguments (bins/nnue_train/src/trainer_simple.rs:392-600).

    The reference applies one weight decay and one learning rate to every
    group; the per-kind fields exist for symmetry with LayerStackConfig.
    """

    ft_in: int
    max_active: int
    piece_inputs: int = 0
    ft_out: int = 256
    l1_out: int = 32
    l2_out: int = 32
    max_batch: int = 16384
    optimizer: str = "adamw"
    weight_decay: float = 0.01
    device: int = 0
    keep_grads: bool = False

    def to_c(self) -> TataraTrainerConfig:
        wd = self.weight_decay
        return TataraTrainerConfig(
            arch=1,
            device=self.device,
            max_batch=self.max_batch,
            ft_in=self.ft_in,
            max_active=self.max_active,
            piece_inputs=self.piece_inputs,
            ft_out=self.ft_out,
            l1_out=self.l1_out,
            l2_out=self.l2_out,
            num_buckets=1,
            optimizer=OPTIMIZERS[self.optimizer],
            ft_weight_decay=wd,
            dense_weight_decay=wd,
            bias_weight_decay=wd,
            ft_lr_mult=1.0,
            dense_lr_mult=1.0,
            bias_lr_mult=1.0,
            keep_grads=1 if self.keep_grads else 0,
        )

    @property
    def train_ft_in(self) -> int:
        return self.ft_in + self.piece_inputs


def oom_remedy(config) -> str:
    """The actionable message of a trainer whose buffers did not fit in GPU
    memory (gpu_oom_error, bins/nnue_train/src/training.rs:100-146): the
    configuration that sizes the buffers, then the ways to shrink them.  The
    f16 forward modes are reported but not recommended (they trade accuracy);
    f16 optimizer moments are, as they only save memory."""
    layerstack = isinstance(config, LayerStackConfig)
    flag, dim = ("--ft-out", config.ft_out) if layerstack else ("--l1", config.ft_out)
    fp16 = getattr(config, "ft_fp16", False), getattr(config, "ft_fp16_out", False)
    opt16 = getattr(config, "fp16_opt_state", False)
    lines = [f"GPU out of memory while allocating training buffers (batch-size={config.max_batch}, "
             f"{flag}={dim}, ft-fp16={str(fp16[0]).lower()}, ft-fp16-out={str(fp16[1]).lower()}, "
             f"fp16-opt-state={str(opt16).lower()}).",
             "Reduce GPU memory by one or more of:"]
    if not opt16:
        lines.append("  - add `--fp16-opt-state` (f16 optimizer moments, about half their memory)")
    lines.append(f"  - lower `{flag}` (the FT output width; the buffers grow about linearly with it)")
    lines.append("  - smaller `--batch-size`")
    return "\n".join(lines)


class _Trainer:
    """Shared TrainerBackend surface over an opaque C trainer handle."""

    GROUPS: tuple = ()

    def __init__(self, config):
        self.config = config
        self._lib = _lib.load()
        h = C.c_void_p()
        cfg = config.to_c()
        try:
            check(self._lib.tatara_trainer_create(C.byref(cfg), C.byref(h)))
        except OutOfMemory as e:
            # the library freed whatever the failed create had allocated
            raise OutOfMemory(e.status, f"{e.message}\n{oom_remedy(config)}") from None
        self._h = h.value
        self._keep = None  # host arrays referenced by the in-flight step

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.tatara_trainer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- TrainerBackend -----------------------------------------------------
    def train_step(self, batch, bucket_idx=None, lr: float = 8.75e-4, wdl_lambda: float = 0.0,
                   loss=Sigmoid()) -> float:
        """One training step; returns the previous step's sum of squared errors."""
        if isinstance(batch, DeviceBatch):
            cb = batch.to_c()
        else:
            cb, self._keep = _host_batch(batch, bucket_idx)
        cl = loss.to_c()
        out = C.c_double()
        check(self._lib.tatara_trainer_train_step(self._h, C.byref(cb), lr, wdl_lambda,
                                                  C.byref(cl), C.byref(out)))
        return out.value

    def flush_pending_loss(self) -> float:
        out = C.c_double()
        check(self._lib.tatara_trainer_flush_pending_loss(self._h, C.byref(out)))
        return out.value

    def validate_step(self, batch, bucket_idx=None, wdl_lambda: float = 0.0, loss=Sigmoid()):
        """Forward + loss only: returns (sum_sq_err, net_output)."""
        if isinstance(batch, DeviceBatch):
            cb = batch.to_c()
            n = batch.n_pos
        else:
            cb, self._keep = _host_batch(batch, bucket_idx)
            n = batch.n_positions
        cl = loss.to_c()
        sse = C.c_double()
        net = np.zeros(n, dtype=np.float32)
        check(self._lib.tatara_trainer_validate_step(
            self._h, C.byref(cb), wdl_lambda, C.byref(cl), C.byref(sse),
            net.ctypes.data_as(_lib.c_f32p)))
        return sse.value, net

    # -- state access (parity tests, checkpoints) --------------------------
    @property
    def step_count(self) -> int:
        out = C.c_uint64()
        check(self._lib.tatara_trainer_step_count(self._h, C.byref(out)))
        return out.value

    def tensor_size(self, name: str) -> int:
        out = C.c_uint64()
        check(self._lib.tatara_trainer_tensor_size(self._h, name.encode(), C.byref(out)))
        return out.value

    def get(self, name: str, which: str = "w") -> np.ndarray:
        n = self.tensor_size(name)
        out = np.empty(n, dtype=np.float32)
        check(self._lib.tatara_trainer_get_tensor(self._h, name.encode(), WHICH[which],
                                                  out.ctypes.data_as(_lib.c_f32p), n))
        return out

    def set(self, name: str, values: np.ndarray, which: str = "w") -> None:
        v = np.ascontiguousarray(values, dtype=np.float32).ravel()
        check(self._lib.tatara_trainer_set_tensor(self._h, name.encode(), WHICH[which],
                                                  v.ctypes.data_as(_lib.c_f32p), v.size))

    def activation(self, name: str, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        check(self._lib.tatara_trainer_get_activation(self._h, name.encode(),
                                                      out.ctypes.data_as(_lib.c_f32p), n))
        return out

    PHASES = ("prep", "ft_forward", "dense_forward", "dense_backward", "ft_grad_update",
              "ft_virtual_fold", "dense_opt")

    def set_profiling(self, enable: bool) -> None:
        """Per-phase GPU timing with HIP events on the trainer's stream."""
        check(self._lib.tatara_trainer_set_profiling(self._h, 1 if enable else 0))

    def phase_times(self) -> tuple[dict, int]:
        """Summed milliseconds per phase and the number of profiled steps."""
        ms = (C.c_double * len(self.PHASES))()
        steps = C.c_uint64()
        check(self._lib.tatara_trainer_phase_times(self._h, ms, len(self.PHASES), C.byref(steps)))
        return dict(zip(self.PHASES, list(ms))), steps.value

    def state(self) -> dict:
        return {g: {k: self.get(g, k) for k in ("w", "m", "v", "slow")} for g in self.GROUPS}


    def save_resume_checkpoint(self, path, feature_set, bucket_mode, superbatch: int, run_id: str = "",
                               lr_horizon=None) -> None:
        """save_raw_checkpoint (RNRC v8, bins/nnue_train/src/ckpt.rs:614-699): every
        group's w, m, v, slow and the step counter, written atomically.
        bucket_mode: "kingrank9" / "progress8kpabs" for LayerStack, None for Simple."""
        from .checkpoint import BUCKET_MODES, FEATURE_SETS

        fs = FEATURE_SETS[feature_set] if isinstance(feature_set, str) else int(feature_set)
        check(self._lib.tatara_trainer_save_resume(self._h, os.fsencode(path), fs, BUCKET_MODES[bucket_mode],
                                                   int(superbatch), run_id.encode(), int(lr_horizon or 0)))

    def load_resume_checkpoint(self, path, feature_set, bucket_mode):
        """load_raw_checkpoint: restores every group and the step counter and
        rebuilds the forward table; returns (superbatch, producer run id or
        None, LR horizon or None) as RawCkptResumeState (ckpt.rs:134-137)."""
        from ._lib import TataraCkptHeader
        from .checkpoint import BUCKET_MODES, FEATURE_SETS

        fs = FEATURE_SETS[feature_set] if isinstance(feature_set, str) else int(feature_set)
        h = TataraCkptHeader()
        check(self._lib.tatara_trainer_load_resume(self._h, os.fsencode(path), fs, BUCKET_MODES[bucket_mode],
                                                   C.byref(h)))
        return h.superbatch, (h.run_id.decode() or None), (h.lr_horizon or None)

    def _export(self, path, feature_set, fv_scale) -> None:
        from .dataloader import FEATURE_SETS

        fs = FEATURE_SETS[feature_set] if isinstance(feature_set, str) else int(feature_set)
        check(self._lib.tatara_trainer_export_quantised(self._h, os.fsencode(path), fs,
                                                        int(fv_scale is not None), int(fv_scale or 0)))


def _round_half_away(x: float) -> int:
    """Rust f32/f64 `round` of an exactly representable value."""
    return int(math.floor(x + 0.5)) if x >= 0 else -int(math.floor(-x + 0.5))


def simple_fv_scale(scale: float) -> int:
    """simple_fv_scale (crates/nnue-format/src/simple_weights.rs:90-95):
    round((127 * 64) as f32 / scale) in f32."""
    return _round_half_away(float(np.float32(127 * 64) / np.float32(scale)))


def layerstack_export_fv_scale(override, loss, score_scale: float):
    """layerstack_export_fv_scale (bins/nnue_train/src/training.rs:72-86): the
    override, else round(8128 / score_scale) in f32 for the sigmoid loss, else
    None (WRM)."""
    if override is not None:
        return int(override)
    if isinstance(loss, Sigmoid):
        return _round_half_away(float(np.float32(127 * 64) / np.float32(score_scale)))
    return None


class LayerStackTrainer(_Trainer):
    """TrainerBackend for the LayerStack architecture on one MI355X."""

    GROUPS = GROUPS

    def __init__(self, config: LayerStackConfig):
        super().__init__(config)

    def fp16_clamp_count(self) -> tuple[int, int]:
        """read_fp16_clamp_count: cumulative (dft values clamped, dft values written)."""
        c, e = C.c_uint64(), C.c_uint64()
        check(self._lib.tatara_trainer_fp16_clamp_count(self._h, C.byref(c), C.byref(e)))
        return c.value, e.value

    def save_quantised(self, path, feature_set, fv_scale=None) -> None:
        """LayerStackWeights::save_quantised of the current weights (OutputFormat::Tatara);
        fv_scale None omits the arch string's fv_scale token."""
        self._export(path, feature_set, fv_scale)


class SimpleTrainer(_Trainer):
    """TrainerBackend for the Simple architecture on one MI355X (no buckets)."""

    GROUPS = SIMPLE_GROUPS

    def __init__(self, config: SimpleConfig):
        super().__init__(config)

    def train_step(self, batch, lr: float = 1e-3, wdl_lambda: float = 0.0, loss=None) -> float:
        return super().train_step(batch, None, lr, wdl_lambda, Wrm() if loss is None else loss)

    def validate_step(self, batch, wdl_lambda: float = 0.0, loss=None):
        return super().validate_step(batch, None, wdl_lambda, Wrm() if loss is None else loss)

    def save_quantised(self, path, feature_set, fv_scale: int) -> None:
        """SimpleWeights::save_quantised (CReLU) of the current weights; fv_scale is
        simple_fv_scale(scale) in the reference trainer."""
        if fv_scale is None:
            raise ValueError("the Simple format always carries fv_scale")
        self._export(path, feature_set, int(fv_scale))
