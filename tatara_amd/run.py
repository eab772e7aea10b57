"""Superbatch driver and schedules over the C ABI.

The schedule classes mirror crates/nnue-train/src/schedule.rs (the same
names and fields) and evaluate through the library (`tatara_lr_at`,
`tatara_wdl_at`); `run` drives a trainer through `tatara_train_run`
(crates/nnue-train/src/trainer.rs:759-1211): superbatches start..=end of
batches_per_superbatch PSV batches, lagged-loss accounting with a flush per
superbatch, quantised and resume checkpoints every save_rate superbatches and
at the end, pruning of old resume checkpoints, and <output_dir>/control.json
read at the start of every superbatch (trainer.rs:640-744): a
`{"target_superbatches": N}` with start <= N < end_superbatch stops the run
after superbatch max(N, current), saving there and appending the applied
target to <output_dir>/control_history.jsonl; the lr / wdl schedules keep the
configured end as their horizon.
"""
from __future__ import annotations

import ctypes as C
import sys
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional

import numpy as np

from . import _lib
from ._lib import (TataraLrSchedule, TataraRunConfig, TataraRunSuperbatch, TataraWdlSchedule, check)
from .dataloader import BUCKET_MODES, FEATURE_SETS

LR_CONSTANT, LR_STEP, LR_DROP, LR_LINEAR, LR_COSINE, LR_EXPONENTIAL, LR_ONE_CYCLE = range(7)
WDL_CONSTANT, WDL_LINEAR = range(2)


def _f(x: float) -> str:
    """An f32 field as the schedules' Display impls print it."""
    from .experiment import rust_display

    return rust_display(x)


class _LrBase:
    """An LrScheduler: `lr(batch, superbatch)` and `horizon()`."""

    def _c(self) -> TataraLrSchedule:  # pragma: no cover - overridden
        raise NotImplementedError

    def to_c(self) -> TataraLrSchedule:
        s = self._c()
        self._keep = s  # the structure a `next` pointer may reference
        return s

    def lr(self, batch: int, superbatch: int) -> float:
        out = C.c_float()
        check(_lib.load().tatara_lr_at(C.byref(self.to_c()), batch, superbatch, C.byref(out)))
        return out.value

    def horizon(self) -> Optional[int]:
        h, has = C.c_uint64(), C.c_int32()
        check(_lib.load().tatara_lr_horizon(C.byref(self.to_c()), C.byref(h), C.byref(has)))
        return h.value if has.value else None

    def with_warmup(self, warmup_batches: int) -> "WarmupLR":
        """LrSchedulerEnum::with_warmup."""
        return WarmupLR(self, warmup_batches)


@dataclass
class ConstantLR(_LrBase):
    value: float

    def _c(self):
        return TataraLrSchedule(kind=LR_CONSTANT, start=self.value)

    def __str__(self):  # schedule.rs:50-54
        return f"constant {_f(self.value)}"


@dataclass
class StepLR(_LrBase):
    start: float
    gamma: float
    step: int

    def _c(self):
        return TataraLrSchedule(kind=LR_STEP, start=self.start, gamma=self.gamma, period=self.step)

    def __str__(self):  # schedule.rs:100-108
        return f"start {_f(self.start)} gamma {_f(self.gamma)} drop every {self.step} superbatches"


@dataclass
class DropLR(_LrBase):
    start: float
    gamma: float
    drop: int

    def _c(self):
        return TataraLrSchedule(kind=LR_DROP, start=self.start, gamma=self.gamma, period=self.drop)

    def __str__(self):  # schedule.rs:74-82
        return f"start {_f(self.start)} gamma {_f(self.gamma)} drop at {self.drop} superbatches"


@dataclass
class LinearDecayLR(_LrBase):
    initial_lr: float
    final_lr: float
    final_superbatch: int

    def _c(self):
        return TataraLrSchedule(kind=LR_LINEAR, start=self.initial_lr, gamma=self.final_lr,
                                period=self.final_superbatch)

    def __str__(self):  # schedule.rs:132-140
        return (f"start at {_f(self.initial_lr)} and linearly decay to {_f(self.final_lr)} at superbatch "
                f"{self.final_superbatch}")


@dataclass
class CosineDecayLR(_LrBase):
    initial_lr: float
    final_lr: float
    final_superbatch: int

    def _c(self):
        return TataraLrSchedule(kind=LR_COSINE, start=self.initial_lr, gamma=self.final_lr,
                                period=self.final_superbatch)

    def __str__(self):  # schedule.rs:165-173
        return (f"start at {_f(self.initial_lr)} and cosine decay to {_f(self.final_lr)} at superbatch "
                f"{self.final_superbatch}")


@dataclass
class ExponentialDecayLR(_LrBase):
    initial_lr: float
    final_lr: float
    final_superbatch: int

    def _c(self):
        return TataraLrSchedule(kind=LR_EXPONENTIAL, start=self.initial_lr, gamma=self.final_lr,
                                period=self.final_superbatch)

    def __str__(self):  # schedule.rs:197-205
        return (f"start at {_f(self.initial_lr)} and exponentially decay to {_f(self.final_lr)} at superbatch "
                f"{self.final_superbatch}")


class OneCycleLR(_LrBase):
    """OneCycleLR::new(max_lr, warmup_pct, div_factor, final_div_factor, total_superbatch)."""

    def __init__(self, max_lr: float, warmup_pct: float, div_factor: float, final_div_factor: float,
                 total_superbatch: int):
        s = TataraLrSchedule()
        check(_lib.load().tatara_lr_schedule_one_cycle(max_lr, warmup_pct, div_factor, final_div_factor,
                                                      total_superbatch, C.byref(s)))
        self.initial_lr, self.max_lr, self.final_lr = s.start, s.max_lr, s.gamma
        self.warmup_superbatch, self.total_superbatch = s.period, s.total

    def _c(self):
        return TataraLrSchedule(kind=LR_ONE_CYCLE, start=self.initial_lr, gamma=self.final_lr, max_lr=self.max_lr,
                                period=self.warmup_superbatch, total=self.total_superbatch)

    def __str__(self):  # schedule.rs:282-294
        return (f"one-cycle {_f(self.initial_lr)} \u2192 max {_f(self.max_lr)} (warmup to superbatch "
                f"{self.warmup_superbatch}) \u2192 cosine anneal to {_f(self.final_lr)} at superbatch "
                f"{self.total_superbatch}")


@dataclass
class WarmupLR(_LrBase):
    inner: _LrBase
    warmup_batches: int

    def _c(self):
        s = self.inner.to_c()
        s = TataraLrSchedule.from_buffer_copy(s)
        s.warmup_batches = self.warmup_batches
        self._inner_keep = self.inner
        return s

    def __str__(self):  # schedule.rs:321-329
        return f"{self.inner}, warmup over {self.warmup_batches} batches"


@dataclass
class SequenceLR(_LrBase):
    first: _LrBase
    second: _LrBase
    first_scheduler_final_superbatch: int

    def _c(self):
        s = TataraLrSchedule.from_buffer_copy(self.first.to_c())
        self._second = self.second.to_c()
        s.next = C.pointer(self._second)
        s.next_after = self.first_scheduler_final_superbatch
        return s

    def __str__(self):  # schedule.rs:350-358
        return f"{self.first}, then after {self.first_scheduler_final_superbatch} superbatches, {self.second}"


class _WdlBase:
    """A WdlScheduler: `blend(batch, superbatch, max)`."""

    def _c(self) -> TataraWdlSchedule:  # pragma: no cover - overridden
        raise NotImplementedError

    def to_c(self) -> TataraWdlSchedule:
        s = self._c()
        self._keep = s
        return s

    def blend(self, batch: int, superbatch: int, max_superbatch: int) -> float:
        out = C.c_float()
        check(_lib.load().tatara_wdl_at(C.byref(self.to_c()), batch, superbatch, max_superbatch, C.byref(out)))
        return out.value


@dataclass
class ConstantWDL(_WdlBase):
    value: float

    def _c(self):
        return TataraWdlSchedule(kind=WDL_CONSTANT, start=self.value)

    def __str__(self):  # schedule.rs:451-455
        return f"constant {_f(self.value)}"


@dataclass
class LinearWDL(_WdlBase):
    start: float
    end: float

    def _c(self):
        return TataraWdlSchedule(kind=WDL_LINEAR, start=self.start, end=self.end)

    def __str__(self):  # schedule.rs:472-476
        return f"linear taper start {_f(self.start)} end {_f(self.end)}"


@dataclass
class WarmupWDL(_WdlBase):
    inner: _WdlBase
    warmup_batches: int

    def _c(self):
        s = TataraWdlSchedule.from_buffer_copy(self.inner.to_c())
        s.warmup_batches = self.warmup_batches
        return s

    def __str__(self):  # schedule.rs:496-504
        return f"{self.inner}, warmup over {self.warmup_batches} batches"


@dataclass
class SequenceWDL(_WdlBase):
    first: _WdlBase
    second: _WdlBase
    first_scheduler_final_superbatch: int

    def _c(self):
        s = TataraWdlSchedule.from_buffer_copy(self.first.to_c())
        self._second = self.second.to_c()
        s.next = C.pointer(self._second)
        s.next_after = self.first_scheduler_final_superbatch
        return s

    def __str__(self):  # schedule.rs:526-534
        return f"{self.first}, then after {self.first_scheduler_final_superbatch} superbatches, {self.second}"


@dataclass
class TrainingConfig:
    """The TrainingConfig fields the driver uses (trainer.rs:395-490)."""

    net_id: str
    feature_set: str
    output_dir: str
    start_superbatch: int = 1
    end_superbatch: int = 1
    batches_per_superbatch: int = 1
    batch_size: int = 16384
    save_rate: int = 1
    fv_scale: Optional[int] = None
    keep_raw_checkpoints: Optional[int] = None
    bucket_mode: str = "none"
    num_buckets: int = 1
    progress_weights: Optional[object] = None  # DeviceArray of f32, for progress8kpabs
    run_id: str = ""
    print_progress: bool = True
    # the run's experiment.json (tatara_amd.experiment.ExperimentLogger), or None
    experiment: Optional[object] = None


@dataclass
class RunResult:
    superbatches: list = field(default_factory=list)  # dicts per superbatch
    lr_seen: np.ndarray = None
    wdl_seen: np.ndarray = None


def run(trainer, data_path, lr_scheduler, wdl_scheduler, cfg: TrainingConfig, loss) -> RunResult:
    """run (trainer.rs:759-1211) through the library's driver."""
    Path(cfg.output_dir).mkdir(parents=True, exist_ok=True)
    n_sb = cfg.end_superbatch - cfg.start_superbatch + 1
    steps = max(n_sb, 0) * cfg.batches_per_superbatch
    rep = (TataraRunSuperbatch * max(n_sb, 1))()
    n_rep = C.c_uint64()
    lr_seen = np.zeros(max(steps, 1), np.float32)
    wdl_seen = np.zeros(max(steps, 1), np.float32)
    c = TataraRunConfig()
    c.data_path = str(data_path).encode()
    c.output_dir = str(cfg.output_dir).encode()
    c.net_id = cfg.net_id.encode()
    c.run_id = cfg.run_id.encode()
    c.start_superbatch, c.end_superbatch = cfg.start_superbatch, cfg.end_superbatch
    c.batches_per_superbatch, c.batch_size, c.save_rate = cfg.batches_per_superbatch, cfg.batch_size, cfg.save_rate
    c.has_fv_scale = int(cfg.fv_scale is not None)
    c.fv_scale = cfg.fv_scale or 0
    c.has_keep_raw = int(cfg.keep_raw_checkpoints is not None)
    c.keep_raw_checkpoints = cfg.keep_raw_checkpoints or 0
    c.feature_set = FEATURE_SETS[cfg.feature_set]
    c.bucket_mode = BUCKET_MODES[cfg.bucket_mode]
    c.num_buckets = cfg.num_buckets
    c.progress_weights = cfg.progress_weights.ptr if cfg.progress_weights is not None else None
    c.print_progress = int(cfg.print_progress)
    c.experiment = cfg.experiment.handle if cfg.experiment is not None else None
    lr_c, wdl_c, loss_c = lr_scheduler.to_c(), wdl_scheduler.to_c(), loss.to_c()
    try:
        check(trainer._lib.tatara_train_run(
            trainer._h, C.byref(c), C.byref(lr_c), C.byref(wdl_c), C.byref(loss_c), rep, len(rep), C.byref(n_rep),
            lr_seen.ctypes.data_as(C.POINTER(C.c_float)), wdl_seen.ctypes.data_as(C.POINTER(C.c_float)),
            steps))
    except Exception:
        # an interrupted run keeps status "running" with results.interrupted
        # set (training.rs:912-923)
        if cfg.experiment is not None:
            cfg.experiment.mark_interrupted()
            try:
                cfg.experiment.write()
            except Exception as e:  # reported, as a failed write is
                print(f"[train] warning: failed to write experiment log {cfg.experiment.path}: {e}",
                      file=sys.stderr)
        raise
    out = RunResult(lr_seen=lr_seen[:steps], wdl_seen=wdl_seen[:steps])
    for r in rep[:n_rep.value]:
        out.superbatches.append(dict(superbatch=r.superbatch, positions=r.positions, loss_sum=r.loss_sum,
                                     mean_loss=r.mean_loss, seconds=r.seconds, lr=r.lr, wdl=r.wdl,
                                     saved=bool(r.saved)))
    return out
