"""experiment.json, the structured log of a training run, over the C ABI.

`ExperimentLogger` mirrors crates/nnue-train/src/experiment.rs's logger
(the same method names and meaning): the library holds the document and
writes it (`tatara_experiment_*`), and `run()` in tatara_amd/run.py hands
it to the superbatch driver, which writes it at the start, when control.json
applies a new target, after every superbatch and at the end.  The "params"
object belongs to whoever holds the run's options (the reference's CLI,
bins/nnue_train/src/training.rs:1492-1575 for LayerStack, :1676-1745 for
Simple); `layerstack_params` / `simple_params` build it from this package's
configs with the reference's field names and order, f32 values written as
serde_json writes an f32.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import sys
import time
from pathlib import Path
from typing import Optional

import numpy as np

from . import _lib
from ._lib import TataraExperimentInit, check

PSV_RECORD_BYTES = 40
LAYERSTACK_QA, LAYERSTACK_QB = 127, 64  # nnue-format layerstack_weights.rs:100-101
SIMPLE_QB = 64                          # simple_weights.rs:71; QA from the activation (:147-152)


class F32(float):
    """A value the reference holds as f32: written with the shortest digits
    that read back as the same f32."""


def _digits(x: float, f32: bool) -> tuple[bool, str, int]:
    """Sign, shortest round-trip significant digits and the exponent of the first."""
    v = np.float32(x) if f32 else np.float64(x)
    s = np.format_float_scientific(v, unique=True, trim="-")
    mant, e = s.split("e")
    neg = mant.startswith("-")
    digits = mant.lstrip("-").replace(".", "").rstrip("0") or "0"
    return neg, digits, int(e)


def rust_display(x: float, f32: bool = True) -> str:
    """Rust's `{}` of a float: the shortest digits, positional, no exponent,
    no trailing ".0" (what the schedules' Display impls print)."""
    if math.isnan(x):
        return "NaN"
    if math.isinf(x):
        return "inf" if x > 0 else "-inf"
    if x == 0:
        return "-0" if math.copysign(1.0, x) < 0 else "0"
    neg, d, e = _digits(x, f32)
    if e >= len(d) - 1:
        s = d + "0" * (e - len(d) + 1)
    elif e >= 0:
        s = d[:e + 1] + "." + d[e + 1:]
    else:
        s = "0." + "0" * (-e - 1) + d
    return ("-" if neg else "") + s


def json_float(x: float, f32: bool = False) -> str:
    """A finite float as serde_json writes it (ryu's layouts)."""
    if x == 0:
        return "-0.0" if math.copysign(1.0, x) < 0 else "0.0"
    neg, d, e = _digits(x, f32)
    n, kk = len(d), e + 1
    k = kk - n
    if k >= 0 and kk <= 16:
        s = d + "0" * k + ".0"
    elif 0 < kk <= 16:
        s = d[:kk] + "." + d[kk:]
    elif -5 < kk <= 0:
        s = "0." + "0" * (-kk) + d
    elif n == 1:
        s = f"{d}e{kk - 1}"
    else:
        s = f"{d[0]}.{d[1:]}e{kk - 1}"
    return ("-" if neg else "") + s


def _json_str(s: str) -> str:
    out = ['"']
    short = {'"': '\\"', "\\": "\\\\", "\b": "\\b", "\f": "\\f", "\n": "\\n", "\r": "\\r", "\t": "\\t"}
    for ch in s:
        if ch in short:
            out.append(short[ch])
        elif ord(ch) < 0x20:
            out.append(f"\\u{ord(ch):04x}")
        else:
            out.append(ch)
    return "".join(out) + '"'


def dumps(obj, depth: int = 0) -> str:
    """serde_json::to_string_pretty of a dict / list / scalar tree (F32 and
    np.float32 values as f32, other floats as f64)."""
    pad = "  " * (depth + 1)
    if isinstance(obj, dict):
        if not obj:
            return "{}"
        items = [f"{pad}{_json_str(str(k))}: {dumps(v, depth + 1)}" for k, v in obj.items()]
        return "{\n" + ",\n".join(items) + "\n" + "  " * depth + "}"
    if isinstance(obj, (list, tuple)):
        if not obj:
            return "[]"
        return "[\n" + ",\n".join(pad + dumps(v, depth + 1) for v in obj) + "\n" + "  " * depth + "]"
    if obj is None:
        return "null"
    if isinstance(obj, (bool, np.bool_)):
        return "true" if obj else "false"
    if isinstance(obj, (int, np.integer)):
        return str(int(obj))
    if isinstance(obj, (F32, np.float32)):
        return json_float(float(obj), f32=True)
    if isinstance(obj, (float, np.floating)):
        return json_float(float(obj))
    if isinstance(obj, str):
        return _json_str(obj)
    raise TypeError(f"cannot serialise {type(obj).__name__}")


def format_utc_iso(epoch_secs: int) -> str:
    buf = C.create_string_buffer(32)
    check(_lib.load().tatara_format_utc_iso(epoch_secs, buf))
    return buf.value.decode()


def format_utc_compact(epoch_secs: int) -> str:
    buf = C.create_string_buffer(32)
    check(_lib.load().tatara_format_utc_compact(epoch_secs, buf))
    return buf.value.decode()


def default_id(net_id: str, start_epoch_secs: int, pid: Optional[int] = None) -> str:
    """The run id: net id, UTC start time, process id (training.rs:1458-1466)."""
    return f"{net_id}-{format_utc_compact(start_epoch_secs)}-{os.getpid() if pid is None else pid}"


class ExperimentLogger:
    """ExperimentLogger (experiment.rs:356-540) over the library's document."""

    def __init__(self, path, id: str, name: str, params: dict, data_name: str, data_positions: int,
                 command: Optional[str] = None, commit: Optional[str] = None, lineage: Optional[dict] = None,
                 fv_scale: Optional[int] = None, start_epoch_secs: Optional[int] = None,
                 generator_version: Optional[str] = None):
        self._lib = _lib.load()
        self.path = str(path)
        self.id = id
        init = TataraExperimentInit()
        self._keep = [s.encode() if s is not None else None for s in
                      (self.path, id, name, commit, command if command is not None else " ".join(sys.argv),
                       generator_version, dumps(params), data_name)]
        (init.path, init.id, init.name, init.commit, init.command, init.generator_version, init.params_json,
         init.data_name) = self._keep
        init.start_epoch_secs = int(time.time()) if start_epoch_secs is None else start_epoch_secs
        if lineage is not None:
            init.has_lineage = 1
            parent = lineage.get("parent_id")
            ck = lineage["resumed_from_checkpoint"].encode()
            self._keep += [parent.encode() if parent is not None else None, ck]
            init.lineage_parent_id, init.lineage_checkpoint = self._keep[-2], self._keep[-1]
            init.lineage_superbatch = lineage["resumed_from_superbatch"]
        init.data_positions = data_positions
        init.has_fv_scale = int(fv_scale is not None)
        init.fv_scale = fv_scale or 0
        h = C.c_void_p()
        check(self._lib.tatara_experiment_create(C.byref(init), C.byref(h)))
        self._h = h

    @classmethod
    def for_data(cls, path, id: str, name: str, params: dict, data_path, test_tail_positions: int = 0, **kw):
        """DataInfo from the PSV file (build_data_info, training.rs:1604-1618):
        its basename and record count, less a held-out tail."""
        total = os.path.getsize(data_path) // PSV_RECORD_BYTES if os.path.exists(data_path) else 0
        train = total - test_tail_positions if 0 < test_tail_positions < total else total
        return cls(path, id, name, params, Path(data_path).name, train, **kw)

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def set_target_superbatches(self, target: int):
        check(self._lib.tatara_experiment_set_target_superbatches(self._h, target))

    def record_superbatch(self, superbatch: int, mean_loss: float, sb_positions: int, elapsed_seconds: float,
                          test_loss: Optional[float] = None, test_accuracy: Optional[float] = None):
        tl = C.byref(C.c_double(test_loss)) if test_loss is not None else None
        ta = C.byref(C.c_double(test_accuracy)) if test_accuracy is not None else None
        check(self._lib.tatara_experiment_record_superbatch(self._h, superbatch, mean_loss, sb_positions,
                                                            elapsed_seconds, tl, ta))

    def note_checkpoint(self, file_name: str):
        check(self._lib.tatara_experiment_note_checkpoint(self._h, file_name.encode()))

    def mark_finished(self, elapsed_seconds: float):
        check(self._lib.tatara_experiment_mark_finished(self._h, elapsed_seconds))

    def mark_interrupted(self):
        check(self._lib.tatara_experiment_mark_interrupted(self._h))

    def write(self):
        check(self._lib.tatara_experiment_write(self._h))

    def close(self):
        if getattr(self, "_h", None):
            self._lib.tatara_experiment_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _loss_params(loss) -> tuple[dict, F32]:
    """loss_kind and the wrm_* fields (only for the WRM loss), and `scale`."""
    from .trainer import Wrm

    if isinstance(loss, Wrm):
        p = {"loss_kind": "wrm", "wrm_in_scaling": F32(loss.in_scaling), "wrm_in_offset": F32(loss.in_offset),
             "wrm_nnue2score": F32(loss.nnue2score), "wrm_target_offset": F32(loss.target_offset),
             "wrm_target_scaling": F32(loss.target_scaling), "wrm_pow_exp": F32(loss.pow_exp),
             "wrm_qp_asymmetry": F32(loss.qp_asymmetry), "wrm_weight_boost_w1": F32(loss.weight_boost_w1),
             "wrm_weight_boost_w2": F32(loss.weight_boost_w2)}
        return p, F32(loss.nnue2score)
    return {"loss_kind": "sigmoid"}, F32(1.0 / loss.scale)


def _schedule_params(lr_scheduler, wdl_scheduler) -> dict:
    """lr / lr_gamma / lr_step as the step schedule's raw values (the first
    schedule's start for the others), the effective schedule's description,
    and the WDL lambda (start_wdl / end_wdl for a linear taper)."""
    from .run import ConstantWDL, DropLR, LinearWDL, StepLR

    first = lr_scheduler
    while hasattr(first, "inner") or hasattr(first, "first"):
        first = getattr(first, "inner", None) or getattr(first, "first")
    lr = getattr(first, "start", None)
    if lr is None:
        lr = getattr(first, "initial_lr", getattr(first, "value", 0.0))
    gamma = getattr(first, "gamma", 1.0) if isinstance(first, (StepLR, DropLR)) else 1.0
    step = first.step if isinstance(first, StepLR) else 1
    out = {"lr": F32(lr), "lr_gamma": F32(gamma), "lr_step": max(int(step), 1), "lr_schedule": str(lr_scheduler)}
    w = wdl_scheduler
    while hasattr(w, "inner"):
        w = w.inner
    out["wdl"] = F32(w.value if isinstance(w, ConstantWDL) else 0.0)
    if isinstance(w, LinearWDL):
        out["start_wdl"], out["end_wdl"] = F32(w.start), F32(w.end)
    return out


def _optim_params(cfg) -> dict:
    """weight_decay, and the per-group values only when any group overrides
    them (OptimGroupConfig::resolve, training.rs:1484-1545)."""
    wd = F32(cfg.weight_decay)
    out = {"weight_decay": wd}
    groups = [getattr(cfg, k, None) for k in ("ft_weight_decay", "dense_weight_decay", "bias_weight_decay")]
    mults = [getattr(cfg, k, 1.0) for k in ("ft_lr_mult", "dense_lr_mult", "bias_lr_mult")]
    if any(g is not None for g in groups) or any(m != 1.0 for m in mults):
        for name, g in zip(("ft", "dense", "bias"), groups):
            out[f"{name}_weight_decay"] = F32(wd if g is None else g)
        for name, m in zip(("ft", "dense", "bias"), mults):
            out[f"{name}_lr_mult"] = F32(m)
    return out


def _tail(cfg, threads: int) -> dict:
    return {"tf32": bool(getattr(cfg, "tf32", False)), "ft_fp16": bool(getattr(cfg, "ft_fp16", False)),
            "ft_fp16_out": bool(getattr(cfg, "ft_fp16_out", False)),
            "fp16_opt_state": bool(getattr(cfg, "fp16_opt_state", False)),
            # the driver reads the PSV file in order, one reader, no shuffle window
            "teacher_shuffle_buffer_mib": 0, "teacher_shuffle": False, "teacher_shuffle_seed": 0,
            "threads": threads}


def layerstack_params(cfg, run_cfg, loss, lr_scheduler, wdl_scheduler, ft_in: int,
                      progress_coeff: Optional[str] = None, threads: int = 1) -> dict:
    """The params object of a LayerStack run (training.rs:1492-1575)."""
    lp, scale = _loss_params(loss)
    p = {"architecture": f"LayerStack-{cfg.ft_out}-{cfg.l1_out}-{cfg.l2_out}-{cfg.num_buckets}bucket",
         "feature_set": run_cfg.feature_set, "ft_in": ft_in}
    if cfg.piece_inputs:
        p["ft_factorize"] = True
    p.update({"l0": cfg.ft_out, "l1": cfg.l1_out, "l2": cfg.l2_out, "num_buckets": cfg.num_buckets,
              "optimizer": cfg.optimizer.lower(), "bucket_mode": run_cfg.bucket_mode})
    if progress_coeff is not None:
        p["progress_coeff"] = Path(progress_coeff).name
    sp = _schedule_params(lr_scheduler, wdl_scheduler)
    p.update({k: sp[k] for k in ("lr", "lr_gamma", "lr_step", "lr_schedule")})
    p.update({"batch_size": run_cfg.batch_size, "batches_per_superbatch": run_cfg.batches_per_superbatch,
              "superbatches": run_cfg.end_superbatch, "start_superbatch": run_cfg.start_superbatch,
              "wdl": sp["wdl"]})
    for k in ("start_wdl", "end_wdl"):
        if k in sp:
            p[k] = sp[k]
    p["scale"] = scale
    p.update(_optim_params(cfg))
    p.update({"qa": LAYERSTACK_QA, "qb": LAYERSTACK_QB})
    p.update(lp)
    p.update(_tail(cfg, threads))
    return p


def simple_params(cfg, run_cfg, loss, lr_scheduler, wdl_scheduler, ft_in: int, activation: str = "crelu",
                  threads: int = 1) -> dict:
    """The params object of a Simple run (training.rs:1676-1745)."""
    lp, scale = _loss_params(loss)
    p = {"architecture": f"simple-{run_cfg.feature_set}-{cfg.ft_out}x2-{cfg.l1_out}-{cfg.l2_out}-{activation}",
         "feature_set": run_cfg.feature_set, "ft_in": ft_in}
    if cfg.piece_inputs:
        p["ft_factorize"] = True
    p.update({"l0": cfg.ft_out, "l1": cfg.l1_out, "l2": cfg.l2_out, "optimizer": cfg.optimizer.lower(),
              "activation": activation})
    sp = _schedule_params(lr_scheduler, wdl_scheduler)
    p.update({k: sp[k] for k in ("lr", "lr_gamma", "lr_step", "lr_schedule")})
    p.update({"batch_size": run_cfg.batch_size, "batches_per_superbatch": run_cfg.batches_per_superbatch,
              "superbatches": run_cfg.end_superbatch, "start_superbatch": run_cfg.start_superbatch,
              "wdl": sp["wdl"]})
    for k in ("start_wdl", "end_wdl"):
        if k in sp:
            p[k] = sp[k]
    p["scale"] = scale
    p.update(_optim_params(cfg))
    p.update({"qa": 255 if activation == "screlu" else 127, "qb": SIMPLE_QB})
    p.update(lp)
    p.update(_tail(cfg, threads))
    return p
