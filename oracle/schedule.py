"""CPU restatement of the learning-rate and WDL-lambda schedules.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the
library's schedules (tatara_lr_at / tatara_wdl_at); nothing in the product
imports it.

Follows crates/nnue-train/src/schedule.rs: ConstantLR (:43-47), DropLR
(:64-71), StepLR (:92-97), LinearDecayLR (:118-125), CosineDecayLR
(:150-158), ExponentialDecayLR (:183-190), OneCycleLR::new (:233-253) and
lr (:260-275), WarmupLR (:303-313), SequenceLR (:339-347), ConstantWDL
(:446-448), LinearWDL (:465-469), WarmupWDL (:486-493), SequenceWDL
(:515-524).  Every operation is one float32 operation in the reference's
order (numpy float32 scalars); `usize as f32` rounds to nearest; cos and
powf are glibc's cosf / powf (what Rust's f32 methods call on linux-gnu),
and f32::powi is restated as compiler-rt's __powisf2 (square and multiply
over the exponent's bits).
"""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np

F = np.float32
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.cosf.restype = ctypes.c_float
_libm.cosf.argtypes = [ctypes.c_float]
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
_libm.roundf.restype = ctypes.c_float
_libm.roundf.argtypes = [ctypes.c_float]

PI = F(np.pi)  # std::f32::consts::PI


def cosf(x) -> np.float32:
    return F(_libm.cosf(float(F(x))))


def powf(x, y) -> np.float32:
    return F(_libm.powf(float(F(x)), float(F(y))))


def powi(a, b: int) -> np.float32:
    """compiler-rt __powisf2."""
    a = F(a)
    recip = b < 0
    r = F(1.0)
    while True:
        if b & 1:
            r = F(r * a)
        b = int(b / 2)  # C division truncates toward zero
        if b == 0:
            break
        a = F(a * a)
    return F(F(1.0) / r) if recip else r


def usize_f32(n: int) -> np.float32:
    return F(n)  # numpy rounds an integer to the nearest float32


def cosine_interp(start, end, p) -> np.float32:
    return F(F(end) + F(F(F(0.5) * F(F(start) - F(end))) * F(F(1.0) + cosf(F(PI * F(p))))))


class ConstantLR:
    def __init__(self, value):
        self.value = F(value)

    def lr(self, batch, sb):
        return self.value

    def horizon(self):
        return None


class DropLR:
    def __init__(self, start, gamma, drop):
        self.start, self.gamma, self.drop = F(start), F(gamma), drop

    def lr(self, batch, sb):
        return F(self.start * self.gamma) if sb > self.drop else self.start

    def horizon(self):
        return None


class StepLR:
    def __init__(self, start, gamma, step):
        self.start, self.gamma, self.step = F(start), F(gamma), step

    def lr(self, batch, sb):
        steps = max(sb - 1, 0) // self.step
        return F(self.start * powi(self.gamma, steps))

    def horizon(self):
        return None


class _Decay:
    def __init__(self, initial_lr, final_lr, final_superbatch):
        self.initial_lr, self.final_lr, self.final_superbatch = F(initial_lr), F(final_lr), final_superbatch

    def horizon(self):
        return self.final_superbatch


class LinearDecayLR(_Decay):
    def lr(self, batch, sb):
        if sb >= self.final_superbatch:
            return self.final_lr
        lam = F(usize_f32(sb) / usize_f32(self.final_superbatch))
        return F(self.initial_lr + F(lam * F(self.final_lr - self.initial_lr)))


class CosineDecayLR(_Decay):
    def lr(self, batch, sb):
        if sb >= self.final_superbatch:
            return self.final_lr
        progress = F(usize_f32(sb) / usize_f32(self.final_superbatch))
        lam = F(F(1.0) - F(F(0.5) * F(F(1.0) + cosf(F(PI * progress)))))
        return F(self.initial_lr + F(lam * F(self.final_lr - self.initial_lr)))


class ExponentialDecayLR(_Decay):
    def lr(self, batch, sb):
        if sb >= self.final_superbatch:
            return self.final_lr
        lam = F(usize_f32(sb) / usize_f32(self.final_superbatch))
        return F(self.initial_lr * powf(F(self.final_lr / self.initial_lr), lam))


class OneCycleLR:
    def __init__(self, max_lr, warmup_pct, div_factor, final_div_factor, total_superbatch):
        self.max_lr = F(max_lr)
        self.initial_lr = F(self.max_lr / F(div_factor))
        self.final_lr = F(self.initial_lr / F(final_div_factor))
        w = F(_libm.roundf(float(F(F(warmup_pct) * usize_f32(total_superbatch)))))
        w = min(max(w, F(0.0)), usize_f32(total_superbatch))
        self.warmup_superbatch = 0 if np.isnan(w) else int(w)
        self.total_superbatch = total_superbatch

    def lr(self, batch, sb):
        if sb <= self.warmup_superbatch:
            denom = usize_f32(max(self.warmup_superbatch, 1))
            return cosine_interp(self.initial_lr, self.max_lr, F(usize_f32(sb) / denom))
        if sb >= self.total_superbatch:
            return self.final_lr
        denom = usize_f32(max(self.total_superbatch - self.warmup_superbatch, 1))
        return cosine_interp(self.max_lr, self.final_lr, F(usize_f32(sb - self.warmup_superbatch) / denom))

    def horizon(self):
        return self.total_superbatch


class WarmupLR:
    def __init__(self, inner, warmup_batches):
        self.inner, self.warmup_batches = inner, warmup_batches

    def lr(self, batch, sb):
        base = self.inner.lr(batch, sb)
        if sb == 1 and batch < self.warmup_batches:
            return F(base / usize_f32(self.warmup_batches - batch))
        return base

    def horizon(self):
        return self.inner.horizon()


class SequenceLR:
    def __init__(self, first, second, first_scheduler_final_superbatch):
        self.first, self.second, self.mid = first, second, first_scheduler_final_superbatch

    def lr(self, batch, sb):
        return self.first.lr(batch, sb) if sb <= self.mid else self.second.lr(batch, sb - self.mid)

    def horizon(self):
        return None  # the trait's default


class ConstantWDL:
    def __init__(self, value):
        self.value = F(value)

    def blend(self, batch, sb, mx):
        return self.value


class LinearWDL:
    def __init__(self, start, end):
        self.start, self.end = F(start), F(end)

    def blend(self, batch, sb, mx):
        grad = F(F(self.end - self.start) / usize_f32(max(mx - 1, 1)))
        return F(self.start + F(grad * usize_f32(sb - 1)))


class WarmupWDL:
    def __init__(self, inner, warmup_batches):
        self.inner, self.warmup_batches = inner, warmup_batches

    def blend(self, batch, sb, mx):
        base = self.inner.blend(batch, sb, mx)
        if sb == 1 and batch < self.warmup_batches:
            return F(base / usize_f32(self.warmup_batches - batch))
        return base


class SequenceWDL:
    def __init__(self, first, second, first_scheduler_final_superbatch):
        self.first, self.second, self.mid = first, second, first_scheduler_final_superbatch

    def blend(self, batch, sb, mx):
        if sb <= self.mid:
            return self.first.blend(batch, sb, self.mid)
        return self.second.blend(batch, sb - self.mid, mx - self.mid)
