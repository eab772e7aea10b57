"""CPU oracle of one LayerStack training step (test infrastructure only).

Chains the restated reference CPU kernels of oracle/ffi.py in the launch
order of GpuTrainer::{forward, backward, optimizer_step}
(bins/nnue_train/src/trainer_layerstack.rs:2038-4489), on host arrays:

forward   :2113-2290  FT gather x2 (comb table when factorized) + FT post
          :2308-2463  per-bucket L1 (dense_mm_fwd_bucket_cpu on original rows;
                      the reference's bucket sort only reorders rows)
          :2489-2628  L1 shared (dense_mm_fwd_cpu) + L1 tail
          :2630-2830  L2, L3, loss
backward  :2886-3936  L3, L2, L1 tail, L1 shared, per-bucket L1, FT post,
                      FT weight gradient (stm then nstm), factorizer reduce
optimizer :4034-4489  RAdam on ft_w then the 9 uniform groups, lookahead
                      every 6 steps (Ranger), fold for the next forward

Also provides the default LayerStack initialisation
(crates/nnue-train/src/init.rs:252-266, trainer_layerstack.rs:844-870).

Precision: the reference's PrecisionFlags (bins/nnue_train/src/
trainer_common.rs:49-61) place f16 roundings at fixed points of the step; the
f16 kernels (native_kernels.cu) compute in f32 between them, so the f32 CPU
functions applied to f16-rounded inputs restate them (the reference's own
fp16 kernel tests check them that way, gpu_cpu_equivalence_tests.rs:
2489-2690):
  ft_fp16         forward table = f16(comb) or f16(weights)
                  (ft_fold_virtual_f16 / cast_f32_to_f16 / the f16 mirror)
  ft_fp16_out     FT raw sums = f16(sum); dft = f16(clamp(g * 2^14 b,
                  +-65504)) (ft_post_perspective_grad_fused_fp16, :2304-2352);
                  FT weight gradient from the f16 dft x 1/(2^14 b)
                  (gather_and_sum_per_feature_*_fp16, :1030-1100)
  fp16_opt_state  ft_w moments stored f16(m 2^28), f16(v 2^40) and read back
                  divided by the scale (radam_step_f16state, :1118-1170)
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import ffi

FT_POST_SCALE = np.float32(127.0 / 128.0)
L1_SQR_SCALE = np.float32(127.0 / 128.0)
BETA2 = 0.999
EPS = 1e-8
ALPHA = 0.5
RANGER_K = 6
N_SMA_THRESHOLD = 5.0
QUANT = np.float32(127.0 / 64.0)
F32_MIN = float(np.finfo(np.float32).min)
F32_MAX = float(np.finfo(np.float32).max)

# (name, kind, quantised clamp) in uniform_optim_group_layout order
# (trainer_layerstack.rs:676-705); kind: dense / bias
UNIFORM_GROUPS = (
    ("ft_b", "bias", False),
    ("l1_w", "dense", True),
    ("l1_b", "bias", True),
    ("l1_shared_weight", "dense", True),
    ("l1_shared_bias", "bias", True),
    ("l2_w", "dense", True),
    ("l2_b", "bias", True),
    ("l3_w", "dense", True),
    ("l3_b", "bias", False),
)


F16_MAX = np.float32(65504.0)
DFT_BASE_SCALE = np.float32(16384.0)       # FT_DFT_FP16_BASE_SCALE (arch.rs)
M_SCALE = np.float32(2.0 ** 28)            # FT_OPT_M_SCALE
V_SCALE = np.float32(2.0 ** 40)            # FT_OPT_V_SCALE


@dataclass
class Precision:
    ft_fp16: bool = False
    ft_fp16_out: bool = False
    fp16_opt_state: bool = False
    # TF32-class L1 products (the reference's --tf32, cuBLAS TF32 GEMMs,
    # trainer_layerstack.rs:2388-2510, 3335-3540), as the HIP trainer forms
    # them on gfx950 (no TF32 matrix instructions): `combined` rounded to f16
    # once and held so; forward products of it with f16-rounded weights, the
    # bucket bias added after the bucket sum; the weight gradients take that
    # f16 `combined` with f32 dl1, the input gradient f32 dl1 and f32
    # weights; f32 sums throughout.
    tf32: bool = False

    @classmethod
    def all_optim(cls):
        return cls(True, True, True, True)


FP32 = Precision()


def f16(x) -> np.ndarray:
    """Round to f16 (nearest even, overflow to inf) and widen back to f32."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def to_f16_state(st: dict) -> dict:
    """ft_w moments as stored with fp16_opt_state: f16(m 2^28), f16(v 2^40), as f32 values."""
    ft = st["ft_w"]
    ft["m16"] = f16(np.clip(ft["m"] * M_SCALE, -F16_MAX, F16_MAX))
    ft["v16"] = f16(np.minimum(ft["v"] * V_SCALE, F16_MAX))
    return st


@dataclass
class LsShape:
    ft_in: int
    max_active: int
    piece_inputs: int
    ft_out: int
    l1: int
    l2: int
    nb: int

    @property
    def train_ft_in(self):
        return self.ft_in + self.piece_inputs

    @property
    def l1e(self):
        return self.l1 - 1

    @property
    def l2_in(self):
        return 2 * self.l1e

    def sizes(self):
        return {
            "ft_w": self.train_ft_in * self.ft_out,
            "ft_b": self.ft_out,
            "l1_w": self.nb * self.l1 * self.ft_out,
            "l1_b": self.nb * self.l1,
            "l1_shared_weight": self.ft_out * self.l1,
            "l1_shared_bias": self.l1,
            "l2_w": self.nb * self.l2 * self.l2_in,
            "l2_b": self.nb * self.l2,
            "l3_w": self.nb * self.l2,
            "l3_b": self.nb,
        }


def default_init(sh: LsShape) -> dict:
    """LayerStackInit::default_uniform weights (FT virtual rows zero)."""
    s = sh.sizes()
    ft = ffi.init_sample(sh.ft_in * sh.ft_out, sh.ft_in, "uniform", "fanin", 1.0, 0x100)
    ft = np.concatenate([ft, np.zeros(s["ft_w"] - ft.size, dtype=np.float32)])
    w = {
        "ft_w": ft,
        "ft_b": np.zeros(s["ft_b"], np.float32),
        "l1_w": ffi.init_sample(s["l1_w"], sh.ft_out, "uniform", "abs", 0.01, 0x101),
        "l1_b": np.zeros(s["l1_b"], np.float32),
        "l1_shared_weight": ffi.init_sample(s["l1_shared_weight"], sh.ft_out, "uniform", "abs", 0.01, 0x102),
        "l1_shared_bias": np.zeros(s["l1_shared_bias"], np.float32),
        "l2_w": ffi.init_sample(s["l2_w"], sh.l2_in, "uniform", "abs", 0.01, 0x103),
        "l2_b": np.zeros(s["l2_b"], np.float32),
        "l3_w": ffi.init_sample(s["l3_w"], sh.l2, "uniform", "abs", 0.01, 0x104),
        "l3_b": np.zeros(s["l3_b"], np.float32),
    }
    return {k: {"w": v, "m": np.zeros_like(v), "v": np.zeros_like(v), "slow": np.zeros_like(v)}
            for k, v in w.items()}


@dataclass
class OptConfig:
    optimizer: str = "ranger"
    weight_decay: float = 0.01
    ft_wd: float | None = None
    dense_wd: float | None = None
    bias_wd: float | None = None
    ft_lr_mult: float = 1.0
    dense_lr_mult: float = 1.0
    bias_lr_mult: float = 1.0

    def group(self, kind: str, lr: float):
        wd = {"ft": self.ft_wd, "dense": self.dense_wd, "bias": self.bias_wd}[kind]
        mult = {"ft": self.ft_lr_mult, "dense": self.dense_lr_mult, "bias": self.bias_lr_mult}[kind]
        return (self.weight_decay if wd is None else wd), np.float32(np.float32(lr) * np.float32(mult))

    @property
    def beta1(self):
        return 0.99 if self.optimizer == "ranger" else 0.9

    def step_size_denom(self, step):
        if self.optimizer == "adamw":
            return 1.0, 1
        return ffi.radam_step_size_denom(step, self.beta1, BETA2, N_SMA_THRESHOLD)


def forward(sh: LsShape, st: dict, batch: dict, wdl_lambda: float, loss: dict, prec: Precision = FP32):
    """Forward + loss.  Returns (intermediates, loss_acc)."""
    b = batch["stm"].shape[0]
    ma = sh.max_active
    ft_w = st["ft_w"]["w"]
    if sh.piece_inputs:
        w_fwd = ffi.ft_fold_virtual(ft_w, sh.ft_in, sh.ft_out, sh.piece_inputs)
    else:
        w_fwd = ft_w[: sh.ft_in * sh.ft_out]
    if prec.ft_fp16:
        w_fwd = f16(w_fwd)
    a = {}
    a["ft_stm"] = ffi.sparse_ft_forward(w_fwd, batch["stm"], batch["nnz"], b, sh.ft_out, sh.ft_in, ma)
    a["ft_nstm"] = ffi.sparse_ft_forward(w_fwd, batch["nstm"], batch["nnz"], b, sh.ft_out, sh.ft_in, ma)
    if prec.ft_fp16_out:
        a["ft_stm"], a["ft_nstm"] = f16(a["ft_stm"]), f16(a["ft_nstm"])
    a["combined"] = ffi.ft_post_perspective_fwd(a["ft_stm"], a["ft_nstm"], st["ft_b"]["w"], b,
                                                sh.ft_out, FT_POST_SCALE)
    bk = batch["bucket"]
    if prec.tf32:
        a["combined"] = f16(a["combined"])
        zero_b = np.zeros_like(st["l1_b"]["w"])
        l1b = ffi.dense_mm_fwd_bucket(a["combined"], f16(st["l1_w"]["w"]), zero_b, bk, b, sh.ft_out, sh.l1,
                                      sh.nb).reshape(b, sh.l1)
        valid = (bk >= 0) & (bk < sh.nb)
        l1b[valid] += st["l1_b"]["w"].reshape(sh.nb, sh.l1)[bk[valid]]
        a["l1_bucket"] = l1b.reshape(-1)
        a["l1_shared"] = ffi.dense_mm_fwd(a["combined"], f16(st["l1_shared_weight"]["w"]),
                                          st["l1_shared_bias"]["w"], b, sh.ft_out, sh.l1)
    else:
        a["l1_bucket"] = ffi.dense_mm_fwd_bucket(a["combined"], st["l1_w"]["w"], st["l1_b"]["w"], bk, b,
                                                 sh.ft_out, sh.l1, sh.nb)
        a["l1_shared"] = ffi.dense_mm_fwd(a["combined"], st["l1_shared_weight"]["w"],
                                          st["l1_shared_bias"]["w"], b, sh.ft_out, sh.l1)
    a["l1_total"] = ffi.elementwise_add(a["l1_bucket"], a["l1_shared"])
    a["l1_main"] = ffi.slice_extract_2d(a["l1_total"], b, sh.l1, 0, sh.l1e)
    a["l1_skip"] = ffi.slice_extract_2d(a["l1_total"], b, sh.l1, sh.l1e, 1)
    a["l1_sqr"] = ffi.abs_pow2_scale_fwd(a["l1_main"], L1_SQR_SCALE)
    a["l2_pre"] = ffi.concat_l1sqr_main_fwd(a["l1_sqr"], a["l1_main"], b, sh.l1e, sh.l1e)
    a["l2_input"] = ffi.crelu_fwd(a["l2_pre"])
    a["l2_out"] = ffi.dense_mm_fwd_bucket(a["l2_input"], st["l2_w"]["w"], st["l2_b"]["w"], bk, b,
                                          sh.l2_in, sh.l2, sh.nb)
    a["l2_acted"] = ffi.crelu_fwd(a["l2_out"])
    a["l3_out"] = ffi.dense_mm_fwd_bucket(a["l2_acted"], st["l3_w"]["w"], st["l3_b"]["w"], bk, b,
                                          sh.l2, 1, sh.nb)
    a["net"] = ffi.elementwise_add(a["l3_out"], a["l1_skip"])
    norm = np.full(b, np.float32(1.0) / np.float32(b), dtype=np.float32)
    if loss["kind"] == "sigmoid":
        a["dy"], acc = ffi.loss_wdl(a["net"], batch["score"], batch["wdl"], norm, wdl_lambda,
                                    loss["scale"])
    else:
        ext = loss["pow_exp"] != 2.0 or loss["qp_asymmetry"] != 0.0 or loss["w1"] != 0.0
        a["dy"], acc = ffi.loss_wrm(a["net"], batch["score"], batch["wdl"], norm, wdl_lambda,
                                    loss["nnue2score"], loss["in_scaling"], loss["in_offset"],
                                    loss["target_offset"], loss["target_scaling"], loss["pow_exp"],
                                    loss["qp_asymmetry"], loss["w1"], loss["w2"], ext)
    return a, acc


def backward(sh: LsShape, st: dict, batch: dict, a: dict, prec: Precision = FP32) -> dict:
    """Gradients of every group (the reference grad buffers after backward)."""
    b = batch["stm"].shape[0]
    bk = batch["bucket"]
    s = sh.sizes()
    g = {}
    dy = a["dy"]
    dl2_acted = ffi.dense_mm_bwd_input_bucket(dy, st["l3_w"]["w"], bk, b, sh.l2, 1, sh.nb)
    g["l3_w"] = ffi.dense_mm_bwd_weight_bucket(a["l2_acted"], dy, bk, b, sh.l2, 1, sh.nb)
    g["l3_b"] = ffi.bias_grad_bucket(dy, bk, np.zeros(s["l3_b"], np.float32), b, 1, sh.nb)
    dl2_out = ffi.crelu_grad(a["l2_out"], dl2_acted)
    dl2_input = ffi.dense_mm_bwd_input_bucket(dl2_out, st["l2_w"]["w"], bk, b, sh.l2_in, sh.l2, sh.nb)
    g["l2_w"] = ffi.dense_mm_bwd_weight_bucket(a["l2_input"], dl2_out, bk, b, sh.l2_in, sh.l2, sh.nb)
    g["l2_b"] = ffi.bias_grad_bucket(dl2_out, bk, np.zeros(s["l2_b"], np.float32), b, sh.l2, sh.nb)
    dl2_pre = ffi.crelu_grad(a["l2_pre"], dl2_input)
    dl1_sqr, dl1_main_from_concat = ffi.concat_l1sqr_main_grad(dl2_pre, b, sh.l1e)
    dl1_main_from_sqr = ffi.abs_pow2_scale_grad(a["l1_main"], dl1_sqr, L1_SQR_SCALE)
    dl1_main = ffi.elementwise_add(dl1_main_from_concat, dl1_main_from_sqr)
    dl1_total = np.zeros(b * sh.l1, dtype=np.float32)
    ffi.slice_scatter_2d(dl1_main, dl1_total, b, sh.l1e, sh.l1, 0)
    ffi.slice_scatter_2d(dy, dl1_total, b, 1, sh.l1, sh.l1e)
    a["dl1_total"] = dl1_total
    # (under tf32 `combined` is the f16 value the forward held)
    dcomb_shared = ffi.dense_mm_bwd_input(dl1_total, st["l1_shared_weight"]["w"], b, sh.ft_out, sh.l1)
    g["l1_shared_weight"] = ffi.dense_mm_bwd_weight(a["combined"], dl1_total, b, sh.ft_out, sh.l1)
    g["l1_shared_bias"] = ffi.bias_grad(dl1_total, np.zeros(sh.l1, np.float32), b, sh.l1)
    g["l1_w"] = ffi.dense_mm_bwd_weight_bucket(a["combined"], dl1_total, bk, b, sh.ft_out, sh.l1, sh.nb)
    dcomb_l1 = ffi.dense_mm_bwd_input_bucket(dl1_total, st["l1_w"]["w"], bk, b, sh.ft_out, sh.l1, sh.nb)
    g["l1_b"] = ffi.bias_grad_bucket(dl1_total, bk, np.zeros(s["l1_b"], np.float32), b, sh.l1, sh.nb)
    dcomb = ffi.elementwise_add(dcomb_l1, dcomb_shared)
    a["dcombined"] = dcomb
    ft_b_grad = np.zeros(sh.ft_out, np.float32)
    a["dft_stm"] = ffi.ft_post_perspective_grad(dcomb, a["ft_stm"], st["ft_b"]["w"], ft_b_grad, b,
                                                sh.ft_out, 0, sh.ft_out, FT_POST_SCALE)
    a["dft_nstm"] = ffi.ft_post_perspective_grad(dcomb, a["ft_nstm"], st["ft_b"]["w"], ft_b_grad, b,
                                                 sh.ft_out, sh.ft_out // 2, sh.ft_out, FT_POST_SCALE)
    g["ft_b"] = ft_b_grad
    ft_grad = np.zeros(s["ft_w"], np.float32)
    if prec.ft_fp16_out:
        scale = DFT_BASE_SCALE * np.float32(b)
        inv = np.float32(1.0) / scale
        a["dft_scale"] = scale
        a["clamps"] = 0
        for k in ("dft_stm", "dft_nstm"):
            scaled = a[k] * scale
            a["clamps"] += int(np.count_nonzero(np.abs(scaled) > F16_MAX))
            a[k + "16"] = f16(np.clip(scaled, -F16_MAX, F16_MAX))
        ffi.ft_grad_fp16(a["dft_stm16"], batch["stm"], batch["nnz"], ft_grad, b, sh.ft_out, sh.ft_in,
                         sh.max_active, inv, add=False)
        ffi.ft_grad_fp16(a["dft_nstm16"], batch["nstm"], batch["nnz"], ft_grad, b, sh.ft_out, sh.ft_in,
                         sh.max_active, inv, add=True)
    else:
        ffi.sparse_ft_backward_nnz(a["dft_stm"], batch["stm"], batch["nnz"], ft_grad, b, sh.ft_out,
                                   sh.ft_in, sh.max_active)
        ffi.sparse_ft_backward_nnz(a["dft_nstm"], batch["nstm"], batch["nnz"], ft_grad, b, sh.ft_out,
                                   sh.ft_in, sh.max_active)
    if sh.piece_inputs:
        ffi.ft_reduce_virtual_grad(ft_grad, sh.ft_in, sh.ft_out, sh.piece_inputs)
    g["ft_w"] = ft_grad
    return g


def optimizer_step(sh: LsShape, st: dict, grads: dict, opt: OptConfig, lr: float, step: int,
                   prec: Precision = FP32):
    """RAdam/Ranger/AdamW over every group (step is the new 1-based count)."""
    ss, denom = opt.step_size_denom(step)
    beta1 = opt.beta1
    order = [("ft_w", "ft", False)] + list(UNIFORM_GROUPS)
    for name, kind, quant in order:
        wd, lr_g = opt.group(kind, lr)
        lo, hi = (-float(QUANT), float(QUANT)) if quant else (F32_MIN, F32_MAX)
        grad = np.ascontiguousarray(grads[name], dtype=np.float32).copy()
        if name == "ft_w" and prec.fp16_opt_state:
            ft = st["ft_w"]
            m = ft["m16"] / M_SCALE
            v = ft["v16"] / V_SCALE
            ffi.radam_step(ft["w"], m, v, grad, lr_g, ss, denom, wd, beta1, BETA2, EPS, lo, hi)
            ft["m16"] = f16(np.clip(m * M_SCALE, -F16_MAX, F16_MAX))
            with np.errstate(invalid="ignore"):
                sv = v * V_SCALE
            ft["v16"] = f16(np.where(sv > F16_MAX, F16_MAX, sv))  # a NaN stays NaN
            ft["m"], ft["v"] = ft["m16"] / M_SCALE, ft["v16"] / V_SCALE
            continue
        ffi.radam_step(st[name]["w"], st[name]["m"], st[name]["v"], grad, lr_g, ss, denom, wd, beta1,
                       BETA2, EPS, lo, hi)
    if opt.optimizer == "ranger" and step % RANGER_K == 0:
        for name, _, _ in order:
            ffi.ranger_lookahead_lerp(st[name]["w"], st[name]["slow"], ALPHA)


def train_step(sh: LsShape, st: dict, batch: dict, opt: OptConfig, lr: float, wdl_lambda: float,
               loss: dict, step: int, prec: Precision = FP32):
    """Full step; mutates st.  Returns (loss_acc, intermediates, grads).  With
    fp16_opt_state, st["ft_w"] must carry "m16" / "v16" (to_f16_state)."""
    a, acc = forward(sh, st, batch, wdl_lambda, loss, prec)
    g = backward(sh, st, batch, a, prec)
    optimizer_step(sh, st, g, opt, lr, step, prec)
    return acc, a, g
