"""CPU oracle of one Simple (FT -> L1 -> L2 -> L3, CReLU) training step.

Test infrastructure only: chains the restated reference CPU kernels of
oracle/ffi.py in the launch order of SimpleGpuTrainer
(bins/nnue_train/src/trainer_simple.rs), on host arrays:

forward   :1023-1055  FT gather x2 (comb table when factorized)
          :1056-1240  simple_ft_post_fused_crelu per perspective
                      (ft_out += bias in place, combined[b][off + c] = clamp(x, 0, 1);
                      crates/cuda-native-runtime/kernels/native_kernels.cu:1406-1427)
          :1240-1400  L1, L2, L3 as row-major x . W (+ bias) with CReLU between
                      (cuBLAS sgemm_fwd_rowmajor + bias_add_per_row, whose CPU
                      counterpart is dense_mm_fwd_cpu with W [in][out])
          :1401-1506  loss_wdl / loss_wrm (+ wrm_weight_sum)
backward  :1509-2347  L3, L2, L1 (x . W^T, x^T . dy, bias sums, crelu_grad),
                      simple_bwd_ft_act_crelu_fused, simple_bias_grad_dual,
                      FT weight gradient stm then nstm, factorizer reduce
optimizer :2359-2690  RAdam on the 8 groups (one weight decay, one lr; quantised
                      clamp on l1_w, l1_b, l2_w, l2_b, l3_w), lookahead every 6
                      steps (Ranger) on all groups, fold for the next forward

Initial weights: SimpleInit::default_uniform (crates/nnue-train/src/init.rs:290-303)
sampled with the fan-ins of trainer_simple.rs:454-463, FT factorizer rows
appended as zeros, slow weights equal to the initial weights (:474-489).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import ffi
from .layerstack import ALPHA, BETA2, EPS, F32_MAX, F32_MIN, N_SMA_THRESHOLD, QUANT, RANGER_K

SEEDS = tuple(0x5071E001 + k for k in range(8))

# (name, quantised clamp) in run_optimizer_step order (trainer_simple.rs:2443-2520)
GROUPS = (
    ("ft_w", False),
    ("ft_b", False),
    ("l1_w", True),
    ("l1_b", True),
    ("l2_w", True),
    ("l2_b", True),
    ("l3_w", True),
    ("l3_b", False),
)


@dataclass
class SimpleShape:
    ft_in: int
    max_active: int
    piece_inputs: int
    ft_out: int
    l1: int
    l2: int

    @property
    def train_ft_in(self):
        return self.ft_in + self.piece_inputs

    @property
    def l1_in(self):
        return 2 * self.ft_out

    def sizes(self):
        return {
            "ft_w": self.train_ft_in * self.ft_out,
            "ft_b": self.ft_out,
            "l1_w": self.l1_in * self.l1,
            "l1_b": self.l1,
            "l2_w": self.l1 * self.l2,
            "l2_b": self.l2,
            "l3_w": self.l2,
            "l3_b": 1,
        }


def default_init(sh: SimpleShape) -> dict:
    s = sh.sizes()
    ft = ffi.init_sample(sh.ft_in * sh.ft_out, sh.ft_in, "uniform", "abs", 0.01, SEEDS[0])
    ft = np.concatenate([ft, np.zeros(s["ft_w"] - ft.size, dtype=np.float32)])
    fan = {"ft_b": sh.ft_in, "l1_w": sh.l1_in, "l1_b": sh.l1_in, "l2_w": sh.l1, "l2_b": sh.l1,
           "l3_w": sh.l2, "l3_b": sh.l2}
    w = {"ft_w": ft}
    for k, (name, _) in enumerate(GROUPS[1:], start=1):
        w[name] = ffi.init_sample(s[name], fan[name], "uniform", "abs", 0.01, SEEDS[k])
    return {k: {"w": v, "m": np.zeros_like(v), "v": np.zeros_like(v), "slow": v.copy()}
            for k, v in w.items()}


@dataclass
class OptConfig:
    optimizer: str = "adamw"
    weight_decay: float = 0.01

    @property
    def beta1(self):
        return 0.99 if self.optimizer == "ranger" else 0.9

    def step_size_denom(self, step):
        if self.optimizer == "adamw":
            return 1.0, 1
        return ffi.radam_step_size_denom(step, self.beta1, BETA2, N_SMA_THRESHOLD)


def _loss(a, batch, wdl_lambda, loss, b):
    norm = np.full(b, np.float32(1.0) / np.float32(b), dtype=np.float32)
    if loss["kind"] == "sigmoid":
        return ffi.loss_wdl(a["net"], batch["score"], batch["wdl"], norm, wdl_lambda, loss["scale"])
    ext = loss["pow_exp"] != 2.0 or loss["qp_asymmetry"] != 0.0 or loss["w1"] != 0.0
    return ffi.loss_wrm(a["net"], batch["score"], batch["wdl"], norm, wdl_lambda,
                        loss["nnue2score"], loss["in_scaling"], loss["in_offset"],
                        loss["target_offset"], loss["target_scaling"], loss["pow_exp"],
                        loss["qp_asymmetry"], loss["w1"], loss["w2"], ext)


def forward(sh: SimpleShape, st: dict, batch: dict, wdl_lambda: float, loss: dict):
    b = batch["stm"].shape[0]
    ma = sh.max_active
    ft_w = st["ft_w"]["w"]
    if sh.piece_inputs:
        w_fwd = ffi.ft_fold_virtual(ft_w, sh.ft_in, sh.ft_out, sh.piece_inputs)
    else:
        w_fwd = ft_w[: sh.ft_in * sh.ft_out]
    a = {}
    bias = st["ft_b"]["w"]
    raw_s = ffi.sparse_ft_forward(w_fwd, batch["stm"], batch["nnz"], b, sh.ft_out, sh.ft_in, ma)
    raw_n = ffi.sparse_ft_forward(w_fwd, batch["nstm"], batch["nnz"], b, sh.ft_out, sh.ft_in, ma)
    # simple_ft_post_fused_crelu: x = raw + bias (one f32 add), stored back in place
    a["ft_stm"] = (raw_s.reshape(b, sh.ft_out) + bias[None, :]).astype(np.float32).ravel()
    a["ft_nstm"] = (raw_n.reshape(b, sh.ft_out) + bias[None, :]).astype(np.float32).ravel()
    comb = np.empty((b, 2 * sh.ft_out), np.float32)
    comb[:, : sh.ft_out] = ffi.crelu_fwd(a["ft_stm"]).reshape(b, sh.ft_out)
    comb[:, sh.ft_out:] = ffi.crelu_fwd(a["ft_nstm"]).reshape(b, sh.ft_out)
    a["combined"] = comb.ravel()
    a["l1_pre"] = ffi.dense_mm_fwd(a["combined"], st["l1_w"]["w"], st["l1_b"]["w"], b, sh.l1_in, sh.l1)
    a["l1_act"] = ffi.crelu_fwd(a["l1_pre"])
    a["l2_pre"] = ffi.dense_mm_fwd(a["l1_act"], st["l2_w"]["w"], st["l2_b"]["w"], b, sh.l1, sh.l2)
    a["l2_act"] = ffi.crelu_fwd(a["l2_pre"])
    a["net"] = ffi.dense_mm_fwd(a["l2_act"], st["l3_w"]["w"], st["l3_b"]["w"], b, sh.l2, 1)
    a["dy"], acc = _loss(a, batch, wdl_lambda, loss, b)
    return a, acc


def backward(sh: SimpleShape, st: dict, batch: dict, a: dict) -> dict:
    b = batch["stm"].shape[0]
    s = sh.sizes()
    g = {}
    dy = a["dy"]
    dl2_act = ffi.dense_mm_bwd_input(dy, st["l3_w"]["w"], b, sh.l2, 1)
    g["l3_w"] = ffi.dense_mm_bwd_weight(a["l2_act"], dy, b, sh.l2, 1)
    g["l3_b"] = ffi.bias_grad(dy, np.zeros(1, np.float32), b, 1)
    dl2_pre = ffi.crelu_grad(a["l2_pre"], dl2_act)
    dl1_act = ffi.dense_mm_bwd_input(dl2_pre, st["l2_w"]["w"], b, sh.l1, sh.l2)
    g["l2_w"] = ffi.dense_mm_bwd_weight(a["l1_act"], dl2_pre, b, sh.l1, sh.l2)
    g["l2_b"] = ffi.bias_grad(dl2_pre, np.zeros(sh.l2, np.float32), b, sh.l2)
    dl1_pre = ffi.crelu_grad(a["l1_pre"], dl1_act)
    a["dl1_pre"] = dl1_pre
    dcomb = ffi.dense_mm_bwd_input(dl1_pre, st["l1_w"]["w"], b, sh.l1_in, sh.l1)
    g["l1_w"] = ffi.dense_mm_bwd_weight(a["combined"], dl1_pre, b, sh.l1_in, sh.l1)
    g["l1_b"] = ffi.bias_grad(dl1_pre, np.zeros(sh.l1, np.float32), b, sh.l1)
    dc = dcomb.reshape(b, 2 * sh.ft_out)
    a["dcombined"] = dcomb
    # simple_bwd_ft_act_crelu_fused (native_kernels.cu:1452): gradient passes where 0 < x < 1
    a["dft_stm"] = ffi.crelu_grad(a["ft_stm"], np.ascontiguousarray(dc[:, : sh.ft_out]).ravel())
    a["dft_nstm"] = ffi.crelu_grad(a["ft_nstm"], np.ascontiguousarray(dc[:, sh.ft_out:]).ravel())
    # simple_bias_grad_dual (native_kernels.cu:1572): per row stm + nstm, summed over rows
    both = (a["dft_stm"] + a["dft_nstm"]).astype(np.float32)
    g["ft_b"] = ffi.bias_grad(both, np.zeros(sh.ft_out, np.float32), b, sh.ft_out)
    ft_grad = np.zeros(s["ft_w"], np.float32)
    ffi.sparse_ft_backward_nnz(a["dft_stm"], batch["stm"], batch["nnz"], ft_grad, b, sh.ft_out,
                               sh.ft_in, sh.max_active)
    ffi.sparse_ft_backward_nnz(a["dft_nstm"], batch["nstm"], batch["nnz"], ft_grad, b, sh.ft_out,
                               sh.ft_in, sh.max_active)
    if sh.piece_inputs:
        ffi.ft_reduce_virtual_grad(ft_grad, sh.ft_in, sh.ft_out, sh.piece_inputs)
    g["ft_w"] = ft_grad
    return g


def optimizer_step(sh: SimpleShape, st: dict, grads: dict, opt: OptConfig, lr: float, step: int):
    ss, denom = opt.step_size_denom(step)
    for name, quant in GROUPS:
        lo, hi = (-float(QUANT), float(QUANT)) if quant else (F32_MIN, F32_MAX)
        grad = np.ascontiguousarray(grads[name], dtype=np.float32).copy()
        ffi.radam_step(st[name]["w"], st[name]["m"], st[name]["v"], grad, np.float32(lr), ss, denom,
                       opt.weight_decay, opt.beta1, BETA2, EPS, lo, hi)
    if opt.optimizer == "ranger" and step % RANGER_K == 0:
        for name, _ in GROUPS:
            ffi.ranger_lookahead_lerp(st[name]["w"], st[name]["slow"], ALPHA)


def train_step(sh: SimpleShape, st: dict, batch: dict, opt: OptConfig, lr: float, wdl_lambda: float,
               loss: dict, step: int):
    """Full step; mutates st.  Returns (loss_acc, intermediates, grads)."""
    a, acc = forward(sh, st, batch, wdl_lambda, loss)
    g = backward(sh, st, batch, a)
    optimizer_step(sh, st, g, opt, lr, step)
    return acc, a, g
