#!/usr/bin/env python3
"""Training-step throughput of the MI355X backend on the BASELINE headline workload.

Default workload: LayerStack, halfka-hm-merged
with the factorizer, ft-out 1536 / l1 16 / l2 32, fp32, batch 65536, 8
output buckets, Ranger, sigmoid-MSE loss at scale 1/290 (the LayerStack
default), on one GPU.  `--workload ls768` runs configs[2] (ft-out 768 / l1 8,
9 buckets) and `--workload simple` configs[1] (Simple HalfKP 256x2-32-32,
AdamW lr 1e-3 wd 0.01, WRM with every scaling at 290 as README.md:57-62
runs it).  A step is one forward + backward + optimizer pass over one
batch; 8 distinct seeded synthetic batches are uploaded to HBM before the
timed region and cycled (inputs resident in HBM, as the metric asks).

Method (after native-bench, bins/nnue_train/src/native_bench.rs:550-575):
W warm-up steps, synchronize, then exactly K timed steps bracketed by a
device synchronize on both sides, host wall clock.  The same K steps are then
timed with host batches (numpy arrays every step, through the trainer's
pinned upload ring, as native-bench passes a host BatchData per step) and
reported beside the resident figure.  A profiled pass times every phase with
HIP events on the trainer's own stream.

Roofline: every kernel of the step has a compulsory-byte count (each input
read once, each output written once, a gathered table counted once;
`compulsory_bytes`).  `roofline.achieved` is the dominant FT kernel's
compulsory bytes over its average launch time; `traffic` is the HBM bytes it
actually moves (rocprofv3 counters, profiles/hbm_traffic.md); the logical
rate of the per-occurrence count (every gathered row once per occurrence) is
kept as `logical_GBps`.  The run
fails loudly if compulsory bytes / time exceed the HBM peak for the dominant
kernel or the whole step.  The CPU baseline is the oracle step (restated
reference CPU kernels, OpenMP) timed on bounded samples on this host: all
cores, one thread, configs[0]'s CPU-only run, and a GPU cross-check of the
first step's outputs.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0

# name -> workload; ref = the reference's published fp32 pos/s at b=65536 on
# RTX 5090 (the reference's README.md:41-43)
WORKLOADS = {
    "ls1536": dict(
        metric="train pos/s @ batch 65536 (LayerStack ft-1536, 1 GPU); FT gather % HBM peak",
        arch="layerstack", spec="halfka-hm-merged", ft_out=1536, l1=16, l2=32, nb=8,
        bucket_mode="progress8kpabs", optimizer="ranger", lr=8.75e-4, ref=2.45e6, ref_src="README.md:41",
        desc="LayerStack halfka-hm-merged ft-out 1536/16/32 fp32, batch 65536, progress8kpabs "
             "(8 buckets, seeded progress weights ~ N(0, 0.01)), Ranger, sigmoid loss 1/290, "
             "factorizer on (BASELINE configs[3])"),
    "ls1536_mixed": dict(
        metric="train pos/s @ batch 65536 (LayerStack ft-1536 --all-optim, 1 GPU); FT gather % HBM peak",
        arch="layerstack", spec="halfka-hm-merged", ft_out=1536, l1=16, l2=32, nb=8,
        bucket_mode="progress8kpabs", optimizer="ranger", lr=8.75e-4, ref=3.13e6, ref_src="README.md:41",
        all_optim=True,
        desc="LayerStack halfka-hm-merged ft-out 1536/16/32 in mixed precision (the --all-optim FT modes: "
             "f16 forward table, f16 FT activations and gradients with loss scale 2^14*b, f16 ft_w moments; "
             "f32 master weights and dense layers), batch 65536, progress8kpabs (8 buckets), Ranger, "
             "sigmoid loss 1/290, factorizer on (BASELINE configs[4])"),
    "ls768": dict(
        metric="train pos/s @ batch 65536 (LayerStack ft-768, 1 GPU); FT gather % HBM peak",
        arch="layerstack", spec="halfka-hm-merged", ft_out=768, l1=8, l2=32, nb=9,
        bucket_mode="kingrank9", optimizer="ranger", lr=8.75e-4, ref=4.24e6, ref_src="README.md:42",
        desc="LayerStack halfka-hm-merged ft-out 768/8/32 fp32, batch 65536, kingrank9 (9 buckets), "
             "Ranger, sigmoid loss 1/290, factorizer on (BASELINE configs[2])"),
    "simple": dict(
        metric="train pos/s @ batch 65536 (Simple HalfKP 256x2-32-32, 1 GPU); FT gather % HBM peak",
        arch="simple", spec="halfkp", ft_out=256, l1=32, l2=32, nb=1,
        bucket_mode="none", optimizer="adamw", lr=1e-3, ref=11.29e6, ref_src="README.md:43",
        desc="Simple HalfKP 256x2-32-32 fp32 crelu, batch 65536, AdamW lr 1e-3 wd 0.01, "
             "WRM with every scaling 290, factorizer on (BASELINE configs[1])"),
}


def hbm_traffic(workload: str, kernel: str):
    """(HBM bytes per launch, commit, kernel-source digest) of a kernel from
    the committed counter summary.

    profiles/hbm_traffic.md holds FETCH_SIZE / WRITE_SIZE per dispatch from
    two rocprofv3 --pmc passes of this script, scaled by a plain-copy
    calibration, with the commit and the `source_digest` of the kernels
    measured; (None, None, None) when the kernel was not profiled.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) == 9 and cells[0] == workload and cells[1].startswith(kernel):
                    return int(cells[6]), cells[7], cells[8]
    except OSError:
        pass
    return None, None, None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def logical_bytes(host_batches, ft_out, ft_in, max_active, lookahead_frac, out_rows, f16=False):
    """Per-launch logical bytes of the two FT kernels (every gathered row counted
    once per occurrence), averaged
    over the batches.  Rows served by L2 / Infinity Cache are counted, so this
    rate can exceed the HBM peak; it is reported beside the roofline, not as it.

    ft_forward: gathered rows of both perspectives + the per-perspective sums
    and combined written (out_rows rows of ft_out values per position: 3 for
    LayerStack, 4 for Simple) + index rows + nnz.  FT gradient + update:
    gathered dft rows (one per occurrence) + occurrence list + w, m, v read and
    written for every real row (+ slow on lookahead steps) + the gradient
    written.  f16 (--all-optim): gathered rows, raw sums, dft, moments and
    `combined` are 2 bytes."""
    nnz_total = np.mean([float(h["nnz"].sum()) for h in host_batches])
    b = host_batches[0]["nnz"].size
    s16 = 2.0 if f16 else 4.0
    gather = 2.0 * nnz_total * ft_out * s16
    outs = (2 * s16 + (s16 if f16 else 4.0) * (out_rows - 2)) * b * ft_out
    fwd = gather + outs + 2.0 * b * max_active * 4 + 4.0 * b
    cells = float(ft_in) * ft_out
    grad = (gather + 2.0 * nnz_total * 4 + cells * (2 * 4.0 + 4 * s16) + lookahead_frac * 2.0 * 4.0 * cells
            + 4.0 * cells)
    return fwd, grad


def scan_mask_words(piece_inputs: int) -> int:
    """Hit-mask words per schedule entry of the block-scan FT backward: feature
    groups of at most 8 waves x 16 features per king block, one word per wave."""
    n_groups = -(-piece_inputs // 128)
    return 8 * n_groups


def compulsory_bytes(w: dict, spec: dict, b: int, scan: bool, lookahead_frac: float) -> dict:
    """Compulsory HBM bytes per launch of every kernel of one step, by phase.

    A kernel's compulsory bytes are what any implementation of it must move:
    each input it needs read once and each output written once; a gathered
    table or activation counts once, however many positions gather it (L2 and
    the Infinity Cache serve the repeats).  Their sum over the step is a lower
    bound on the step's HBM traffic, so compulsory bytes / time <= 8 TB/s for
    any kernel and for the whole step.  Small per-workgroup partials (< 1% of
    the step) are left out, which keeps it a lower bound.
    """
    f16 = bool(w.get("all_optim"))
    ft_in, pi, ma = spec["ft_in"], spec["piece_inputs"], spec["max_active"]
    fo = w["ft_out"]
    s_tab = s_o = s_d = s_m = 2 if f16 else 4
    s_c = 2 if f16 else 4  # `combined` (held as f16 with --all-optim's tf32)
    real, virt = float(ft_in) * fo, float(pi) * fo
    idx = 2.0 * b * ma * 4 + 4.0 * b              # index rows + nnz
    sched = 2.0 * b * 4                            # king-block schedule
    cell = 8.0 + 4.0 * s_m + lookahead_frac * 8.0  # w, m, v read + written (+ slow on lookahead steps)
    masks = scan_mask_words(pi) * 2.0 * b * 4 if scan else 0.0
    occ = 0.0 if scan else 2.0 * b * ma * 4 + 8.0 * ft_in  # occurrence values + offsets
    out = {}
    if w["arch"] == "layerstack":
        l1, nb = w["l1"], w["nb"]
        P = -(-(b + (nb + 1) * 16) // 16) * 16
        out["prep"] = idx + sched + 4.0 * b + (masks + idx + sched if scan else 2 * occ)
        out["ft_forward"] = real * s_tab + idx + sched + 4.0 * fo + 2.0 * b * fo * s_o + s_c * b * fo
        out["dense_forward"] = s_c * b * fo + 4.0 * (nb * l1 * fo + fo * l1) + 4.0 * P * 3 * l1 + 12.0 * b
        out["dense_backward"] = s_c * b * fo + 2.0 * b * fo * s_o + 4.0 * P * l1 + 2.0 * b * fo * s_d
        out["ft_grad_update"] = 2.0 * b * fo * s_d + masks + sched + occ + real * (cell + 4.0)
        out["ft_virtual_fold"] = (8.0 + s_tab) * real + virt * (cell + 4.0)
        out["dense_opt"] = 4.0 * 4 * (nb * l1 * fo + fo * l1)
    else:
        l1 = w["l1"]
        out["prep"] = idx + sched + (masks + idx + sched if scan else 2 * occ)
        out["ft_forward"] = real * 4 + idx + sched + 4.0 * fo + 2.0 * b * fo * 4 + 2.0 * b * 2 * fo * 4
        out["dense_forward"] = 4.0 * b * 2 * fo + 4.0 * 2 * fo * l1 + 4.0 * b * 3 * l1 + 12.0 * b
        out["dense_backward"] = 4.0 * b * 2 * fo + 2.0 * b * fo * 4 + 4.0 * b * l1 + 2.0 * b * fo * 4
        out["ft_grad_update"] = 2.0 * b * fo * 4 + masks + sched + occ + real * (cell + 4.0)
        out["ft_virtual_fold"] = 12.0 * real + virt * (cell + 4.0)
        out["dense_opt"] = 4.0 * 4 * 2 * fo * l1
    return out


WRM290 = {"kind": "wrm", "nnue2score": 290.0, "in_scaling": 290.0, "in_offset": 0.0,
          "target_offset": 0.0, "target_scaling": 290.0, "pow_exp": 2.0, "qp_asymmetry": 0.0,
          "w1": 0.0, "w2": 0.5}
SIGMOID = {"kind": "sigmoid", "scale": 1.0 / 290.0}


def host_facts() -> dict:
    """The CPU the baseline ran on: logical CPUs, the ones this process may use,
    and the model name from /proc/cpuinfo."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count()
    return {"nproc": os.cpu_count(), "affinity_cores": affinity, "cpu_model": model}


def default_cpu_threads() -> int:
    """The cores this process may use, capped by OMP_NUM_THREADS when it is set
    (the GPU box gives one GPU's job a 16-core share whatever nproc shows)."""
    n = host_facts()["affinity_cores"] or 1
    env = os.environ.get("OMP_NUM_THREADS")
    return min(n, int(env)) if env and env.isdigit() and int(env) > 0 else n


def oracle_workload(w: dict, spec: dict):
    """(shape, fresh state, optimizer config, one-step function) of the oracle for a workload."""
    if w["arch"] == "layerstack":
        from oracle import layerstack as ols

        sh = ols.LsShape(ft_in=spec["ft_in"], max_active=spec["max_active"], piece_inputs=spec["piece_inputs"],
                         ft_out=w["ft_out"], l1=w["l1"], l2=w["l2"], nb=w["nb"])
        prec = ols.Precision.all_optim() if w.get("all_optim") else ols.Precision()
        opt = ols.OptConfig(optimizer=w["optimizer"], weight_decay=0.01)

        def fresh():
            st = ols.default_init(sh)
            return ols.to_f16_state(st) if prec.fp16_opt_state else st

        def one(st, bd, step):
            return ols.train_step(sh, st, bd, opt, w["lr"], 0.0, SIGMOID, step, prec)
    else:
        from oracle import simple as osi

        sh = osi.SimpleShape(ft_in=spec["ft_in"], max_active=spec["max_active"],
                             piece_inputs=spec["piece_inputs"], ft_out=w["ft_out"], l1=w["l1"], l2=w["l2"])
        opt = osi.OptConfig(optimizer=w["optimizer"], weight_decay=0.01)

        def fresh():
            return osi.default_init(sh)

        def one(st, bd, step):
            return osi.train_step(sh, st, bd, opt, w["lr"], 0.0, WRM290, step)
    return sh, fresh, one


def host_slice(w: dict, spec: dict, hb: dict, n: int) -> dict:
    ma = spec["max_active"]
    return dict(stm=np.ascontiguousarray(hb["stm"].reshape(-1, ma)[:n]),
                nstm=np.ascontiguousarray(hb["nstm"].reshape(-1, ma)[:n]), nnz=hb["nnz"][:n].copy(),
                bucket=hb["bucket"][:n].copy() if w["arch"] == "layerstack" else None,
                score=hb["score"][:n].copy(), wdl=hb["wdl"][:n].copy())


def timed_steps(one, st, bd, min_seconds: float, max_steps: int, min_steps: int = 1):
    """Consecutive oracle steps until about min_seconds of work (returns steps, seconds)."""
    steps, t0 = 0, time.perf_counter()
    while True:
        steps += 1
        one(st, bd, steps)
        dt = time.perf_counter() - t0
        if steps >= max_steps or (steps >= min_steps and dt >= min_seconds):
            return steps, dt


def gpu_check(w: dict, spec: dict, bd: dict, acc: float, a: dict, st1: dict) -> dict:
    """One GPU step on the CPU sample's batch from the same initial weights, against
    the oracle's first step: net output, loss, and post-step weights of every group
    (1e-5 relative / 1e-6 absolute)."""
    from tatara_amd.trainer import (Batch, LayerStackConfig, LayerStackTrainer, Sigmoid, SimpleConfig,
                                    SimpleTrainer, Wrm)

    n = bd["nnz"].size
    batch = Batch(bd["stm"], bd["nstm"], bd["nnz"], bd["score"], bd["wdl"])
    if w["arch"] == "layerstack":
        cfg = LayerStackConfig(ft_in=spec["ft_in"], max_active=spec["max_active"], piece_inputs=spec["piece_inputs"],
                               ft_out=w["ft_out"], l1_out=w["l1"], l2_out=w["l2"], num_buckets=w["nb"], max_batch=n,
                               optimizer=w["optimizer"], weight_decay=0.01)
        if w.get("all_optim"):
            cfg = cfg.all_optim()
        t = LayerStackTrainer(cfg)
        step = lambda: t.train_step(batch, bd["bucket"], w["lr"], 0.0, Sigmoid(1.0 / 290.0))  # noqa: E731
    else:
        cfg = SimpleConfig(ft_in=spec["ft_in"], max_active=spec["max_active"], piece_inputs=spec["piece_inputs"],
                           ft_out=w["ft_out"], l1_out=w["l1"], l2_out=w["l2"], max_batch=n,
                           optimizer=w["optimizer"], weight_decay=0.01)
        t = SimpleTrainer(cfg)
        wrm = Wrm(nnue2score=290.0, in_scaling=290.0, in_offset=0.0, target_offset=0.0, target_scaling=290.0)
        step = lambda: t.train_step(batch, w["lr"], 0.0, wrm)  # noqa: E731

    def worst(got, exp, rtol=1e-5, atol=1e-6):
        got, exp = np.asarray(got, np.float64), np.asarray(exp, np.float64)
        return float(np.max(np.abs(got - exp) / (atol + rtol * np.abs(exp)))) if exp.size else 0.0

    with t:
        step()
        loss = t.flush_pending_loss()
        net = worst(t.activation("net_output", n), a["net"])
        comb_n = n * w["ft_out"] * (1 if w["arch"] == "layerstack" else 2)
        comb_exact = bool(np.array_equal(t.activation("combined", comb_n), a["combined"]))
        weights = {g: float(f"{worst(t.get(g), st1[g]['w']):.3g}") for g in st1}
    ratios = [net] + list(weights.values())
    return {"batch": n, "combined_bit_exact": comb_exact, "net_output_worst_ratio": float(f"{net:.3g}"),
            "loss_rel_diff": float(f"{abs(loss - acc) / max(abs(acc), 1e-30):.3g}"),
            "post_step_weights_worst_ratio": weights,
            "within_north_star": comb_exact and max(ratios) <= 1.0,
            "bar": "|gpu - cpu| / (1e-6 + 1e-5 |cpu|) <= 1 elementwise"}


def cpu_baseline(w: dict, spec: dict, hb: dict, threads: int, min_seconds: float = 12.0,
                 max_steps: int = 40) -> dict:
    """The oracle step (restated reference CPU kernels, OpenMP) on this host, on
    bounded samples of the same workload: all cores (the value), one thread,
    configs[0]'s CPU-only run, and a GPU cross-check of the first step."""
    from oracle import ffi

    facts = host_facts()
    n = 16384 if w["arch"] == "layerstack" else 32768
    bd = host_slice(w, spec, hb, n)
    sh, fresh, one = oracle_workload(w, spec)
    n_ft = (spec["ft_in"] + spec["piece_inputs"]) * w["ft_out"]

    used = ffi.set_threads(threads)
    st = fresh()
    # the first step doubles as the GPU cross-check's reference
    t0 = time.perf_counter()
    acc, a, _ = one(st, bd, 1)
    first = time.perf_counter() - t0
    st1 = {g: {"w": v["w"].copy()} for g, v in st.items()}
    try:
        check = gpu_check(w, spec, bd, acc, a, st1)
    except Exception as e:  # the baseline must not hide the GPU result
        check = {"error": repr(e)}
    del a, st1
    steps, dt = timed_steps(lambda s_, b_, k: one(s_, b_, k + 1), st, bd, max(min_seconds - first, 0.0),
                            max_steps - 1)
    steps, dt = steps + 1, dt + first
    value = steps * n / dt

    # one thread, a smaller sample of the same workload (two steps: the dense
    # optimizer pass over every FT parameter is a fixed cost per step)
    ffi.set_threads(1)
    n1 = 4096
    st = fresh()
    steps1, dt1 = timed_steps(one, st, host_slice(w, spec, hb, n1), 0.0, 2, 2)
    del st

    # Simple HalfKP 256x2-32-32, WRM 290, AdamW, batch 4096, one
    # superbatch of 64 steps, CPU only (8 distinct seeded batches cycled)
    ffi.set_threads(threads)
    cfg0 = configs0_cpu_run()
    return {
        "value": round(value, 1),
        "unit": "pos/s",
        "cores": used,
        "kind": "port",
        "sample": f"{steps} consecutive full oracle steps (fwd+bwd+{w['optimizer']} over all {n_ft / 1e6:.1f}M "
                  f"FT params) at b={n} of the same workload on {used} threads, {dt:.1f} s",
        "host": facts,
        "single_thread": {"value": round(steps1 * n1 / dt1, 1), "unit": "pos/s", "cores": 1,
                          "sample": f"{steps1} consecutive full oracle steps at b={n1}, {dt1:.1f} s"},
        "configs0_cpu_run": cfg0,
        "gpu_check": check,
    }


def configs0_cpu_run(steps: int = 64, b: int = 4096) -> dict:
    """BASELINE configs[0] on the CPU reference path: Simple HalfKP 256x2-32-32 fp32,
    crelu, WRM at 290, AdamW (lr 1e-3, wd 0.01), batch 4096, one superbatch of
    64 steps, on seeded synthetic PSV positions decoded by the oracle."""
    from oracle import ffi
    from oracle import features as ofe
    from tatara_amd.psv import synthetic_psv

    w = WORKLOADS["simple"]
    info = ofe.feature_set_info("halfkp")
    spec = dict(ft_in=info["ft_in"], max_active=info["max_active"], piece_inputs=info["piece_inputs"])
    _, fresh, one = oracle_workload(w, spec)
    batches = []
    for i in range(8):
        bd = ofe.psv_to_batch(synthetic_psv(b, seed=40000 + i), "halfkp")
        batches.append(dict(stm=bd["stm"], nstm=bd["nstm"], nnz=bd["nnz"], bucket=None, score=bd["score"],
                            wdl=bd["wdl"]))
    st = fresh()
    t0 = time.perf_counter()
    loss = 0.0
    for k in range(steps):
        loss += one(st, batches[k % 8], k + 1)[0]
    dt = time.perf_counter() - t0
    return {"value": round(steps * b / dt, 1), "unit": "pos/s", "threads": ffi.set_threads(0) or None,
            "steps": steps, "batch": b, "seconds": round(dt, 2),
            "mean_loss": float(f"{loss / (steps * b):.6g}"),
            "workload": "configs[0]: Simple HalfKP 256x2-32-32 fp32 crelu, WRM 290, AdamW lr 1e-3 wd 0.01, "
                        "b=4096, 1 superbatch of 64 steps (8 seeded synthetic PSV batches cycled)"}


def quantised_view(t) -> dict:
    """The integer values save_quantised would write (layerstack_weights.rs:568-829),
    computed from the trainer's f32 weights: FT i16 = round(127 w) with the
    factorizer folded in, L1 (bucket + shared) i8 = round(64 w).  Rounding is
    half away from zero, as Rust's f64::round."""
    def rnd(x):
        x = np.asarray(x, np.float64)
        return np.sign(x) * np.floor(np.abs(x) + 0.5)

    cfg = t.config
    ft = t.get("ft_w").reshape(-1, cfg.ft_out)
    real = ft[: cfg.ft_in].copy()
    if cfg.piece_inputs:
        real += np.tile(ft[cfg.ft_in:], (cfg.ft_in // cfg.piece_inputs, 1))
    l1 = t.get("l1_w").reshape(cfg.num_buckets, cfg.l1_out, cfg.ft_out)
    l1s = t.get("l1_shared_weight").reshape(cfg.ft_out, cfg.l1_out)
    merged = (l1 + l1s.T[None]).astype(np.float32)
    return {"ft_i16": np.clip(rnd(127.0 * real), -32768, 32767),
            "l1_i8": np.clip(rnd(64.0 * merged), -128, 127)}


def teacher_scores(hb: dict, ft_in: int, seed: int = 11, scale: float = 60.0) -> np.ndarray:
    """A learnable stand-in for the PSV scores (the synthetic ones are noise):
    a fixed random piece-square teacher, score = scale * (sum of t[f] over the
    side to move's active features - the same over the other side's), clipped
    to +-3000, t ~ N(0, 1) per feature index (seeded)."""
    t = np.random.default_rng(seed).standard_normal(ft_in)
    b = hb["nnz"].size
    stm, nstm = hb["stm"].reshape(b, -1), hb["nstm"].reshape(b, -1)
    valid = np.arange(stm.shape[1])[None, :] < hb["nnz"][:, None]

    def side(idx):
        ok = valid & (idx >= 0) & (idx < ft_in)
        return np.where(ok, t[np.clip(idx, 0, ft_in - 1)], 0.0).sum(axis=1)

    return np.clip(scale * (side(stm) - side(nstm)), -3000.0, 3000.0).astype(np.float32)


def drift_report(w: dict, spec: dict, dev: list, host_batches: list, b: int, steps_per_sb: int) -> dict:
    """f32 vs mixed precision over 8 superbatches from the same initial weights and
    batches.  The synthetic PSV scores carry nothing the net can learn (the loss
    stays flat and the weights barely leave their initial scale, where the FT
    table quantises to all zeros), so the batches' scores are replaced by a
    fixed piece-square teacher (teacher_scores): the positions, features,
    buckets, shape, optimizer and lr stay configs[4]'s.  Reported: both loss
    curves, the exported-net integer tables (FT i16, merged L1 i8) of both runs
    and how many of them differ, the f32 master weights' relative drift per
    group, and the raw net outputs on a held-out batch (the last of the set,
    never trained on), with the mixed-minus-f32 difference set against the
    f32 run's own change from its initial outputs."""
    from tatara_amd.trainer import GROUPS, DeviceArray, LayerStackConfig, LayerStackTrainer, Sigmoid

    base = LayerStackConfig(ft_in=spec["ft_in"], max_active=spec["max_active"], piece_inputs=spec["piece_inputs"],
                            ft_out=w["ft_out"], l1_out=w["l1"], l2_out=w["l2"], num_buckets=w["nb"], max_batch=b,
                            optimizer=w["optimizer"], weight_decay=0.01)
    loss = Sigmoid(1.0 / 290.0)
    taught = []
    for d, hb in zip(dev, host_batches):
        arrays = dict(d.arrays)
        arrays["score"] = DeviceArray(teacher_scores(hb, spec["ft_in"]))
        taught.append(dataclasses.replace(d, arrays=arrays))
    train, held = (taught[:-1], taught[-1]) if len(taught) > 1 else (taught, taught[0])
    curves, views, weights, nets, start, init = {}, {}, {}, {}, {}, {}
    for name, cfg in (("f32", base), ("mixed", base.all_optim())):
        with LayerStackTrainer(cfg) as t:
            if name == "f32":
                init = {g: t.get(g).astype(np.float64) for g in GROUPS}
            start[name] = t.validate_step(held, None, 0.0, loss)[1]
            # train_step returns the previous step's loss; the flush returns the last
            per_step = [t.train_step(train[i % len(train)], None, w["lr"], 0.0, loss)
                        for i in range(8 * steps_per_sb)]
            per_step = per_step[1:] + [t.flush_pending_loss()]
            sb_loss = [float(np.sum(per_step[k * steps_per_sb:(k + 1) * steps_per_sb])) / (steps_per_sb * b)
                       for k in range(8)]
            views[name] = quantised_view(t)
            weights[name] = {g: t.get(g).astype(np.float64) for g in GROUPS}
            nets[name] = t.validate_step(held, None, 0.0, loss)[1].astype(np.float64)
            if name == "mixed":
                clamps, elems = t.fp16_clamp_count()
        curves[name] = sb_loss

    def rel_l2(x, ref):
        d = float(np.linalg.norm(x - ref))
        n = float(np.linalg.norm(ref))
        return d / n if n else d

    w_drift = {g: float(f"{rel_l2(weights['mixed'][g], weights['f32'][g]):.4g}") for g in GROUPS}
    f32_move = {g: float(f"{rel_l2(weights['f32'][g], init[g]):.4g}") for g in GROUPS}
    ft_diff = np.abs(views["f32"]["ft_i16"] - views["mixed"]["ft_i16"])
    l1_diff = np.abs(views["f32"]["l1_i8"] - views["mixed"]["l1_i8"])
    rel = [abs(m - f) / f for f, m in zip(curves["f32"], curves["mixed"]) if f]
    net_d = nets["mixed"] - nets["f32"]
    net_move = nets["f32"] - start["f32"].astype(np.float64)
    move_rms = float(np.sqrt(np.mean(net_move ** 2)))
    drift_rms = float(np.sqrt(np.mean(net_d ** 2)))
    ft_nz = float(np.count_nonzero(views["f32"]["ft_i16"])) / ft_diff.size
    return {
        "superbatches": 8, "steps_per_superbatch": steps_per_sb, "positions_per_superbatch": steps_per_sb * b,
        "lr": w["lr"], "optimizer": w["optimizer"],
        "target": "teacher scores: 60 x (sum of N(0,1) piece-square values over the side to move's active "
                  "features - the other side's), clipped to +-3000, wdl_lambda 0 (the PSV positions, features "
                  "and buckets of the bench; the synthetic PSV scores are noise)",
        "loss_f32": [float(f"{x:.9g}") for x in curves["f32"]],
        "loss_mixed": [float(f"{x:.9g}") for x in curves["mixed"]],
        "loss_rel_diff_max": float(f"{max(rel):.3g}"),
        "weights_rel_l2_mixed_vs_f32": w_drift,
        "weights_rel_l2_f32_trained_vs_init": f32_move,
        "net_output_heldout": {
            "f32_rms": float(np.sqrt(np.mean(nets["f32"] ** 2))),
            "f32_rms_change_from_init": move_rms,
            "mixed_minus_f32_rms": drift_rms,
            "mixed_minus_f32_max_abs": float(np.max(np.abs(net_d))),
            "drift_over_f32_change": float(f"{drift_rms / move_rms:.4g}") if move_rms else None,
            "corr_of_training_change": float(np.corrcoef(net_move, nets["mixed"] - start["mixed"])[0, 1]),
        },
        "ft_i16_nonzero_frac": ft_nz,
        "ft_i16_nonzero_frac_mixed": float(np.count_nonzero(views["mixed"]["ft_i16"])) / ft_diff.size,
        "ft_i16_differing_frac": float(np.count_nonzero(ft_diff)) / ft_diff.size,
        "ft_i16_differing_frac_of_nonzero": (float(np.count_nonzero(ft_diff)) /
                                             max(1, int(np.count_nonzero(views["f32"]["ft_i16"])))),
        "ft_i16_max_abs_diff": int(ft_diff.max()),
        "l1_i8_nonzero_frac": float(np.count_nonzero(views["f32"]["l1_i8"])) / l1_diff.size,
        "l1_i8_differing_frac": float(np.count_nonzero(l1_diff)) / l1_diff.size,
        "l1_i8_max_abs_diff": int(l1_diff.max()),
        "dft_clamps": int(clamps), "dft_values_written": int(elems),
    }


def time_export(t, w: dict, spec: dict, args) -> dict:
    """Times the quantised export (LayerStackWeights / SimpleWeights::save_quantised)
    of the trainer's current weights to a temporary file: GPU quantisation, D2H of
    the quantised stream and the file write, end to end.  With the CPU baseline,
    the oracle exporter (one thread, from host f32 weights already downloaded)
    writes the same file and the bytes are compared."""
    import tempfile

    fv = 28
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "net.bin")
        times = []
        for _ in range(args.export_reps):
            t0 = time.perf_counter()
            t.save_quantised(path, w["spec"], fv_scale=fv)
            times.append(time.perf_counter() - t0)
        with open(path, "rb") as f:
            got = f.read()
    out = {"ms_min": round(1e3 * min(times), 2), "ms_median": round(1e3 * float(np.median(times)), 2),
           "bytes": len(got), "reps": args.export_reps, "format": w["arch"]}
    if not args.no_cpu_baseline:
        from oracle import export as ox

        weights = {g: t.get(g) for g in t.GROUPS}
        t0 = time.perf_counter()
        weights["ft_w"] = ox.coalesce(weights["ft_w"], spec["ft_in"], spec["piece_inputs"], w["ft_out"])
        from tatara_amd.dataloader import FEATURE_SETS, feature_set_info

        fs = FEATURE_SETS[w["spec"]]
        fh = feature_set_info(w["spec"])["feature_hash"]
        if w["arch"] == "layerstack":
            want = ox.ls_save_quantised(fs, fh, spec["ft_in"], w["ft_out"], w["l1"], w["l2"], w["nb"], weights,
                                        fv_scale=fv)
        else:
            weights["l1_w"] = weights["l1_w"].reshape(2 * w["ft_out"], w["l1"]).T.copy()
            weights["l2_w"] = weights["l2_w"].reshape(w["l1"], w["l2"]).T.copy()
            want = ox.simple_save_quantised(fs, fh, spec["ft_in"], w["ft_out"], w["l1"], w["l2"], weights,
                                            fv_scale=fv)
        out["cpu_oracle_ms"] = round(1e3 * (time.perf_counter() - t0), 1)
        out["cpu_oracle_threads"] = 1
        out["identical_to_oracle"] = got == want
    return out


def run_loop_throughput(w: dict, cfg, records: list, b: int, pw, superbatches: int = 2) -> dict:
    """End-to-end training throughput through tatara_train_run (the superbatch
    driver, trainer.rs:759-1211): the bench's PSV batches written to one file
    under /tmp, read back by the driver's reader thread into a pinned
    two-slot ring, uploaded (40 B per position), decoded to indices and
    buckets on the GPU, and trained, `superbatches` superbatches of
    len(records) batches from a fresh trainer.  `value` is positions over the
    superbatches' own seconds, as the reference's `[train] ... pos/s` line
    reports it (trainer.rs:1080-1096: the file read, upload, decode and steps
    of the superbatch, up to its loss flush); `with_checkpoints` adds the
    final .bin export and resume checkpoint the driver writes at the end."""
    import shutil
    import tempfile

    from tatara_amd import run as R
    from tatara_amd.trainer import LayerStackTrainer, Sigmoid, SimpleTrainer, Wrm, simple_fv_scale

    d = tempfile.mkdtemp(prefix="tatara_bench_run_", dir="/tmp")
    try:
        path = os.path.join(d, "bench.psv")
        with open(path, "wb") as f:
            for r in records:
                f.write(np.ascontiguousarray(r).tobytes())
        layerstack = w["arch"] == "layerstack"
        rc = R.TrainingConfig(net_id="bench", feature_set=w["spec"], output_dir=os.path.join(d, "out"),
                              start_superbatch=1, end_superbatch=superbatches,
                              batches_per_superbatch=len(records), batch_size=b, save_rate=1 << 30,
                              fv_scale=None if layerstack else simple_fv_scale(290.0),
                              bucket_mode=w["bucket_mode"], num_buckets=w["nb"],
                              progress_weights=pw.dev if pw is not None else None, print_progress=False)
        if layerstack:
            trainer, loss = LayerStackTrainer(cfg), Sigmoid(1.0 / 290.0)
        else:
            trainer = SimpleTrainer(cfg)
            loss = Wrm(nnue2score=290.0, in_scaling=290.0, in_offset=0.0, target_offset=0.0, target_scaling=290.0)
        with trainer as t:
            t0 = time.perf_counter()
            res = R.run(t, path, R.ConstantLR(w["lr"]), R.ConstantWDL(0.0), rc, loss)
            wall = time.perf_counter() - t0
        sbs = res.superbatches
        pos = sum(r["positions"] for r in sbs)
        secs = sum(r["seconds"] for r in sbs)
        return {"value": round(pos / secs, 1), "unit": "pos/s",
                "per_superbatch_pos_s": [round(r["positions"] / r["seconds"], 1) for r in sbs],
                "with_checkpoints": {"value": round(pos / wall, 1), "unit": "pos/s", "seconds": round(wall, 3)},
                "positions": pos, "superbatches": len(sbs), "batches_per_superbatch": len(records),
                "mean_loss_last": round(sbs[-1]["mean_loss"], 6),
                "path": "tatara_train_run: PSV file in /tmp -> pinned ring -> H2D 40 B/pos -> GPU decode "
                        "-> king-blocked train_step; a fresh trainer"}
    except Exception as e:  # the run figure must not hide the resident result
        return {"value": None, "error": repr(e)}
    finally:
        shutil.rmtree(d, ignore_errors=True)


def make_trainer(w: dict, spec: dict, b: int):
    """The workload's trainer at batch capacity b: (config, trainer, loss,
    step(trainer, device_batch))."""
    from tatara_amd.trainer import (LayerStackConfig, LayerStackTrainer, Sigmoid, SimpleConfig,
                                    SimpleTrainer, Wrm)

    lr = w["lr"]
    if w["arch"] == "layerstack":
        cfg = LayerStackConfig(ft_in=spec["ft_in"], max_active=spec["max_active"],
                               piece_inputs=spec["piece_inputs"], ft_out=w["ft_out"], l1_out=w["l1"],
                               l2_out=w["l2"], num_buckets=w["nb"], max_batch=b,
                               optimizer=w["optimizer"], weight_decay=0.01)
        if w.get("all_optim"):
            cfg = cfg.all_optim()
        loss = Sigmoid(1.0 / 290.0)
        return cfg, LayerStackTrainer(cfg), loss, lambda t, db: t.train_step(db, None, lr, 0.0, loss)
    cfg = SimpleConfig(ft_in=spec["ft_in"], max_active=spec["max_active"],
                       piece_inputs=spec["piece_inputs"], ft_out=w["ft_out"], l1_out=w["l1"],
                       l2_out=w["l2"], max_batch=b, optimizer=w["optimizer"], weight_decay=0.01)
    loss = Wrm(nnue2score=290.0, in_scaling=290.0, in_offset=0.0, target_offset=0.0, target_scaling=290.0)
    return cfg, SimpleTrainer(cfg), loss, lambda t, db: t.train_step(db, lr, 0.0, loss)


def other_workloads(names: list, b: int, steps: int, warmup: int, n_batches: int = 2) -> dict:
    """The other BASELINE workloads, measured the way `value` is: resident
    GPU-decoded batches cycled, warm-up steps, then `steps` timed steps
    bracketed by device synchronisations (host wall clock).  A workload
    that fails is reported with its error; the headline line still prints."""
    out = {}
    for name in names:
        try:
            out[name] = one_workload(name, b, steps, warmup, n_batches)
        except Exception as e:  # noqa: BLE001 - a secondary figure must not cost the headline line
            out[name] = {"value": None, "error": repr(e)}
            log(f"{name}: {e!r}")
    return out


def one_workload(name: str, b: int, steps: int, warmup: int, n_batches: int) -> dict:
    """Resident-batch throughput of one workload (see other_workloads)."""
    from tatara_amd import _lib
    from tatara_amd.dataloader import ProgressWeights, feature_set_info, psv_to_device_batch
    from tatara_amd.psv import synthetic_progress_weights, synthetic_psv

    lib = _lib.load()
    w = WORKLOADS[name]
    info = feature_set_info(w["spec"])
    spec = dict(ft_in=info["ft_in"], max_active=info["max_active"], piece_inputs=info["piece_inputs"])
    pw = ProgressWeights(synthetic_progress_weights(seed=7)) if w["bucket_mode"] == "progress8kpabs" else None
    dev = [psv_to_device_batch(synthetic_psv(b, seed=1000 + i), w["spec"], w["bucket_mode"], w["nb"], pw)
           for i in range(n_batches)]
    _, trainer, _, step = make_trainer(w, spec, b)
    with trainer as t:
        for i in range(warmup):
            step(t, dev[i % len(dev)])
        t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        t0 = time.perf_counter()
        for i in range(steps):
            step(t, dev[i % len(dev)])
        t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        elapsed = time.perf_counter() - t0
    pos_s = b * steps / elapsed
    log(f"{name}: {pos_s:,.0f} pos/s ({1000.0 * elapsed / steps:.3f} ms/step)")
    return {"value": round(pos_s, 1), "unit": "pos/s", "ms_per_step": round(1000.0 * elapsed / steps, 4),
            "steps": steps, "warmup": warmup, "vs_baseline": round(pos_s / w["ref"], 4),
            "vs_baseline_ref": f"RTX 5090 {w['ref'] / 1e6:.2f}M pos/s (reference {w['ref_src']})",
            "dtype": "f16+f32" if w.get("all_optim") else "f32", "workload": w["desc"]}


def git_commit() -> str:
    """The commit of this checkout (.git/HEAD read directly; git may be absent),
    or "unknown"."""
    root = os.path.dirname(os.path.abspath(__file__))
    try:
        with open(os.path.join(root, ".git", "HEAD")) as f:
            head = f.read().strip()
        if head.startswith("ref: "):
            ref = head[5:]
            p = os.path.join(root, ".git", ref)
            if os.path.exists(p):
                with open(p) as f:
                    return f.read().strip()[:12]
            with open(os.path.join(root, ".git", "packed-refs")) as f:
                for line in f:
                    if line.strip().endswith(" " + ref):
                        return line.split()[0][:12]
            return "unknown"
        return head[:12]
    except OSError:
        return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="ls1536")
    ap.add_argument("--batch", type=int, default=65536)
    ap.add_argument("--n-batches", type=int, default=8)
    ap.add_argument("--profile-steps", type=int, default=12)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="oracle threads for the CPU baseline (default: the cores this process may use, "
                         "capped by OMP_NUM_THREADS)")
    ap.add_argument("--drift", type=int, default=0, metavar="STEPS_PER_SUPERBATCH",
                    help="mixed-precision workloads: train the f32 and the mixed trainer from the same "
                         "initial weights over 8 superbatches of this many steps and report the loss "
                         "curves and the drift of the quantised net")
    ap.add_argument("--export-reps", type=int, default=0,
                    help="also time this many quantised exports (.bin) of the trained weights")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="first run a plain device copy of this many MiB (counter calibration)")
    ap.add_argument("--chain-ab-rounds", type=int, default=4,
                    help="alternating rounds of --steps steps with the occurrence-list sort chain skipped "
                         "(king-blocked batches) and queued (gated off on the device); 0 skips the comparison")
    ap.add_argument("--no-run-loop", action="store_true",
                    help="skip the end-to-end tatara_train_run figure (PSV file -> decode -> steps)")
    ap.add_argument("--no-other-workloads", action="store_true",
                    help="skip the short throughput runs of the other BASELINE workloads "
                         "(other_workloads in the JSON line)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build targets a single MI355X "
              f"(--gpus {args.gpus} is not supported; multi-GPU sharding is a design "
              f"note only)", file=sys.stderr)
        return 2

    from tatara_amd import _lib
    from tatara_amd.dataloader import (ProgressWeights, device_batch_to_host, feature_set_info,
                                       psv_to_device_batch)
    from tatara_amd.psv import synthetic_progress_weights, synthetic_psv
    from tatara_amd.trainer import (Batch, LayerStackConfig, LayerStackTrainer, Sigmoid,
                                    SimpleConfig, SimpleTrainer, Wrm)

    w = WORKLOADS[args.workload]
    lib = _lib.load()
    if args.copy_calibration_mb:
        import ctypes as C

        nbytes = args.copy_calibration_mb << 20
        src, dst = C.c_void_p(), C.c_void_p()
        _lib.check(lib.tatara_malloc(C.byref(src), nbytes))
        _lib.check(lib.tatara_malloc(C.byref(dst), nbytes))
        _lib.check(lib.tatara_memset(src.value, 1, nbytes))
        for _ in range(3):
            _lib.check(lib.tatara_op_copy(dst.value, src.value, nbytes))
        _lib.check(lib.tatara_free(src.value))
        _lib.check(lib.tatara_free(dst.value))
        log(f"copied {args.copy_calibration_mb} MiB x3 (counter calibration)")
    info = feature_set_info(w["spec"])
    spec = dict(ft_in=info["ft_in"], max_active=info["max_active"], piece_inputs=info["piece_inputs"])
    b = args.batch
    log(f"{args.workload}: generating {args.n_batches} x {b} synthetic PSV positions")
    records = [synthetic_psv(b, seed=1000 + i) for i in range(args.n_batches)]
    pw = ProgressWeights(synthetic_progress_weights(seed=7)) if w["bucket_mode"] == "progress8kpabs" else None
    # PSV -> feature indices + buckets on the GPU (the dataloader step)
    t_dec = time.perf_counter()
    dev = [psv_to_device_batch(r, w["spec"], w["bucket_mode"], w["nb"], pw) for r in records]
    decode_ms = 1000.0 * (time.perf_counter() - t_dec) / len(dev)
    host_batches = [device_batch_to_host(d) for d in dev]
    log(f"decoded on the GPU: {decode_ms:.2f} ms per batch of {b} (incl. 40 B/pos upload); "
        f"mean nnz {np.mean([h['nnz'].mean() for h in host_batches]):.1f}; bucket histogram "
        f"{np.bincount(host_batches[0]['bucket'], minlength=w['nb']).tolist()}")
    lr = w["lr"]
    cfg, trainer, loss, step = make_trainer(w, spec, b)
    with trainer as t:
        log(f"warm-up {args.warmup} steps")
        for i in range(args.warmup):
            step(t, dev[i % len(dev)])
        t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        log(f"timing {args.steps} steps")
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(t, dev[i % len(dev)])
        last = t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        elapsed = time.perf_counter() - t0
        ms_per_step = 1000.0 * elapsed / args.steps
        pos_s = b * args.steps / elapsed
        log(f"{pos_s:,.0f} pos/s  ({ms_per_step:.3f} ms/step), last loss {last:.4f}")

        # the same resident batches without the king-blocked statement
        # (on_device = 1): the step also queues the occurrence-list sort chain
        # (keys, radix passes, offsets), which the device flag then gates
        # off.  Alternating rounds of each, medians compared.
        gated = [dataclasses.replace(d, king_blocked=False) for d in dev]
        ab = {"skipped": [], "queued": []}
        for rnd in range(args.chain_ab_rounds):
            order = (("skipped", dev), ("queued", gated)) if rnd % 2 == 0 else (("queued", gated), ("skipped", dev))
            for name, bs in order:
                for i in range(args.warmup):
                    step(t, bs[i % len(bs)])
                t.flush_pending_loss()
                _lib.check(lib.tatara_synchronize())
                t0 = time.perf_counter()
                for i in range(args.steps):
                    step(t, bs[i % len(bs)])
                t.flush_pending_loss()
                _lib.check(lib.tatara_synchronize())
                ab[name].append(1000.0 * (time.perf_counter() - t0) / args.steps)
        if args.chain_ab_rounds:
            log(f"sort chain skipped / queued: {np.median(ab['skipped']):.4f} / {np.median(ab['queued']):.4f} "
                f"ms/step (medians of {args.chain_ab_rounds} alternating rounds)")

        # the drop-in path: host batches (on_device = 0) every step, copied into
        # the trainer's pinned upload ring and uploaded on its copy stream, as
        # native-bench passes a host BatchData per step
        host_objs = [(Batch(h["stm"].reshape(b, -1), h["nstm"].reshape(b, -1), h["nnz"], h["score"], h["wdl"]),
                      h["bucket"]) for h in host_batches]
        if w["arch"] == "layerstack":
            hstep = lambda t, hb: t.train_step(hb[0], hb[1], lr, 0.0, loss)  # noqa: E731
        else:
            hstep = lambda t, hb: t.train_step(hb[0], lr, 0.0, loss)  # noqa: E731
        for i in range(args.warmup):
            hstep(t, host_objs[i % len(host_objs)])
        t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        t0 = time.perf_counter()
        for i in range(args.steps):
            hstep(t, host_objs[i % len(host_objs)])
        t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        h_elapsed = time.perf_counter() - t0
        host_pos_s = b * args.steps / h_elapsed
        h2d = sum(a.nbytes for k, a in host_batches[0].items() if k != "bucket" or w["arch"] == "layerstack")
        log(f"host batches: {host_pos_s:,.0f} pos/s ({1000.0 * h_elapsed / args.steps:.3f} ms/step, "
            f"{h2d / 1e6:.1f} MB H2D per step)")

        # phase profile (HIP events on the trainer's stream)
        t.set_profiling(True)
        for i in range(args.profile_steps):
            step(t, dev[i % len(dev)])
        t.flush_pending_loss()
        phases, nprof = t.phase_times()
        t.set_profiling(False)
        step_count = t.step_count
        export = time_export(t, w, spec, args) if args.export_reps > 0 else None
    run_loop = None
    if not args.no_run_loop:
        log(f"run loop: tatara_train_run, 2 superbatches of {len(records)} batches from a PSV file")
        run_loop = run_loop_throughput(w, cfg, records, b, pw)
        log(f"run loop: {run_loop.get('value')} pos/s")
    phase_avg = {k: v / max(nprof, 1) for k, v in phases.items()}
    drift = None
    if args.drift and w.get("all_optim"):
        log(f"drift: f32 vs mixed, 8 superbatches of {args.drift} steps")
        drift = drift_report(w, spec, dev, host_batches, b, args.drift)
    log("phases (ms/step): " + ", ".join(f"{k} {v:.3f}" for k, v in phase_avg.items()))

    la = 1.0 / 6.0 if w["optimizer"] == "ranger" else 0.0
    f16 = bool(w.get("all_optim"))
    fwd_logical, grad_logical = logical_bytes(host_batches, w["ft_out"], spec["ft_in"], spec["max_active"],
                                              lookahead_frac=la, out_rows=3 if w["arch"] == "layerstack" else 4,
                                              f16=f16)
    # the f16 forward table is gathered by the eight-column pair kernel; the
    # trainers run the FT gradient as a block scan for an f32 dft (factorized
    # feature sets; LayerStack from two 256-column chunks, Simple from one),
    # else from occurrence lists
    fwd_kernel = "ft_forward_pair16_kernel" if f16 else "ft_forward_kernel"
    min_scan_cols = 256 if w["arch"] == "simple" else 512
    # the block scan (f32 dft) or its matrix-core form (f16 dft) takes every
    # king-bucketed batch from min_scan_cols columns up
    scan = w["ft_out"] >= min_scan_cols
    grad_kernel = ("ft_grad_mfma_kernel" if f16 else "ft_grad_scan_kernel") if scan else "ft_grad_update_kernel"
    comp = compulsory_bytes(w, spec, b, scan, la)
    step_bytes = sum(comp.values())
    step_frac = step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS
    if step_frac > 1.0:
        raise SystemExit(f"compulsory bytes per step / ms_per_step = {step_frac:.3f} of the HBM peak: the byte "
                         f"model or the timing is wrong")
    kernels = {
        fwd_kernel: (phase_avg["ft_forward"], comp["ft_forward"], fwd_logical),
        grad_kernel: (phase_avg["ft_grad_update"], comp["ft_grad_update"], grad_logical),
    }
    dom = max(kernels, key=lambda k: kernels[k][0])
    ms, byts, logical = kernels[dom]
    achieved = byts / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    if achieved > HBM_PEAK_GBS:
        raise SystemExit(f"{dom}: compulsory bytes / launch time = {achieved:.0f} GB/s exceeds the HBM peak")
    traffic, traffic_commit, traffic_digest = hbm_traffic(args.workload, dom)
    from tatara_amd.build import source_digest

    digest = source_digest()
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "avg_launch_ms": round(ms, 4),
        "compulsory_bytes_per_launch": int(byts),
        # the HBM bytes the kernel actually moves (rocprofv3 counters) and its
        # logical bytes (every gathered row once per occurrence, L2 /
        # Infinity Cache hits included)
        "hbm_GBps": round(traffic / (ms * 1e-3) / 1e9, 1) if (traffic and ms > 0) else None,
        "traffic_over_compulsory": round(traffic / byts, 3) if traffic else None,
        "logical_GBps": round(logical / (ms * 1e-3) / 1e9, 1) if ms > 0 else None,
        "traffic_source": "profiles/hbm_traffic.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; copy-calibrated)",
        # the commit and kernel-source digest the traffic row was measured
        # with, beside this run's: a stale row shows as traffic_current false
        "traffic_commit": traffic_commit,
        "traffic_source_digest": traffic_digest,
        "source_digest": digest,
        "traffic_current": traffic_digest == digest,
        "commit": git_commit(),
    }
    other = {k: {"avg_launch_ms": round(v[0], 4),
                 "compulsory_GB": round(v[1] / 1e9, 4),
                 "compulsory_frac": round(v[1] / (v[0] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if v[0] > 0 else None,
                 "logical_GBps": round(v[2] / (v[0] * 1e-3) / 1e9, 1) if v[0] > 0 else None,
                 "hbm_bytes": hbm_traffic(args.workload, k)[0]}
             for k, v in kernels.items()}
    phases_out = {k: {"ms": round(v, 4), "compulsory_GB": round(comp[k] / 1e9, 4),
                      "compulsory_frac": round(comp[k] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if v > 0 else None}
                  for k, v in phase_avg.items()}

    others = None
    if not args.no_other_workloads:
        others = other_workloads([n for n in WORKLOADS if n != args.workload], b, min(args.steps, 20),
                                 args.warmup)
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle step)")
        try:
            cpu = cpu_baseline(w, spec, host_batches[0], args.cpu_threads or default_cpu_threads())
        except Exception as e:  # the baseline must not hide the GPU result
            cpu = {"value": None, "error": repr(e)}

    line = {
        "metric": w["metric"],
        "value": round(pos_s, 1),
        "unit": "pos/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(pos_s / w["ref"], 4),
        "dtype": "f16+f32" if w.get("all_optim") else "f32",
        "data": f"synthetic: seeded PSV positions (40 pieces, 15% in hand, 10% promoted), decoded to "
                f"{w['spec']} indices and {w['bucket_mode']} buckets on the GPU, resident in HBM",
        "config": {
            "workload": w["desc"],
            "global_batch": b,
            "ft_out": w["ft_out"], "l1": w["l1"], "l2": w["l2"], "num_buckets": w["nb"],
            "n_batches_cycled": args.n_batches,
            "vs_baseline_ref": f"RTX 5090 fp32 {w['ref'] / 1e6:.2f}M pos/s (reference {w['ref_src']})",
            "step_count_end": step_count,
        },
        "roofline": roofline,
        "step_hbm": {"compulsory_GB": round(step_bytes / 1e9, 3),
                     "compulsory_TBps": round(step_bytes / (ms_per_step * 1e-3) / 1e12, 3),
                     "frac": round(step_frac, 4)},
        "host_batches": {"value": round(host_pos_s, 1), "unit": "pos/s",
                         "ms_per_step": round(1000.0 * h_elapsed / args.steps, 4),
                         "ratio_to_resident": round(host_pos_s / pos_s, 4),
                         "h2d_MB_per_step": round(h2d / 1e6, 2),
                         "path": "host arrays every step (on_device = 0): pinned two-slot upload ring, "
                                 "copy stream, event-gated"},
        "sort_chain_ab": None if not args.chain_ab_rounds else {
            "skipped_ms_median": round(float(np.median(ab["skipped"])), 4),
            "queued_ms_median": round(float(np.median(ab["queued"])), 4),
            "skipped_ms": [round(x, 4) for x in ab["skipped"]],
            "queued_ms": [round(x, 4) for x in ab["queued"]],
            "rounds": args.chain_ab_rounds, "steps_per_round": args.steps,
            "path": "the resident batches passed as on_device = 2 (king-blocked: no occurrence-list sort "
                    "chain queued, as `value` runs them) and as on_device = 1 (the chain queued each step "
                    "and gated off on the device), in alternating rounds"},
        "kernels": other,
        "phases": phases_out,
        "psv_decode_ms_per_batch": round(decode_ms, 3),
        "cpu_baseline": cpu,
    }
    if export is not None:
        line["export"] = export
    if drift is not None:
        line["drift_vs_f32"] = drift
    if run_loop is not None:
        line["run_loop"] = run_loop
    if others is not None:
        line["other_workloads"] = others
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
