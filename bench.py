#!/usr/bin/env python3
"""Training-step throughput of the MI355X backend on the BASELINE headline workload.

Workload: LayerStack, halfka-hm-merged with the
factorizer, ft-out 1536 / l1 16 / l2 32, fp32, batch 65536, 8 output
buckets, Ranger, sigmoid-MSE loss at scale 1/290 (the LayerStack default),
on one GPU.  A step is one forward + backward + optimizer pass over one
batch; 8 distinct seeded synthetic batches are uploaded to HBM before the
timed region and cycled (inputs resident in HBM, as the metric asks).

Method (after native-bench, bins/nnue_train/src/native_bench.rs:550-575):
W warm-up steps, synchronize, then exactly K timed steps bracketed by a
device synchronize on both sides, host wall clock.  A second, profiled pass
times every phase with HIP events on the trainer's own stream; the dominant
kernel's average duration gives `roofline.achieved` from its algorithmic
bytes.  The CPU baseline is the oracle step (restated reference CPU
kernels, OpenMP) timed on a bounded sample on this host.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "train pos/s @ batch 65536 (LayerStack ft-1536, 1 GPU); FT gather % HBM peak"
HBM_PEAK_GBS = 8000.0
REF_RTX5090_FP32 = 2.45e6  # BASELINE.md section 1 (README.md:41), LayerStack 1536 fp32


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(batches, ft_out, ft_in, max_active, lookahead_frac):
    """Per-launch algorithmic bytes of the two FT kernels, averaged over the batches.

    ft_forward: gathered fp32 rows of both perspectives + raw sums (x2) and
    combined written + index rows + nnz.
    ft_grad_update: gathered fp32 dft rows (one per occurrence) + occurrence
    list + w, m, v read and written for every real row (+ slow on the
    lookahead step, 1 in 6) + the row gradient written for the virtual rows.
    """
    nnz_total = np.mean([float(b.nnz.sum()) for b, _ in batches])
    b = batches[0][0].n_positions
    gather = 2.0 * nnz_total * ft_out * 4
    fwd = gather + 3.0 * b * ft_out * 4 + 2.0 * b * max_active * 4 + 4.0 * b
    rows = ft_in * ft_out * 4.0
    grad = gather + 2.0 * nnz_total * 4 + 6.0 * rows + lookahead_frac * 2.0 * rows + rows
    return fwd, grad


def cpu_baseline(batch, bucket, threads: int) -> dict:
    """Oracle (CPU restatement) step on this host, bounded sample."""
    from oracle import ffi
    from oracle import layerstack as ols

    used = ffi.set_threads(threads)
    n = 16384
    sh = ols.LsShape(ft_in=45 * 1629, max_active=40, piece_inputs=1629, ft_out=1536, l1=16, l2=32, nb=8)
    st = ols.default_init(sh)
    bd = dict(stm=batch.stm_indices[:n], nstm=batch.nstm_indices[:n], nnz=batch.nnz[:n],
              bucket=bucket[:n], score=batch.score[:n], wdl=batch.wdl[:n])
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    loss = {"kind": "sigmoid", "scale": 1.0 / 290.0}
    t0 = time.perf_counter()
    ols.train_step(sh, st, bd, opt, 8.75e-4, 0.0, loss, 1)
    dt = time.perf_counter() - t0
    return {
        "value": round(n / dt, 1),
        "unit": "pos/s",
        "cores": used,
        "kind": "port",
        "sample": f"1 full oracle step (fwd+bwd+Ranger over all 115.1M FT params) at b={n} "
                  f"of the same workload, {dt:.1f} s",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=65536)
    ap.add_argument("--n-batches", type=int, default=8)
    ap.add_argument("--profile-steps", type=int, default=12)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "16")))
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="first run a plain device copy of this many MiB (counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build targets a single MI355X "
              f"(--gpus {args.gpus} is not supported; multi-GPU sharding is a design "
              f"note in DESIGN.md)", file=sys.stderr)
        return 2

    from tatara_amd import _lib
    from tatara_amd.synthetic import HALFKA_HM_MERGED, structured_batch
    from tatara_amd.trainer import DeviceBatch, LayerStackConfig, LayerStackTrainer, Sigmoid

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
    spec = HALFKA_HM_MERGED
    b = args.batch
    log(f"generating {args.n_batches} synthetic batches of {b} positions")
    batches = [structured_batch(b, spec, num_buckets=8, seed=1000 + i) for i in range(args.n_batches)]
    cfg = LayerStackConfig(ft_in=spec["ft_in"], max_active=spec["max_active"],
                           piece_inputs=spec["piece_inputs"], ft_out=1536, l1_out=16, l2_out=32,
                           num_buckets=8, max_batch=b, optimizer="ranger", weight_decay=0.01)
    loss = Sigmoid(1.0 / 290.0)
    lr = 8.75e-4
    with LayerStackTrainer(cfg) as t:
        dev = [DeviceBatch.upload(bt, bk) for bt, bk in batches]
        log(f"warm-up {args.warmup} steps")
        for i in range(args.warmup):
            t.train_step(dev[i % len(dev)], None, lr, 0.0, loss)
        t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        log(f"timing {args.steps} steps")
        t0 = time.perf_counter()
        for i in range(args.steps):
            t.train_step(dev[i % len(dev)], None, lr, 0.0, loss)
        last = t.flush_pending_loss()
        _lib.check(lib.tatara_synchronize())
        elapsed = time.perf_counter() - t0
        ms_per_step = 1000.0 * elapsed / args.steps
        pos_s = b * args.steps / elapsed
        log(f"{pos_s:,.0f} pos/s  ({ms_per_step:.3f} ms/step), last loss {last:.4f}")

        # phase profile (HIP events on the trainer's stream)
        t.set_profiling(True)
        for i in range(args.profile_steps):
            t.train_step(dev[i % len(dev)], None, lr, 0.0, loss)
        t.flush_pending_loss()
        phases, nprof = t.phase_times()
        t.set_profiling(False)
        step_count = t.step_count
    phase_avg = {k: v / max(nprof, 1) for k, v in phases.items()}
    log("phases (ms/step): " + ", ".join(f"{k} {v:.3f}" for k, v in phase_avg.items()))

    fwd_bytes, grad_bytes = algorithmic_bytes(batches, 1536, spec["ft_in"], spec["max_active"],
                                              lookahead_frac=1.0 / 6.0)
    kernels = {
        "ft_forward_kernel": (phase_avg["ft_forward"], fwd_bytes),
        "ft_grad_update_kernel": (phase_avg["ft_grad_update"], grad_bytes),
    }
    dom = max(kernels, key=lambda k: kernels[k][0])
    ms, byts = kernels[dom]
    achieved = byts / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": None,
        "avg_launch_ms": round(ms, 4),
        "algorithmic_bytes_per_launch": int(byts),
    }
    other = {k: {"avg_launch_ms": round(v[0], 4),
                 "algorithmic_GBps": round(v[1] / (v[0] * 1e-3) / 1e9, 1) if v[0] > 0 else None}
             for k, v in kernels.items()}

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle step)")
        try:
            cpu = cpu_baseline(batches[0][0], batches[0][1], args.cpu_threads)
        except Exception as e:  # the baseline must not hide the GPU result
            cpu = {"value": None, "error": repr(e)}

    line = {
        "metric": METRIC,
        "value": round(pos_s, 1),
        "unit": "pos/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(pos_s / REF_RTX5090_FP32, 4),
        "dtype": "f32",
        "data": "synthetic (seeded king-blocked halfka-hm-merged index batches, resident in HBM)",
        "config": {
            "workload": "LayerStack halfka-hm-merged ft-out 1536/16/32 fp32, batch 65536, "
                        "8 buckets, Ranger, sigmoid loss 1/290, factorizer on (BASELINE configs[3])",
            "global_batch": b,
            "ft_out": 1536, "l1": 16, "l2": 32, "num_buckets": 8,
            "n_batches_cycled": args.n_batches,
            "vs_baseline_ref": "RTX 5090 fp32 2.45M pos/s (BASELINE.md, README.md:41)",
            "step_count_end": step_count,
        },
        "roofline": roofline,
        "kernels": other,
        "phases_ms": {k: round(v, 4) for k, v in phase_avg.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
