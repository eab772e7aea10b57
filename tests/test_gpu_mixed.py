"""Mixed precision (the reference's --ft-fp16 / --ft-fp16-out / --fp16-opt-state
modes) on the GPU vs the oracle step with the same f16 rounding points
(oracle/layerstack.py, Precision).

Bars:
  - FT raw sums and `combined`: bit-exact (the same f32 slot-order sums of the
    same f16 rows, rounded once to f16; with tf32 `combined` is held as f16,
    rounded once from the same f32 value);
  - the f16 dft (scaled by 2^14 b): within 2e-3 relative, the bar of the
    reference's own fp16 kernel tests (gpu_cpu_equivalence_tests.rs:2791),
    plus one f16 subnormal step: the dense backward upstream is within 1e-5,
    which can move a value across an f16 rounding boundary;
  - net output, loss and post-step weights: 1e-5 relative / 1e-6 absolute;
  - f16 moments: within 2e-3 relative (one f16 step) of the oracle's stored
    values, plus one f16 subnormal step divided by the scale and a floor of
    1e-5 (after one step) / 1e-4 (after seven) of the tensor's largest
    magnitude: a cell whose dft values sit in the f16 subnormal range (scaled
    values below 2^-14) carries up to one subnormal step, 2^-24 / (2^14 b),
    per occurrence in its gradient, which is several percent of a tiny
    moment and accumulates over steps;
  - the dft clamp counter: equal to the oracle's count up to the values that
    sit within 1e-5 of the clamp threshold;
  - with an f16 dft the ft_w gradient is also allowed 2^-11 A (A the
    cell's sum of |dft| over its h occurrences: each value may sit one f16
    step from the oracle's), and the matrix-core FT backward (king-bucketed
    rows, ft_out >= 512), which sums each cell in another order than the
    oracle, another (h + n_stages + 2) 2^-23 A; the f16 moments inherit that
    gradient bound through (1 - beta1) and (1 - beta2) (2 |g| + bound).
"""
import numpy as np
import pytest

from oracle import ffi
from oracle import layerstack as ols
from tatara_amd.trainer import GROUPS, LayerStackTrainer, Sigmoid

from test_gpu_trainer import as_dict, batch_for, close, loss_dict, make

pytestmark = pytest.mark.gpu

FLAGS = {
    "fp16_fwd": ols.Precision(True, False, False),
    "fp16_fwd_out": ols.Precision(True, True, False),
    "fp16_state": ols.Precision(False, False, True),
    "tf32": ols.Precision(tf32=True),
    "all_optim": ols.Precision.all_optim(),
}
SUB16 = 2.0 ** -24  # smallest f16 subnormal


def mixed(prec: ols.Precision, **kw):
    sh, cfg = make(**kw)
    import dataclasses

    cfg = dataclasses.replace(cfg, ft_fp16=prec.ft_fp16, ft_fp16_out=prec.ft_fp16_out,
                              fp16_opt_state=prec.fp16_opt_state, tf32=prec.tf32)
    return sh, cfg


def oracle_state(sh, prec):
    st = ols.default_init(sh)
    return ols.to_f16_state(st) if prec.fp16_opt_state else st


def f16_grad_bound(sh, batch, a, b, mfma):
    """Per-cell bound on the ft_w gradient's difference from the oracle with
    an f16 dft: 2^-11 A (each of the cell's dft values may sit one f16 step
    from the oracle's, the dense backward upstream being within 1e-5), plus
    (h + n_stages + 2) 2^-23 A when the trainer sums on the matrix cores
    (another order than the oracle's sequential sum); A is the cell's sum of
    |dft16| / scale over its h occurrences and n_stages the 64-row MFMA
    stages of a king block (at most ceil(2b / 64)); virtual rows sum their
    real rows' bounds."""
    inv = float(1.0 / a["dft_scale"])
    A = np.zeros(sh.train_ft_in * sh.ft_out, np.float32)
    h = np.zeros(sh.train_ft_in * sh.ft_out, np.float32)
    for k, idx in (("dft_stm16", "stm"), ("dft_nstm16", "nstm")):
        mag = np.abs(a[k].astype(np.float32))
        ffi.ft_grad_fp16(mag, batch[idx], batch["nnz"], A, b, sh.ft_out, sh.ft_in, sh.max_active, inv,
                         add=idx == "nstm")
        ffi.ft_grad_fp16(np.ones_like(mag), batch[idx], batch["nnz"], h, b, sh.ft_out, sh.ft_in, sh.max_active,
                         1.0, add=idx == "nstm")
    if sh.piece_inputs:
        ffi.ft_reduce_virtual_grad(A, sh.ft_in, sh.ft_out, sh.piece_inputs)
        ffi.ft_reduce_virtual_grad(h, sh.ft_in, sh.ft_out, sh.piece_inputs)
    n_stages = -(-2 * b // 64)
    order = (h.astype(np.float64) + n_stages + 2) * 2.0 ** -23 if mfma else 0.0
    return (2.0 ** -11 + order) * A.astype(np.float64)


def check_moments(t, st, prec, what, floor=1e-5, g=None, g_bound=None, opt=None):
    """f16 ft_w moments within one f16 step; with g_bound (the ft_w gradient's
    own bound, g the oracle gradient) the moments also inherit it: m through
    (1 - beta1), v through (1 - beta2) (2 |g| + g_bound)."""
    for name in GROUPS:
        for k in ("m", "v"):
            got, exp = t.get(name, k), st[name][k]
            if name == "ft_w" and prec.fp16_opt_state:
                scale = ols.M_SCALE if k == "m" else ols.V_SCALE
                extra = 0.0
                if g_bound is not None:
                    extra = ((1 - opt.beta1) * g_bound if k == "m"
                             else (1 - ols.BETA2) * (2 * np.abs(g) + g_bound) * g_bound)
                close(got, exp, 2e-3, atol=SUB16 / float(scale) + extra, atol_frac=floor,
                      what=f"{what} {name}.{k} (f16)")
            else:
                close(got, exp, 1e-5, atol_frac=1e-5, what=f"{what} {name}.{k}")


# ft_out 256: occurrence lists (sequential sums); 512 with a factorizer: the
# block scan, or with an f16 dft its matrix-core form (f32 sums in the
# matrix core's order, within the same 1e-3 gradient bar)
CASES = [(m, f, 256) for m in FLAGS for f in (True, False)] + [("fp16_fwd_out", True, 512),
                                                               ("all_optim", True, 512)]


@pytest.mark.parametrize("mode,factorize,ft_out", CASES,
                         ids=[f"{m}-{'factorized' if f else 'plain'}-{o}" for m, f, o in CASES])
def test_one_step_matches_oracle(gpu, mode, factorize, ft_out):
    prec = FLAGS[mode]
    sh, cfg = mixed(prec, factorize=factorize, ft_out=ft_out)
    b = cfg.max_batch
    batch, bucket = batch_for(11, b, sh.nb)
    lr, lam, loss = 8.75e-4, 0.25, Sigmoid()
    with LayerStackTrainer(cfg) as t:
        t.train_step(batch, bucket, lr, lam, loss)
        st = oracle_state(sh, prec)
        opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
        acc, a, g = ols.train_step(sh, st, as_dict(batch, bucket), opt, lr, lam, loss_dict(loss), 1, prec)
        bf = b * sh.ft_out
        assert np.array_equal(t.activation("ft_stm_out", bf), a["ft_stm"])
        assert np.array_equal(t.activation("ft_nstm_out", bf), a["ft_nstm"])
        assert np.array_equal(t.activation("combined", bf), a["combined"])
        close(t.activation("net_output", b), a["net"], 1e-5, atol=1e-6, what="net_output")
        for k in ("dft_stm", "dft_nstm"):
            if prec.ft_fp16_out:
                close(t.activation(k, bf), a[k + "16"], 2e-3, atol=SUB16, what=k + " (f16, scaled)")
            else:
                dmax = max(np.abs(a[k]).max(), 1e-30)
                close(t.activation(k, bf), a[k], 1e-4, atol=1e-5 * dmax, what=k)
        bd = as_dict(batch, bucket)
        gb = f16_grad_bound(sh, bd, a, b, mfma=factorize and ft_out >= 512) if prec.ft_fp16_out else None
        close(t.get("ft_w", "grad"), g["ft_w"], 1e-3 if prec.ft_fp16_out else 1e-4, atol_frac=1e-5,
              atol=gb if gb is not None else 0.0, what="grad ft_w")
        for name in GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"{name}.w")
        check_moments(t, st, prec, "step 1", g=g["ft_w"], g_bound=gb, opt=opt)
        close([t.flush_pending_loss()], [acc], 1e-6, what="loss")
        clamps, elems = t.fp16_clamp_count()
        assert elems == (2 * b * sh.ft_out if prec.ft_fp16_out else 0)
        assert clamps == 0


@pytest.mark.parametrize("l1,l2,ft_out", [(32, 64, 512), (8, 16, 512), (32, 16, 256), (16, 32, 640)])
def test_all_optim_dense_shapes(gpu, l1, l2, ft_out):
    """--all-optim at l1 = 32 (two 16-output blocks in the TF32 L1 forward,
    the f16-dft L1 input gradient with 32 weights per column), l1 = 8, and
    ft_out 640 (the matrix-core backward's last chunk half empty): one step
    against the oracle with the same bars as the other shapes."""
    prec = FLAGS["all_optim"]
    sh, cfg = mixed(prec, ft_out=ft_out, l1=l1, l2=l2)
    b = cfg.max_batch
    batch, bucket = batch_for(17, b, sh.nb)
    with LayerStackTrainer(cfg) as t:
        t.train_step(batch, bucket, 8.75e-4, 0.25, Sigmoid())
        st = oracle_state(sh, prec)
        opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
        acc, a, g = ols.train_step(sh, st, as_dict(batch, bucket), opt, 8.75e-4, 0.25, loss_dict(Sigmoid()), 1,
                                   prec)
        bf = b * sh.ft_out
        assert np.array_equal(t.activation("combined", bf), a["combined"])
        close(t.activation("net_output", b), a["net"], 1e-5, atol=1e-6, what="net_output")
        for k in ("dft_stm", "dft_nstm"):
            close(t.activation(k, bf), a[k + "16"], 2e-3, atol=SUB16, what=k + " (f16, scaled)")
        bd = as_dict(batch, bucket)
        gb = f16_grad_bound(sh, bd, a, b, mfma=ft_out >= 512)
        close(t.get("ft_w", "grad"), g["ft_w"], 1e-3, atol_frac=1e-5, atol=gb, what="grad ft_w")
        for name in GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"{name}.w")
        check_moments(t, st, prec, "step 1", g=g["ft_w"], g_bound=gb, opt=opt)
        close([t.flush_pending_loss()], [acc], 1e-6, what="loss")


@pytest.mark.parametrize("ft_out", [256, 512])
def test_all_optim_seven_steps_with_lookahead(gpu, ft_out):
    prec = ols.Precision.all_optim()
    sh, cfg = mixed(prec, ft_out=ft_out)
    b = cfg.max_batch
    st = oracle_state(sh, prec)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    loss = Sigmoid()
    losses_gpu, losses_ref = [], []
    with LayerStackTrainer(cfg) as t:
        for step in range(1, 8):  # lookahead fires at step 6
            batch, bucket = batch_for(200 + step % 3, b, sh.nb)
            lagged = t.train_step(batch, bucket, 1e-3, 0.0, loss)
            if step > 1:
                losses_gpu.append(lagged)
            acc, _, _ = ols.train_step(sh, st, as_dict(batch, bucket), opt, 1e-3, 0.0, loss_dict(loss), step,
                                       prec)
            losses_ref.append(acc)
        losses_gpu.append(t.flush_pending_loss())
        close(losses_gpu, losses_ref, 1e-5, what="lagged losses")
        for name in GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"{name}.w after 7 steps")
            close(t.get(name, "slow"), st[name]["slow"], 1e-5, atol=1e-6, what=f"{name}.slow")
        check_moments(t, st, prec, "step 7", floor=1e-4)


def test_all_optim_rows_across_king_blocks(gpu):
    """Mixed precision with ft_out 512 (the matrix-core FT backward): a batch
    with features of several king blocks in a row and a repeated feature is
    flagged on the device and takes the gated occurrence sort and the f16
    occurrence-list kernel; the next batch takes the matrix cores again."""
    from tatara_amd.trainer import Batch
    prec = ols.Precision.all_optim()
    sh, cfg = mixed(prec, ft_out=512)
    b = cfg.max_batch
    rng = np.random.default_rng(23)
    batch, bucket = batch_for(12, b, sh.nb)
    stm = batch.stm_indices.copy()
    stm[:, 0] = rng.integers(0, sh.ft_in, b)
    nstm = batch.nstm_indices.copy()
    nstm[5, 3] = nstm[5, 2]
    cross = Batch(stm, nstm, batch.nnz, batch.score, batch.wdl)
    st = oracle_state(sh, prec)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    with LayerStackTrainer(cfg) as t:
        for step, (bt, bk) in enumerate([(cross, bucket), batch_for(13, b, sh.nb)], start=1):
            t.train_step(bt, bk, 1e-3, 0.0, Sigmoid())
            bd = as_dict(bt, bk)
            _, a, g = ols.train_step(sh, st, bd, opt, 1e-3, 0.0, loss_dict(Sigmoid()), step, prec)
            for name in ("ft_w", "ft_b"):
                close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"step {step} {name}.w")
            # step 1: occurrence lists (sequential sums, as the oracle); step 2: matrix cores
            gb = f16_grad_bound(sh, bd, a, b, mfma=step == 2)
            check_moments(t, st, prec, f"step {step}", g=g["ft_w"], g_bound=gb, opt=opt)


def test_dft_clamp_counter(gpu):
    """A steep loss (sigmoid scale 10) and +-10 skip-column L1 weights push the
    scaled FT gradient past 65504; the clamps are counted and the stored values
    capped, as in the oracle."""
    prec = ols.Precision.all_optim()
    sh, cfg = mixed(prec, b=16)
    b = cfg.max_batch
    batch, bucket = batch_for(3, b, sh.nb, invalid_buckets=False)
    loss = Sigmoid(scale=10.0)
    st = oracle_state(sh, prec)
    w = st["l1_shared_weight"]["w"].reshape(sh.ft_out, sh.l1)
    w[:, sh.l1 - 1] = np.where(np.arange(sh.ft_out) % 2 == 0, 10.0, -10.0)
    with LayerStackTrainer(cfg) as t:
        t.set("l1_shared_weight", st["l1_shared_weight"]["w"])
        t.train_step(batch, bucket, 1e-3, 0.0, loss)
        opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
        _, a, _ = ols.train_step(sh, st, as_dict(batch, bucket), opt, 1e-3, 0.0, loss_dict(loss), 1, prec)
        clamps, elems = t.fp16_clamp_count()
        assert elems == 2 * b * sh.ft_out
        # values within 1e-5 of the threshold may land on either side
        near = sum(int(np.count_nonzero(np.abs(np.abs(a[k] * a["dft_scale"]) - 65504.0) < 65504.0 * 1e-5))
                   for k in ("dft_stm", "dft_nstm"))
        assert a["clamps"] > 50 and abs(clamps - a["clamps"]) <= near, (clamps, a["clamps"], near)
        got = t.activation("dft_stm", b * sh.ft_out)
        assert np.abs(got).max() == 65504.0
        close(got, a["dft_stm16"], 2e-3, atol=SUB16, what="clamped dft_stm")
        for name in GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"{name}.w")


def test_fp16_out_requires_fp16_forward(gpu):
    sh, cfg = mixed(ols.Precision(False, True, False))
    with pytest.raises(Exception, match="ft_fp16_out requires ft_fp16"):
        LayerStackTrainer(cfg)


def test_f16_moment_round_trip(gpu):
    """set/get of f16 moments: x -> f16(clamp(x 2^28)) -> f16 / 2^28
    (MomentBuf::from_host_f32 / to_host_f32)."""
    sh, cfg = mixed(ols.Precision(False, False, True))
    with LayerStackTrainer(cfg) as t:
        n = t.tensor_size("ft_w")
        x = np.random.default_rng(0).normal(0, 1e-5, n).astype(np.float32)
        x[:4] = [1.0, -1.0, 1e-12, 0.0]  # 1.0 * 2^28 saturates at 65504
        t.set("ft_w", x, "m")
        want = ols.f16(np.clip(x * ols.M_SCALE, -65504, 65504)) / ols.M_SCALE
        assert np.array_equal(t.get("ft_w", "m"), want)
