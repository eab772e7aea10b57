"""LayerStack training-step parity: HIP trainer vs the CPU oracle step (GPU).

Bars:
  - initial weights and the FT forward (raw sums, combined): bit-exact;
  - net output, gradients, post-step weights and optimizer state: within
    1e-5 relative / 1e-6 absolute, looser where a
    batch-reduced sum is compared element-wise against a different order;
  - the step is deterministic: two runs give bit-identical state.
"""
import numpy as np
import pytest

from oracle import layerstack as ols
from tatara_amd.synthetic import small_spec, structured_batch, HALFKA_HM_MERGED
from tatara_amd.trainer import (DeviceBatch, LayerStackConfig, LayerStackTrainer, Sigmoid, Wrm,
                                GROUPS)

pytestmark = pytest.mark.gpu

SPEC = small_spec(king_buckets=10, piece_inputs=64, max_active=40)


def close(got, exp, rtol, atol_frac=0.0, atol=0.0, what=""):
    got = np.asarray(got, np.float64)
    exp = np.asarray(exp, np.float64)
    scale = np.abs(exp).max() if exp.size else 0.0
    tol = atol + atol_frac * scale + rtol * np.abs(exp)
    err = np.abs(got - exp)
    bad = err > tol
    if bad.any():
        ratio = np.where(tol > 0, err / np.where(tol > 0, tol, 1.0), np.inf)
        i = int(np.argmax(np.where(bad, ratio, -1.0)))
        raise AssertionError(
            f"{what}: {bad.sum()} / {bad.size} outside tolerance; worst at {i}: got {got.ravel()[i]:.9g}, "
            f"exp {exp.ravel()[i]:.9g}, err {err.ravel()[i]:.3e} > tol {tol.ravel()[i]:.3e} "
            f"(largest abs err {err.max():.3e})")


def make(nb=8, ft_out=256, l1=16, optimizer="ranger", b=256, keep=True, factorize=True, l2=32):
    sh = ols.LsShape(ft_in=SPEC["ft_in"], max_active=SPEC["max_active"],
                     piece_inputs=SPEC["piece_inputs"] if factorize else 0, ft_out=ft_out, l1=l1,
                     l2=l2, nb=nb)
    cfg = LayerStackConfig(ft_in=sh.ft_in, max_active=sh.max_active, piece_inputs=sh.piece_inputs,
                           ft_out=ft_out, l1_out=l1, l2_out=l2, num_buckets=nb, max_batch=b,
                           optimizer=optimizer, keep_grads=keep)
    return sh, cfg


def batch_for(seed, b, nb, invalid_buckets=True):
    batch, bucket = structured_batch(b, SPEC, num_buckets=nb, seed=seed, nnz_min=30)
    if invalid_buckets:
        bucket[3] = -1
        bucket[7] = nb  # out of range -> no bucket layers
    return batch, bucket


def as_dict(batch, bucket):
    return dict(stm=batch.stm_indices, nstm=batch.nstm_indices, nnz=batch.nnz, bucket=bucket,
                score=batch.score, wdl=batch.wdl)


def loss_dict(loss):
    if isinstance(loss, Sigmoid):
        return {"kind": "sigmoid", "scale": loss.scale}
    return {"kind": "wrm", "nnue2score": loss.nnue2score, "in_scaling": loss.in_scaling,
            "in_offset": loss.in_offset, "target_offset": loss.target_offset,
            "target_scaling": loss.target_scaling, "pow_exp": loss.pow_exp,
            "qp_asymmetry": loss.qp_asymmetry, "w1": loss.weight_boost_w1,
            "w2": loss.weight_boost_w2}


def test_initial_weights_bit_exact(gpu):
    sh, cfg = make()
    with LayerStackTrainer(cfg) as t:
        st = ols.default_init(sh)
        for g in GROUPS:
            assert np.array_equal(t.get(g), st[g]["w"]), g
            assert not t.get(g, "m").any() and not t.get(g, "slow").any()


@pytest.mark.parametrize("loss", [Sigmoid(), Wrm(), Wrm(pow_exp=2.5, qp_asymmetry=0.2, weight_boost_w1=1.0)],
                         ids=["sigmoid", "wrm", "wrm_ext"])
@pytest.mark.parametrize("optimizer", ["ranger", "adamw"])
def test_one_step_matches_oracle(gpu, loss, optimizer):
    sh, cfg = make(optimizer=optimizer)
    b = cfg.max_batch
    batch, bucket = batch_for(1, b, sh.nb)
    lr, lam = 8.75e-4, 0.25
    with LayerStackTrainer(cfg) as t:
        assert t.train_step(batch, bucket, lr, lam, loss) == 0.0
        st = ols.default_init(sh)
        opt = ols.OptConfig(optimizer=optimizer, weight_decay=0.01)
        acc, a, g = ols.train_step(sh, st, as_dict(batch, bucket), opt, lr, lam, loss_dict(loss), 1)
        # forward: bit-exact FT path
        bf = b * sh.ft_out
        assert np.array_equal(t.activation("ft_stm_out", bf), a["ft_stm"])
        assert np.array_equal(t.activation("ft_nstm_out", bf), a["ft_nstm"])
        assert np.array_equal(t.activation("combined", bf), a["combined"])
        close(t.activation("net_output", b), a["net"], 1e-5, atol=1e-6, what="net_output")
        dmax = max(np.abs(a["dft_stm"]).max(), 1e-30)
        close(t.activation("dft_stm", bf), a["dft_stm"], 1e-4, atol=1e-5 * dmax, what="dft_stm")
        close(t.activation("dft_nstm", bf), a["dft_nstm"], 1e-4, atol=1e-5 * dmax, what="dft_nstm")
        # gradients (kept for the check)
        for name in GROUPS:
            close(t.get(name, "grad"), g[name], 1e-4, atol_frac=1e-5, what=f"grad {name}")
        # post-step state
        for name in GROUPS:
            for k in ("w", "m", "v"):
                close(t.get(name, k), st[name][k], 1e-5, atol=1e-6 if k == "w" else 0.0,
                      atol_frac=1e-5 if k != "w" else 0.0, what=f"{name}.{k}")
        close([t.flush_pending_loss()], [acc], 1e-6, what="loss")
        assert t.step_count == 1


def test_rows_across_king_blocks_and_repeated_features(gpu):
    """Index rows that are not king-bucketed (features of several blocks in
    one row) or repeat a feature: the step takes the occurrence-list FT
    backward and still matches the oracle; the next king-bucketed batch
    takes the block scan again (ft_out of two 256-column chunks)."""
    from tatara_amd.trainer import Batch
    sh, cfg = make(optimizer="ranger", ft_out=512)
    b = cfg.max_batch
    rng = np.random.default_rng(21)
    batch, bucket = batch_for(2, b, sh.nb)
    stm = batch.stm_indices.copy()
    stm[:, 0] = rng.integers(0, sh.ft_in, b)  # first slot from any block
    nstm = batch.nstm_indices.copy()
    nstm[5, 3] = nstm[5, 2]                   # a repeated feature
    mixed = Batch(stm, nstm, batch.nnz, batch.score, batch.wdl)
    st = ols.default_init(sh)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    with LayerStackTrainer(cfg) as t:
        for step, (bt, bk) in enumerate([(mixed, bucket), batch_for(3, b, sh.nb)], start=1):
            t.train_step(bt, bk, 1e-3, 0.0, Sigmoid())
            _, a, _ = ols.train_step(sh, st, as_dict(bt, bk), opt, 1e-3, 0.0, loss_dict(Sigmoid()), step)
            # the forward's rows with a feature outside their king block are
            # summed from global memory: still bit-exact
            bf = b * sh.ft_out
            assert np.array_equal(t.activation("ft_stm_out", bf), a["ft_stm"]), step
            assert np.array_equal(t.activation("ft_nstm_out", bf), a["ft_nstm"]), step
            assert np.array_equal(t.activation("combined", bf), a["combined"]), step
            for name in ("ft_w", "ft_b"):
                for k in ("w", "m", "v"):
                    close(t.get(name, k), st[name][k], 1e-5, atol=1e-6 if k == "w" else 0.0,
                          atol_frac=1e-5 if k != "w" else 0.0, what=f"step {step} {name}.{k}")


@pytest.mark.parametrize("ft_out", [256, 512], ids=["occurrence_lists", "block_scan"])
def test_multi_step_ranger_with_lookahead(gpu, ft_out):
    sh, cfg = make(optimizer="ranger", ft_out=ft_out)
    b = cfg.max_batch
    st = ols.default_init(sh)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    loss = Sigmoid()
    losses_gpu, losses_ref = [], []
    with LayerStackTrainer(cfg) as t:
        for step in range(1, 8):  # lookahead fires at step 6
            batch, bucket = batch_for(100 + step % 3, b, sh.nb)
            lagged = t.train_step(batch, bucket, 1e-3, 0.0, loss)
            if step > 1:
                losses_gpu.append(lagged)
            acc, _, _ = ols.train_step(sh, st, as_dict(batch, bucket), opt, 1e-3, 0.0, loss_dict(loss), step)
            losses_ref.append(acc)
        losses_gpu.append(t.flush_pending_loss())
        close(losses_gpu, losses_ref, 1e-5, what="lagged losses")
        for name in GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"{name}.w after 7 steps")
            close(t.get(name, "slow"), st[name]["slow"], 1e-5, atol=1e-6, what=f"{name}.slow")


def test_unfactorized_and_l1_8(gpu):
    sh, cfg = make(factorize=False, l1=8, nb=9, optimizer="radam")
    b = cfg.max_batch
    batch, bucket = batch_for(5, b, sh.nb)
    with LayerStackTrainer(cfg) as t:
        t.train_step(batch, bucket, 1e-3, 0.5, Sigmoid())
        st = ols.default_init(sh)
        opt = ols.OptConfig(optimizer="radam")
        acc, a, g = ols.train_step(sh, st, as_dict(batch, bucket), opt, 1e-3, 0.5, loss_dict(Sigmoid()), 1)
        assert np.array_equal(t.activation("combined", b * sh.ft_out), a["combined"])
        for name in GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=name)


SHAPES = [(l1, l2) for l1 in (8, 16, 32) for l2 in (16, 32, 64)]


@pytest.mark.parametrize("l1,l2", SHAPES, ids=[f"l1_{a}-l2_{b}" for a, b in SHAPES])
def test_dense_shapes_match_oracle(gpu, l1, l2):
    """Every (l1, l2) with kernels (l1 in {8, 16, 32}, l2 in {16, 32, 64}):
    two Ranger steps against the oracle, with the one-step bars for the
    activations, gradients and post-step weights."""
    sh, cfg = make(l1=l1, l2=l2)
    b = cfg.max_batch
    st = ols.default_init(sh)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    loss = Sigmoid()
    with LayerStackTrainer(cfg) as t:
        for step in (1, 2):
            batch, bucket = batch_for(30 + step, b, sh.nb)
            t.train_step(batch, bucket, 8.75e-4, 0.25, loss)
            acc, a, g = ols.train_step(sh, st, as_dict(batch, bucket), opt, 8.75e-4, 0.25, loss_dict(loss), step)
            bf = b * sh.ft_out
            assert np.array_equal(t.activation("combined", bf), a["combined"])
            close(t.activation("net_output", b), a["net"], 1e-5, atol=1e-6, what=f"step {step} net_output")
            dmax = max(np.abs(a["dft_stm"]).max(), 1e-30)
            close(t.activation("dft_stm", bf), a["dft_stm"], 1e-4, atol=1e-5 * dmax, what=f"step {step} dft_stm")
            for name in GROUPS:
                close(t.get(name, "grad"), g[name], 1e-4, atol_frac=1e-5, what=f"step {step} grad {name}")
                close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"step {step} {name}.w")
        assert t.tensor_size("l2_w") == sh.nb * l2 * 2 * (l1 - 1)


@pytest.mark.parametrize("ft_out", [384, 640, 1152])
def test_ft_out_multiples_of_128(gpu, ft_out):
    """ft_out a multiple of 128 but not of 256 (the reference's --ft-out rule,
    training.rs:497-503): the last 256-column chunk of the dft is half
    empty (the block scan from 512 up, the occurrence lists below), and the
    FT-post gradient takes one column per lane.  Two Ranger steps against
    the oracle."""
    sh, cfg = make(ft_out=ft_out)
    b = cfg.max_batch
    st = ols.default_init(sh)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    with LayerStackTrainer(cfg) as t:
        for step in (1, 2):
            batch, bucket = batch_for(50 + step, b, sh.nb)
            t.train_step(batch, bucket, 8.75e-4, 0.25, Sigmoid())
            _, a, g = ols.train_step(sh, st, as_dict(batch, bucket), opt, 8.75e-4, 0.25, loss_dict(Sigmoid()), step)
            bf = b * sh.ft_out
            assert np.array_equal(t.activation("ft_stm_out", bf), a["ft_stm"])
            assert np.array_equal(t.activation("combined", bf), a["combined"])
            for name in GROUPS:
                close(t.get(name, "grad"), g[name], 1e-4, atol_frac=1e-5, what=f"step {step} grad {name}")
                close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"step {step} {name}.w")


@pytest.mark.parametrize("l1,l2", [(24, 32), (16, 48), (4, 32), (64, 32), (16, 128)])
def test_dense_shapes_without_kernels_are_rejected(gpu, l1, l2):
    from tatara_amd._lib import TataraError
    _, cfg = make(l1=l1, l2=l2)
    with pytest.raises(TataraError, match="l1 must be 8, 16 or 32 and l2 16, 32 or 64"):
        LayerStackTrainer(cfg)


def test_validate_step_and_ragged_batch(gpu):
    sh, cfg = make(b=512)
    batch, bucket = batch_for(7, 160, sh.nb)  # smaller than capacity, multiple of 16
    with LayerStackTrainer(cfg) as t:
        sse, net = t.validate_step(batch, bucket, 0.0, Sigmoid())
        st = ols.default_init(sh)
        a, acc = ols.forward(sh, st, as_dict(batch, bucket), 0.0, loss_dict(Sigmoid()))
        close(net, a["net"], 1e-5, atol=1e-6, what="validate net")
        close([sse], [acc], 1e-6, what="validate sse")
        assert t.step_count == 0
        # a batch that is not a multiple of 16 is rejected
        bad, bb = batch_for(7, 24, sh.nb)
        from tatara_amd._lib import TataraError
        with pytest.raises(TataraError):
            t.train_step(bad.__class__(bad.stm_indices[:20], bad.nstm_indices[:20], bad.nnz[:20],
                                       bad.score[:20], bad.wdl[:20]), bb[:20])


def test_device_batch_and_determinism(gpu):
    sh, cfg = make(keep=False)
    b = cfg.max_batch
    batches = [batch_for(s, b, sh.nb) for s in (11, 12, 13)]
    states = []
    for run in range(2):
        with LayerStackTrainer(cfg) as t:
            dbs = [DeviceBatch.upload(bt, bk) for bt, bk in batches]
            for db in dbs:
                t.train_step(db, None, 1e-3, 0.0, Sigmoid())
            t.flush_pending_loss()
            states.append({g: t.get(g) for g in GROUPS})
    for g in GROUPS:
        assert np.array_equal(states[0][g], states[1][g]), g


def test_full_shape_step_properties(gpu):
    """LS ft-1536/16/32, halfka-hm-merged shape, b=4096: finite, deterministic, learns."""
    spec = HALFKA_HM_MERGED
    b = 4096
    cfg = LayerStackConfig(ft_in=spec["ft_in"], max_active=40, piece_inputs=spec["piece_inputs"],
                           ft_out=1536, num_buckets=8, max_batch=b, optimizer="ranger")
    batch, bucket = structured_batch(b, spec, num_buckets=8, seed=3)
    with LayerStackTrainer(cfg) as t:
        db = DeviceBatch.upload(batch, bucket)
        sse0, _ = t.validate_step(db, None, 0.0, Sigmoid())
        for _ in range(5):
            t.train_step(db, None, 5e-3, 0.0, Sigmoid())
        t.flush_pending_loss()
        sse1, net = t.validate_step(db, None, 0.0, Sigmoid())
        assert np.isfinite(net).all()
        assert sse1 < sse0
        w = t.get("ft_w")
        assert np.isfinite(w).all()


def test_host_batches_through_the_upload_ring(gpu):
    """Host batches (on_device = 0) go through the pinned two-slot upload ring
    on the copy stream: the caller may overwrite its arrays as soon as
    train_step returns, and the trained state equals a run on device-resident
    copies of the same batches bit for bit (ragged sizes, consecutive steps
    reusing each ring slot)."""
    from tatara_amd.trainer import Batch
    sh, cfg = make(keep=False, b=512)
    sizes = [512, 160, 512, 256, 96, 512]
    batches = [batch_for(20 + i, n, sh.nb) for i, n in enumerate(sizes)]
    states, losses = [], []
    for mode in ("host", "device"):
        with LayerStackTrainer(cfg) as t:
            got = []
            for bt, bk in batches:
                if mode == "host":
                    hb = Batch(bt.stm_indices.copy(), bt.nstm_indices.copy(), bt.nnz.copy(), bt.score.copy(),
                               bt.wdl.copy())
                    hk = bk.copy()
                    got.append(t.train_step(hb, hk, 1e-3, 0.0, Sigmoid()))
                    for a in (hb.stm_indices, hb.nstm_indices, hk):
                        a[...] = 0
                    hb.score[...] = 1e9
                else:
                    got.append(t.train_step(DeviceBatch.upload(bt, bk), None, 1e-3, 0.0, Sigmoid()))
            got.append(t.flush_pending_loss())
            losses.append(got)
            states.append({g: t.get(g) for g in GROUPS})
    assert losses[0] == losses[1]
    for g in GROUPS:
        assert np.array_equal(states[0][g], states[1][g]), g


@pytest.mark.parametrize("ft_out", [512, 256], ids=["block_scan", "occurrence_lists"])
def test_king_blocked_batches(gpu, ft_out):
    """Device batches passed as king-blocked (on_device = 2: no occurrence-list
    fallback queued) train bit-identically to the same batches passed with
    on_device = 1, with the block scan and with the occurrence lists."""
    sh, cfg = make(keep=False, ft_out=ft_out)
    b = cfg.max_batch
    batches = [batch_for(s, b, sh.nb) for s in (31, 32, 33, 34, 35, 36, 37)]
    states, losses = [], []
    for king_blocked in (False, True):
        with LayerStackTrainer(cfg) as t:
            got = []
            for bt, bk in batches:
                db = DeviceBatch.upload(bt, bk)
                db.king_blocked = king_blocked
                assert db.to_c().on_device == (2 if king_blocked else 1)
                got.append(t.train_step(db, None, 1e-3, 0.0, Sigmoid()))
            got.append(t.flush_pending_loss())
            losses.append(got)
            states.append({g: (t.get(g), t.get(g, "m"), t.get(g, "v")) for g in GROUPS})
    assert losses[0] == losses[1]
    for g in GROUPS:
        for a0, a1 in zip(states[0][g], states[1][g]):
            assert np.array_equal(a0, a1), g


def test_king_blocked_batch_that_is_not_is_reported(gpu):
    """A batch passed as king-blocked whose rows span king blocks or repeat a
    feature (the caller's statement is false): the step trains without the FT
    weight gradient, the next flush reports TATARA_ERR_STATE, and the trainer
    goes on: later king-blocked batches train as before and flush cleanly."""
    from tatara_amd import _lib
    from tatara_amd.trainer import Batch
    sh, cfg = make(keep=False, ft_out=512)
    b = cfg.max_batch
    batch, bucket = batch_for(41, b, sh.nb)
    nstm = batch.nstm_indices.copy()
    nstm[5, 3] = nstm[5, 2]  # a repeated feature
    bad = DeviceBatch.upload(Batch(batch.stm_indices, nstm, batch.nnz, batch.score, batch.wdl), bucket)
    bad.king_blocked = True
    good = DeviceBatch.upload(*batch_for(42, b, sh.nb))
    good.king_blocked = True
    with LayerStackTrainer(cfg) as t:
        w0 = t.get("ft_w")
        t.train_step(bad, None, 1e-3, 0.0, Sigmoid())
        with pytest.raises(_lib.TataraError) as ei:
            t.flush_pending_loss()
        assert ei.value.status == -4 and "on_device = 1" in str(ei.value)
        t.train_step(good, None, 1e-3, 0.0, Sigmoid())
        assert np.isfinite(t.flush_pending_loss())
        assert not np.array_equal(t.get("ft_w"), w0)


@pytest.mark.parametrize("kb,pi,ma", [(10, 64, 44), (2, 1791, 40), (2, 1800, 40)],
                         ids=["max_active_44", "pi_1791", "pi_1800_row_gather"])
def test_forward_table_shapes(gpu, kb, pi, ma):
    """The block-resident forward at its shape limits: max_active above 40
    (twelve slot quads per row, rows padded to 48 slots), the largest king
    block it holds in LDS (1791 rows), and one row more (the row gather runs
    instead).  Forward bit-exact, post-step FT weights within tolerance."""
    spec = small_spec(king_buckets=kb, piece_inputs=pi, max_active=ma)
    sh = ols.LsShape(ft_in=spec["ft_in"], max_active=ma, piece_inputs=pi, ft_out=256, l1=16, l2=32, nb=8)
    cfg = LayerStackConfig(ft_in=sh.ft_in, max_active=ma, piece_inputs=pi, ft_out=256, l1_out=16, l2_out=32,
                           num_buckets=8, max_batch=256, optimizer="ranger", keep_grads=True)
    batch, bucket = structured_batch(256, spec, num_buckets=8, seed=31, nnz_min=ma - 10)
    st = ols.default_init(sh)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    with LayerStackTrainer(cfg) as t:
        t.train_step(batch, bucket, 1e-3, 0.0, Sigmoid())
        _, a, _ = ols.train_step(sh, st, as_dict(batch, bucket), opt, 1e-3, 0.0, loss_dict(Sigmoid()), 1)
        bf = 256 * 256
        assert np.array_equal(t.activation("ft_stm_out", bf), a["ft_stm"])
        assert np.array_equal(t.activation("ft_nstm_out", bf), a["ft_nstm"])
        assert np.array_equal(t.activation("combined", bf), a["combined"])
        for k in ("w", "m", "v"):
            close(t.get("ft_w", k), st["ft_w"][k], 1e-5, atol=1e-6 if k == "w" else 0.0,
                  atol_frac=1e-5 if k != "w" else 0.0, what=f"ft_w.{k}")
