"""Simple-architecture training-step parity: HIP trainer vs the CPU oracle step (GPU).

Bars (as for LayerStack):
  - initial weights and slow weights, the FT forward (sums + bias, combined):
    bit-exact;
  - L1 pre-activation, net output, dft, gradients, post-step weights and
    optimizer state: within 1e-5 relative / 1e-6 absolute (looser only where
    a batch-reduced sum is compared against a different summation order);
  - the step is deterministic: two runs give bit-identical state.
"""
import numpy as np
import pytest

from oracle import simple as osi
from tatara_amd.synthetic import HALFKP, small_spec, structured_batch
from tatara_amd.trainer import (SIMPLE_GROUPS, DeviceBatch, Sigmoid, SimpleConfig, SimpleTrainer,
                                Wrm)

pytestmark = pytest.mark.gpu

SPEC = small_spec(king_buckets=10, piece_inputs=64, max_active=38)
# README.md:57-62: the Simple trainer runs the WRM with every scaling at 290
WRM290 = Wrm(nnue2score=290.0, in_scaling=290.0, in_offset=0.0, target_offset=0.0, target_scaling=290.0)


def close(got, exp, rtol, atol_frac=0.0, atol=0.0, what=""):
    got = np.asarray(got, np.float64)
    exp = np.asarray(exp, np.float64)
    scale = np.abs(exp).max() if exp.size else 0.0
    tol = atol + atol_frac * scale + rtol * np.abs(exp)
    err = np.abs(got - exp)
    bad = err > tol
    assert not bad.any(), (
        f"{what}: {bad.sum()} / {bad.size} outside tolerance; worst abs err {err.max():.3e} "
        f"at {int(err.argmax())} (got {got.ravel()[err.argmax()]:.9g}, exp {exp.ravel()[err.argmax()]:.9g})"
    )


def make(ft_out=128, l1=32, optimizer="adamw", b=256, keep=True, factorize=True, l2=32):
    sh = osi.SimpleShape(ft_in=SPEC["ft_in"], max_active=SPEC["max_active"],
                         piece_inputs=SPEC["piece_inputs"] if factorize else 0, ft_out=ft_out, l1=l1,
                         l2=l2)
    cfg = SimpleConfig(ft_in=sh.ft_in, max_active=sh.max_active, piece_inputs=sh.piece_inputs,
                       ft_out=ft_out, l1_out=l1, l2_out=l2, max_batch=b, optimizer=optimizer,
                       weight_decay=0.01, keep_grads=keep)
    return sh, cfg


def batch_for(seed, b):
    batch, _ = structured_batch(b, SPEC, num_buckets=1, seed=seed, nnz_min=30)
    return batch


def as_dict(batch):
    return dict(stm=batch.stm_indices, nstm=batch.nstm_indices, nnz=batch.nnz, bucket=None,
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
    with SimpleTrainer(cfg) as t:
        st = osi.default_init(sh)
        for g in SIMPLE_GROUPS:
            assert np.array_equal(t.get(g), st[g]["w"]), g
            assert np.array_equal(t.get(g, "slow"), st[g]["slow"]), g
            assert not t.get(g, "m").any()


@pytest.mark.parametrize("loss", [WRM290, Wrm(), Sigmoid(), Wrm(pow_exp=2.5, qp_asymmetry=0.2, weight_boost_w1=1.0)],
                         ids=["wrm290", "wrm", "sigmoid", "wrm_ext"])
@pytest.mark.parametrize("optimizer", ["adamw", "ranger"])
def test_one_step_matches_oracle(gpu, loss, optimizer):
    sh, cfg = make(optimizer=optimizer)
    b = cfg.max_batch
    batch = batch_for(1, b)
    lr, lam = 1e-3, 0.25
    with SimpleTrainer(cfg) as t:
        assert t.train_step(batch, lr, lam, loss) == 0.0
        st = osi.default_init(sh)
        opt = osi.OptConfig(optimizer=optimizer, weight_decay=0.01)
        acc, a, g = osi.train_step(sh, st, as_dict(batch), opt, lr, lam, loss_dict(loss), 1)
        bf = b * sh.ft_out
        assert np.array_equal(t.activation("ft_stm_out", bf), a["ft_stm"])
        assert np.array_equal(t.activation("ft_nstm_out", bf), a["ft_nstm"])
        assert np.array_equal(t.activation("combined", 2 * bf), a["combined"])
        close(t.activation("l1_pre", b * sh.l1), a["l1_pre"], 1e-5, atol=1e-6, what="l1_pre")
        close(t.activation("net_output", b), a["net"], 1e-5, atol=1e-6, what="net_output")
        dmax = max(np.abs(a["dft_stm"]).max(), 1e-30)
        close(t.activation("dft_stm", bf), a["dft_stm"], 1e-4, atol=1e-5 * dmax, what="dft_stm")
        close(t.activation("dft_nstm", bf), a["dft_nstm"], 1e-4, atol=1e-5 * dmax, what="dft_nstm")
        for name in SIMPLE_GROUPS:
            close(t.get(name, "grad"), g[name], 1e-4, atol_frac=1e-5, what=f"grad {name}")
        for name in SIMPLE_GROUPS:
            for k in ("w", "m", "v"):
                close(t.get(name, k), st[name][k], 1e-5, atol=1e-6 if k == "w" else 0.0,
                      atol_frac=1e-5 if k != "w" else 0.0, what=f"{name}.{k}")
        close([t.flush_pending_loss()], [acc], 1e-6, what="loss")
        assert t.step_count == 1


@pytest.mark.parametrize("ft_out", [128, 256])  # occurrence lists / block scan FT backward
def test_multi_step_ranger_with_lookahead(gpu, ft_out):
    sh, cfg = make(optimizer="ranger", ft_out=ft_out)
    b = cfg.max_batch
    st = osi.default_init(sh)
    opt = osi.OptConfig(optimizer="ranger", weight_decay=0.01)
    losses_gpu, losses_ref = [], []
    with SimpleTrainer(cfg) as t:
        for step in range(1, 8):  # lookahead fires at step 6
            batch = batch_for(100 + step % 3, b)
            lagged = t.train_step(batch, 1e-3, 0.0, WRM290)
            if step > 1:
                losses_gpu.append(lagged)
            acc, _, _ = osi.train_step(sh, st, as_dict(batch), opt, 1e-3, 0.0, loss_dict(WRM290), step)
            losses_ref.append(acc)
        losses_gpu.append(t.flush_pending_loss())
        close(losses_gpu, losses_ref, 1e-5, what="lagged losses")
        for name in SIMPLE_GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"{name}.w after 7 steps")
            close(t.get(name, "slow"), st[name]["slow"], 1e-5, atol=1e-6, what=f"{name}.slow")


def test_rows_across_king_blocks_and_repeated_features(gpu):
    """Index rows with features of several king blocks or a repeated feature:
    the hit-mask pass flags the batch on the device, the gated occurrence
    sort and occurrence-list kernel run instead of the block scan, and the
    step still matches the oracle; the next king-bucketed batch takes the
    block scan again (ft_out 256)."""
    from tatara_amd.trainer import Batch
    sh, cfg = make(optimizer="ranger", ft_out=256)
    b = cfg.max_batch
    rng = np.random.default_rng(22)
    batch = batch_for(4, b)
    stm = batch.stm_indices.copy()
    stm[:, 0] = rng.integers(0, sh.ft_in, b)  # first slot from any block
    nstm = batch.nstm_indices.copy()
    nstm[7, 3] = nstm[7, 2]                   # a repeated feature
    mixed = Batch(stm, nstm, batch.nnz, batch.score, batch.wdl)
    st = osi.default_init(sh)
    opt = osi.OptConfig(optimizer="ranger", weight_decay=0.01)
    with SimpleTrainer(cfg) as t:
        for step, bt in enumerate([mixed, batch_for(5, b), mixed], start=1):
            t.train_step(bt, 1e-3, 0.0, WRM290)
            osi.train_step(sh, st, as_dict(bt), opt, 1e-3, 0.0, loss_dict(WRM290), step)
            for k in ("w", "m", "v"):
                close(t.get("ft_w", k), st["ft_w"][k], 1e-5, atol=1e-6 if k == "w" else 0.0,
                      atol_frac=1e-5 if k != "w" else 0.0, what=f"step {step} ft_w.{k}")


def test_unfactorized_l1_16_ragged_batch(gpu):
    """No factorizer, l1 = 16, RAdam, and a batch that is not a multiple of 16."""
    sh, cfg = make(factorize=False, l1=16, optimizer="radam", ft_out=64, b=256)
    batch = batch_for(5, 200)
    with SimpleTrainer(cfg) as t:
        t.train_step(batch, 1e-3, 0.5, WRM290)
        st = osi.default_init(sh)
        opt = osi.OptConfig(optimizer="radam")
        acc, a, g = osi.train_step(sh, st, as_dict(batch), opt, 1e-3, 0.5, loss_dict(WRM290), 1)
        assert np.array_equal(t.activation("combined", 200 * 2 * sh.ft_out), a["combined"])
        close(t.activation("net_output", 200), a["net"], 1e-5, atol=1e-6, what="net")
        for name in SIMPLE_GROUPS:
            close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=name)
        close([t.flush_pending_loss()], [acc], 1e-6, what="loss")


# (ft_out, l1, l2): the README's 512x2-8-64, and the other l1 / l2 with kernels
SIMPLE_SHAPES = [(512, 8, 64), (128, 8, 16), (128, 16, 16), (128, 16, 64), (128, 32, 16), (256, 32, 64),
                 (128, 8, 32)]


@pytest.mark.parametrize("ft_out,l1,l2", SIMPLE_SHAPES, ids=[f"{a}x2-{b}-{c}" for a, b, c in SIMPLE_SHAPES])
def test_dense_shapes_match_oracle(gpu, ft_out, l1, l2):
    """Two Ranger steps at each shape against the oracle (one-step bars)."""
    sh, cfg = make(ft_out=ft_out, l1=l1, l2=l2, optimizer="ranger")
    b = cfg.max_batch
    st = osi.default_init(sh)
    opt = osi.OptConfig(optimizer="ranger", weight_decay=0.01)
    with SimpleTrainer(cfg) as t:
        for step in (1, 2):
            batch = batch_for(40 + step, b)
            t.train_step(batch, 1e-3, 0.25, WRM290)
            acc, a, g = osi.train_step(sh, st, as_dict(batch), opt, 1e-3, 0.25, loss_dict(WRM290), step)
            bf = b * sh.ft_out
            assert np.array_equal(t.activation("combined", 2 * bf), a["combined"])
            close(t.activation("l1_pre", b * l1), a["l1_pre"], 1e-5, atol=1e-6, what=f"step {step} l1_pre")
            close(t.activation("net_output", b), a["net"], 1e-5, atol=1e-6, what=f"step {step} net_output")
            for name in SIMPLE_GROUPS:
                close(t.get(name, "grad"), g[name], 1e-4, atol_frac=1e-5, what=f"step {step} grad {name}")
                close(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"step {step} {name}.w")


@pytest.mark.parametrize("l1,l2", [(4, 32), (24, 32), (32, 48), (64, 64)])
def test_dense_shapes_without_kernels_are_rejected(gpu, l1, l2):
    from tatara_amd._lib import TataraError
    _, cfg = make(l1=l1, l2=l2)
    with pytest.raises(TataraError, match="l1 must be 8, 16 or 32 and l2 16, 32 or 64"):
        SimpleTrainer(cfg)


def test_validate_step(gpu):
    sh, cfg = make(b=512)
    batch = batch_for(7, 77)
    with SimpleTrainer(cfg) as t:
        sse, net = t.validate_step(batch, 0.0, WRM290)
        st = osi.default_init(sh)
        a, acc = osi.forward(sh, st, as_dict(batch), 0.0, loss_dict(WRM290))
        close(net, a["net"], 1e-5, atol=1e-6, what="validate net")
        close([sse], [acc], 1e-6, what="validate sse")
        assert t.step_count == 0


def test_device_batch_and_determinism(gpu):
    sh, cfg = make(keep=False)
    b = cfg.max_batch
    batches = [batch_for(s, b) for s in (11, 12, 13)]
    states = []
    for run in range(2):
        with SimpleTrainer(cfg) as t:
            dbs = [DeviceBatch.upload(bt) for bt in batches]
            for db in dbs:
                t.train_step(db, 1e-3, 0.0, WRM290)
            t.flush_pending_loss()
            states.append({g: t.get(g) for g in SIMPLE_GROUPS})
    for g in SIMPLE_GROUPS:
        assert np.array_equal(states[0][g], states[1][g]), g


def test_full_shape_halfkp_256_learns(gpu):
    """Simple HalfKP 256x2-32-32 at its real shape (factorizer on), b=4096, AdamW."""
    spec = HALFKP
    b = 4096
    cfg = SimpleConfig(ft_in=spec["ft_in"], max_active=spec["max_active"],
                       piece_inputs=spec["piece_inputs"], ft_out=256, l1_out=32, l2_out=32,
                       max_batch=b, optimizer="adamw", weight_decay=0.01)
    batch, _ = structured_batch(b, spec, num_buckets=1, seed=3)
    with SimpleTrainer(cfg) as t:
        db = DeviceBatch.upload(batch)
        sse0, _ = t.validate_step(db, 0.0, WRM290)
        for _ in range(5):
            t.train_step(db, 1e-3, 0.0, WRM290)
        t.flush_pending_loss()
        sse1, net = t.validate_step(db, 0.0, WRM290)
        assert np.isfinite(net).all()
        assert sse1 < sse0
        assert np.isfinite(t.get("ft_w")).all()


def test_host_batches_through_the_upload_ring(gpu):
    """Host batches through the pinned upload ring equal device batches bit for
    bit, with the caller's arrays overwritten right after each train_step."""
    from tatara_amd.trainer import Batch
    sh, cfg = make(keep=False, b=512)
    batches = [batch_for(30 + i, n) for i, n in enumerate([512, 200, 512, 37, 512])]
    states, losses = [], []
    for mode in ("host", "device"):
        with SimpleTrainer(cfg) as t:
            got = []
            for bt in batches:
                if mode == "host":
                    hb = Batch(bt.stm_indices.copy(), bt.nstm_indices.copy(), bt.nnz.copy(), bt.score.copy(),
                               bt.wdl.copy())
                    got.append(t.train_step(hb, 1e-3, 0.0, WRM290))
                    hb.stm_indices[...] = 0
                    hb.nstm_indices[...] = 0
                    hb.score[...] = 1e9
                else:
                    got.append(t.train_step(DeviceBatch.upload(bt), 1e-3, 0.0, WRM290))
            got.append(t.flush_pending_loss())
            losses.append(got)
            states.append({g: t.get(g) for g in SIMPLE_GROUPS})
    assert losses[0] == losses[1]
    for g in SIMPLE_GROUPS:
        assert np.array_equal(states[0][g], states[1][g]), g


def test_king_blocked_batches(gpu):
    """Simple: device batches passed as king-blocked (on_device = 2, no
    occurrence-list fallback queued) train bit-identically to on_device = 1
    (block scan at 256 columns); a batch that repeats a feature is reported
    by the next flush."""
    from tatara_amd import _lib
    from tatara_amd.trainer import Batch
    sh, cfg = make(keep=False, ft_out=256)
    b = cfg.max_batch
    batches = [batch_for(s, b) for s in (51, 52, 53, 54, 55, 56, 57)]
    states = []
    for king_blocked in (False, True):
        with SimpleTrainer(cfg) as t:
            for bt in batches:
                db = DeviceBatch.upload(bt)
                db.king_blocked = king_blocked
                t.train_step(db, 1e-3, 0.0, WRM290)
            t.flush_pending_loss()
            states.append({g: (t.get(g), t.get(g, "m"), t.get(g, "v")) for g in SIMPLE_GROUPS})
    for g in SIMPLE_GROUPS:
        for a0, a1 in zip(states[0][g], states[1][g]):
            assert np.array_equal(a0, a1), g
    bt = batches[0]
    stm = bt.stm_indices.copy()
    stm[7, 1] = stm[7, 0]
    bad = DeviceBatch.upload(Batch(stm, bt.nstm_indices, bt.nnz, bt.score, bt.wdl))
    bad.king_blocked = True
    with SimpleTrainer(cfg) as t:
        t.train_step(bad, 1e-3, 0.0, WRM290)
        with pytest.raises(_lib.TataraError) as ei:
            t.flush_pending_loss()
        assert ei.value.status == -4


@pytest.mark.parametrize("ma", [44, 38], ids=["max_active_44", "max_active_38"])
def test_forward_slot_padding_and_rows_across_blocks(gpu, ma):
    """The block-resident concat forward with rows padded to 48 slots
    (max_active 44) and to 40 (38), including a row with a feature outside
    its king block (summed again from global memory): bit-exact, and the
    post-step FT weights within tolerance."""
    from tatara_amd.trainer import Batch
    spec = small_spec(king_buckets=10, piece_inputs=64, max_active=ma)
    sh = osi.SimpleShape(ft_in=spec["ft_in"], max_active=ma, piece_inputs=64, ft_out=128, l1=32, l2=32)
    cfg = SimpleConfig(ft_in=sh.ft_in, max_active=ma, piece_inputs=64, ft_out=128, l1_out=32, l2_out=32,
                       max_batch=256, optimizer="adamw", weight_decay=0.01, keep_grads=True)
    batch, _ = structured_batch(256, spec, num_buckets=1, seed=41, nnz_min=ma - 10)
    stm = batch.stm_indices.copy()
    stm[9, 1] = (int(stm[9, 0]) // 64 + 1) % 10 * 64 + 5  # a feature of another block
    batch = Batch(stm, batch.nstm_indices, batch.nnz, batch.score, batch.wdl)
    st = osi.default_init(sh)
    opt = osi.OptConfig(optimizer="adamw", weight_decay=0.01)
    with SimpleTrainer(cfg) as t:
        t.train_step(batch, 1e-3, 0.0, WRM290)
        _, a, _ = osi.train_step(sh, st, as_dict(batch), opt, 1e-3, 0.0, loss_dict(WRM290), 1)
        bf = 256 * sh.ft_out
        assert np.array_equal(t.activation("ft_stm_out", bf), a["ft_stm"])
        assert np.array_equal(t.activation("ft_nstm_out", bf), a["ft_nstm"])
        assert np.array_equal(t.activation("combined", 2 * bf), a["combined"])
        for k in ("w", "m", "v"):
            close(t.get("ft_w", k), st["ft_w"][k], 1e-5, atol=1e-6 if k == "w" else 0.0,
                  atol_frac=1e-5 if k != "w" else 0.0, what=f"ft_w.{k}")
