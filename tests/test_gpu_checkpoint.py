"""Raw resume checkpoints (RNRC v8) of the GPU trainers against the oracle's
file reader / writer (oracle/checkpoint.py), and resume determinism.

Bars (all exact):
  - a saved file parses with the oracle reader into the trainer's header
    fields and, group by group in the reference order, the trainer's w, m, v
    and slow (f16 moments as f16 * (1 / scale), MomentBuf::to_host_f32);
  - an oracle-written file loads into exactly its arrays (f16 moments:
    f16(clamp(x * scale, +-65504)), MomentBuf::from_host_f32), the step
    counter, and a forward table rebuilt from the loaded weights;
  - training resumed from a checkpoint is bit-identical to the uninterrupted
    run (weights, moments, slow weights and losses; across a Ranger lookahead
    step), for LayerStack f32, LayerStack --all-optim and Simple - the
    trainers are deterministic, so nothing less is acceptable;
  - a mismatching or truncated file is rejected before any state changes.
"""
import numpy as np
import pytest

from oracle import checkpoint as oc
from tatara_amd.synthetic import HALFKA_HM_MERGED, HALFKP, structured_batch
from tatara_amd._lib import TataraError
from tatara_amd.trainer import (GROUPS, SIMPLE_GROUPS, LayerStackConfig, LayerStackTrainer, Sigmoid,
                                SimpleConfig, SimpleTrainer, Wrm)

pytestmark = pytest.mark.gpu

NB = 8
M_SCALE, V_SCALE = 2.0 ** 28, 2.0 ** 40  # FT_OPT_M_SCALE / FT_OPT_V_SCALE


def ls_cfg(ft_out=128, factorize=True, **kw):
    s = HALFKA_HM_MERGED
    return LayerStackConfig(ft_in=s["ft_in"], max_active=s["max_active"],
                            piece_inputs=s["piece_inputs"] if factorize else 0, ft_out=ft_out, l1_out=16,
                            l2_out=32, num_buckets=NB, max_batch=256, optimizer="ranger", **kw)


def simple_cfg(ft_out=128):
    s = HALFKP
    return SimpleConfig(ft_in=s["ft_in"], max_active=s["max_active"], piece_inputs=s["piece_inputs"],
                        ft_out=ft_out, l1_out=32, l2_out=32, max_batch=256, optimizer="ranger")


def ls_batches(n, b=256):
    return [structured_batch(b, HALFKA_HM_MERGED, num_buckets=NB, seed=100 + i, nnz_min=30) for i in range(n)]


def simple_batches(n, b=256):
    return [structured_batch(b, HALFKP, num_buckets=1, seed=200 + i, nnz_min=30)[0] for i in range(n)]


def ls_arch(cfg, mode="progress8kpabs"):
    return oc.layerstack("halfka-hm-merged", cfg.ft_out, cfg.l1_out, cfg.l2_out, cfg.num_buckets, mode,
                         cfg.piece_inputs > 0)


def simple_arch(cfg):
    return oc.simple("halfkp", cfg.ft_out, cfg.l1_out, cfg.l2_out, cfg.piece_inputs > 0)


def state(t):
    return {g: {k: t.get(g, k) for k in ("w", "m", "v", "slow")} for g in t.GROUPS}


def same_state(a, b, what):
    for g in a:
        for k in a[g]:
            assert np.array_equal(a[g][k], b[g][k], equal_nan=True), f"{what}: {g}.{k}"


def ls_step(t, bb, lr=8.75e-4):
    batch, bucket = bb
    return t.train_step(batch, bucket, lr, 0.0, Sigmoid(1 / 290))


def simple_step(t, batch, lr=1e-3):
    return t.train_step(batch, lr, 0.0, Wrm())


@pytest.mark.parametrize("precision", ["f32", "all_optim"])
def test_layerstack_save_matches_state_and_oracle_reader(gpu, tmp_path, precision):
    cfg = ls_cfg()
    if precision == "all_optim":
        cfg = cfg.all_optim()
    path = tmp_path / "ls.ckpt"
    with LayerStackTrainer(cfg) as t:
        for bb in ls_batches(3):
            ls_step(t, bb)
        t.save_resume_checkpoint(path, "halfka-hm-merged", "kingrank9", 5, "net-run-7", 42)
        h, groups = oc.load_file(path, ls_arch(cfg, "kingrank9"), [(g, t.tensor_size(g)) for g in GROUPS])
        assert (h["version"], h["superbatch"], h["step_count"], h["run_id"], h["lr_horizon"]) == \
            (8, 5, 3, "net-run-7", 42)
        assert [g.name for g in groups] == list(GROUPS)
        for g in groups:
            for k in ("w", "m", "v", "slow"):
                assert np.array_equal(getattr(g, k), t.get(g.name, k)), f"{g.name}.{k}"
        # the moments really are nonzero after three steps (the f16 v of these
        # tiny gradients, ~1e-25 * 2^40, underflows f16 to zero)
        assert np.count_nonzero(groups[0].m)
        assert precision == "all_optim" or np.count_nonzero(groups[0].v)
    assert not (tmp_path / "ls.ckpt.tmp").exists()


def test_simple_save_matches_state_and_oracle_reader(gpu, tmp_path):
    cfg = simple_cfg()
    path = tmp_path / "simple.ckpt"
    with SimpleTrainer(cfg) as t:
        for batch in simple_batches(2):
            simple_step(t, batch)
        t.save_resume_checkpoint(path, "halfkp", None, 1, "", None)
        h, groups = oc.load_file(path, simple_arch(cfg), [(g, t.tensor_size(g)) for g in SIMPLE_GROUPS])
        assert (h["superbatch"], h["step_count"], h["run_id"], h["lr_horizon"]) == (1, 2, None, None)
        for g in groups:
            for k in ("w", "m", "v", "slow"):
                assert np.array_equal(getattr(g, k), t.get(g.name, k)), f"{g.name}.{k}"


@pytest.mark.parametrize("precision", ["f32", "all_optim"])
def test_layerstack_load_oracle_file(gpu, tmp_path, precision):
    cfg = ls_cfg()
    if precision == "all_optim":
        cfg = cfg.all_optim()
    rng = np.random.default_rng(5)
    path = tmp_path / "in.ckpt"
    with LayerStackTrainer(cfg) as t:
        groups = []
        for g in GROUPS:
            n = t.tensor_size(g)
            scale = 0.05 if g != "ft_w" else 0.01
            arrs = [rng.normal(0, scale, n).astype(np.float32), rng.normal(0, 1e-4, n).astype(np.float32),
                    np.abs(rng.normal(0, 1e-8, n)).astype(np.float32), rng.normal(0, scale, n).astype(np.float32)]
            if g == "ft_w":
                arrs[1][:3] = [1e-3, -1.0, 3e-9]  # beyond +-65504 / 2^28: clamped in f16 state
                arrs[2][:2] = [1e-3, 7e-14]
            groups.append(oc.Group(g, *arrs))
        oc.save_file(path, ls_arch(cfg), "producer", 9, 123, None, groups)
        assert t.load_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs") == (9, "producer", None)
        assert t.step_count == 123
        for g in groups:
            for k in ("w", "m", "v", "slow"):
                exp = getattr(g, k)
                if precision == "all_optim" and g.name == "ft_w" and k in ("m", "v"):
                    exp = oc.f16_moment_round_trip(exp, M_SCALE if k == "m" else V_SCALE)
                assert np.array_equal(t.get(g.name, k), exp), f"{g.name}.{k}"
        # the forward table follows the loaded weights: the same net output as a
        # trainer whose weights were set tensor by tensor
        batch, bucket = ls_batches(1)[0]
        _, net = t.validate_step(batch, bucket, 0.0, Sigmoid(1 / 290))
    with LayerStackTrainer(cfg) as ref:
        for g in groups:
            ref.set(g.name, g.w)
        _, net_ref = ref.validate_step(batch, bucket, 0.0, Sigmoid(1 / 290))
    assert np.array_equal(net, net_ref)
    assert np.abs(net).max() > 0


@pytest.mark.parametrize("precision", ["f32", "all_optim"])
def test_layerstack_resume_is_bit_identical(gpu, tmp_path, precision):
    cfg = ls_cfg()
    if precision == "all_optim":
        cfg = cfg.all_optim()
    bs = ls_batches(6)
    path = tmp_path / "resume.ckpt"
    with LayerStackTrainer(cfg) as a:
        for i in range(4):
            ls_step(a, bs[i % len(bs)])
        a.flush_pending_loss()
        a.save_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs", 1, "run-a", 10)
        # steps 5..9 cross the lookahead at step 6
        losses_a = [ls_step(a, bs[i % len(bs)]) for i in range(4, 9)][1:] + [a.flush_pending_loss()]
        end_a = state(a)
        steps_a = a.step_count
    with LayerStackTrainer(cfg) as b:
        ls_step(b, bs[5])  # state that the load must replace
        b.flush_pending_loss()
        assert b.load_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs") == (1, "run-a", 10)
        assert b.step_count == 4
        losses_b = [ls_step(b, bs[i % len(bs)]) for i in range(4, 9)][1:] + [b.flush_pending_loss()]
        same_state(end_a, state(b), f"resumed LayerStack ({precision})")
        assert b.step_count == steps_a == 9
    assert losses_a == losses_b


def test_simple_resume_is_bit_identical(gpu, tmp_path):
    cfg = simple_cfg()
    bs = simple_batches(4)
    path = tmp_path / "resume.ckpt"
    with SimpleTrainer(cfg) as a:
        for i in range(3):
            simple_step(a, bs[i % 4])
        a.flush_pending_loss()
        a.save_resume_checkpoint(path, "halfkp", None, 2)
        losses_a = [simple_step(a, bs[i % 4]) for i in range(3, 8)][1:] + [a.flush_pending_loss()]
        end_a = state(a)
    with SimpleTrainer(cfg) as b:
        assert b.load_resume_checkpoint(path, "halfkp", None) == (2, None, None)
        losses_b = [simple_step(b, bs[i % 4]) for i in range(3, 8)][1:] + [b.flush_pending_loss()]
        same_state(end_a, state(b), "resumed Simple")
    assert losses_a == losses_b


def test_f32_checkpoint_into_f16_state_trainer(gpu, tmp_path):
    path = tmp_path / "f32.ckpt"
    with LayerStackTrainer(ls_cfg()) as a:
        for bb in ls_batches(2):
            ls_step(a, bb)
        a.save_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs", 0)
        st = state(a)
    with LayerStackTrainer(ls_cfg().all_optim()) as b:
        b.load_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs")
        assert np.array_equal(b.get("ft_w", "m"), oc.f16_moment_round_trip(st["ft_w"]["m"], M_SCALE))
        assert np.array_equal(b.get("ft_w", "v"), oc.f16_moment_round_trip(st["ft_w"]["v"], V_SCALE))
        assert np.array_equal(b.get("ft_w"), st["ft_w"]["w"])
        assert np.array_equal(b.get("l1_w", "m"), st["l1_w"]["m"])


def test_mismatch_and_truncation_leave_state_unchanged(gpu, tmp_path):
    path = tmp_path / "ls.ckpt"
    with LayerStackTrainer(ls_cfg()) as a:
        ls_step(a, ls_batches(1)[0])
        a.save_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs", 0)
    data = path.read_bytes()
    with LayerStackTrainer(ls_cfg(ft_out=256)) as other:
        with pytest.raises(TataraError, match="ft_out mismatch: got 128, want 256"):
            other.load_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs")
    with LayerStackTrainer(ls_cfg(factorize=False)) as other:
        with pytest.raises(TataraError, match="ft-factorize mismatch"):
            other.load_resume_checkpoint(path, "halfka-hm-merged", "progress8kpabs")
    with LayerStackTrainer(ls_cfg()) as t:
        before = state(t)
        with pytest.raises(TataraError, match="bucket mode 'progress8kpabs' does not match --bucket-mode 'kingrank9'"):
            t.load_resume_checkpoint(path, "halfka-hm-merged", "kingrank9")
        cut = tmp_path / "cut.ckpt"
        cut.write_bytes(data[:-1])
        with pytest.raises(TataraError, match="truncated while reading group l3_b slow"):
            t.load_resume_checkpoint(cut, "halfka-hm-merged", "progress8kpabs")
        n_ftw = t.tensor_size("ft_w")
        hdr = len(data) - sum(8 + 16 * t.tensor_size(g) for g in GROUPS)
        cut.write_bytes(data[:hdr + 8 + 4 * n_ftw + 100])
        with pytest.raises(TataraError, match="truncated while reading group ft_w m"):
            t.load_resume_checkpoint(cut, "halfka-hm-merged", "progress8kpabs")
        bad = bytearray(data)
        bad[hdr:hdr + 8] = (n_ftw + 1).to_bytes(8, "little")
        cut.write_bytes(bytes(bad))
        with pytest.raises(TataraError, match="group ft_w len mismatch"):
            t.load_resume_checkpoint(cut, "halfka-hm-merged", "progress8kpabs")
        same_state(before, state(t), "state after rejected loads")
        assert t.step_count == 0
        # trailing bytes are allowed
        cut.write_bytes(data + b"\0" * 7)
        t.load_resume_checkpoint(cut, "halfka-hm-merged", "progress8kpabs")
        assert t.step_count == 1
