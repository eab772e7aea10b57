"""Superbatch driver (tatara_train_run) on the GPU.

Pins: the driver equals a hand-written loop over the same PSV batches
(GPU decode + train_step with the oracle schedule's lr / wdl, lagged loss
summed per superbatch and flushed at its end) bit for bit, in weights and
loss sums; the lr / wdl values it used equal the oracle schedule's; the
checkpoint cadence, names and resume headers, the start-superbatch offset
(crates/nnue-train/src/trainer.rs run_with_start_superbatch_offset test:
start 3, end 5, save_rate 2 saves 4 and 5 only) and the pruning of old
resume checkpoints follow trainer.rs:759-1283; bad data files and configs
are rejected before any step.
"""
import json

import numpy as np
import pytest

import oracle.schedule as osch
from tatara_amd import run as R
from tatara_amd._lib import TataraError
from tatara_amd.dataloader import feature_set_info, psv_to_device_batch
from tatara_amd.psv import synthetic_psv
from tatara_amd.trainer import (LayerStackConfig, LayerStackTrainer, SimpleConfig, SimpleTrainer, Sigmoid,
                                Wrm)

pytestmark = pytest.mark.gpu

B = 256


def simple_cfg():
    info = feature_set_info("halfkp")
    return SimpleConfig(ft_in=info["ft_in"], max_active=info["max_active"], ft_out=32, l1_out=32, l2_out=32,
                        max_batch=B, optimizer="adamw")


def write_psv(tmp_path, n, seed=7):
    path = tmp_path / "data.psv"
    recs = synthetic_psv(n, seed)
    recs.tofile(path)
    return path, recs


def manual(trainer, recs, start, end, bps, lr_o, wdl_o, loss, feature_set="halfkp", bucket_mode="none", nb=1):
    """The driver's loop written out with the Python API."""
    n = recs.shape[0]
    cursor = 0
    sums = []
    for sb in range(start, end + 1):
        s = 0.0
        for b in range(bps):
            idx = (cursor + np.arange(B)) % n
            cursor = (cursor + B) % n
            db = psv_to_device_batch(recs[idx], feature_set, bucket_mode, nb)
            lr = float(lr_o.lr(b, sb))
            wdl = float(wdl_o.blend(b, sb, end))
            if isinstance(trainer, SimpleTrainer):
                s += trainer.train_step(db, lr=lr, wdl_lambda=wdl, loss=loss)
            else:
                s += trainer.train_step(db, None, lr=lr, wdl_lambda=wdl, loss=loss)
        s += trainer.flush_pending_loss()
        sums.append(s)
    return sums


def test_run_equals_manual_loop_and_checkpoints(gpu, tmp_path):
    path, recs = write_psv(tmp_path, 3 * B + 40)  # the file ends mid-batch: reading starts over
    cfg = R.TrainingConfig(net_id="net", feature_set="halfkp", output_dir=str(tmp_path / "out"),
                           start_superbatch=1, end_superbatch=3, batches_per_superbatch=2, batch_size=B,
                           save_rate=2, fv_scale=16, print_progress=True)
    lr_p, wdl_p = R.StepLR(1e-3, 0.5, 1), R.LinearWDL(0.0, 1.0)
    lr_o, wdl_o = osch.StepLR(1e-3, 0.5, 1), osch.LinearWDL(0.0, 1.0)
    loss = Wrm()
    with SimpleTrainer(simple_cfg()) as t1, SimpleTrainer(simple_cfg()) as t2:
        res = R.run(t1, path, lr_p, wdl_p, cfg, loss)
        sums = manual(t2, recs, 1, 3, 2, lr_o, wdl_o, loss)
        assert [r["superbatch"] for r in res.superbatches] == [1, 2, 3]
        assert [r["positions"] for r in res.superbatches] == [2 * B] * 3
        assert [r["saved"] for r in res.superbatches] == [False, True, True]
        assert [r["loss_sum"] for r in res.superbatches] == sums
        for r in res.superbatches:
            assert r["mean_loss"] == r["loss_sum"] / r["positions"]
        exp_lr = [np.float32(lr_o.lr(b, sb)) for sb in (1, 2, 3) for b in (0, 1)]
        exp_wdl = [np.float32(wdl_o.blend(b, sb, 3)) for sb in (1, 2, 3) for b in (0, 1)]
        assert res.lr_seen.tobytes() == np.array(exp_lr, np.float32).tobytes()
        assert res.wdl_seen.tobytes() == np.array(exp_wdl, np.float32).tobytes()
        assert t1.step_count == t2.step_count == 6
        for g in t1.GROUPS:
            for k in ("w", "m", "v"):
                assert np.array_equal(t1.get(g, k), t2.get(g, k)), (g, k)
        out = tmp_path / "out"
        names = sorted(p.name for p in out.iterdir())
        assert names == ["net-2.bin", "net-2.ckpt", "net-3.bin", "net-3.ckpt"]
        # the last checkpoints hold the final state
        t2.save_quantised(str(tmp_path / "manual.bin"), "halfkp", 16)
        assert (out / "net-3.bin").read_bytes() == (tmp_path / "manual.bin").read_bytes()
    with SimpleTrainer(simple_cfg()) as t3:
        sb, run_id, horizon = t3.load_resume_checkpoint(str(out / "net-3.ckpt"), "halfkp", None)
        assert (sb, run_id, horizon) == (3, None, None)
        assert t3.step_count == 6


def test_start_superbatch_offset_saves_only_from_offset(gpu, tmp_path):
    path, _ = write_psv(tmp_path, 2 * B)
    cfg = R.TrainingConfig(net_id="offset", feature_set="halfkp", output_dir=str(tmp_path / "out"),
                           start_superbatch=3, end_superbatch=5, batches_per_superbatch=1, batch_size=B,
                           save_rate=2, run_id="run-a", fv_scale=16,
                           print_progress=False)
    lr = R.CosineDecayLR(2e-3, 1e-5, 5)
    with SimpleTrainer(simple_cfg()) as t:
        res = R.run(t, path, lr, R.ConstantWDL(0.25), cfg, Wrm())
        assert [r["superbatch"] for r in res.superbatches] == [3, 4, 5]
        assert [r["saved"] for r in res.superbatches] == [False, True, True]
        o = osch.CosineDecayLR(2e-3, 1e-5, 5)
        assert res.lr_seen.tolist() == [float(o.lr(0, sb)) for sb in (3, 4, 5)]
        assert [r["lr"] for r in res.superbatches] == res.lr_seen.tolist()
        assert set(res.wdl_seen.tolist()) == {0.25}
        names = sorted(p.name for p in (tmp_path / "out").iterdir())
        assert names == ["offset-4.bin", "offset-4.ckpt", "offset-5.bin", "offset-5.ckpt"]
    with SimpleTrainer(simple_cfg()) as t:
        sb, run_id, horizon = t.load_resume_checkpoint(str(tmp_path / "out" / "offset-4.ckpt"), "halfkp", None)
        assert (sb, run_id, horizon) == (4, "run-a", 5)


def test_keep_raw_checkpoints_prunes_oldest(gpu, tmp_path):
    path, _ = write_psv(tmp_path, B)
    out = tmp_path / "out"
    out.mkdir()
    (out / "keep-9.ckpt.tmp").write_bytes(b"x")  # not a resume checkpoint name: untouched
    (out / "other-1.ckpt").write_bytes(b"x")  # another net id: untouched
    cfg = R.TrainingConfig(net_id="keep", feature_set="halfkp", output_dir=str(out), start_superbatch=1,
                           end_superbatch=4, batches_per_superbatch=1, batch_size=B, save_rate=1,
                           keep_raw_checkpoints=2, fv_scale=16, print_progress=False)
    with SimpleTrainer(simple_cfg()) as t:
        R.run(t, path, R.ConstantLR(1e-3), R.ConstantWDL(0.0), cfg, Wrm())
    names = sorted(p.name for p in out.iterdir())
    assert names == ["keep-1.bin", "keep-2.bin", "keep-3.bin", "keep-3.ckpt", "keep-4.bin", "keep-4.ckpt",
                     "keep-9.ckpt.tmp", "other-1.ckpt"]


def test_layerstack_kingrank9_run_equals_manual_loop(gpu, tmp_path):
    info = feature_set_info("halfka-hm-merged")
    lcfg = LayerStackConfig(ft_in=info["ft_in"], max_active=info["max_active"], ft_out=128, l1_out=16,
                            l2_out=32, num_buckets=9, max_batch=B, optimizer="ranger")
    path, recs = write_psv(tmp_path, 2 * B, seed=11)
    cfg = R.TrainingConfig(net_id="ls", feature_set="halfka-hm-merged", output_dir=str(tmp_path / "out"),
                           start_superbatch=1, end_superbatch=2, batches_per_superbatch=3, batch_size=B,
                           save_rate=100, bucket_mode="kingrank9", num_buckets=9, print_progress=False)
    lr_p = R.WarmupLR(R.OneCycleLR(3e-3, 0.5, 25.0, 1e4, 2), 2)
    lr_o = osch.WarmupLR(osch.OneCycleLR(3e-3, 0.5, 25.0, 1e4, 2), 2)
    loss = Sigmoid()
    with LayerStackTrainer(lcfg) as t1, LayerStackTrainer(lcfg) as t2:
        res = R.run(t1, path, lr_p, R.ConstantWDL(0.3), cfg, loss)
        sums = manual(t2, recs, 1, 2, 3, lr_o, osch.ConstantWDL(0.3), loss, "halfka-hm-merged", "kingrank9", 9)
        assert [r["loss_sum"] for r in res.superbatches] == sums
        for g in t1.GROUPS:
            assert np.array_equal(t1.get(g), t2.get(g)), g
        assert sorted(p.name for p in (tmp_path / "out").iterdir()) == ["ls-2.bin", "ls-2.ckpt"]
    with LayerStackTrainer(lcfg) as t3:
        sb, _, horizon = t3.load_resume_checkpoint(str(tmp_path / "out" / "ls-2.ckpt"), "halfka-hm-merged",
                                                   "kingrank9")
        assert (sb, horizon) == (2, 2)


def test_rejects_bad_data_and_config(gpu, tmp_path):
    bad = tmp_path / "bad.psv"
    bad.write_bytes(b"\0" * 41)
    empty = tmp_path / "empty.psv"
    empty.write_bytes(b"")
    good, _ = write_psv(tmp_path, B)
    base = dict(net_id="x", feature_set="halfkp", output_dir=str(tmp_path / "out"), batch_size=B,
                fv_scale=16, print_progress=False)
    with SimpleTrainer(simple_cfg()) as t:
        for path, extra, msg in [(bad, {}, "multiple of the PSV record size"),
                                 (empty, {}, "no PSV records"),
                                 (tmp_path / "missing.psv", {}, "cannot open"),
                                 (good, {"start_superbatch": 0}, "start_superbatch"),
                                 (good, {"start_superbatch": 3, "end_superbatch": 2}, "end_superbatch"),
                                 (good, {"save_rate": 0}, "save_rate")]:
            cfg = R.TrainingConfig(**base, **extra)
            with pytest.raises(TataraError, match=msg):
                R.run(t, path, R.ConstantLR(1e-3), R.ConstantWDL(0.0), cfg, Wrm())
        assert t.step_count == 0


def control_run(tmp_path, name, control, start, end, save_rate, lr, wdl, bps=2):
    """One run with <output_dir>/control.json holding `control` (None: no file)."""
    path, _ = write_psv(tmp_path, 2 * B)
    out = tmp_path / name
    out.mkdir()
    if control is not None:
        (out / "control.json").write_text(control)
    cfg = R.TrainingConfig(net_id="test", feature_set="halfkp", output_dir=str(out), start_superbatch=start,
                           end_superbatch=end, batches_per_superbatch=bps, batch_size=B, save_rate=save_rate,
                           fv_scale=16, print_progress=False)
    with SimpleTrainer(simple_cfg()) as t:
        res = R.run(t, path, lr, wdl, cfg, Wrm())
        steps = t.step_count
    return res, out, steps


def test_control_stops_after_current_superbatch(gpu, tmp_path):
    # trainer.rs:1805 control_stops_after_current_superbatch_and_records_completion
    res, out, steps = control_run(tmp_path, "stop", '{"target_superbatches": 1}', 1, 3, 10,
                                  R.StepLR(1e-3, 0.9, 1), R.ConstantWDL(0.0))
    assert steps == 2
    assert [(r["superbatch"], r["saved"]) for r in res.superbatches] == [(1, True)]
    assert sorted(p.name for p in out.iterdir()) == ["control.json", "control_history.jsonl", "test-1.bin",
                                                     "test-1.ckpt"]
    records = [json.loads(s) for s in (out / "control_history.jsonl").read_text().splitlines()]
    assert len(records) == 1
    assert (records[0]["type"], records[0]["target_superbatches"], records[0]["superbatch"]) == ("control", 1, 1)
    assert records[0]["timestamp"].endswith("Z")


@pytest.mark.parametrize("target,ran,saved", [(2, [3, 4, 5], "test-5"), (4, [3, 4], "test-4")])
def test_control_on_a_resumed_run(gpu, tmp_path, target, ran, saved):
    # trainer.rs:1914 stale_control_before_resume_start_is_ignored,
    # trainer.rs:1960 valid_control_after_resume_start_stops_at_target
    res, out, steps = control_run(tmp_path, "resume", json.dumps({"target_superbatches": target}), 3, 5, 10,
                                  R.StepLR(1e-3, 0.9, 1), R.ConstantWDL(0.0))
    assert [r["superbatch"] for r in res.superbatches] == ran
    assert steps == 2 * len(ran)
    assert sorted(p.name for p in out.iterdir() if p.suffix in (".bin", ".ckpt")) == [saved + ".bin",
                                                                                     saved + ".ckpt"]
    hist = out / "control_history.jsonl"
    assert hist.exists() == (target == 4)
    if target == 4:
        assert len(hist.read_text().splitlines()) == 1


@pytest.mark.parametrize("control", [None, "{ not json", '{"target_superbatches": 3}',
                                     '{"target_superbatches": 99}'])
def test_ignored_control_runs_to_the_configured_end(gpu, tmp_path, control):
    # trainer.rs:2010 missing_unreadable_and_malformed_control_do_not_stop_training,
    # trainer.rs:2054 control_target_at_or_above_configured_end_is_noop
    res, out, steps = control_run(tmp_path, "noop", control, 1, 3, 10, R.ConstantLR(1e-3), R.ConstantWDL(0.0))
    assert [r["superbatch"] for r in res.superbatches] == [1, 2, 3] and steps == 6
    assert not (out / "control_history.jsonl").exists()


def test_control_keeps_the_schedule_horizon(gpu, tmp_path):
    # trainer.rs:2134 control_keeps_original_lr_and_wdl_schedule_horizon
    lr, wdl = R.LinearDecayLR(1e-3, 1e-4, 4), R.LinearWDL(0.1, 0.9)
    base, _, _ = control_run(tmp_path, "base", None, 1, 4, 10, lr, wdl)
    ctl, out, steps = control_run(tmp_path, "ctl", '{"target_superbatches": 2, "unknown_field": true}', 1, 4, 10,
                                  lr, wdl)
    assert [r["superbatch"] for r in ctl.superbatches] == [1, 2] and steps == 4
    assert ctl.lr_seen[:4].tobytes() == base.lr_seen[:4].tobytes()
    assert ctl.wdl_seen[:4].tobytes() == base.wdl_seen[:4].tobytes()
    assert [r["loss_sum"] for r in ctl.superbatches] == [r["loss_sum"] for r in base.superbatches[:2]]


def _logger(out, run_id, data_path, cfg, lr, wdl, loss):
    from tatara_amd import experiment as X

    info = feature_set_info("halfkp")
    params = X.simple_params(simple_cfg(), cfg, loss, lr, wdl, ft_in=info["ft_in"])
    return X.ExperimentLogger.for_data(out / "experiments" / f"{run_id}.json", run_id, cfg.net_id, params,
                                       data_path, command="pytest", start_epoch_secs=1_700_000_000,
                                       fv_scale=cfg.fv_scale)


def test_run_writes_experiment_json(gpu, tmp_path):
    # trainer.rs:1746 run_writes_experiment_json: start 1, end 3, save_rate 2
    import oracle.experiment as oex

    path, recs = write_psv(tmp_path, 3 * B + 40)
    out = tmp_path / "out"
    lr, wdl, loss = R.StepLR(1e-3, 0.9, 1), R.ConstantWDL(0.0), Wrm()
    cfg = R.TrainingConfig(net_id="net", feature_set="halfkp", output_dir=str(out), start_superbatch=1,
                           end_superbatch=3, batches_per_superbatch=2, batch_size=B, save_rate=2, fv_scale=16,
                           print_progress=False, run_id="ignored-when-logged")
    log = _logger(out, "exp-test", path, cfg, lr, wdl, loss)
    cfg.experiment = log
    with SimpleTrainer(simple_cfg()) as t:
        res = R.run(t, path, lr, wdl, cfg, loss)
    doc = json.loads((out / "experiments" / "exp-test.json").read_text())
    assert doc["status"] == "completed" and doc["results"]["interrupted"] is False
    assert len(doc["history"]) == 3
    assert doc["checkpoints"] == ["net-2.bin", "net-2.ckpt", "net-3.bin", "net-3.ckpt"]
    # the oracle document after the same calls, the wall-clock fields apart
    ora = oex.Experiment("exp-test", "net", 1_700_000_000, "pytest", doc["params"], "data.psv", 3 * B + 40,
                         fv_scale=16, generator_version=doc["generator"]["version"])
    for r in res.superbatches:
        ora.record_superbatch(r["superbatch"], r["mean_loss"], r["positions"], 1.0)
        if r["saved"]:
            for ext in ("bin", "ckpt"):
                ora.note_checkpoint(f"net-{r['superbatch']}.{ext}")
    ora.mark_finished(1.0)
    want = ora.document()
    for d in (doc, want):
        d["last_updated_at"] = None
        d["results"]["training_time_seconds"] = d["results"]["mean_pos_per_sec"] = None
    assert doc == want
    assert doc["params"]["lr_schedule"] == "start 0.001 gamma 0.9 drop every 1 superbatches"
    # resume checkpoints carry the experiment's id as the producer run id
    with SimpleTrainer(simple_cfg()) as t3:
        for sb in (2, 3):
            got_sb, run_id, _ = t3.load_resume_checkpoint(str(out / f"net-{sb}.ckpt"), "halfkp", None)
            assert (got_sb, run_id) == (sb, "exp-test")
    log.close()


def test_control_stop_records_target_in_experiment_json(gpu, tmp_path):
    # trainer.rs:1805 control_stops_after_current_superbatch_and_records_completion
    path, _ = write_psv(tmp_path, 2 * B)
    out = tmp_path / "stop"
    out.mkdir()
    (out / "control.json").write_text('{"target_superbatches": 1}')
    lr, wdl, loss = R.StepLR(1e-3, 0.9, 1), R.ConstantWDL(0.0), Wrm()
    cfg = R.TrainingConfig(net_id="test", feature_set="halfkp", output_dir=str(out), start_superbatch=1,
                           end_superbatch=3, batches_per_superbatch=2, batch_size=B, save_rate=10, fv_scale=16,
                           print_progress=False)
    log = _logger(out, "control-stop", path, cfg, lr, wdl, loss)
    cfg.experiment = log
    with SimpleTrainer(simple_cfg()) as t:
        R.run(t, path, lr, wdl, cfg, loss)
    doc = json.loads((out / "experiments" / "control-stop.json").read_text())
    assert doc["status"] == "completed"
    assert doc["results"]["target_superbatches"] == 1
    assert len(doc["history"]) == 1
    assert doc["checkpoints"] == ["test-1.bin", "test-1.ckpt"]
    log.close()


def test_failed_run_marks_experiment_interrupted(gpu, tmp_path):
    # training.rs:912-923: an error leaves status "running" with interrupted set
    bad = tmp_path / "bad.psv"
    bad.write_bytes(b"\x00" * 39)  # not a whole record
    out = tmp_path / "out"
    lr, wdl, loss = R.ConstantLR(1e-3), R.ConstantWDL(0.0), Wrm()
    cfg = R.TrainingConfig(net_id="net", feature_set="halfkp", output_dir=str(out), start_superbatch=1,
                           end_superbatch=2, batches_per_superbatch=1, batch_size=B, print_progress=False)
    log = _logger(out, "failed", bad, cfg, lr, wdl, loss)
    cfg.experiment = log
    with SimpleTrainer(simple_cfg()) as t, pytest.raises(TataraError):
        R.run(t, bad, lr, wdl, cfg, loss)
    doc = json.loads((out / "experiments" / "failed.json").read_text())
    assert doc["status"] == "running" and doc["results"]["interrupted"] is True
    assert doc["history"] == []
    log.close()
