"""experiment.json from the library (tatara_experiment_*, host code, CPU
only) against the oracle (oracle/experiment.py) and the reference's own
logger tests (crates/nnue-train/src/experiment.rs:606-919).

  - the UTC formatting entry points equal the oracle on known values and
    random times;
  - the written document, parsed, equals the oracle's document after the
    same calls (the reference's test sequences and random ones with
    non-finite losses, held-out metrics, targets, checkpoints, interruption),
    `last_updated_at` apart (the wall clock at the last update);
  - the text is serde_json's pretty layout: two-space indent, fields in
    declaration order, each f64 as the shortest digits that read back
    exactly, in ryu's layouts ("0.04", "1e-7", "100000.0", "1.5e16"); f32
    params with the shortest f32 digits ("0.000875");
  - write() is atomic (temp file renamed; parent directories created; no
    temp file left) and reports a failure;
  - the params builders and schedule descriptions follow the reference's
    sample (experiment.rs:641-708).
The run-level cases (tatara_train_run writing it) are in tests/test_gpu_run.py.
"""
import json
import math
import os
import random
import re

import numpy as np
import pytest

from oracle import experiment as oex
from tatara_amd import experiment as tex
from tatara_amd.run import (ConstantLR, ConstantWDL, LinearDecayLR, LinearWDL, SequenceLR, StepLR, TrainingConfig,
                            WarmupLR)
from tatara_amd.trainer import LayerStackConfig, SimpleConfig, Sigmoid, Wrm

ISO = re.compile(r"^\d{4}-\d{2}-\d{2}T\d{2}:\d{2}:\d{2}Z$")
PARAMS = {"architecture": "LayerStack-1536-16-32-9bucket", "lr": tex.F32(8.75e-4), "batch_size": 65536,
          "loss_kind": "wrm", "tf32": False}


def _pair(tmp_path, **kw):
    args = dict(id="rshogi-20260517t041530z", name="rshogi", start_epoch_secs=1_747_000_000,
                command="nnue-train --data teacher.psv", params=PARAMS, data_name="teacher.psv",
                data_positions=800_000_000, fv_scale=16, commit="7beb263")
    args.update(kw)
    path = tmp_path / "experiments" / f"{args['id']}.json"
    lib = tex.ExperimentLogger(path, args["id"], args["name"], args["params"], args["data_name"],
                               args["data_positions"], command=args["command"], commit=args["commit"],
                               lineage=args.get("lineage"), fv_scale=args["fv_scale"],
                               start_epoch_secs=args["start_epoch_secs"], generator_version="9.9.9")
    ora_params = json.loads(tex.dumps(args["params"]))
    ora = oex.Experiment(args["id"], args["name"], args["start_epoch_secs"], args["command"], ora_params,
                         args["data_name"], args["data_positions"], fv_scale=args["fv_scale"],
                         commit=args["commit"], lineage=args.get("lineage"), generator_version="9.9.9")
    return lib, ora, path


def _compare(lib, ora, path):
    lib.write()
    text = path.read_text()
    got = json.loads(text)
    want = ora.document()
    assert ISO.match(got["last_updated_at"])
    got["last_updated_at"] = want["last_updated_at"] = None
    assert got == want
    assert list(got) == list(want)
    assert list(got["results"]) == list(want["results"])
    return text


@pytest.mark.parametrize("epoch", [0, 1, 86399, 951782400, 1_700_000_000, 4107542399, 253402300799])
def test_utc_formatting_matches_the_oracle(epoch):
    assert tex.format_utc_iso(epoch) == oex.format_utc_iso(epoch)
    assert tex.format_utc_compact(epoch) == oex.format_utc_compact(epoch)


def test_utc_formatting_at_random():
    rng = random.Random(11)
    for _ in range(2000):
        e = rng.randrange(0, 253402300800)
        assert tex.format_utc_iso(e) == oex.format_utc_iso(e)
        assert tex.format_utc_compact(e) == oex.format_utc_compact(e)


def test_new_document_is_running_with_empty_history(tmp_path):
    lib, ora, path = _pair(tmp_path)
    text = _compare(lib, ora, path)
    got = json.loads(text)
    assert got["status"] == "running" and got["schema_version"] == 2 and got["history"] == []
    assert got["date"] == tex.format_utc_iso(1_747_000_000) == got["date"]
    assert got["generator"] == {"name": "tatara", "version": "9.9.9"}


def test_reference_sequence(tmp_path):
    lib, ora, path = _pair(tmp_path)
    for sb, loss, t in ((1, 0.04, 10.0), (2, 0.03, 20.0), (3, 0.035, 30.0)):
        lib.record_superbatch(sb, loss, 1_000_000, t)
        ora.record_superbatch(sb, loss, 1_000_000, t)
    got = json.loads(_compare(lib, ora, path))
    assert got["results"]["best_loss"] == 0.03 and got["results"]["best_loss_superbatch"] == 2
    assert got["results"]["mean_pos_per_sec"] == 100_000 and got["data"]["total_positions"] == 3_000_000


def test_non_finite_loss_and_held_out_metrics(tmp_path, capfd):
    lib, ora, path = _pair(tmp_path)
    seq = [(1, 0.04, 1_000, 1.0, 0.05, 0.81), (2, 0.03, 1_000, 2.0, 0.042, 0.84),
           (3, 0.02, 1_000, 3.0, math.inf, 0.9), (4, math.nan, 1_000, 4.0, None, None),
           (5, -math.inf, 1_000, 5.0, math.nan, None)]
    for s in seq:
        lib.record_superbatch(*s)
        ora.record_superbatch(*s)
    _compare(lib, ora, path)
    err = capfd.readouterr().err
    assert "superbatch 4 loss is non-finite (NaN); recording 0.0 in experiment.json" in err
    assert "superbatch 5 loss is non-finite (-inf)" in err


def test_random_sequences(tmp_path):
    rng = random.Random(5)
    for trial in range(20):
        lineage = None
        if trial % 3 == 1:
            lineage = {"parent_id": None if trial % 2 else "parent-run", "resumed_from_checkpoint": "net-4.ckpt",
                       "resumed_from_superbatch": 4}
        lib, ora, path = _pair(tmp_path / str(trial), lineage=lineage,
                               commit=None if trial % 2 else "abc1234",
                               fv_scale=None if trial % 4 == 3 else rng.randrange(1, 1000),
                               data_positions=rng.choice([0, 1, 123_456_789]))
        for sb in range(1, rng.randrange(1, 12)):
            loss = rng.choice([rng.random() * 0.1, rng.uniform(-1e-30, 1e30), math.nan, 0.0, 1e-300])
            tl = rng.choice([None, rng.random(), math.inf])
            ta = rng.choice([None, rng.random(), math.nan])
            el = rng.choice([rng.uniform(0.0, 1e5), 0.0, -3.0, 2.5, math.nan])
            pos = rng.choice([0, 65536 * 6104, 2 ** 64 - 1])
            lib.record_superbatch(sb, loss, pos, el, tl, ta)
            ora.record_superbatch(sb, loss, pos, el, tl, ta)
            if rng.random() < 0.3:
                for name in (f"net-{sb}.bin", f"net-{sb}.ckpt"):
                    lib.note_checkpoint(name)
                    ora.note_checkpoint(name)
            if rng.random() < 0.2:
                lib.set_target_superbatches(sb + 2)
                ora.set_target_superbatches(sb + 2)
        if trial % 2:
            lib.mark_interrupted()
            ora.mark_interrupted()
        else:
            t = rng.uniform(0, 1e4)
            lib.mark_finished(t)
            ora.mark_finished(t)
        _compare(lib, ora, path)
        lib.close()


def test_text_layout(tmp_path):
    lib, ora, path = _pair(tmp_path, data_positions=1000)
    for sb, loss in enumerate([0.04, 1e-7, 1.5e-7, 100000.0, 1.5e16, 1.2345678901234568e17, 0.00001, 1e-6,
                               0.1 + 0.2, 123.456, 5e-324], start=1):
        lib.record_superbatch(sb, loss, 10, 1.0)
    lib.note_checkpoint("net-1.bin")
    lib.write()
    text = path.read_text()
    assert text.endswith("}\n")
    losses = re.findall(r'"loss": ([^,\n]+)', text)
    assert losses == ["0.04", "1e-7", "1.5e-7", "100000.0", "1.5e16", "1.2345678901234568e17", "0.00001", "1e-6",
                      "0.30000000000000004", "123.456", "5e-324"]
    for s in losses:  # the same text as the host mirror's formatter, and exact
        assert tex.json_float(float(s)) == s
    assert '"lr": 0.000875,' in text  # the f32 param, shortest f32 digits
    assert '\n  "params": {\n    "architecture": "LayerStack-1536-16-32-9bucket",\n' in text
    assert '\n  "history": [\n    {\n      "superbatch": 1,\n      "loss": 0.04\n    },\n' in text
    assert '\n  "checkpoints": [\n    "net-1.bin"\n  ]\n}\n' in text
    assert '"fv_scale": 16,' in text


def test_float_formatting_round_trips():
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(2000) * 10.0 ** rng.integers(-300, 300, 2000),
                           rng.random(500), [1.0, 0.5, 1e16, 1e17, 9.999999999999999e15, 2.0 ** -1074]])
    for v in vals:
        s = tex.json_float(float(v))
        assert float(s) == float(v), s
        with np.errstate(over="ignore"):
            v32 = np.float32(v)
        if np.isfinite(v32) and v32 != 0:
            f = tex.json_float(float(v32), f32=True)
            assert np.float32(float(f)) == v32, f


def test_write_is_atomic_and_reports_failure(tmp_path):
    lib, ora, path = _pair(tmp_path / "a" / "b")
    lib.write()
    assert path.is_file() and not os.path.exists(str(path) + ".tmp")
    json.loads(path.read_text())
    lib.record_superbatch(1, 0.5, 1, 1.0)
    lib.write()  # rewritten whole, still valid
    assert json.loads(path.read_text())["history"][0]["loss"] == 0.5
    blocker = tmp_path / "file"
    blocker.write_text("x")
    bad = tex.ExperimentLogger(blocker / "sub" / "x.json", "i", "n", {}, "d", 0, command="c",
                               start_epoch_secs=0)
    with pytest.raises(tex._lib.TataraError, match="io error: experiment.json"):
        bad.write()


def test_create_rejects_a_params_value_that_is_not_an_object(tmp_path):
    from tatara_amd._lib import TataraExperimentInit

    init = TataraExperimentInit(path=b"x.json", id=b"i", name=b"n", command=b"c", params_json=b"[1, 2]",
                                data_name=b"d")
    import ctypes as C

    h = C.c_void_p()
    assert tex._lib.load().tatara_experiment_create(C.byref(init), C.byref(h)) != 0


def test_schedule_descriptions_and_params_builders():
    # experiment.rs:641-708's sample: lr 8.75e-4, gamma 0.995, step 1
    assert str(StepLR(8.75e-4, 0.995, 1)) == "start 0.000875 gamma 0.995 drop every 1 superbatches"
    assert str(ConstantWDL(0.0)) == "constant 0" and str(LinearWDL(0.0, 0.75)) == "linear taper start 0 end 0.75"
    lr = WarmupLR(SequenceLR(ConstantLR(1e-3), LinearDecayLR(1e-3, 1e-5, 100), 10), 50)
    assert str(lr) == ("constant 0.001, then after 10 superbatches, start at 0.001 and linearly decay to "
                       "0.00001 at superbatch 100, warmup over 50 batches")
    cfg = LayerStackConfig(ft_in=73305, max_active=40, piece_inputs=1629, num_buckets=9)
    run_cfg = TrainingConfig(net_id="rshogi", feature_set="halfka-hm-merged", output_dir="/tmp/x",
                             end_superbatch=400, batches_per_superbatch=6104, batch_size=65536,
                             bucket_mode="progress8kpabs", num_buckets=9)
    p = tex.layerstack_params(cfg.all_optim(), run_cfg, Wrm(), StepLR(8.75e-4, 0.995, 1), ConstantWDL(0.0),
                              ft_in=73305, progress_coeff="/data/progress.bin", threads=16)
    q = json.loads(tex.dumps(p))
    assert q["architecture"] == "LayerStack-1536-16-32-9bucket" and q["ft_factorize"] is True
    assert q["lr"] == 0.000875 and q["lr_gamma"] == 0.995 and q["lr_step"] == 1
    assert q["lr_schedule"] == "start 0.000875 gamma 0.995 drop every 1 superbatches"
    assert (q["qa"], q["qb"], q["scale"], q["loss_kind"]) == (127, 64, 600.0, "wrm")
    assert q["wrm_in_scaling"] == 340.0 and q["wrm_weight_boost_w2"] == 0.5
    assert q["tf32"] and q["ft_fp16"] and q["ft_fp16_out"] and q["fp16_opt_state"]
    assert q["progress_coeff"] == "progress.bin" and q["bucket_mode"] == "progress8kpabs"
    assert "ft_weight_decay" not in q and q["weight_decay"] == pytest.approx(0.01)
    keys = list(q)
    assert keys.index("lr_schedule") < keys.index("batch_size") < keys.index("scale") < keys.index("qa")
    s = tex.simple_params(SimpleConfig(ft_in=125388, max_active=38), TrainingConfig(
        net_id="s", feature_set="halfkp", output_dir="/tmp/x"), Sigmoid(1.0 / 290.0), ConstantLR(1e-3),
        ConstantWDL(0.0), ft_in=125388)
    s = json.loads(tex.dumps(s))
    assert s["architecture"] == "simple-halfkp-256x2-32-32-crelu" and s["activation"] == "crelu"
    assert s["loss_kind"] == "sigmoid" and "wrm_in_scaling" not in s and s["scale"] == 290.0
    assert "num_buckets" not in s and "bucket_mode" not in s and "ft_factorize" not in s
