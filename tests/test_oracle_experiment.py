"""The experiment-log oracle (oracle/experiment.py) pinned independently of
its own formulas.

  - UTC formatting: the reference's known values (experiment.rs:728-739:
    epoch 0, 1_700_000_000 = 2023-11-14T22:13:20Z, compact
    "20231114t221320z"), and civil_from_epoch against Python's own calendar
    (datetime) on leap days, century years and random times;
  - the logger's aggregation, on the reference's own test sequences
    (experiment.rs:751-827): best loss and its superbatch, total positions,
    mean pos/s, dataset passes; a NaN loss recorded as 0.0 and never best;
    held-out metrics, a non-finite test loss dropped; interruption keeping
    status "running"; optional fields left out when absent;
  - planted mistakes (a March-based month off by one, a non-finite loss
    taken as best, an unrounded rate) fail these checks.
CPU only.
"""
import datetime
import math
import random

import pytest

from oracle import experiment as oex


def _doc(**kw):
    args = dict(id="rshogi-20260517t041530z", name="rshogi", start_epoch_secs=1_747_000_000,
                command="nnue-train --data teacher.psv", params={"lr": 0.000875}, data_name="teacher.psv",
                data_positions=800_000_000, fv_scale=16, commit="7beb263")
    args.update(kw)
    return oex.Experiment(**args)


def test_known_utc_values():
    assert oex.civil_from_epoch(0) == (1970, 1, 1, 0, 0, 0)
    assert oex.civil_from_epoch(1_700_000_000) == (2023, 11, 14, 22, 13, 20)
    assert oex.format_utc_iso(0) == "1970-01-01T00:00:00Z"
    assert oex.format_utc_iso(1_700_000_000) == "2023-11-14T22:13:20Z"
    assert oex.format_utc_compact(1_700_000_000) == "20231114t221320z"


def _calendar(epoch):
    d = datetime.datetime(1970, 1, 1, tzinfo=datetime.timezone.utc) + datetime.timedelta(seconds=epoch)
    return d.year, d.month, d.day, d.hour, d.minute, d.second


@pytest.mark.parametrize("date", ["2000-02-29", "2000-03-01", "2100-02-28", "2100-03-01", "2400-02-29",
                                  "1999-12-31", "2024-12-31", "9999-12-31", "2038-01-19"])
def test_civil_from_epoch_against_the_calendar_on_edges(date):
    d = datetime.datetime.fromisoformat(date).replace(tzinfo=datetime.timezone.utc)
    for secs in (0, 1, 86399):
        e = int(d.timestamp()) + secs
        assert oex.civil_from_epoch(e) == _calendar(e)


def test_civil_from_epoch_against_the_calendar_at_random():
    rng = random.Random(7)
    for _ in range(20000):
        e = rng.randrange(0, 253402300800)  # up to 9999-12-31
        assert oex.civil_from_epoch(e) == _calendar(e)


def test_planted_month_offset_fails_the_calendar():
    def wrong(epoch):
        y, mo, d, h, mi, s = oex.civil_from_epoch(epoch)
        return y, (mo % 12) + 1 if mo == 2 else mo, d, h, mi, s  # February mislabelled

    e = int(datetime.datetime(2023, 2, 10, tzinfo=datetime.timezone.utc).timestamp())
    assert wrong(e) != _calendar(e)


def test_record_superbatch_aggregates_like_the_reference_test():
    x = _doc()
    x.record_superbatch(1, 0.04, 1_000_000, 10.0)
    x.record_superbatch(2, 0.03, 1_000_000, 20.0)
    x.record_superbatch(3, 0.035, 1_000_000, 30.0)
    d = x.document()
    assert len(d["history"]) == 3
    assert d["results"]["best_loss"] == 0.03 and d["results"]["best_loss_superbatch"] == 2
    assert d["data"]["total_positions"] == 3_000_000
    assert d["results"]["mean_pos_per_sec"] == 100_000
    assert abs(d["data"]["dataset_passes"] - 0.00375) < 1e-9
    assert d["results"]["training_time_seconds"] == 30


def test_non_finite_loss_is_recorded_as_zero_and_never_best():
    x = _doc()
    x.record_superbatch(1, math.nan, 1_000, 1.0)
    d = x.document()
    assert d["history"][0]["loss"] == 0.0
    assert "best_loss" not in d["results"]
    # a planted mistake: taking the recorded 0.0 as the best loss
    assert not ("best_loss" in d["results"] and d["results"]["best_loss"] == 0.0)


def test_validation_metrics_like_the_reference_test():
    x = _doc()
    x.record_superbatch(1, 0.04, 1_000, 1.0, 0.05, 0.81)
    x.record_superbatch(2, 0.03, 1_000, 2.0, 0.042, 0.84)
    x.record_superbatch(3, 0.02, 1_000, 3.0, math.inf, 0.9)
    d = x.document()
    assert d["history"][0]["test_loss"] == 0.05 and d["history"][0]["test_accuracy"] == 0.81
    assert "test_loss" not in d["history"][2] and d["history"][2]["test_accuracy"] == 0.9
    assert d["results"]["best_test_loss"] == 0.042 and d["results"]["best_test_loss_superbatch"] == 2


def test_validation_metrics_omitted_when_never_recorded():
    x = _doc()
    x.record_superbatch(1, 0.04, 1_000, 1.0)
    d = x.document()
    assert "test_loss" not in d["history"][0] and "test_accuracy" not in d["history"][0]
    assert "best_test_loss" not in d["results"]


def test_mark_interrupted_keeps_running_status():
    x = _doc()
    x.record_superbatch(1, 0.04, 1_000, 1.0)
    x.mark_interrupted()
    d = x.document()
    assert d["status"] == "running" and d["results"]["interrupted"] is True
    x.mark_finished(12.4)
    d = x.document()
    assert d["status"] == "completed" and d["results"]["training_time_seconds"] == 12


def test_optional_fields_omitted_and_order():
    x = _doc(commit=None)
    d = x.document()
    assert "commit" not in d and "lineage" not in d
    assert "target_superbatches" not in d["results"]
    assert list(d) == ["schema_version", "generator", "id", "name", "date", "status", "last_updated_at",
                       "command", "params", "data", "results", "history", "checkpoints"]
    assert d["results"]["fv_scale"] == 16 and d["schema_version"] == 2
    y = _doc(lineage={"parent_id": None, "resumed_from_checkpoint": "net-3.ckpt", "resumed_from_superbatch": 3},
             fv_scale=None)
    e = y.document()
    assert e["lineage"] == {"resumed_from_checkpoint": "net-3.ckpt", "resumed_from_superbatch": 3}
    assert e["results"]["fv_scale"] is None
    y.set_target_superbatches(5)
    assert y.document()["results"]["target_superbatches"] == 5


def test_rate_rounding_half_away_from_zero():
    x = _doc(data_positions=0)
    x.record_superbatch(1, 0.1, 5, 2.0)  # 2.5 pos/s -> 3; elapsed 2.0 -> 2
    d = x.document()
    assert d["results"]["mean_pos_per_sec"] == 3
    assert d["data"]["dataset_passes"] == 0.0
    # a planted mistake: Python's round() (half to even) gives 2
    assert round(5 / 2.0) != d["results"]["mean_pos_per_sec"]
    x.record_superbatch(2, 0.1, 0, 0.0)  # zero elapsed: rate 0
    assert x.document()["results"]["mean_pos_per_sec"] == 0
