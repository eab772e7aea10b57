"""CPU restatement of the structured run log (experiment.json).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the
library's experiment log (tatara_experiment_* and the run driver's use of
it); nothing in the product imports it.

Follows crates/nnue-train/src/experiment.rs: the document and its field
order (:47-292, ExperimentDoc::new :293-340), ExperimentLogger's updates
(set_target_superbatches :392-396, record_superbatch :398-487,
note_checkpoint :489-492, mark_finished :494-499, mark_interrupted
:501-507) and the UTC formatting (format_utc_iso :562-567,
format_utc_compact :569-576, civil_from_epoch :578-603).  The document is a
Python dict in serialisation order, optional fields left out when absent;
`last_updated_at` is the wall clock at each update and is left to the
caller to compare.  Rust's f64::round (half away from zero) and
`as u64` (saturating) are restated as such.
"""
from __future__ import annotations

import math

SCHEMA_VERSION = 2


def civil_from_epoch(epoch_secs: int) -> tuple[int, int, int, int, int, int]:
    """(year, month, day, hour, minute, second) UTC of a UNIX time in seconds.

    The date is Howard Hinnant's published civil_from_days algorithm
    ("chrono-Compatible Low-Level Date Algorithms"; the reference names it at
    crates/nnue-train/src/experiment.rs:577): 400-year eras from 0000-03-01,
    the year of the era, the day of a March-based year, and the month from the
    153-day five-month pattern."""
    days, rem = divmod(epoch_secs, 86400)
    hour, minute, second = rem // 3600, rem % 3600 // 60, rem % 60
    z = days + 719468
    era = (z if z >= 0 else z - 146096) // 146097
    doe = z - era * 146097
    yoe = (doe - doe // 1460 + doe // 36524 - doe // 146096) // 365
    year = yoe + era * 400
    doy = doe - (365 * yoe + yoe // 4 - yoe // 100)
    mp = (5 * doy + 2) // 153
    day = doy - (153 * mp + 2) // 5 + 1
    month = mp + 3 if mp < 10 else mp - 9
    return (year + 1 if month <= 2 else year), month, day, hour, minute, second


def format_utc_iso(epoch_secs: int) -> str:
    y, mo, d, h, mi, s = civil_from_epoch(epoch_secs)
    return f"{y:04}-{mo:02}-{d:02}T{h:02}:{mi:02}:{s:02}Z"


def format_utc_compact(epoch_secs: int) -> str:
    y, mo, d, h, mi, s = civil_from_epoch(epoch_secs)
    return f"{y:04}{mo:02}{d:02}t{h:02}{mi:02}{s:02}z"


def _round_half_away(x: float) -> float:
    return math.floor(x + 0.5) if x >= 0 else -math.floor(-x + 0.5)


def _as_u64(x: float) -> int:
    if x != x or x <= 0:
        return 0
    return min(int(x), 2 ** 64 - 1)


class Experiment:
    """ExperimentLogger's document, updated as the logger updates it."""

    def __init__(self, id, name, start_epoch_secs, command, params, data_name, data_positions, fv_scale=None,
                 commit=None, lineage=None, generator_version=""):
        self.doc = {
            "schema_version": SCHEMA_VERSION,
            "generator": {"name": "tatara", "version": generator_version},
            "id": id,
            "name": name,
            "date": format_utc_iso(start_epoch_secs),
            "status": "running",
            "last_updated_at": format_utc_iso(start_epoch_secs),
        }
        if commit is not None:
            self.doc["commit"] = commit
        self.doc["command"] = command
        if lineage is not None:
            lin = {}
            if lineage.get("parent_id") is not None:
                lin["parent_id"] = lineage["parent_id"]
            lin["resumed_from_checkpoint"] = lineage["resumed_from_checkpoint"]
            lin["resumed_from_superbatch"] = lineage["resumed_from_superbatch"]
            self.doc["lineage"] = lin
        self.doc["params"] = params
        self.doc["data"] = {"name": data_name, "positions": data_positions, "total_positions": 0,
                            "dataset_passes": 0.0}
        self._results = {"training_time_seconds": 0, "fv_scale": fv_scale, "target_superbatches": None,
                         "best_loss": None, "best_loss_superbatch": None, "best_test_loss": None,
                         "best_test_loss_superbatch": None, "mean_pos_per_sec": 0, "interrupted": False}
        self.doc["results"] = None
        self.doc["history"] = []
        self.doc["checkpoints"] = []
        self.positions_trained = 0
        self.warnings = []

    def set_target_superbatches(self, target: int):
        self._results["target_superbatches"] = target

    def record_superbatch(self, superbatch, mean_loss, sb_positions, elapsed_seconds, test_loss=None,
                          test_accuracy=None):
        self.positions_trained = min(self.positions_trained + sb_positions, 2 ** 64 - 1)
        finite = math.isfinite(mean_loss)
        if not finite:
            self.warnings.append(superbatch)
        if test_loss is not None and not math.isfinite(test_loss):
            test_loss = None
        if test_accuracy is not None and not math.isfinite(test_accuracy):
            test_accuracy = None
        entry = {"superbatch": superbatch, "loss": mean_loss if finite else 0.0}
        if test_loss is not None:
            entry["test_loss"] = test_loss
        if test_accuracy is not None:
            entry["test_accuracy"] = test_accuracy
        self.doc["history"].append(entry)
        r = self._results
        if finite and (r["best_loss"] is None or mean_loss < r["best_loss"]):
            r["best_loss"], r["best_loss_superbatch"] = mean_loss, superbatch
        if test_loss is not None and (r["best_test_loss"] is None or test_loss < r["best_test_loss"]):
            r["best_test_loss"], r["best_test_loss_superbatch"] = test_loss, superbatch
        elapsed = elapsed_seconds if elapsed_seconds > 0.0 else 0.0  # f64::max(x, 0.0), NaN -> 0.0
        r["training_time_seconds"] = _as_u64(_round_half_away(elapsed))
        r["mean_pos_per_sec"] = _as_u64(_round_half_away(self.positions_trained / elapsed)) if elapsed > 0 else 0
        d = self.doc["data"]
        d["total_positions"] = self.positions_trained
        d["dataset_passes"] = self.positions_trained / d["positions"] if d["positions"] > 0 else 0.0

    def note_checkpoint(self, file_name: str):
        self.doc["checkpoints"].append(file_name)

    def mark_finished(self, elapsed_seconds: float):
        self.doc["status"] = "completed"
        e = elapsed_seconds if elapsed_seconds > 0.0 else 0.0
        self._results["training_time_seconds"] = _as_u64(_round_half_away(e))

    def mark_interrupted(self):
        self._results["interrupted"] = True

    def document(self) -> dict:
        """The document as serialised: optional results fields only when set."""
        r = self._results
        res = {"training_time_seconds": r["training_time_seconds"], "fv_scale": r["fv_scale"]}
        for k in ("target_superbatches", "best_loss", "best_loss_superbatch", "best_test_loss",
                  "best_test_loss_superbatch"):
            if r[k] is not None:
                res[k] = r[k]
        res["mean_pos_per_sec"] = r["mean_pos_per_sec"]
        res["interrupted"] = r["interrupted"]
        out = dict(self.doc)
        out["results"] = res
        out["history"] = [dict(h) for h in self.doc["history"]]
        out["checkpoints"] = list(self.doc["checkpoints"])
        return out
