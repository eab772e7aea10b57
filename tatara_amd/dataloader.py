"""PSV records -> training batches on the GPU (the dataloader's feature step).

Mirrors the reference dataloader's per-position work
(Batch::push_decoded, crates/nnue-train/src/dataloader.rs:444-497, and
BucketMode::bucket_board, :303-328) over the C ABI's tatara_psv_to_batch: the
host hands over 40-byte PackedSfenValue records and gets a device-resident
batch (index rows, nnz, score, wdl, bucket) that LayerStackTrainer /
SimpleTrainer consume directly.  Feature sets and bucket modes use the
reference's names.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import check
from .trainer import DeviceArray, DeviceBatch

FEATURE_SETS = {"halfkp": 0, "halfka-split": 1, "halfka-merged": 2, "halfka-hm-split": 3,
                "halfka-hm-merged": 4}
BUCKET_MODES = {"none": 0, "kingrank9": 1, "progress8kpabs": 2}
KPABS_WEIGHTS = 81 * 1548


def feature_set_info(name: str) -> dict:
    """FeatureSetSpec dimensions and hash (crates/shogi-features/src/feature_set.rs)."""
    lib = _lib.load()
    kb, pi, fi, ma = (C.c_int32() for _ in range(4))
    h = C.c_uint32()
    check(lib.tatara_feature_set_info(FEATURE_SETS[name], C.byref(kb), C.byref(pi), C.byref(fi),
                                      C.byref(ma), C.byref(h)))
    return dict(king_buckets=kb.value, piece_inputs=pi.value, ft_in=fi.value, max_active=ma.value,
                feature_hash=h.value)


class ProgressWeights:
    """ShogiProgressKPAbs::load_from_bin: 81*1548 f64 values kept as f32 on the device."""

    def __init__(self, values_f64):
        v = np.asarray(values_f64, dtype=np.float64).ravel()
        if v.size != KPABS_WEIGHTS:
            raise ValueError(f"progress.bin size mismatch: got {v.size} values, expected {KPABS_WEIGHTS}")
        self.host = v.astype(np.float32)  # f64 -> f32 rounds to nearest, as `as f32` does
        self.dev = DeviceArray(self.host)

    @classmethod
    def load_from_bin(cls, path) -> "ProgressWeights":
        raw = np.fromfile(path, dtype="<f8")
        return cls(raw)


# feature sets whose friend- and enemy-king planes are one (halfka-*-merged):
# a record with both kings on one square gives that feature twice
MERGED_KING_PLANES = ("halfka-merged", "halfka-hm-merged")


def king_squares(records) -> tuple[np.ndarray, np.ndarray]:
    """The two 7-bit king squares of each record: bits 1..7 and 8..14 of its
    LSB-first bit stream (after the side-to-move bit, packed_sfen.rs:387-430)."""
    rec = np.ascontiguousarray(records, dtype=np.uint8).reshape(-1, 40)
    w = rec[:, 0].astype(np.uint32) | (rec[:, 1].astype(np.uint32) << 8)
    return (w >> 1) & 127, (w >> 8) & 127


def records_king_blocked(records, feature_set: str) -> bool:
    """Whether the decoded rows of these records are king-blocked (every
    feature in its perspective's king block, none twice).  Board, hand and
    king features occupy disjoint ranges of a block and one square holds one
    piece, so only the merged king plane can repeat a feature: when both kings
    are on one square."""
    if feature_set not in MERGED_KING_PLANES:
        return True
    a, b = king_squares(records)
    return not bool(np.any((a == b) & (a < 81)))


def psv_to_device_batch(records, feature_set: str, bucket_mode: str = "none", num_buckets: int = 1,
                        progress: ProgressWeights | None = None) -> DeviceBatch:
    """Decodes [n, 40] uint8 records on the GPU into a DeviceBatch (+ bucket)."""
    rec = np.ascontiguousarray(records, dtype=np.uint8).reshape(-1, 40)
    n = rec.shape[0]
    info = feature_set_info(feature_set)
    ma = info["max_active"]
    if bucket_mode == "progress8kpabs" and progress is None:
        raise ValueError("progress buckets need ProgressWeights")
    src = DeviceArray(rec)
    db = DeviceBatch(n, ma)
    db.arrays = {
        "stm": DeviceArray.empty((n, ma), np.int32),
        "nstm": DeviceArray.empty((n, ma), np.int32),
        "nnz": DeviceArray.empty((n,), np.int32),
        "score": DeviceArray.empty((n,), np.float32),
        "wdl": DeviceArray.empty((n,), np.float32),
        "bucket": DeviceArray.empty((n,), np.int32),
    }
    a = db.arrays
    lib = _lib.load()
    check(lib.tatara_psv_to_batch(src.ptr, n, FEATURE_SETS[feature_set], BUCKET_MODES[bucket_mode],
                                  num_buckets, progress.dev.ptr if progress is not None else None,
                                  a["stm"].ptr, a["nstm"].ptr, a["nnz"].ptr, a["bucket"].ptr,
                                  a["score"].ptr, a["wdl"].ptr))
    src.free()
    db.king_blocked = records_king_blocked(rec, feature_set)
    return db


def device_batch_to_host(db: DeviceBatch) -> dict:
    return {k: v.to_host() for k, v in db.arrays.items()}
