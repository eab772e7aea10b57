"""ctypes binding of the CPU feature oracle (oracle/features.cpp).

TEST INFRASTRUCTURE ONLY: the checker for PSV decoding, feature-index
extraction and bucket assignment; imported by tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg.  The product never uses it.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .ffi import lib

FEATURE_SETS = ("halfkp", "halfka-split", "halfka-merged", "halfka-hm-split", "halfka-hm-merged")
BUCKET_MODES = {"none": 0, "kingrank9": 1, "progress": 2}


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def feature_set_info(fs) -> dict:
    i = FEATURE_SETS.index(fs) if isinstance(fs, str) else int(fs)
    out = np.zeros(4, np.int32)
    rc = lib().orc_feature_set_info(C.c_int(i), out.ctypes.data_as(C.POINTER(C.c_int32)))
    if rc != 0:
        raise ValueError(fs)
    return dict(king_buckets=int(out[0]), piece_inputs=int(out[1]), ft_in=int(out[2]),
                max_active=int(out[3]))


def psv_decode(psv) -> dict:
    """Decoded boards: ptype/color [n, 81], hand [n, 2, 7], stm, kings, score, result, ply."""
    psv = _u8(psv).reshape(-1, 40)
    n = psv.shape[0]
    out = np.zeros((n, 182), np.int32)
    lib().orc_psv_decode(psv.ctypes.data_as(C.c_void_p), C.c_int64(n),
                         out.ctypes.data_as(C.POINTER(C.c_int32)))
    return dict(ptype=out[:, :81], color=out[:, 81:162], hand=out[:, 162:176].reshape(n, 2, 7),
                stm=out[:, 176], bking=out[:, 177], wking=out[:, 178], score=out[:, 179],
                result=out[:, 180], ply=out[:, 181])


def psv_to_batch(psv, fs, bucket_mode="none", num_buckets=1, weights=None) -> dict:
    """Batch::push_decoded for every record (+ bucket); index rows padded with -1."""
    psv = _u8(psv).reshape(-1, 40)
    n = psv.shape[0]
    i = FEATURE_SETS.index(fs) if isinstance(fs, str) else int(fs)
    ma = feature_set_info(i)["max_active"]
    stm = np.zeros((n, ma), np.int32)
    nstm = np.zeros((n, ma), np.int32)
    nnz = np.zeros(n, np.int32)
    bucket = np.zeros(n, np.int32)
    score = np.zeros(n, np.float32)
    wdl = np.zeros(n, np.float32)
    prog = np.zeros(n, np.float32)
    w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
    P = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    rc = lib().orc_psv_to_batch(P(psv), C.c_int64(n), C.c_int(i), C.c_int(BUCKET_MODES[bucket_mode]),
                                C.c_int(num_buckets), P(w) if w is not None else None, P(stm), P(nstm),
                                P(nnz), P(bucket), P(score), P(wdl), P(prog))
    if rc != 0:
        raise ValueError(fs)
    return dict(stm=stm, nstm=nstm, nnz=nnz, bucket=bucket, score=score, wdl=wdl, progress=prog)


def board_rows(ptype, color, hand, stm, score=0, result=0, ply=0) -> np.ndarray:
    """Boards as the 182-value rows of psv_decode (kings read from ptype/color)."""
    ptype = np.atleast_2d(np.asarray(ptype, np.int32))
    color = np.atleast_2d(np.asarray(color, np.int32))
    n = ptype.shape[0]
    hand = np.asarray(hand, np.int32).reshape(n, 2, 7)
    rows = np.zeros((n, 182), np.int32)
    rows[:, :81] = ptype
    rows[:, 81:162] = color
    rows[:, 162:176] = hand.reshape(n, 14)
    rows[:, 176] = np.asarray(stm).reshape(-1)
    for c, col in ((0, 177), (1, 178)):
        m = (ptype == 8) & (color == c)
        rows[:, col] = np.where(m.any(1), m.argmax(1), 81)
    rows[:, 179] = score
    rows[:, 180] = result
    rows[:, 181] = ply
    return rows


def boards_to_batch(rows, fs, bucket_mode="none", num_buckets=1, weights=None) -> dict:
    """Batch::push_decoded over decoded boards (rows from board_rows / psv_decode layout)."""
    rows = np.ascontiguousarray(rows, dtype=np.int32).reshape(-1, 182)
    n = rows.shape[0]
    i = FEATURE_SETS.index(fs) if isinstance(fs, str) else int(fs)
    ma = feature_set_info(i)["max_active"]
    out = dict(stm=np.zeros((n, ma), np.int32), nstm=np.zeros((n, ma), np.int32),
               nnz=np.zeros(n, np.int32), bucket=np.zeros(n, np.int32), score=np.zeros(n, np.float32),
               wdl=np.zeros(n, np.float32), progress=np.zeros(n, np.float32))
    w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
    P = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    rc = lib().orc_boards_to_batch(P(rows), C.c_int64(n), C.c_int(i), C.c_int(BUCKET_MODES[bucket_mode]),
                                   C.c_int(num_buckets), P(w) if w is not None else None, P(out["stm"]),
                                   P(out["nstm"]), P(out["nnz"]), P(out["bucket"]), P(out["score"]),
                                   P(out["wdl"]), P(out["progress"]))
    if rc != 0:
        raise ValueError(fs)
    return out


def expf(x) -> np.ndarray:
    """glibc expf, elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_expf(x.ctypes.data_as(C.c_void_p), y.ctypes.data_as(C.c_void_p), C.c_int64(x.size))
    return y


def kpabs_indices(record) -> np.ndarray:
    rec = _u8(record).reshape(40)
    out = np.zeros(128, np.int32)
    n = lib().orc_kpabs_indices(rec.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.POINTER(C.c_int32)),
                                C.c_int(128))
    return out[:n].copy()
