"""Seeded synthetic training batches at the index level.

`structured_batch` produces index rows with the structure of a king-bucketed
feature set (HalfKA_hm / HalfKP): every active index of a position's
perspective lies in that perspective's king block
(king_bucket * piece_inputs + packed piece), pieces are distinct within a
perspective, and the last slots carry the king features.  It is the
index-level analogue of BatchData::smoke_dummy
(bins/nnue_train/src/trainer_common.rs:185-221), which draws indices
uniformly and therefore has none of the locality of real batches.
Scores ~ N(0, 600) clipped to +-3000, results uniform over {0, 0.5, 1}
(the BASELINE synthetic label distribution).
"""
from __future__ import annotations

import numpy as np

from .trainer import Batch

# feature-set shapes (crates/shogi-features/src/feature_set.rs:103-185)
# piece_lo/piece_hi bound the packed non-king pieces; king_lo the merged king
# plane (None: the feature set has no king feature)
HALFKA_HM_MERGED = dict(ft_in=45 * 1629, piece_inputs=1629, max_active=40, king_buckets=45,
                        piece_lo=1, piece_hi=1548, king_lo=1548)
HALFKP = dict(ft_in=81 * 1548, piece_inputs=1548, max_active=38, king_buckets=81,
              piece_lo=1, piece_hi=1548, king_lo=None)


def small_spec(king_buckets: int = 10, piece_inputs: int = 64, max_active: int = 40) -> dict:
    """A reduced feature-set shape with the same structure (for parity tests)."""
    return dict(ft_in=king_buckets * piece_inputs, piece_inputs=piece_inputs,
                max_active=max_active, king_buckets=king_buckets, piece_lo=0,
                piece_hi=piece_inputs - 2, king_lo=piece_inputs - 2)


def _distinct_rows(rng, n: int, k: int, lo: int, hi: int) -> np.ndarray:
    """n rows of k distinct integers in [lo, hi).

    Dense draws (k comparable to the range) take the first k entries of a
    random permutation per row; sparse draws redraw the rows that repeat.
    """
    span = hi - lo
    if k > span:
        raise ValueError(f"cannot draw {k} distinct values from {span}")
    if k * k > 6 * span:  # P(no repeat) = exp(-k^2 / 2 span) < 5%: rejection would crawl
        out = np.empty((n, k), dtype=np.int64)
        for r0 in range(0, n, 4096):
            r1 = min(n, r0 + 4096)
            out[r0:r1] = np.argsort(rng.random((r1 - r0, span)), axis=1)[:, :k] + lo
        return out
    out = rng.integers(lo, hi, (n, k))
    todo = np.arange(n)
    while todo.size:
        s = np.sort(out[todo], axis=1)
        bad = (s[:, 1:] == s[:, :-1]).any(axis=1)
        todo = todo[bad]
        out[todo] = rng.integers(lo, hi, (todo.size, k))
    return out


def structured_batch(n_pos: int, spec: dict = HALFKA_HM_MERGED, num_buckets: int = 8,
                     seed: int = 0, nnz_min: int | None = None):
    """Returns (Batch, bucket_idx)."""
    rng = np.random.default_rng(seed)
    pi, kb_n, ma = spec["piece_inputs"], spec["king_buckets"], spec["max_active"]
    has_king = spec["king_lo"] is not None
    n_piece_slots = ma - (2 if has_king else 0)
    lo = nnz_min if nnz_min is not None else ma
    nnz = rng.integers(lo, ma + 1, n_pos).astype(np.int32)
    out = []
    for _persp in range(2):
        kb = rng.integers(0, kb_n, n_pos).astype(np.int64)
        pieces = _distinct_rows(rng, n_pos, n_piece_slots, spec["piece_lo"], spec["piece_hi"])
        rows = [pieces]
        if has_king:
            k0, nk = spec["king_lo"], pi - spec["king_lo"]
            kings = _distinct_rows(rng, n_pos, 2, k0, k0 + nk)
            rows.append(kings)
        packed = np.concatenate(rows, axis=1)
        idx = (kb[:, None] * pi + packed).astype(np.int32)
        slot = np.arange(ma)[None, :]
        idx = np.where(slot < nnz[:, None], idx, -1).astype(np.int32)
        out.append(idx)
    score = np.clip(rng.normal(0.0, 600.0, n_pos), -3000, 3000).astype(np.float32)
    wdl = rng.choice(np.array([0.0, 0.5, 1.0], np.float32), n_pos)
    bucket = rng.integers(0, num_buckets, n_pos).astype(np.int32)
    return Batch(out[0], out[1], nnz, score, wdl), bucket
