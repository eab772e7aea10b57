"""Pins the CPU feature oracle (oracle/features.cpp) to the reference's own tests.

Sources (crates/shogi-format, crates/shogi-features):
  - sample.psv (100 records, tests/golden/sample.psv; tests/psv_smoke.rs) and
    the Huffman / bit-stream KATs of src/packed_sfen.rs:709-835;
  - for_each_board_piece emission order (packed_sfen.rs:835-923);
  - golden kings-only indices (tests/feature_set.rs:283-320), the nnue-pytorch
    index formulas for halfkp / halfka-split (:118-226), range / injectivity /
    fold / perspective-swap / mirror invariants (:322-569);
  - kingrank9 SFEN fixtures (src/kingrank9.rs:78-104);
  - zero-weight progress = 0.5 -> bucket 4 (src/progress_kpabs.rs:230-270).
A byte-exact re-encode of every sample.psv record (decoder and the
independent encoder of tatara_amd/psv.py) pins the decoder bit for bit.
"""
import ctypes
import ctypes.util
from pathlib import Path

import numpy as np
import pytest

from oracle import features as of
from tatara_amd import psv

GOLDEN = Path(__file__).resolve().parent / "golden"
FS = of.FEATURE_SETS


def sample():
    raw = np.fromfile(GOLDEN / "sample.psv", dtype=np.uint8)
    assert raw.size == 4000
    return raw.reshape(100, 40)


def sq(file, rank):
    return file * 9 + rank


def board(stm, bk, wk, pieces=(), hand=None):
    pt = np.zeros(81, int)
    col = np.zeros(81, int)
    pt[bk], col[bk] = 8, 0
    pt[wk], col[wk] = 8, 1
    for c, t, s in pieces:
        pt[s], col[s] = t, c
    h = np.zeros((2, 7), int) if hand is None else hand
    return of.board_rows(pt, col, h, stm)


def feats(rows, fs):
    o = of.boards_to_batch(rows, fs)
    return [list(zip(o["stm"][i][: o["nnz"][i]].tolist(), o["nstm"][i][: o["nnz"][i]].tolist()))
            for i in range(len(o["nnz"]))]


# -- PSV decode (packed_sfen.rs, psv_smoke.rs) ------------------------------------------------
def test_sample_psv_records_are_sane():
    d = of.psv_decode(sample())
    assert np.all(np.abs(d["score"]) <= 32600) and np.all(d["ply"] <= 1024)
    assert set(np.unique(d["result"]).tolist()) <= {-1, 0, 1}
    assert np.all(d["bking"] < 81) and np.all(d["wking"] < 81)
    full = {1: 18, 2: 4, 3: 4, 4: 4, 7: 4, 5: 2, 6: 2}
    base = np.array([0, 1, 2, 3, 4, 5, 6, 7, 8, 1, 2, 3, 4, 5, 6])
    for i in range(100):
        b = base[d["ptype"][i]]
        for t, want in full.items():
            hand = d["hand"][i, :, psv.HAND_TYPES.index(t)].sum()
            assert (b == t).sum() + hand == want, (i, t)
        assert (d["ptype"][i] == 8).sum() == 2


def test_sample_psv_reencodes_byte_for_byte():
    raw = sample()
    d = of.psv_decode(raw)
    enc = psv.encode(d["ptype"], d["color"], d["hand"], d["stm"], d["score"], d["result"], d["ply"])
    enc[:, 34:36] = raw[:, 34:36]  # move16 is not decoded
    assert np.array_equal(enc, raw)


class BitWriter:
    def __init__(self):
        self.bits = []

    def put(self, value, n):
        self.bits += [(value >> i) & 1 for i in range(n)]

    def record(self):
        b = np.zeros(256, np.uint8)
        b[: len(self.bits)] = self.bits[:256]
        out = np.zeros(40, np.uint8)
        out[:32] = np.packbits(b, bitorder="little")
        return out


def _header(w, stm=0, bk=80, wk=79):
    w.put(stm, 1)
    w.put(bk, 7)
    w.put(wk, 7)


@pytest.mark.parametrize("bits,nbits,ptype,color", [
    (0b0000, 1, 0, 0),       # empty square: 0 (test_huffman_decode_empty)
    (0b0001, 4, 1, 0),       # black pawn: 01 + unpromoted + black
    (0b1101, 4, 9, 1),       # white promoted pawn: 01 + promoted + white
    (0b001111, 6, 7, 0),     # black gold: 01111 + black (no promotion bit)
])
def test_board_square_huffman_kats(bits, nbits, ptype, color):
    w = BitWriter()
    _header(w)
    w.put(bits, nbits)
    d = of.psv_decode(w.record())
    assert d["ptype"][0, 0] == ptype and (ptype == 0 or d["color"][0, 0] == color)


@pytest.mark.parametrize("bits,nbits,hand_idx,counted", [
    (0b000, 3, 0, True),         # hand pawn: 0 + box 0 + black
    (0b00111, 5, 4, True),       # hand gold: 0111 + black
    (0b010, 3, 0, False),        # piece-box pawn: 0 + box 1 + black -> ignored
    (0b0111111, 7, 6, False),    # piece-box rook: 11111 + box 1 + black -> ignored
])
def test_hand_huffman_kats(bits, nbits, hand_idx, counted):
    w = BitWriter()
    _header(w)
    w.put(0, 79)        # 79 empty squares
    w.put(bits, nbits)  # the entry under test
    # fill the rest with piece-box lances (001 + box 1 + black 0 = 5 bits) and
    # piece-box pawns (3 bits) so nothing else is counted
    while 256 - len(w.bits) >= 5 and (256 - len(w.bits)) % 3 != 0:
        w.put(0b01001, 5)
    while 256 - len(w.bits) >= 3:
        w.put(0b010, 3)
    assert len(w.bits) == 256
    d = of.psv_decode(w.record())
    want = np.zeros((2, 7), int)
    if counted:
        want[0, hand_idx] = 1
    assert np.array_equal(d["hand"][0], want)


def test_hand_loop_stops_at_bit_256():
    # an all-zero stream: both kings on square 0, 80 empty squares (bits 15..94),
    # then 3-bit black hand pawns; the last one starts at bit 254 and its
    # colour bit is read past the end as 0 (BitStream::read_bit), so 54 pawns
    d = of.psv_decode(np.zeros(40, np.uint8))
    assert d["bking"][0] == 0 and d["wking"][0] == 0
    assert d["hand"][0, 0, 0] == 54 and d["hand"][0].sum() == 54


# -- emission order (packed_sfen.rs:835-923) ---------------------------------------------------
def test_board_piece_emission_order():
    pieces = [(0, 1, sq(f, 6)) for f in range(9)] + [(1, 1, sq(f, 2)) for f in range(9)]
    pieces += [(0, 4, sq(0, 7)), (1, 14, sq(8, 1))]
    rows = board(0, sq(4, 8), sq(4, 0), pieces)
    f = feats(rows, "halfkp")[0]
    assert len(f) == 20
    kb = sq(4, 8) * 1548
    got = [s - kb for s, _ in f]
    want = [90 + sq(fl, 6) for fl in range(9)] + [171 + sq(fl, 2) for fl in range(9)]
    want += [576 + sq(0, 7), 1467 + sq(8, 1)]  # black silver (F_SILVER), white dragon (E_DRAGON)
    assert got == want


# -- golden indices (tests/feature_set.rs:283-320) ------------------------------------------------
@pytest.mark.parametrize("fs,bk,wk,want", [
    ("halfka-hm-merged", sq(4, 8), sq(4, 0), [(73268, 73268), (73260, 73260)]),
    ("halfka-merged", sq(0, 0), sq(8, 8), [(1548, 1548), (1628, 1628)]),
    ("halfka-hm-split", sq(6, 2), sq(2, 6), [(35768, 35768), (35889, 35889)]),
])
def test_golden_kings_only(fs, bk, wk, want):
    assert feats(board(0, bk, wk), fs)[0] == want


def test_feature_set_dimensions():
    want = {"halfkp": (81, 1548, 125388, 38), "halfka-split": (81, 1710, 138510, 40),
            "halfka-merged": (81, 1629, 131949, 40), "halfka-hm-split": (45, 1710, 76950, 40),
            "halfka-hm-merged": (45, 1629, 73305, 40)}
    for fs, (kb, pi, fi, ma) in want.items():
        assert of.feature_set_info(fs) == dict(king_buckets=kb, piece_inputs=pi, ft_in=fi, max_active=ma)


# -- nnue-pytorch index formulas (tests/feature_set.rs:118-226) ------------------------------------
_BASE_F = {1: 90, 2: 252, 3: 414, 4: 576, 7: 738, 5: 900, 13: 1062, 6: 1224, 14: 1386,
           9: 738, 10: 738, 11: 738, 12: 738}
_HAND_F = [1, 39, 49, 59, 69, 79, 85]
_HAND_E = [20, 44, 54, 64, 74, 82, 88]
_ORDER = [1, 2, 3, 4, 7, 5, 6, 9, 10, 11, 12, 13, 14]


def _formula(d, i, with_kings, ft_stride):
    """Independent restatement: king_sq * stride + bonapiece, perspective-rotated."""
    stm = int(d["stm"][i])
    kings = (int(d["bking"][i]), int(d["wking"][i]))

    def rot(s, p):
        return s if p == 0 else 80 - s

    def bp_board(t, c, s, p):
        f = _BASE_F[t]
        return (f if c == p else f + 81) + rot(s, p)

    out = []
    for p in (stm, 1 - stm):
        ksq = rot(kings[p], p)
        idx = []
        for t in _ORDER:
            for c in (0, 1):
                for s in range(81):
                    if d["ptype"][i, s] == t and d["color"][i, s] == c:
                        idx.append(ksq * ft_stride + bp_board(t, c, s, p))
        if with_kings:
            idx.append(ksq * ft_stride + 1548 + rot(kings[p], p))
            idx.append(ksq * ft_stride + 1629 + rot(kings[1 - p], p))
        for owner in (0, 1):
            for hi in range(7):
                for k in range(int(d["hand"][i, owner, hi])):
                    idx.append(ksq * ft_stride + (_HAND_F if owner == p else _HAND_E)[hi] + k)
        out.append(idx)
    return list(zip(out[0], out[1]))


@pytest.mark.parametrize("fs,with_kings,stride", [("halfkp", False, 1548), ("halfka-split", True, 1710)])
def test_reference_index_formula(fs, with_kings, stride):
    recs = np.concatenate([sample(), psv.synthetic_psv(300, seed=7)])
    d = of.psv_decode(recs)
    o = of.psv_to_batch(recs, fs)
    for i in range(len(recs)):
        got = list(zip(o["stm"][i][: o["nnz"][i]].tolist(), o["nstm"][i][: o["nnz"][i]].tolist()))
        assert got == _formula(d, i, with_kings, stride), i


# -- invariants over all five feature sets ----------------------------------------------------------
def _all():
    recs = np.concatenate([sample(), psv.synthetic_psv(200, seed=8)])
    return recs, of.psv_decode(recs)


def test_ranges_and_injectivity():
    recs, _ = _all()
    for fs in FS:
        info = of.feature_set_info(fs)
        o = of.psv_to_batch(recs, fs)
        for i in range(len(recs)):
            n = o["nnz"][i]
            assert 0 < n <= info["max_active"]
            for row in (o["stm"][i], o["nstm"][i]):
                v = row[:n]
                assert v.min() >= 0 and v.max() < info["ft_in"]
                assert len(set(v.tolist())) == n
                assert np.all(row[n:] == -1)


@pytest.mark.parametrize("split,merged", [("halfka-split", "halfka-merged"), ("halfka-hm-split", "halfka-hm-merged")])
def test_merged_is_split_plus_enemy_king_fold(split, merged):
    recs, _ = _all()
    a = of.psv_to_batch(recs, split)
    b = of.psv_to_batch(recs, merged)
    pa, pb = of.feature_set_info(split)["piece_inputs"], of.feature_set_info(merged)["piece_inputs"]
    assert np.array_equal(a["nnz"], b["nnz"])
    for key in ("stm", "nstm"):
        for i in range(len(recs)):
            n = a["nnz"][i]
            ka, ppa = np.divmod(a[key][i][:n], pa)
            kb, ppb = np.divmod(b[key][i][:n], pb)
            assert np.array_equal(ka, kb)
            assert np.array_equal(np.where(ppa >= 1629, ppa - 81, ppa), ppb)


def test_perspective_swap():
    recs, d = _all()
    for fs in FS:
        rows = of.board_rows(d["ptype"], d["color"], d["hand"], d["stm"])
        rows_sw = rows.copy()
        rows_sw[:, 176] = 1 - rows_sw[:, 176]
        f0, f1 = feats(rows, fs), feats(rows_sw, fs)
        for x, y in zip(f0, f1):
            assert sorted((n, s) for s, n in x) == sorted(y)


def _mirror(rows):
    out = rows.copy()
    for s in range(81):
        m = (8 - s // 9) * 9 + s % 9
        out[:, m] = rows[:, s]
        out[:, 81 + m] = rows[:, 81 + s]
    for col in (177, 178):
        k = rows[:, col]
        out[:, col] = (8 - k // 9) * 9 + k % 9
    return out


def test_horizontal_mirror_invariance():
    pieces = [(0, 1, sq(2, 6)), (0, 7, sq(7, 7)), (1, 6, sq(1, 1)), (1, 4, sq(5, 3))]
    rows = np.concatenate([board(0, sq(6, 8), sq(2, 0), pieces), board(1, sq(1, 7), sq(7, 2), pieces),
                           board(0, sq(0, 4), sq(8, 4), pieces)])
    for fs in ("halfka-hm-split", "halfka-hm-merged"):
        for a, b in zip(feats(rows, fs), feats(_mirror(rows), fs)):
            assert a and sorted(a) == sorted(b)
    one = board(0, sq(6, 8), sq(2, 0), [(0, 1, sq(2, 6))])
    for fs in ("halfka-split", "halfka-merged"):
        assert sorted(feats(one, fs)[0]) != sorted(feats(_mirror(one), fs)[0])


# -- buckets -----------------------------------------------------------------------------------------
@pytest.mark.parametrize("sfen,want", [
    ("lnsgkgsnl/1r5b1/ppppppppp/9/9/9/PPPPPPPPP/1B5R1/LNSGKGSNL b - 1", 8),
    ("lnsg1gsnl/1r2k2b1/ppppppppp/9/9/9/PPPPPPPPP/1B2K2R1/LNSG1GSNL w - 1", 8),
    ("9/9/4K4/9/9/9/4k4/9/9 b - 1", 0),
    ("9/9/9/4K4/4k4/9/9/9/9 b - 1", 4),
    ("lnsgkgsnl/1r5b1/ppppppppp/9/9/9/PPPPPPPPP/1B5R1/LNSGKGSNL w - 1", 8),
])
def test_kingrank9_fixtures(sfen, want):
    pt, col, hand, stm = psv.parse_sfen(sfen)
    o = of.boards_to_batch(of.board_rows(pt, col, hand, stm), "halfkp", "kingrank9")
    assert o["bucket"][0] == want


def test_zero_weight_progress_is_half_and_bucket_4():
    recs = sample()
    w = np.zeros(81 * 1548, np.float32)
    for nb in (8, 9):
        o = of.psv_to_batch(recs, "halfka-hm-merged", "progress", nb, w)
        assert np.all(o["progress"] == 0.5) and np.all(o["bucket"] == 4)


def _libm_expf():
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    return libm.expf


def test_progress_matches_brute_force():
    """Sum of the KP-abs weights in emission order, glibc expf, floor(p * N)."""
    expf = _libm_expf()
    recs = np.concatenate([sample(), psv.synthetic_psv(200, seed=9)])
    w = (np.random.default_rng(3).normal(0, 0.05, 81 * 1548)).astype(np.float32)
    o = of.psv_to_batch(recs, "halfka-hm-merged", "progress", 8, w)
    d = of.psv_decode(recs)
    for i in range(len(recs)):
        idx = of.kpabs_indices(recs[i])
        # an independent index formula: black king square * 1548 + BonaPiece (black view),
        # (80 - white king) * 1548 + BonaPiece (white view)
        assert len(idx) == 2 * (int((d["ptype"][i] > 0).sum()) - 2 + int(d["hand"][i].sum()))
        s = np.float32(0.0)
        for v in idx:
            s = np.float32(s + w[v])
        p = np.float32(1.0) / (np.float32(1.0) + np.float32(expf(float(-s))))
        assert o["progress"][i] == p
        assert o["bucket"][i] == min(7, max(0, int(np.floor(np.float32(p * np.float32(8))))))
    assert len(set(o["bucket"].tolist())) > 2


def test_records_king_blocked():
    """A PSV batch is certified king-blocked unless, in a feature set with
    merged king planes, a record has both kings on one square (its decoded
    rows then hold the king feature twice, which the oracle confirms)."""
    from tatara_amd.dataloader import king_squares, records_king_blocked
    from tatara_amd.psv import synthetic_psv

    rec = synthetic_psv(256, seed=77)
    a, b = king_squares(rec)
    dec = of.psv_decode(rec)
    assert np.array_equal(a, dec["bking"]) and np.array_equal(b, dec["wking"])
    for fs in of.FEATURE_SETS:
        assert records_king_blocked(rec, fs)
    bad = rec.copy()
    w = int(bad[9, 0]) | (int(bad[9, 1]) << 8)
    k0 = (w >> 1) & 127
    w = (w & ~(127 << 8)) | (k0 << 8)
    bad[9, 0], bad[9, 1] = w & 255, (w >> 8) & 255
    assert king_squares(bad)[1][9] == k0
    for fs in of.FEATURE_SETS:
        merged = fs in ("halfka-merged", "halfka-hm-merged")
        assert records_king_blocked(bad, fs) == (not merged), fs
        rows = of.psv_to_batch(bad[9:10], fs)
        for persp in ("stm", "nstm"):
            r = rows[persp][0][: rows["nnz"][0]]
            assert (len(np.unique(r)) < len(r)) == merged, (fs, persp)
