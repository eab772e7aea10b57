"""PackedSfenValue (PSV) records: synthetic positions and a vectorised encoder.

The 40-byte record layout is PackedSfenValue
(crates/shogi-format/src/packed_sfen.rs:255-268): a 256-bit LSB-first
Huffman-coded position (side to move, two 7-bit king squares, the 79 other
squares in index order, then hand pieces), score (i16 LE), move16 (u16 LE),
game_ply (u16 LE), game_result (i8) and one padding byte.  The encoder
writes exactly what ShogiBoard::from_packed_sfen (:387-449) reads back:
board pieces as Huffman code + promoted bit (not gold) + colour bit, hand
pieces as the board code without its first bit + a zero piece-box bit (not
gold) + colour bit.  The reference has no encoder; this one exists to make
seeded synthetic training data (40 pieces, 15 % in hand,
10 % of promotable board pieces promoted, uniform owners and side to move,
score ~ N(0, 600) clipped to +-3000, uniform result).

Boards are numpy arrays: ptype [n, 81] (0 none, 1 pawn, 2 lance, 3 knight,
4 silver, 5 bishop, 6 rook, 7 gold, 8 king, 9..14 promoted pawn, lance,
knight, silver, horse, dragon), color [n, 81] (0 black, 1 white),
hand [n, 2, 7] counts in (pawn, lance, knight, silver, gold, bishop, rook)
order, stm [n].  Squares are file * 9 + rank (file 0 = 1-suji, rank 0 = a).
"""
from __future__ import annotations

import numpy as np

RECORD_BYTES = 40

# Huffman code per base piece type: (LSB-first pattern, length)
_HUFF = {0: (0x00, 1), 1: (0x01, 2), 2: (0x03, 4), 3: (0x0B, 4), 4: (0x07, 4), 5: (0x1F, 6),
         6: (0x3F, 6), 7: (0x0F, 5)}
_UNPROMOTE = np.array([0, 1, 2, 3, 4, 5, 6, 7, 8, 1, 2, 3, 4, 5, 6], np.int64)
HAND_TYPES = (1, 2, 3, 4, 7, 5, 6)  # pawn, lance, knight, silver, gold, bishop, rook


_PAT = np.array([_HUFF[t][0] if t in _HUFF else 0 for t in range(9)], np.int64)
_LEN = np.array([_HUFF[t][1] if t in _HUFF else 0 for t in range(9)], np.int64)


def _board_code(ptype: np.ndarray, color: np.ndarray):
    """(value, length) of every square's board code; kings get length 0."""
    base = _UNPROMOTE[ptype]
    val = _PAT[base]
    tot = _LEN[base]
    has_prom = ((base != 7) & (base != 0) & (base != 8)).astype(np.int64)
    val = val | (((ptype >= 9).astype(np.int64) * has_prom) << tot)
    tot = tot + has_prom
    occupied = ((base != 0) & (base != 8)).astype(np.int64)
    val = val | ((color.astype(np.int64) * occupied) << tot)
    tot = tot + occupied
    is_king = base == 8
    return np.where(is_king, 0, val), np.where(is_king, 0, tot)


def encode(ptype, color, hand, stm, score=None, result=None, ply=None) -> np.ndarray:
    """Encodes boards into [n, 40] uint8 PSV records (all 40 pieces present)."""
    ptype = np.asarray(ptype, np.int64)
    color = np.asarray(color, np.int64)
    hand = np.asarray(hand, np.int64)
    n = ptype.shape[0]
    stm = np.asarray(stm, np.int64).reshape(n)
    kings = []
    for c in (0, 1):
        m = (ptype == 8) & (color == c)
        if not np.all(m.sum(1) == 1):
            raise ValueError("every board needs exactly one king per side")
        kings.append(m.argmax(1))
    fields_v = [stm, kings[0], kings[1]]
    fields_l = [np.ones(n, np.int64), np.full(n, 7), np.full(n, 7)]
    bv, bl = _board_code(ptype, color)
    fields_v += [bv[:, i] for i in range(81)]
    fields_l += [bl[:, i] for i in range(81)]
    # hand entries: up to 38 per position, per owner (black, white) in Huffman
    # table order (pawn, lance, knight, silver, bishop, rook, gold), which
    # reproduces the records of the reference's sample.psv bit for bit
    max_hand = 38
    hv = np.zeros((n, max_hand), np.int64)
    hl = np.zeros((n, max_hand), np.int64)
    slot = np.zeros(n, np.int64)
    rows = np.arange(n)
    for owner in (0, 1):
        for t in (1, 2, 3, 4, 5, 6, 7):
            hi = HAND_TYPES.index(t)
            p, l = _HUFF[t]
            code = p >> 1
            ln = l - 1
            if t != 7:
                ln += 1  # piece-box bit, 0
            val = code | (owner << ln)
            ln += 1
            cnt = hand[:, owner, hi]
            for k in range(int(cnt.max(initial=0))):
                m = cnt > k
                if np.any(slot[m] >= max_hand):
                    raise ValueError("more than 38 pieces in hand")
                hv[rows[m], slot[m]] = val
                hl[rows[m], slot[m]] = ln
                slot[m] += 1
    fields_v += [hv[:, i] for i in range(max_hand)]
    fields_l += [hl[:, i] for i in range(max_hand)]
    V = np.stack(fields_v, 1)
    L = np.stack(fields_l, 1)
    off = np.cumsum(L, 1) - L
    total = L.sum(1)
    if np.any(total > 256):
        raise ValueError("position does not fit 256 bits")
    # OR every field into four little-endian 64-bit words (fields are at most
    # 8 bits long, so a field touches at most two words)
    words = np.zeros((n, 6), np.uint64)
    V = V.astype(np.uint64)
    for j in range(V.shape[1]):
        o = off[:, j].astype(np.uint64)
        wi = (o >> np.uint64(6)).astype(np.int64)
        sh = o & np.uint64(63)
        lo = V[:, j] << sh
        hi = np.where(sh > 0, V[:, j] >> (np.uint64(64) - np.maximum(sh, np.uint64(1))), np.uint64(0))
        words[rows, wi] |= lo
        words[rows, wi + 1] |= hi
    packed = np.ascontiguousarray(words[:, :4].astype("<u8")).view(np.uint8).reshape(n, 32)
    out = np.zeros((n, RECORD_BYTES), np.uint8)
    out[:, :32] = packed
    sc = np.zeros(n, np.int16) if score is None else np.asarray(score, np.int16)
    out[:, 32:34] = sc.view(np.uint8).reshape(n, 2)
    pl = np.zeros(n, np.uint16) if ply is None else np.asarray(ply, np.uint16)
    out[:, 36:38] = pl.view(np.uint8).reshape(n, 2)
    rs = np.zeros(n, np.int8) if result is None else np.asarray(result, np.int8)
    out[:, 38] = rs.view(np.uint8)
    return out


# initial piece set per side's total: 2K handled separately
_SET = ([6] * 2 + [5] * 2 + [7] * 4 + [4] * 4 + [3] * 4 + [2] * 4 + [1] * 18)  # R, B, G, S, N, L, P


def synthetic_positions(n: int, seed: int, p_hand: float = 0.15, p_promote: float = 0.1):
    """Seeded random positions per BASELINE configs[0]; returns a dict of arrays."""
    rng = np.random.default_rng(seed)
    n_pieces = len(_SET)  # 38 non-king pieces
    sq = np.argsort(rng.random((n, 81)), axis=1)[:, : n_pieces + 2]
    ptype = np.zeros((n, 81), np.int64)
    color = np.zeros((n, 81), np.int64)
    rows = np.arange(n)
    ptype[rows, sq[:, 0]] = 8
    color[rows, sq[:, 0]] = 0
    ptype[rows, sq[:, 1]] = 8
    color[rows, sq[:, 1]] = 1
    hand = np.zeros((n, 2, 7), np.int64)
    owner = rng.integers(0, 2, (n, n_pieces))
    to_hand = rng.random((n, n_pieces)) < p_hand
    promote = rng.random((n, n_pieces)) < p_promote
    promo_of = {1: 9, 2: 10, 3: 11, 4: 12, 5: 13, 6: 14}
    for k, t in enumerate(_SET):
        on_board = ~to_hand[:, k]
        s = sq[:, k + 2]
        pt = np.full(n, t)
        if t in promo_of:
            pt = np.where(promote[:, k], promo_of[t], t)
        r = rows[on_board]
        ptype[r, s[on_board]] = pt[on_board]
        color[r, s[on_board]] = owner[on_board, k]
        hi = HAND_TYPES.index(t)
        rh = rows[~on_board]
        np.add.at(hand, (rh, owner[~on_board, k], hi), 1)
    stm = rng.integers(0, 2, n)
    score = np.clip(np.rint(rng.normal(0.0, 600.0, n)), -3000, 3000).astype(np.int16)
    result = rng.integers(-1, 2, n).astype(np.int8)
    ply = rng.integers(1, 256, n).astype(np.uint16)
    return dict(ptype=ptype, color=color, hand=hand, stm=stm, score=score, result=result, ply=ply)


def synthetic_psv(n: int, seed: int) -> np.ndarray:
    """[n, 40] uint8 records of seeded synthetic positions."""
    p = synthetic_positions(n, seed)
    return encode(p["ptype"], p["color"], p["hand"], p["stm"], p["score"], p["result"], p["ply"])


def synthetic_progress_weights(seed: int, std: float = 0.01) -> np.ndarray:
    """A seeded progress.bin stand-in: 81 * 1548 f64 weights ~ N(0, std)."""
    rng = np.random.default_rng(seed)
    return rng.normal(0.0, std, 81 * 1548)


def parse_sfen(sfen: str):
    """Board, hands and side to move of an SFEN string (tests and fixtures)."""
    fields = sfen.split()
    placement, side = fields[0], fields[1]
    hands = fields[2] if len(fields) > 2 else "-"
    ptype = np.zeros(81, np.int64)
    color = np.zeros(81, np.int64)
    letters = {"p": 1, "l": 2, "n": 3, "s": 4, "b": 5, "r": 6, "g": 7, "k": 8}
    promo = {1: 9, 2: 10, 3: 11, 4: 12, 5: 13, 6: 14}
    for rank, row in enumerate(placement.split("/")):
        file_from_left = 0
        plus = False
        for ch in row:
            if ch.isdigit():
                file_from_left += int(ch)
                continue
            if ch == "+":
                plus = True
                continue
            t = letters[ch.lower()]
            if plus:
                t = promo[t]
                plus = False
            file = 8 - file_from_left
            ptype[file * 9 + rank] = t
            color[file * 9 + rank] = 0 if ch.isupper() else 1
            file_from_left += 1
    hand = np.zeros((2, 7), np.int64)
    if hands != "-":
        cnt = ""
        for ch in hands:
            if ch.isdigit():
                cnt += ch
                continue
            t = letters[ch.lower()]
            hand[0 if ch.isupper() else 1, HAND_TYPES.index(t)] += int(cnt) if cnt else 1
            cnt = ""
    return ptype, color, hand, 0 if side == "b" else 1
