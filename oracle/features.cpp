// CPU oracle for PSV decoding, feature-index extraction and bucket assignment.
//
// TEST INFRASTRUCTURE ONLY.  The checker for the HIP product path
// (tatara_amd/csrc/psv_kernels.hip); only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it.
//
// Restates, in the reference's order of operations:
//   - PackedSfenValue layout and ShogiBoard::from_packed_sfen
//     (crates/shogi-format/src/packed_sfen.rs:255-268, :387-449, :559-617):
//     LSB-first bit stream, side to move, two 7-bit king squares, 79 Huffman
//     coded squares, then hand / piece-box entries until bit 256;
//   - BonaPiece::from_piece_square / from_hand_piece and the offset table
//     (crates/shogi-format/src/bona_piece.rs);
//   - ShogiBoard::for_each_board_piece emission order (packed_sfen.rs:493-540):
//     BOARD_PIECE_TYPES order x (Black, White) x ascending square;
//   - FeatureSetSpec::extract_active_features / perspective_ctx /
//     pack_bonapiece for the five feature sets
//     (crates/shogi-features/src/feature_set.rs:103-185, :655-810, :822-841,
//     :972-1002);
//   - kingrank9_bucket_board (crates/shogi-features/src/kingrank9.rs:11-23);
//   - ShogiProgressKPAbs (crates/shogi-features/src/progress_kpabs.rs:53-170):
//     f32 sum of the KP-absolute weights in emission order, glibc expf,
//     floor(p * N) clamped to [0, N-1];
//   - Batch::push_decoded score / wdl (crates/nnue-train/src/dataloader.rs:
//     444-497).

#include <cmath>
#include <cstdint>
#include <cstring>

namespace {

enum : int { kNone = 0, kPawn, kLance, kKnight, kSilver, kBishop, kRook, kGold, kKing,
             kProPawn, kProLance, kProKnight, kProSilver, kHorse, kDragon };

// Huffman codes (LSB-first pattern, length) indexed Huffman piece id:
// 0 none, 1 pawn, 2 lance, 3 knight, 4 silver, 5 bishop, 6 rook, 7 gold.
const uint32_t kCode[8] = {0x00, 0x01, 0x03, 0x0b, 0x07, 0x1f, 0x3f, 0x0f};
const int kLen[8] = {1, 2, 4, 4, 4, 6, 6, 5};
const int kHuffToType[8] = {kNone, kPawn, kLance, kKnight, kSilver, kBishop, kRook, kGold};

const int kBoardTypes[13] = {kPawn, kLance, kKnight, kSilver, kGold, kBishop, kRook,
                             kProPawn, kProLance, kProKnight, kProSilver, kHorse, kDragon};
// Hand index order: pawn, lance, knight, silver, gold, bishop, rook.
const int kHandTypes[7] = {kPawn, kLance, kKnight, kSilver, kGold, kBishop, kRook};

// BonaPiece bases [piece type][is_friend] (bona_piece.rs PIECE_BASE).
const int kF_PAWN = 90, kE_PAWN = 171, kF_LANCE = 252, kE_LANCE = 333, kF_KNIGHT = 414,
          kE_KNIGHT = 495, kF_SILVER = 576, kE_SILVER = 657, kF_GOLD = 738, kE_GOLD = 819,
          kF_BISHOP = 900, kE_BISHOP = 981, kF_HORSE = 1062, kE_HORSE = 1143, kF_ROOK = 1224,
          kE_ROOK = 1305, kF_DRAGON = 1386, kE_DRAGON = 1467;
const int kFE_HAND_END = 90, kFE_OLD_END = 1548, kF_KING = 1548, kE_KING = 1629;
const int kPieceBase[15][2] = {
    {0, 0},
    {kE_PAWN, kF_PAWN},     {kE_LANCE, kF_LANCE}, {kE_KNIGHT, kF_KNIGHT}, {kE_SILVER, kF_SILVER},
    {kE_BISHOP, kF_BISHOP}, {kE_ROOK, kF_ROOK},   {kE_GOLD, kF_GOLD},     {0, 0},
    {kE_GOLD, kF_GOLD},     {kE_GOLD, kF_GOLD},   {kE_GOLD, kF_GOLD},     {kE_GOLD, kF_GOLD},
    {kE_HORSE, kF_HORSE},   {kE_DRAGON, kF_DRAGON}};
// hand bases [hand index][is_friend]
const int kHandBase[7][2] = {{20, 1}, {44, 39}, {54, 49}, {64, 59}, {74, 69}, {82, 79}, {88, 85}};

int hand_index(int pt) {
    for (int i = 0; i < 7; ++i)
        if (kHandTypes[i] == pt) return i;
    return -1;
}

int promote(int pt) {
    switch (pt) {
        case kPawn: return kProPawn;
        case kLance: return kProLance;
        case kKnight: return kProKnight;
        case kSilver: return kProSilver;
        case kBishop: return kHorse;
        case kRook: return kDragon;
        default: return pt;
    }
}

struct Bits {
    const uint8_t* d;
    int cur = 0;
    int bit() {
        if (cur >= 256) return 0;  // BitStream::read_bit past the end reads 0
        const int b = (d[cur >> 3] >> (cur & 7)) & 1;
        ++cur;
        return b;
    }
    uint32_t peek(int n) const {  // zero-padded past the 32 bytes
        uint32_t v = 0;
        for (int i = 0; i < n; ++i) {
            const int c = cur + i;
            if (c < 256) v |= (uint32_t)((d[c >> 3] >> (c & 7)) & 1) << i;
        }
        return v;
    }
};

// the prefix code entry whose pattern matches the low bits of v
int match(uint32_t v, bool hand, int* len) {
    for (int i = hand ? 1 : 0; i < 8; ++i) {
        const uint32_t pat = hand ? kCode[i] >> 1 : kCode[i];
        const int l = hand ? kLen[i] - 1 : kLen[i];
        if ((v & ((1u << l) - 1u)) == pat) {
            *len = l;
            return i;
        }
    }
    *len = 0;
    return 0;
}

struct Board {
    int8_t type[81];
    int8_t color[81];
    uint8_t hand[2][7];
    int stm;
    int king[2];  // square, 81 = none
    int16_t score;
    int8_t result;
    uint16_t ply;
};

void decode(const uint8_t* rec, Board& b) {
    std::memset(&b, 0, sizeof(b));
    b.score = (int16_t)(rec[32] | (rec[33] << 8));
    b.ply = (uint16_t)(rec[36] | (rec[37] << 8));
    b.result = (int8_t)rec[38];
    Bits s{rec};
    b.stm = s.bit();
    int k[2] = {0, 0};
    for (int c = 0; c < 2; ++c)
        for (int i = 0; i < 7; ++i) k[c] |= s.bit() << i;
    b.king[0] = k[0];
    b.king[1] = k[1];
    if (k[0] < 81) { b.type[k[0]] = kKing; b.color[k[0]] = 0; }
    if (k[1] < 81) { b.type[k[1]] = kKing; b.color[k[1]] = 1; }
    for (int sq = 0; sq < 81; ++sq) {
        if (sq == k[0] || sq == k[1]) continue;
        int len;
        const int h = match(s.peek(6), false, &len);
        s.cur += len;
        if (h == 0) { b.type[sq] = kNone; b.color[sq] = 0; continue; }
        const int promoted = h != 7 ? s.bit() : 0;
        const int color = s.bit();
        const int pt = kHuffToType[h];
        b.type[sq] = (int8_t)(promoted ? promote(pt) : pt);
        b.color[sq] = (int8_t)color;
    }
    while (s.cur < 256) {
        int len;
        const int h = match(s.peek(5), true, &len);
        s.cur += len;
        const int piecebox = h != 7 ? s.bit() : 0;
        const int color = s.bit();
        if (piecebox) continue;
        const int hi = hand_index(kHuffToType[h]);
        if (hi >= 0) b.hand[color][hi] += 1;
    }
}

int persp_sq(int sq, int persp) { return persp == 0 ? sq : 80 - sq; }

struct Spec {
    int king_buckets, piece_inputs, max_active;
    bool emit_king, fold_enemy, mirror;
};

bool spec_of(int fs, Spec& s) {
    switch (fs) {
        case 0: s = {81, 1548, 38, false, false, false}; return true;  // halfkp
        case 1: s = {81, 1710, 40, true, false, false}; return true;   // halfka-split
        case 2: s = {81, 1629, 40, true, true, false}; return true;    // halfka-merged
        case 3: s = {45, 1710, 40, true, false, true}; return true;    // halfka-hm-split
        case 4: s = {45, 1629, 40, true, true, true}; return true;     // halfka-hm-merged
        default: return false;
    }
}

struct Ctx {
    int bucket;
    bool mirror;
};

Ctx ctx_of(const Spec& s, int king_sq, int persp) {
    const int ki = persp_sq(king_sq, persp);
    if (!s.mirror) return {ki, false};
    const int file = ki / 9, rank = ki % 9;
    const int fm = file >= 5 ? 8 - file : file;
    return {fm * 9 + rank, file >= 5};
}

int pack(const Spec& s, int bp, bool mirror) {
    int pp = bp;
    if (mirror && pp >= kFE_HAND_END) {
        const int rel = pp - kFE_HAND_END;
        const int pi = rel / 81, sq = rel % 81;
        pp = kFE_HAND_END + pi * 81 + (8 - sq / 9) * 9 + sq % 9;
    }
    if (s.fold_enemy && pp >= kE_KING) pp -= 81;
    return pp;
}

int board_bp(int pt, int color, int sq, int persp) {
    if (pt == kNone || pt == kKing) return 0;
    return kPieceBase[pt][color == persp ? 1 : 0] + persp_sq(sq, persp);
}

int hand_bp(int persp, int owner, int hi, int count) {
    if (count == 0) return 0;
    return kHandBase[hi][owner == persp ? 1 : 0] + count - 1;
}

// for_each_board_piece: BOARD_PIECE_TYPES x (Black, White) x ascending square
template <class F>
void each_board_piece(const Board& b, F f) {
    for (int t = 0; t < 13; ++t)
        for (int c = 0; c < 2; ++c)
            for (int sq = 0; sq < 81; ++sq)
                if (b.type[sq] == kBoardTypes[t] && b.color[sq] == c) f(kBoardTypes[t], c, sq);
}

int extract(const Spec& s, const Board& b, int32_t* so, int32_t* no, int cap) {
    const int stm = b.stm, nstm = 1 - stm;
    const int ks = b.king[stm], kn = b.king[nstm];
    if (ks >= 81 || kn >= 81) return 0;
    const Ctx cs = ctx_of(s, ks, stm), cn = ctx_of(s, kn, nstm);
    int count = 0;
    auto emit = [&](int bs, int bn) {
        if (count < cap) {
            so[count] = cs.bucket * s.piece_inputs + pack(s, bs, cs.mirror);
            no[count] = cn.bucket * s.piece_inputs + pack(s, bn, cn.mirror);
        }
        ++count;
    };
    each_board_piece(b, [&](int pt, int c, int sq) { emit(board_bp(pt, c, sq, stm), board_bp(pt, c, sq, nstm)); });
    if (s.emit_king) {
        emit(kF_KING + persp_sq(ks, stm), kF_KING + persp_sq(kn, nstm));
        emit(kE_KING + persp_sq(kn, stm), kE_KING + persp_sq(ks, nstm));
    }
    for (int owner = 0; owner < 2; ++owner)
        for (int hi = 0; hi < 7; ++hi)
            for (int i = 1; i <= b.hand[owner][hi]; ++i) {
                const int bs = hand_bp(stm, owner, hi, i);
                if (bs != 0) emit(bs, hand_bp(nstm, owner, hi, i));
            }
    return count < cap ? count : cap;
}

int kingrank9(const Board& b) {
    int fk, ek;
    // Square::inverse is u8 arithmetic (wraps in a release build for an
    // invalid king square)
    if (b.stm == 0) { fk = b.king[0]; ek = (uint8_t)(80 - b.king[1]); }
    else { fk = (uint8_t)(80 - b.king[1]); ek = b.king[0]; }
    return (fk % 9) / 3 * 3 + (ek % 9) / 3;
}

float progress(const Board& b, const float* w) {
    if (b.king[0] >= 81 || b.king[1] >= 81) return 1.0f / (1.0f + expf(-0.0f));
    const int sbk = b.king[0], swk = 80 - b.king[1];
    float sum = 0.0f;
    each_board_piece(b, [&](int pt, int c, int sq) {
        const int bb = board_bp(pt, c, sq, 0);
        if (bb != 0) sum += w[sbk * kFE_OLD_END + bb];
        const int bw = board_bp(pt, c, sq, 1);
        if (bw != 0) sum += w[swk * kFE_OLD_END + bw];
    });
    for (int owner = 0; owner < 2; ++owner)
        for (int hi = 0; hi < 7; ++hi)
            for (int i = 1; i <= b.hand[owner][hi]; ++i) {
                const int bb = hand_bp(0, owner, hi, i);
                if (bb != 0) sum += w[sbk * kFE_OLD_END + bb];
                const int bw = hand_bp(1, owner, hi, i);
                if (bw != 0) sum += w[swk * kFE_OLD_END + bw];
            }
    float p = 1.0f / (1.0f + expf(-sum));
    return p < 0.0f ? 0.0f : (p > 1.0f ? 1.0f : p);
}

}  // namespace

extern "C" {

// Shape of a feature set: king buckets, piece inputs, ft_in, max_active.
int orc_feature_set_info(int fs, int32_t* out4) {
    Spec s;
    if (!spec_of(fs, s)) return -1;
    out4[0] = s.king_buckets;
    out4[1] = s.piece_inputs;
    out4[2] = s.king_buckets * s.piece_inputs;
    out4[3] = s.max_active;
    return 0;
}

// Decoded board of each record: type[81], color[81], hand[2][7], stm, kings,
// score, result, ply packed into int32 rows of 81+81+14+6 = 182 values.
void orc_psv_decode(const uint8_t* psv, int64_t n, int32_t* out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        Board b;
        decode(psv + 40 * r, b);
        int32_t* o = out + 182 * r;
        for (int i = 0; i < 81; ++i) o[i] = b.type[i];
        for (int i = 0; i < 81; ++i) o[81 + i] = b.color[i];
        for (int c = 0; c < 2; ++c)
            for (int i = 0; i < 7; ++i) o[162 + 7 * c + i] = b.hand[c][i];
        o[176] = b.stm;
        o[177] = b.king[0];
        o[178] = b.king[1];
        o[179] = b.score;
        o[180] = b.result;
        o[181] = b.ply;
    }
}

static void board_from_row(const int32_t* o, Board& b) {
    std::memset(&b, 0, sizeof(b));
    for (int i = 0; i < 81; ++i) b.type[i] = (int8_t)o[i];
    for (int i = 0; i < 81; ++i) b.color[i] = (int8_t)o[81 + i];
    for (int c = 0; c < 2; ++c)
        for (int i = 0; i < 7; ++i) b.hand[c][i] = (uint8_t)o[162 + 7 * c + i];
    b.stm = o[176];
    b.king[0] = o[177];
    b.king[1] = o[178];
    b.score = (int16_t)o[179];
    b.result = (int8_t)o[180];
    b.ply = (uint16_t)o[181];
}

static void fill(const Spec& s, const Board& b, int64_t r, int bucket_mode, int num_buckets,
                 const float* weights, int32_t* stm, int32_t* nstm, int32_t* nnz, int32_t* bucket,
                 float* score, float* wdl, float* prog) {
    const int ma = s.max_active;
    int32_t* so = stm + r * ma;
    int32_t* no = nstm + r * ma;
    for (int i = 0; i < ma; ++i) so[i] = no[i] = -1;
    nnz[r] = extract(s, b, so, no, ma);
    score[r] = (float)b.score;
    wdl[r] = b.result > 0 ? 1.0f : (b.result < 0 ? 0.0f : 0.5f);
    int bk = 0;
    float p = 0.0f;
    if (bucket_mode == 1) {
        bk = kingrank9(b);
    } else if (bucket_mode == 2) {
        p = progress(b, weights);
        int raw = (int)std::floor(p * (float)num_buckets);
        bk = raw < 0 ? 0 : (raw > num_buckets - 1 ? num_buckets - 1 : raw);
    }
    bucket[r] = bk;
    if (prog) prog[r] = p;
}

// Batch::push_decoded for each record: index rows [n][max_active] (-1 past
// nnz), nnz, score, wdl; bucket by mode (0 none -> 0, 1 kingrank9,
// 2 progress with num_buckets and f32 weights).
int orc_psv_to_batch(const uint8_t* psv, int64_t n, int fs, int bucket_mode, int num_buckets,
                     const float* weights, int32_t* stm, int32_t* nstm, int32_t* nnz,
                     int32_t* bucket, float* score, float* wdl, float* prog) {
    Spec s;
    if (!spec_of(fs, s)) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        Board b;
        decode(psv + 40 * r, b);
        fill(s, b, r, bucket_mode, num_buckets, weights, stm, nstm, nnz, bucket, score, wdl, prog);
    }
    return 0;
}

// The same for already decoded boards, in the 182-value row layout of
// orc_psv_decode (boards that a PSV record cannot hold, e.g. without the
// full piece set).
int orc_boards_to_batch(const int32_t* boards, int64_t n, int fs, int bucket_mode, int num_buckets,
                        const float* weights, int32_t* stm, int32_t* nstm, int32_t* nnz,
                        int32_t* bucket, float* score, float* wdl, float* prog) {
    Spec s;
    if (!spec_of(fs, s)) return -1;
    for (int64_t r = 0; r < n; ++r) {
        Board b;
        board_from_row(boards + 182 * r, b);
        fill(s, b, r, bucket_mode, num_buckets, weights, stm, nstm, nnz, bucket, score, wdl, prog);
    }
    return 0;
}

// glibc expf over an array (what Rust's f32::exp evaluates on linux-gnu).
void orc_expf(const float* x, float* y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

// KP-absolute active indices of one record, in progress-sum order; returns count.
int orc_kpabs_indices(const uint8_t* rec, int32_t* out, int cap) {
    Board b;
    decode(rec, b);
    if (b.king[0] >= 81 || b.king[1] >= 81) return 0;
    const int sbk = b.king[0], swk = 80 - b.king[1];
    int n = 0;
    auto put = [&](int v) { if (n < cap) out[n] = v; ++n; };
    each_board_piece(b, [&](int pt, int c, int sq) {
        const int bb = board_bp(pt, c, sq, 0);
        if (bb != 0) put(sbk * kFE_OLD_END + bb);
        const int bw = board_bp(pt, c, sq, 1);
        if (bw != 0) put(swk * kFE_OLD_END + bw);
    });
    for (int owner = 0; owner < 2; ++owner)
        for (int hi = 0; hi < 7; ++hi)
            for (int i = 1; i <= b.hand[owner][hi]; ++i) {
                const int bb = hand_bp(0, owner, hi, i);
                if (bb != 0) put(sbk * kFE_OLD_END + bb);
                const int bw = hand_bp(1, owner, hi, i);
                if (bw != 0) put(swk * kFE_OLD_END + bw);
            }
    return n;
}

}  // extern "C"
