// PSV records -> training batch on the GPU: Huffman decode, feature-index
// extraction for the five feature sets, kingrank9 / KP-absolute progress
// buckets, score and WDL.
//
// The reference does this on CPU dataloader threads (Batch::push_decoded,
// crates/nnue-train/src/dataloader.rs:444-497, over
// ShogiBoard::from_packed_sfen, crates/shogi-format/src/packed_sfen.rs:387-449,
// and FeatureSetSpec::extract_active_features,
// crates/shogi-features/src/feature_set.rs:655-810).  Here one thread decodes
// one 40-byte record, so the host uploads 40 bytes per position instead of
// two index rows.  Every integer result is the reference's: the emission
// order is for_each_board_piece's (BOARD_PIECE_TYPES x (black, white) x
// ascending square, packed_sfen.rs:493-540), then the two kings, then the
// hands ((black, white) x HAND_PIECE_TYPES x count).
//
// The progress bucket (ShogiProgressKPAbs::bucket_board,
// crates/shogi-features/src/progress_kpabs.rs:140-170) sums the f32 weights
// in the reference's order and evaluates exp with ref_expf(), a restatement of
// glibc's expf method (2^(k/32) table + cubic polynomial in double, the
// FMA-contracted build that glibc selects on x86-64 CPUs with FMA), which
// the reference's f32::exp calls on linux-gnu; the result equals glibc's on
// every non-NaN float.
#include "psv_kernels.hpp"

#include "common.hpp"
#include "ref_expf.hpp"

namespace tatara {

namespace {

__global__ void expf_kernel(const float* __restrict__ x, float* __restrict__ y, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = ref_expf(x[i]);
}

// ---------------------------------------------------------------------------
// pieces and BonaPiece (crates/shogi-format/src/{types,bona_piece}.rs)
// ---------------------------------------------------------------------------
enum : int { kNone = 0, kPawn, kLance, kKnight, kSilver, kBishop, kRook, kGold, kKing,
             kProPawn, kProLance, kProKnight, kProSilver, kHorse, kDragon };
constexpr int kFeHandEnd = 90, kFeOldEnd = 1548, kFKing = 1548, kEKing = 1629;

// board piece base offset [piece type][is_friend] (bona_piece.rs PIECE_BASE)
__constant__ int16_t c_piece_base[15][2] = {
    {0, 0},       {171, 90},    {333, 252},  {495, 414},  {657, 576},
    {981, 900},   {1305, 1224}, {819, 738},  {0, 0},      {819, 738},
    {819, 738},   {819, 738},   {819, 738},  {1143, 1062}, {1467, 1386}};
// hand base offset [hand index][is_friend], hand order pawn, lance, knight,
// silver, gold, bishop, rook
__constant__ int16_t c_hand_base[7][2] = {{20, 1},  {44, 39}, {54, 49}, {64, 59},
                                          {74, 69}, {82, 79}, {88, 85}};
// emission rank of a board piece type (BOARD_PIECE_TYPES order), -1 for none/king
__constant__ int8_t c_type_rank[15] = {-1, 0, 1, 2, 3, 5, 6, 4, -1, 7, 8, 9, 10, 11, 12};
// Huffman id -> piece type (0 none, pawn, lance, knight, silver, bishop, rook, gold)
__constant__ int8_t c_huff_type[8] = {kNone, kPawn, kLance, kKnight, kSilver, kBishop, kRook, kGold};
// hand index of a Huffman id (-1 for none)
__constant__ int8_t c_huff_hand[8] = {-1, 0, 1, 2, 3, 5, 6, 4};

__device__ __forceinline__ int promote(int pt) {
    return (pt >= kPawn && pt <= kSilver) ? pt + 8 : (pt == kBishop ? kHorse : (pt == kRook ? kDragon : pt));
}

// Decodes one board square's Huffman code from the low bits of v (LSB first).
// Returns the Huffman id and sets the code length.
__device__ __forceinline__ int board_code(uint32_t v, int& len) {
    if ((v & 1u) == 0) { len = 1; return 0; }          // 0: none
    if ((v & 3u) == 1u) { len = 2; return 1; }         // 01: pawn
    if ((v & 15u) == 3u) { len = 4; return 2; }        // 0011: lance
    if ((v & 15u) == 11u) { len = 4; return 3; }       // 1011: knight
    if ((v & 15u) == 7u) { len = 4; return 4; }        // 0111: silver
    if ((v & 31u) == 15u) { len = 5; return 7; }       // 01111: gold
    if ((v & 63u) == 31u) { len = 6; return 5; }       // 011111: bishop
    len = 6;                                           // 111111: rook
    return 6;
}

// A hand entry's code: the board code without its first (always 1) bit,
// pawn being the single bit 0.
__device__ __forceinline__ int hand_code(uint32_t v, int& len) {
    if ((v & 1u) == 0) { len = 1; return 1; }          // 0: pawn
    if ((v & 7u) == 1u) { len = 3; return 2; }         // 001: lance
    if ((v & 7u) == 5u) { len = 3; return 3; }         // 101: knight
    if ((v & 7u) == 3u) { len = 3; return 4; }         // 011: silver
    if ((v & 15u) == 7u) { len = 4; return 7; }        // 0111: gold
    if ((v & 31u) == 15u) { len = 5; return 5; }       // 01111: bishop
    len = 5;                                           // 11111: rook
    return 6;
}

struct Bits {
    const uint32_t* w;  // 8 words in LDS, stride kPsvThreads
    int cur;
    // n <= 25 bits at the cursor, zero past bit 256
    __device__ uint32_t peek(int n) const {
        if (cur >= 256) return 0u;
        const int wi = cur >> 5, sh = cur & 31;
        uint64_t v = w[wi * kPsvThreads];
        if (wi + 1 < 8) v |= (uint64_t)w[(wi + 1) * kPsvThreads] << 32;
        return (uint32_t)(v >> sh) & ((1u << n) - 1u);
    }
    __device__ int bit() {
        const int b = (int)peek(1);
        ++cur;
        return b;
    }
};

__device__ __forceinline__ int persp_sq(int sq, int persp) { return persp == 0 ? sq : 80 - sq; }

__device__ __forceinline__ int pack_bp(int bp, bool mirror, bool fold) {
    int pp = bp;
    if (mirror && pp >= kFeHandEnd) {
        const int rel = pp - kFeHandEnd;
        const int pi = rel / 81, s = rel % 81;
        pp = kFeHandEnd + pi * 81 + (8 - s / 9) * 9 + s % 9;
    }
    if (fold && pp >= kEKing) pp -= 81;
    return pp;
}

__device__ __forceinline__ void psv_record(const PsvArgs& a, uint32_t r, int t, uint32_t* s_w, uint8_t* s_board,
                                           uint8_t* s_off, uint8_t* s_slot, int32_t* so, int32_t* no) {
    constexpr int T = kPsvThreads;
    const uint8_t* rec = a.psv + (uint64_t)r * 40;
    const uint32_t* rec32 = reinterpret_cast<const uint32_t*>(rec);
#pragma unroll
    for (int k = 0; k < 8; ++k) s_w[k * T + t] = rec32[k];
    const uint32_t tail0 = rec32[8], tail1 = rec32[9];
    const int16_t score = (int16_t)(tail0 & 0xffffu);
    const int8_t result = (int8_t)(tail1 >> 16 & 0xffu);

    // ---- decode (ShogiBoard::from_packed_sfen) ----
    Bits bs{s_w + t, 0};
    const int stm = bs.bit();
    int king[2] = {0, 0};
    for (int c = 0; c < 2; ++c)
        for (int i = 0; i < 7; ++i) king[c] |= bs.bit() << i;
    uint8_t hand[2][7];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int i = 0; i < 7; ++i) hand[c][i] = 0;
    for (int sq = 0; sq < 81; ++sq) {
        uint8_t v = kNone;
        if (sq == king[1]) {  // placed after the black king, as the reference does
            v = kKing | (1 << 4);
        } else if (sq == king[0]) {
            v = kKing;
        } else {
            int len;
            const int h = board_code(bs.peek(6), len);
            bs.cur += len;
            if (h != 0) {
                const int prom = h != 7 ? bs.bit() : 0;
                const int col = bs.bit();
                const int pt = c_huff_type[h];
                v = (uint8_t)((prom ? promote(pt) : pt) | (col << 4));
            }
        }
        s_board[sq * T + t] = v;
    }
    while (bs.cur < 256) {
        int len;
        const int h = hand_code(bs.peek(5), len);
        bs.cur += len;
        const int box = h != 7 ? bs.bit() : 0;
        const int col = bs.bit();
        if (!box) hand[col][c_huff_hand[h]] += 1;
    }

    // ---- board pieces in emission order (for_each_board_piece) ----
    for (int b = 0; b < 26; ++b) s_off[b * T + t] = 0;
    for (int sq = 0; sq < 81; ++sq) {
        const int v = s_board[sq * T + t];
        const int rk = c_type_rank[v & 15];
        if (rk >= 0) s_off[(rk * 2 + (v >> 4)) * T + t] += 1;
    }
    int n_board = 0;
    for (int b = 0; b < 26; ++b) {
        const int c = s_off[b * T + t];
        s_off[b * T + t] = (uint8_t)n_board;
        n_board += c;
    }
    for (int sq = 0; sq < 81; ++sq) {
        const int v = s_board[sq * T + t];
        const int rk = c_type_rank[v & 15];
        if (rk < 0) continue;
        const int b = rk * 2 + (v >> 4);
        const int slot = s_off[b * T + t];
        s_off[b * T + t] = (uint8_t)(slot + 1);
        s_slot[slot * T + t] = (uint8_t)sq;
    }

    // ---- feature indices (extract_active_features) ----
    const int cap = a.max_active;
    int count = 0;
    const bool kings_ok = king[0] < 81 && king[1] < 81;
    if (kings_ok) {
        const int nstm = 1 - stm;
        const int ks = king[stm], kn = king[nstm];
        int bucket_s, bucket_n;
        bool mir_s = false, mir_n = false;
        {
            const int ki = persp_sq(ks, stm), kj = persp_sq(kn, nstm);
            if (a.mirror) {
                const int fi = ki / 9, fj = kj / 9;
                mir_s = fi >= 5;
                mir_n = fj >= 5;
                bucket_s = (mir_s ? 8 - fi : fi) * 9 + ki % 9;
                bucket_n = (mir_n ? 8 - fj : fj) * 9 + kj % 9;
            } else {
                bucket_s = ki;
                bucket_n = kj;
            }
        }
        const int base_s = bucket_s * a.piece_inputs, base_n = bucket_n * a.piece_inputs;
        const bool fold = a.fold_enemy != 0;
        auto emit = [&](int bp_s, int bp_n) {
            if (count < cap) {
                so[count] = base_s + pack_bp(bp_s, mir_s, fold);
                no[count] = base_n + pack_bp(bp_n, mir_n, fold);
            }
            ++count;
        };
        for (int k = 0; k < n_board; ++k) {
            const int sq = s_slot[k * T + t];
            const int v = s_board[sq * T + t];
            const int pt = v & 15, col = v >> 4;
            emit(c_piece_base[pt][col == stm] + persp_sq(sq, stm),
                 c_piece_base[pt][col == nstm] + persp_sq(sq, nstm));
        }
        if (a.emit_king) {
            emit(kFKing + persp_sq(ks, stm), kFKing + persp_sq(kn, nstm));
            emit(kEKing + persp_sq(kn, stm), kEKing + persp_sq(ks, nstm));
        }
        for (int owner = 0; owner < 2; ++owner)
            for (int hi = 0; hi < 7; ++hi)
                for (int i = 1; i <= hand[owner][hi]; ++i)
                    emit(c_hand_base[hi][owner == stm] + i - 1, c_hand_base[hi][owner == nstm] + i - 1);
    }
    const int nv = count < cap ? count : cap;
    for (int k = nv; k < cap; ++k) {
        so[k] = -1;
        no[k] = -1;
    }
    a.nnz[r] = nv;
    a.score[r] = (float)score;
    a.wdl[r] = result > 0 ? 1.0f : (result < 0 ? 0.0f : 0.5f);

    // ---- bucket (BucketMode::bucket_board) ----
    int bucket = 0;
    if (a.bucket_mode == 1) {
        // kingrank9_bucket_board: ranks from the side to move's view; the
        // u8 square arithmetic wraps as the reference's release build does
        // (only reachable with an invalid king square)
        int fk, ek;
        if (stm == 0) {
            fk = king[0];
            ek = (uint8_t)(80 - king[1]);
        } else {
            fk = (uint8_t)(80 - king[1]);
            ek = king[0];
        }
        bucket = (fk % 9) / 3 * 3 + (ek % 9) / 3;
    } else if (a.bucket_mode == 2) {
        float sum = 0.0f;
        if (kings_ok) {
            const float* w = a.weights;
            const int sbk = king[0] * kFeOldEnd, swk = (80 - king[1]) * kFeOldEnd;
            for (int k = 0; k < n_board; ++k) {
                const int sq = s_slot[k * T + t];
                const int v = s_board[sq * T + t];
                const int pt = v & 15, col = v >> 4;
                sum += w[sbk + c_piece_base[pt][col == 0] + sq];
                sum += w[swk + c_piece_base[pt][col == 1] + 80 - sq];
            }
            for (int owner = 0; owner < 2; ++owner)
                for (int hi = 0; hi < 7; ++hi)
                    for (int i = 1; i <= hand[owner][hi]; ++i) {
                        sum += w[sbk + c_hand_base[hi][owner == 0] + i - 1];
                        sum += w[swk + c_hand_base[hi][owner == 1] + i - 1];
                    }
        }
        float p = 1.0f / (1.0f + ref_expf(-sum));
        p = p < 0.0f ? 0.0f : (p > 1.0f ? 1.0f : p);
        const int raw = (int)floorf(p * (float)a.num_buckets);
        bucket = raw < 0 ? 0 : (raw > a.num_buckets - 1 ? a.num_buckets - 1 : raw);
        if (a.progress) a.progress[r] = p;
    }
    if (a.bucket) a.bucket[r] = bucket;
}

// The per-record work (one thread per record) ends with the record's two
// index rows in LDS; the workgroup then writes its records' rows, which are
// consecutive in memory, as whole rows per store instruction (scattered
// 4-byte stores of one row per lane measured 6.6x the bytes written).
constexpr int kPsvMaxActive = 40;  // the largest feature set's (halfka*: 40, halfkp: 38)
constexpr int kPsvRowPad = kPsvMaxActive + 1;  // odd LDS row stride: no bank conflicts between lanes' rows

__global__ __launch_bounds__(kPsvThreads) void psv_to_batch_kernel(PsvArgs a) {
    constexpr int T = kPsvThreads;
    __shared__ uint32_t s_w[8 * T];          // the 256 position bits of each thread's record
    __shared__ uint8_t s_board[81 * T];      // piece type | colour << 4
    __shared__ uint8_t s_off[26 * T];        // per (type rank, colour): count, then next slot
    __shared__ uint8_t s_slot[81 * T];       // square of each board piece in emission order
    __shared__ int32_t s_idx[2][T * kPsvRowPad];  // the records' stm / nstm index rows
    const int t = threadIdx.x;
    const uint32_t r0 = blockIdx.x * T, r = r0 + t;
    if (r < a.n) psv_record(a, r, t, s_w, s_board, s_off, s_slot, s_idx[0] + t * kPsvRowPad,
                            s_idx[1] + t * kPsvRowPad);
    __syncthreads();
    // row k of the workgroup: lanes j < max_active store its column j
    const uint32_t nrec = a.n - r0 < (uint32_t)T ? a.n - r0 : (uint32_t)T;
    const int cap = a.max_active;
    for (uint32_t k = 0; k < nrec; ++k)
        if (t < cap) {
            a.stm[(uint64_t)(r0 + k) * cap + t] = s_idx[0][k * kPsvRowPad + t];
            a.nstm[(uint64_t)(r0 + k) * cap + t] = s_idx[1][k * kPsvRowPad + t];
        }
}

}  // namespace

int32_t feature_set_shape(int32_t fs, FeatureSetShape& s) {
    switch (fs) {
        case 0: s = {81, 1548, 38, 0, 0, 0, 0x5D69D5B8u}; return kOk;   // halfkp
        case 1: s = {81, 1710, 40, 1, 0, 0, 0x5F134CB8u}; return kOk;   // halfka-split
        case 2: s = {81, 1629, 40, 1, 1, 0, 0xACD68C97u}; return kOk;   // halfka-merged
        case 3: s = {45, 1710, 40, 1, 0, 1, 0x2A46AC09u}; return kOk;   // halfka-hm-split
        case 4: s = {45, 1629, 40, 1, 1, 1, 0x7F134CB8u}; return kOk;   // halfka-hm-merged
        default: TATARA_REQUIRE(false, "unknown feature set");
    }
}

int32_t launch_psv_to_batch(const PsvArgs& a, hipStream_t stream) {
    TATARA_REQUIRE(a.bucket_mode >= 0 && a.bucket_mode <= 2, "unknown bucket mode");
    if (a.bucket_mode == 2) {
        TATARA_REQUIRE(a.num_buckets >= 1 && a.num_buckets <= 256, "num_buckets must be in [1, 256]");
        TATARA_REQUIRE(a.weights, "progress buckets need the KP-absolute weights");
    }
    TATARA_REQUIRE(a.max_active > 0 && a.max_active <= kPsvMaxActive && a.piece_inputs > 0, "feature set shape");
    if (a.n == 0) return kOk;
    psv_to_batch_kernel<<<ceil_div(a.n, kPsvThreads), kPsvThreads, 0, stream>>>(a);
    TATARA_LAUNCHED("psv_to_batch");
    return kOk;
}

int32_t launch_expf(const float* x, float* y, uint64_t n, hipStream_t stream) {
    if (n == 0) return kOk;
    expf_kernel<<<ceil_div(n, 256), 256, 0, stream>>>(x, y, n);
    TATARA_LAUNCHED("expf");
    return kOk;
}

}  // namespace tatara
