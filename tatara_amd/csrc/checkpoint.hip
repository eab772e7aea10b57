// Raw resume checkpoints (RNRC, version 8) of the LayerStack and Simple
// trainers: the header writer and the validating reader that accepts
// versions 1..8 (bins/nnue_train/src/ckpt.rs:18-110, 268-612), and the
// trainers' save / load of every parameter group's w, m, v and slow
// (ckpt.rs:614-757; trainer_layerstack.rs:1440-1726, trainer_simple.rs:
// 2870-2992).  Host code only.
//
// File layout (little-endian): "RNRC", u32 version, feature-set header
// (u32 name length + name, u64 train ft_in, u64 ft_out, u64 max_active,
// u8 factorizer flag, u32 feature hash), u32 run-id length + run id, u32
// arch-kind length + name, u32 bucket-mode length + name, u64 topology count
// + u64 dims, u64 superbatch, u64 step count, u64 LR horizon (0 = none),
// u64 group count; then per group u64 len and four f32 arrays w, m, v, slow.
// f16 moments are written as their true f32 values (f16 / scale) and
// re-quantised on load (MomentBuf::to_host_f32 / from_host_f32,
// trainer_common.rs:78-127).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "checkpoint.hpp"
#include "common.hpp"
#include "psv_kernels.hpp"
#include "trainer_base.hpp"

namespace tatara {

namespace {

constexpr char kMagic[4] = {'R', 'N', 'R', 'C'};
constexpr uint32_t kVersion = 8;
constexpr uint64_t kMaxName = 256;   // name length fields above this are implausible
constexpr uint64_t kMaxRunId = 256;  // MAX_RUN_ID_BYTES

const char* const kFeatureSetNames[] = {"halfkp", "halfka-split", "halfka-merged", "halfka-hm-split",
                                        "halfka-hm-merged"};

void put_u32(std::string& b, uint32_t x) {
    for (int i = 0; i < 4; ++i) b.push_back((char)((x >> (8 * i)) & 0xff));
}
void put_u64(std::string& b, uint64_t x) {
    for (int i = 0; i < 8; ++i) b.push_back((char)((x >> (8 * i)) & 0xff));
}
void put_str(std::string& b, const std::string& s) {
    put_u32(b, (uint32_t)s.size());
    b += s;
}

bool valid_utf8(const std::string& s) {
    size_t i = 0;
    const size_t n = s.size();
    while (i < n) {
        const unsigned char c = (unsigned char)s[i];
        int len;
        uint32_t cp;
        if (c < 0x80) {
            ++i;
            continue;
        } else if ((c & 0xe0) == 0xc0) {
            len = 2;
            cp = c & 0x1f;
        } else if ((c & 0xf0) == 0xe0) {
            len = 3;
            cp = c & 0x0f;
        } else if ((c & 0xf8) == 0xf0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (int k = 1; k < len; ++k) {
            const unsigned char d = (unsigned char)s[i + k];
            if ((d & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (d & 0x3f);
        }
        // overlong forms, surrogates and values past U+10FFFF are not UTF-8
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
            (cp >= 0xd800 && cp <= 0xdfff) || cp > 0x10ffff)
            return false;
        i += len;
    }
    return true;
}

// A byte source with read_exact semantics: a short read is "truncated while
// reading {what}" (read_exact_or_invalid, ckpt.rs:778-796).
class Reader {
   public:
    virtual ~Reader() = default;
    virtual bool read(void* dst, uint64_t n) = 0;

    int32_t exact(void* dst, uint64_t n, const char* what) {
        if (!read(dst, n)) return invalid(std::string("raw checkpoint truncated while reading ") + what);
        return kOk;
    }
    int32_t u32(uint32_t& x, const char* what) {
        uint8_t b[4];
        int32_t st = exact(b, 4, what);
        if (st) return st;
        x = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
        return kOk;
    }
    int32_t u64(uint64_t& x, const char* what) {
        uint8_t b[8];
        int32_t st = exact(b, 8, what);
        if (st) return st;
        x = 0;
        for (int i = 7; i >= 0; --i) x = (x << 8) | b[i];
        return kOk;
    }
    // u32 length (<= limit, else "{what} length {n} is implausible (max {limit})")
    // followed by that many bytes of UTF-8.
    int32_t str(std::string& s, const char* what, uint64_t limit, const char* len_what) {
        uint32_t n = 0;
        int32_t st = u32(n, len_what);
        if (st) return st;
        if (n > limit)
            return invalid("raw checkpoint " + std::string(what) + " length " + std::to_string(n) +
                           " is implausible (max " + std::to_string(limit) + ")");
        s.assign(n, '\0');
        if (n && (st = exact(&s[0], n, what))) return st;
        if (!valid_utf8(s)) return invalid("raw checkpoint " + std::string(what) + " is not valid UTF-8");
        return kOk;
    }

    static int32_t invalid(const std::string& msg) {
        set_error("invalid data: " + msg);
        return kErrInvalid;
    }
};

class MemReader : public Reader {
   public:
    MemReader(const uint8_t* p, uint64_t n) : p_(p), n_(n) {}
    bool read(void* dst, uint64_t n) override {
        if (n > n_ - off_) return false;
        std::memcpy(dst, p_ + off_, n);
        off_ += n;
        return true;
    }
    uint64_t offset() const { return off_; }

   private:
    const uint8_t* p_;
    uint64_t n_, off_ = 0;
};

class FileReader : public Reader {
   public:
    explicit FileReader(FILE* f) : f_(f) {}
    bool read(void* dst, uint64_t n) override {
        if (n == 0) return true;
        const size_t got = std::fread(dst, 1, n, f_);
        off_ += got;
        return got == n;
    }
    uint64_t offset() const { return off_; }

   private:
    FILE* f_;
    uint64_t off_ = 0;
};

std::string hex32(uint32_t x) {
    char b[16];
    std::snprintf(b, sizeof b, "%#010x", x);
    return b;
}

}  // namespace

int32_t ckpt_arch_from_c(const TataraCkptArch& c, CkptArch& a) {
    FeatureSetShape s{};
    int32_t st = feature_set_shape(c.feature_set, s);
    if (st) return st;
    TATARA_REQUIRE(c.arch == TATARA_ARCH_LAYERSTACK || c.arch == TATARA_ARCH_SIMPLE, "unknown arch");
    a.fs_name = kFeatureSetNames[c.feature_set];
    const uint64_t ft_in = (uint64_t)s.king_buckets * s.piece_inputs;
    a.factorize = c.ft_factorize != 0;
    a.train_ft_in = ft_in + (a.factorize ? (uint64_t)s.piece_inputs : 0);
    a.ft_out = c.ft_out;
    a.max_active = (uint64_t)s.max_active;
    a.feature_hash = s.feature_hash;
    a.arch_kind = c.arch == TATARA_ARCH_LAYERSTACK ? "layerstack" : "simple";
    a.has_bucket_mode = c.arch == TATARA_ARCH_LAYERSTACK;
    if (c.arch == TATARA_ARCH_LAYERSTACK) {
        TATARA_REQUIRE(c.bucket_mode == TATARA_BUCKET_KINGRANK9 || c.bucket_mode == TATARA_BUCKET_PROGRESS_KPABS,
                       "a LayerStack checkpoint names its bucket mode (kingrank9 or progress8kpabs)");
        a.bucket_mode = c.bucket_mode == TATARA_BUCKET_KINGRANK9 ? "kingrank9" : "progress8kpabs";
        // layerstack_topology (ckpt.rs:186-199)
        a.topology = {c.ft_out, c.l1_out, c.l2_out, c.num_buckets};
    } else {
        TATARA_REQUIRE(c.bucket_mode == TATARA_BUCKET_NONE, "a Simple checkpoint has no bucket mode");
        a.bucket_mode.clear();
        a.topology = {c.ft_out, c.l1_out, c.l2_out};  // trainer_simple.rs:2881-2885
    }
    return kOk;
}

// write_raw_ckpt_header (ckpt.rs:269-312): always the current version.
std::string ckpt_header_bytes(const CkptArch& a, const std::string& run_id, uint64_t superbatch,
                              uint64_t step_count, uint64_t lr_horizon, uint64_t num_groups) {
    std::string b;
    b.append(kMagic, 4);
    put_u32(b, kVersion);
    put_str(b, a.fs_name);
    put_u64(b, a.train_ft_in);
    put_u64(b, a.ft_out);
    put_u64(b, a.max_active);
    b.push_back(a.factorize ? 1 : 0);
    put_u32(b, a.feature_hash);
    put_str(b, run_id);
    put_str(b, a.arch_kind);
    put_str(b, a.bucket_mode);
    put_u64(b, a.topology.size());
    for (uint64_t d : a.topology) put_u64(b, d);
    put_u64(b, superbatch);
    put_u64(b, step_count);
    put_u64(b, lr_horizon);
    put_u64(b, num_groups);
    return b;
}

namespace {

// read_raw_ckpt_header (ckpt.rs:322-612) against the expected arch.
int32_t read_header(Reader& r, const CkptArch& want, CkptHeader& h) {
    int32_t st;
    char magic[4];
    if ((st = r.exact(magic, 4, "magic"))) return st;
    if (std::memcmp(magic, kMagic, 4) != 0) return Reader::invalid("raw checkpoint magic mismatch");
    uint32_t version = 0;
    if ((st = r.u32(version, "version"))) return st;
    if (version == 0 || version > kVersion)
        return Reader::invalid("raw checkpoint version " + std::to_string(version) +
                               " is not supported (this build reads 1..=" + std::to_string(kVersion) + ")");
    h.version = version;

    if (version >= 2) {
        std::string fs;
        if ((st = r.str(fs, "feature set name", kMaxName, "feature set name length"))) return st;
        uint64_t ft_in = 0, ft_out = 0, max_active = 0;
        if ((st = r.u64(ft_in, "ft_in")) || (st = r.u64(ft_out, "ft_out")) || (st = r.u64(max_active, "max_active")))
            return st;
        bool factorize = false;
        if (version >= 6) {
            uint8_t f = 0;
            if ((st = r.exact(&f, 1, "ft_factorize flag"))) return st;
            factorize = f != 0;
        }
        bool has_hash = false;
        uint32_t hash = 0;
        if (version >= 7) {
            if ((st = r.u32(hash, "feature hash"))) return st;
            has_hash = true;
        }
        if (fs != want.fs_name)
            return Reader::invalid("raw checkpoint feature set mismatch: checkpoint is '" + fs + "', requested '" +
                                   want.fs_name + "' (cannot resume across feature sets)");
        if (factorize != want.factorize)
            return Reader::invalid(std::string("raw checkpoint ft-factorize mismatch: checkpoint ") +
                                   (factorize ? "true" : "false") + ", requested " +
                                   (want.factorize ? "true" : "false") +
                                   " (cannot resume across --ft-factorize on/off)");
        if (has_hash && hash != want.feature_hash)
            return Reader::invalid("raw checkpoint feature hash mismatch: got " + hex32(hash) + ", want " +
                                   hex32(want.feature_hash));
        if (ft_in != want.train_ft_in)
            return Reader::invalid("raw checkpoint ft_in mismatch: got " + std::to_string(ft_in) + ", want " +
                                   std::to_string(want.train_ft_in));
        if (ft_out != want.ft_out)
            return Reader::invalid("raw checkpoint ft_out mismatch: got " + std::to_string(ft_out) + ", want " +
                                   std::to_string(want.ft_out));
        // a factorized file may record twice the base count (ckpt.rs:419-436)
        const bool legacy = want.factorize && max_active == 2 * want.max_active;
        if (max_active != want.max_active && !legacy)
            return Reader::invalid("raw checkpoint max_active mismatch: got " + std::to_string(max_active) +
                                   ", want " + std::to_string(want.max_active));
    } else if (want.fs_name != "halfka-hm-merged") {
        return Reader::invalid("raw checkpoint version 1 is always 'halfka-hm-merged', requested '" + want.fs_name +
                               "' (cannot resume across feature sets)");
    }

    h.run_id.clear();
    if (version >= 3) {
        if ((st = r.str(h.run_id, "producer run id", kMaxRunId, "producer run id length"))) return st;
    }

    if (version >= 4) {
        std::string arch;
        if ((st = r.str(arch, "arch kind name", kMaxName, "arch kind name length"))) return st;
        if (arch != "layerstack" && arch != "simple")
            return Reader::invalid("raw checkpoint has unknown arch kind '" + arch + "'");
        if (arch != want.arch_kind)
            return Reader::invalid("raw checkpoint arch kind mismatch: checkpoint is '" + arch + "', requested '" +
                                   want.arch_kind + "' (cannot resume across architectures)");
        bool has_mode = false;
        std::string mode;
        if (version >= 8) {
            if ((st = r.str(mode, "bucket mode name", kMaxName, "bucket mode name length"))) return st;
            has_mode = !mode.empty();
        } else if (arch == "layerstack") {
            has_mode = true;
            mode = "progress8kpabs";
        }
        if (has_mode != want.has_bucket_mode || (has_mode && mode != want.bucket_mode)) {
            if (has_mode && want.has_bucket_mode)
                return Reader::invalid("checkpoint bucket mode '" + mode + "' does not match --bucket-mode '" +
                                       want.bucket_mode + "'");
            return Reader::invalid("raw checkpoint bucket mode \"" + (has_mode ? mode : std::string()) +
                                   "\" does not match architecture '" + want.arch_kind + "'");
        }
        uint64_t count = 0;
        if ((st = r.u64(count, "topology dim count"))) return st;
        if (count != want.topology.size())
            return Reader::invalid("raw checkpoint topology dim count " + std::to_string(count) + " != expected " +
                                   std::to_string(want.topology.size()));
        for (size_t i = 0; i < want.topology.size(); ++i) {
            uint64_t d = 0;
            if ((st = r.u64(d, "topology dim"))) return st;
            if (d != want.topology[i])
                return Reader::invalid("raw checkpoint topology dim " + std::to_string(i) + " mismatch: got " +
                                       std::to_string(d) + ", want " + std::to_string(want.topology[i]) +
                                       " (network architecture mismatch)");
        }
    } else if (want.arch_kind != "layerstack") {
        return Reader::invalid("raw checkpoint version " + std::to_string(version) +
                               " predates the arch-kind header and is always 'layerstack', requested '" +
                               want.arch_kind + "' (cannot resume across architectures)");
    } else if (want.bucket_mode != "progress8kpabs") {
        return Reader::invalid("checkpoint bucket mode 'progress8kpabs' does not match --bucket-mode '" +
                               want.bucket_mode + "'");
    }

    if ((st = r.u64(h.superbatch, "superbatch")) || (st = r.u64(h.step_count, "step_count"))) return st;
    h.lr_horizon = 0;
    if (version >= 5 && (st = r.u64(h.lr_horizon, "lr_horizon"))) return st;
    if ((st = r.u64(h.num_groups, "num_groups"))) return st;
    return kOk;
}

void header_to_c(const CkptHeader& h, uint64_t bytes, TataraCkptHeader* out) {
    std::memset(out, 0, sizeof *out);
    out->version = h.version;
    out->superbatch = h.superbatch;
    out->step_count = h.step_count;
    out->lr_horizon = h.lr_horizon;
    out->num_groups = h.num_groups;
    out->header_bytes = bytes;
    std::memcpy(out->run_id, h.run_id.data(), h.run_id.size() < kMaxRunId ? h.run_id.size() : kMaxRunId);
}

struct FileCloser {
    FILE* f = nullptr;
    ~FileCloser() {
        if (f) std::fclose(f);
    }
};

}  // namespace

// save_raw_checkpoint_file (ckpt.rs:614-699): header, then every group in the
// format's order, written to "<path>.tmp" and renamed over path.  A run id
// longer than 256 bytes is omitted, as the reference does.
int32_t save_resume_checkpoint(TrainerBase& t, const char* path, const CkptArch& arch,
                               const std::vector<const char*>& groups, uint64_t superbatch, const char* run_id,
                               uint64_t lr_horizon) {
    std::string rid = run_id ? run_id : "";
    if (rid.size() > kMaxRunId) {
        std::fprintf(stderr, "[tatara] warning: producer run id (%zu bytes) exceeds %llu; omitting it from %s\n",
                     rid.size(), (unsigned long long)kMaxRunId, path);
        rid.clear();
    }
    const std::string tmp = std::string(path) + ".tmp";
    auto fail = [&](int32_t st) {
        std::remove(tmp.c_str());
        return st;
    };
    int32_t st;
    {
        FileCloser fc;
        fc.f = std::fopen(tmp.c_str(), "wb");
        if (!fc.f) {
            set_error("io error: cannot create " + tmp);
            return kErrInvalid;
        }
        std::vector<char> iobuf(8u << 20);
        std::setvbuf(fc.f, iobuf.data(), _IOFBF, iobuf.size());
        const std::string hdr =
            ckpt_header_bytes(arch, rid, superbatch, t.step_count, lr_horizon, (uint64_t)groups.size());
        bool ok = std::fwrite(hdr.data(), 1, hdr.size(), fc.f) == hdr.size();
        std::vector<float> host;
        for (const char* name : groups) {
            if (!ok) break;
            ParamGroup* g = t.find(name);
            if (!g) {
                set_error(std::string("raw checkpoint: unknown group ") + name);
                return fail(kErrInvalid);
            }
            std::string len;
            put_u64(len, g->n);
            ok = std::fwrite(len.data(), 1, 8, fc.f) == 8;
            host.resize(g->n);
            for (int which = 0; which < 4 && ok; ++which) {  // w, m, v, slow
                if ((st = t.read_group(*g, which, host.data()))) return fail(st);
                ok = std::fwrite(host.data(), sizeof(float), g->n, fc.f) == g->n;
            }
        }
        if (ok) ok = std::fflush(fc.f) == 0;
        const int closed = std::fclose(fc.f);
        fc.f = nullptr;
        if (!ok || closed != 0) {
            set_error("io error: writing " + tmp + " failed");
            return fail(kErrInvalid);
        }
    }
    if (std::rename(tmp.c_str(), path) != 0) {
        set_error("io error: cannot rename " + tmp + " to " + path);
        return fail(kErrInvalid);
    }
    return kOk;
}

// load_raw_checkpoint_file + the trainers' upload (ckpt.rs:705-754,
// trainer_layerstack.rs:1631-1726): the header is checked against the
// trainer, the group count and every group's length against its groups, and
// the file must hold every group's data before any state changes; then the
// groups are uploaded, the step counter restored and the forward table
// rebuilt.  Trailing bytes are allowed.
int32_t load_resume_checkpoint(TrainerBase& t, const char* path, const CkptArch& arch,
                               const std::vector<const char*>& groups, TataraCkptHeader* out) {
    FileCloser fc;
    fc.f = std::fopen(path, "rb");
    if (!fc.f) {
        set_error(std::string("io error: cannot open ") + path);
        return kErrInvalid;
    }
    FileReader r(fc.f);
    CkptHeader h;
    int32_t st = read_header(r, arch, h);
    if (st) return st;
    if (h.num_groups != groups.size())
        return Reader::invalid("raw checkpoint num_groups " + std::to_string(h.num_groups) + " != expected " +
                               std::to_string(groups.size()));
    const uint64_t data_start = r.offset();
    if (std::fseek(fc.f, 0, SEEK_END) != 0) return Reader::invalid("raw checkpoint seek failed");
    const long end = std::ftell(fc.f);
    if (end < 0) return Reader::invalid("raw checkpoint seek failed");
    const uint64_t size = (uint64_t)end;
    // pass 1: walk the groups as a sequential read would - each length field,
    // its match with the group, then its four arrays - without reading the
    // data, so a short or mismatching file fails before any state changes and
    // names the same field
    std::vector<ParamGroup*> gs;
    uint64_t at = data_start;
    for (const char* name : groups) {
        ParamGroup* g = t.find(name);
        TATARA_REQUIRE(g, std::string("raw checkpoint: unknown group ") + name);
        gs.push_back(g);
        const std::string gname = std::string("group ") + name;
        if (size < at + 8) return Reader::invalid("raw checkpoint truncated while reading " + gname + " len");
        if (std::fseek(fc.f, (long)at, SEEK_SET) != 0) return Reader::invalid("raw checkpoint seek failed");
        FileReader rl(fc.f);
        uint64_t len = 0;
        if ((st = rl.u64(len, (gname + " len").c_str()))) return st;
        if (len != g->n)
            return Reader::invalid("raw checkpoint " + gname + " len mismatch: got " + std::to_string(len) +
                                   ", want " + std::to_string(g->n) + " (network architecture mismatch)");
        at += 8;
        const char* parts[4] = {" w", " m", " v", " slow"};
        for (const char* part : parts) {
            if (size < at + 4 * len) return Reader::invalid("raw checkpoint truncated while reading " + gname + part);
            at += 4 * len;
        }
    }
    // pass 2: upload
    if (std::fseek(fc.f, (long)data_start, SEEK_SET) != 0) return Reader::invalid("raw checkpoint seek failed");
    std::vector<float> host;
    for (ParamGroup* g : gs) {
        FileReader rg(fc.f);
        uint64_t len = 0;
        if ((st = rg.u64(len, "group len"))) return st;
        host.resize(g->n);
        for (int which = 0; which < 4; ++which) {
            if ((st = rg.exact(host.data(), 4 * g->n, "group data"))) return st;
            if ((st = t.write_group(*g, which, host.data()))) return st;
        }
    }
    t.step_count = h.step_count;
    if ((st = t.sync_forward_weights())) return st;
    if (out) header_to_c(h, data_start, out);
    return kOk;
}

}  // namespace tatara

extern "C" {

using namespace tatara;

int32_t tatara_ckpt_write_header(const TataraCkptArch* arch, const char* run_id, uint64_t superbatch,
                                 uint64_t step_count, uint64_t lr_horizon, uint64_t num_groups, uint8_t* out,
                                 uint64_t capacity, uint64_t* out_bytes) {
    TATARA_REQUIRE(arch && out_bytes, "null argument");
    CkptArch a;
    int32_t st = ckpt_arch_from_c(*arch, a);
    if (st) return st;
    std::string rid = run_id ? run_id : "";
    if (rid.size() > kMaxRunId) rid.clear();
    const std::string b = ckpt_header_bytes(a, rid, superbatch, step_count, lr_horizon, num_groups);
    *out_bytes = b.size();
    TATARA_REQUIRE(out || capacity == 0, "null output buffer");
    TATARA_REQUIRE(capacity >= b.size(), "output buffer too small");
    std::memcpy(out, b.data(), b.size());
    return kOk;
}

int32_t tatara_ckpt_read_header(const uint8_t* data, uint64_t n, const TataraCkptArch* expected,
                                TataraCkptHeader* out) {
    TATARA_REQUIRE((data || n == 0) && expected && out, "null argument");
    CkptArch a;
    int32_t st = ckpt_arch_from_c(*expected, a);
    if (st) return st;
    MemReader r(data, n);
    CkptHeader h;
    if ((st = read_header(r, a, h))) return st;
    header_to_c(h, r.offset(), out);
    return kOk;
}

}  // extern "C"
