// Superbatch driver: run (crates/nnue-train/src/trainer.rs:759-1211) over a
// PSV file with the trainer of this library.
//
// Per superbatch sb = start..=end and batch b: lr = LrScheduler::lr(b, sb),
// wdl = WdlScheduler::blend(b, sb, end), the next batch_size records of the
// file (read in order; the file starts over at its end, as PsvEpochReader
// does with one worker, dataloader.rs:724-760), uploaded and decoded on the
// trainer's stream while the previous step still runs, then train_step, whose lagged loss is added to the superbatch's sum; after the
// last batch flush_pending_loss drains the last step's loss into it.  The
// reference's per-superbatch line is printed (loss = sum / positions), and
// checkpoints are written when sb % save_rate == 0 or sb == end: the
// quantised "<net_id>-<sb>.bin" and the resume "<net_id>-<sb>.ckpt" (run id,
// LR horizon), then old ".ckpt" files are pruned to keep_raw_checkpoints
// (prune_old_raw_checkpoints, trainer.rs:1230-1283).  A run with start > 1
// resumes the schedules at that superbatch and reads the data from the start
// of the file, as the reference does.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include <cctype>
#include <cerrno>
#include <cstdlib>
#include <ctime>

#include <dirent.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/tatara_hip.h"
#include "common.hpp"
#include "experiment.hpp"
#include "psv_kernels.hpp"
#include "schedule.hpp"
#include "trainer_base.hpp"

namespace tatara {

namespace {

constexpr uint64_t kPsvBytes = 40;  // PackedSfenValue record (packed_sfen.rs:255-268)

// format_hms (trainer.rs:1285-1300)
std::string format_hms(double secs) {
    if (!(secs >= 0.0) || secs != secs || secs > 1.8e19) return "??";
    const uint64_t total = (uint64_t)secs;
    const uint64_t h = total / 3600, m = (total % 3600) / 60, s = total % 60;
    char buf[64];
    if (h > 0)
        snprintf(buf, sizeof buf, "%lluh%02llum%02llus", (unsigned long long)h, (unsigned long long)m,
                 (unsigned long long)s);
    else if (m > 0)
        snprintf(buf, sizeof buf, "%llum%02llus", (unsigned long long)m, (unsigned long long)s);
    else
        snprintf(buf, sizeof buf, "%llus", (unsigned long long)s);
    return buf;
}

// Rust's `{:.4e}`: four decimals, exponent without sign padding ("8.7500e-4").
std::string rust_exp4(float v) {
    char buf[64];
    snprintf(buf, sizeof buf, "%.4e", (double)v);
    std::string s = buf;
    const size_t e = s.find('e');
    if (e == std::string::npos) return s;
    std::string mant = s.substr(0, e), ex = s.substr(e + 1);
    bool neg = false;
    size_t i = 0;
    if (i < ex.size() && (ex[i] == '+' || ex[i] == '-')) neg = ex[i++] == '-';
    while (i + 1 < ex.size() && ex[i] == '0') ++i;
    return mant + "e" + (neg ? "-" : "") + ex.substr(i);
}

// Sequential PSV reader that starts over at the end of the file.
struct EpochReader {
    FILE* f = nullptr;
    uint64_t records = 0;
    ~EpochReader() {
        if (f) fclose(f);
    }
    int32_t open(const char* path) {
        f = fopen(path, "rb");
        TATARA_REQUIRE(f, std::string("cannot open data file ") + path);
        struct stat st;
        TATARA_REQUIRE(fstat(fileno(f), &st) == 0, "cannot stat the data file");
        const uint64_t size = (uint64_t)st.st_size;
        TATARA_REQUIRE(size % kPsvBytes == 0,
                       "data file size " + std::to_string(size) +
                           " is not a multiple of the PSV record size (40 bytes)");
        records = size / kPsvBytes;
        TATARA_REQUIRE(records > 0, "the data file holds no PSV records");
        return kOk;
    }
    // n records into dst (pinned memory) through a cached staging buffer,
    // where the host checks them: *king_blocked is false when, in a feature
    // set with merged king planes, a record has both kings on one square (its
    // rows would repeat the king feature); board, hand and king features
    // occupy disjoint ranges of a king block otherwise, so every decoded row
    // is king-blocked.  (CPU reads of the pinned buffer itself are uncached.)
    std::vector<uint8_t> stage;
    int32_t read(uint8_t* dst, uint64_t n, bool merged_kings, bool* king_blocked) {
        stage.resize(n * kPsvBytes);
        uint64_t got = 0;
        while (got < n) {
            const size_t r = fread(stage.data() + got * kPsvBytes, kPsvBytes, n - got, f);
            got += r;
            if (got < n) {
                TATARA_REQUIRE(!ferror(f), "read error on the data file");
                rewind(f);  // next epoch
            }
        }
        bool ok = true;
        if (merged_kings) {
            // bit 0: side to move; bits 1..7, 8..14: the king squares (LSB first)
            for (uint64_t i = 0; i < n && ok; ++i) {
                const uint8_t* r = stage.data() + i * kPsvBytes;
                const uint32_t w = (uint32_t)r[0] | ((uint32_t)r[1] << 8);
                const uint32_t k0 = (w >> 1) & 127u, k1 = (w >> 8) & 127u;
                ok = !(k0 == k1 && k0 < 81);
            }
        }
        *king_blocked = ok;
        std::memcpy(dst, stage.data(), n * kPsvBytes);
        return kOk;
    }
};

// prune_old_raw_checkpoints (trainer.rs:1230-1283)
void prune_raw(const std::string& dir, const std::string& net_id, uint64_t keep) {
    if (keep == 0) {
        fprintf(stderr, "[train] warning: keep_raw_checkpoints=0 ignored (would delete all raw checkpoints)\n");
        return;
    }
    DIR* d = opendir(dir.c_str());
    if (!d) {
        fprintf(stderr, "[train] warning: cannot read %s to prune raw checkpoints\n", dir.c_str());
        return;
    }
    const std::string prefix = net_id + "-", suffix = ".ckpt";
    std::vector<std::pair<uint64_t, std::string>> found;
    while (dirent* ent = readdir(d)) {
        const std::string name = ent->d_name;
        if (name.size() <= prefix.size() + suffix.size() || name.compare(0, prefix.size(), prefix) != 0 ||
            name.compare(name.size() - suffix.size(), suffix.size(), suffix) != 0)
            continue;
        std::string num = name.substr(prefix.size(), name.size() - prefix.size() - suffix.size());
        if (!num.empty() && num[0] == '+') num = num.substr(1);  // usize::from_str takes a leading '+'
        if (num.empty() || num.size() > 19 || num.find_first_not_of("0123456789") != std::string::npos) continue;
        found.emplace_back(std::stoull(num), dir + "/" + name);
    }
    closedir(d);
    if (found.size() <= keep) return;
    std::sort(found.begin(), found.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
    for (size_t i = keep; i < found.size(); ++i) {
        if (unlink(found[i].second.c_str()) == 0)
            printf("[train] pruned old raw checkpoint: %s (sb %llu)\n", found[i].second.c_str(),
                   (unsigned long long)found[i].first);
        else
            fprintf(stderr, "[train] warning: failed to prune %s\n", found[i].second.c_str());
    }
}

// ---------------------------------------------------------------------------
// control.json (crates/nnue-train/src/trainer.rs:640-744): at the start of
// every superbatch the driver reads <output_dir>/control.json; a
// {"target_superbatches": N} there moves the run's effective last superbatch
// to N clamped to [current superbatch, configured end] (the LR / WDL
// schedules keep the configured end as their horizon).  Each change is
// printed and appended to control_history.jsonl.  A missing file is silent;
// an unreadable or malformed one, and a stale target below the run's start,
// are reported on stderr and ignored (the stale warning once per value).
// ---------------------------------------------------------------------------

// Recursive-descent JSON reader (RFC 8259 grammar): validates the text and
// reports the raw text of the top-level object's "target_superbatches"
// member, as serde_json deserialises ControlFile { target_superbatches:
// Option<usize> } (unknown fields ignored, a duplicate field an error).
struct JsonReader {
    const char* p;
    const char* end;
    std::string err;
    int depth = 0;

    bool fail(const std::string& m) {
        if (err.empty()) err = m;
        return false;
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool literal(const char* w) {
        const size_t n = std::strlen(w);
        if ((size_t)(end - p) < n || std::strncmp(p, w, n) != 0) return fail("expected value");
        p += n;
        return true;
    }
    bool string(std::string* out) {
        if (p >= end || *p != '"') return fail("expected string");
        ++p;
        while (p < end && *p != '"') {
            const unsigned char ch = (unsigned char)*p;
            if (ch < 0x20) return fail("control character in string");
            if (ch == '\\') {
                ++p;
                if (p >= end) return fail("EOF while parsing a string");
                const char esc = *p;
                if (esc == 'u') {
                    for (int i = 1; i <= 4; ++i)
                        if (p + i >= end || !std::isxdigit((unsigned char)p[i])) return fail("invalid escape");
                    p += 4;
                    if (out) out->push_back('?');
                } else if (std::strchr("\"\\/bfnrt", esc)) {
                    if (out) out->push_back(esc);
                } else {
                    return fail("invalid escape");
                }
                ++p;
                continue;
            }
            if (out) out->push_back((char)ch);
            ++p;
        }
        if (p >= end) return fail("EOF while parsing a string");
        ++p;
        return true;
    }
    bool number() {
        const char* s0 = p;
        if (p < end && *p == '-') ++p;
        if (p >= end || !std::isdigit((unsigned char)*p)) return fail("invalid number");
        if (*p == '0') {
            ++p;
        } else {
            while (p < end && std::isdigit((unsigned char)*p)) ++p;
        }
        if (p < end && *p == '.') {
            ++p;
            if (p >= end || !std::isdigit((unsigned char)*p)) return fail("invalid number");
            while (p < end && std::isdigit((unsigned char)*p)) ++p;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            if (p >= end || !std::isdigit((unsigned char)*p)) return fail("invalid number");
            while (p < end && std::isdigit((unsigned char)*p)) ++p;
        }
        return p > s0;
    }
    bool value(const char** v0 = nullptr, const char** v1 = nullptr) {
        ws();
        if (p >= end) return fail("EOF while parsing a value");
        if (++depth > 128) return fail("recursion limit exceeded");
        const char* s0 = p;
        bool ok;
        switch (*p) {
            case '{': ok = object(nullptr); break;
            case '[': ok = array(); break;
            case '"': ok = string(nullptr); break;
            case 't': ok = literal("true"); break;
            case 'f': ok = literal("false"); break;
            case 'n': ok = literal("null"); break;
            default: ok = number();
        }
        --depth;
        if (v0) *v0 = s0;
        if (v1) *v1 = p;
        return ok;
    }
    bool array() {
        ++p;
        ws();
        if (p < end && *p == ']') {
            ++p;
            return true;
        }
        while (true) {
            if (!value()) return false;
            ws();
            if (p < end && *p == ',') {
                ++p;
                continue;
            }
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            return fail("expected `,` or `]`");
        }
    }
    // target (may be null): receives the raw text of "target_superbatches"
    bool object(std::string* target, bool* seen = nullptr) {
        ++p;
        ws();
        if (p < end && *p == '}') {
            ++p;
            return true;
        }
        while (true) {
            ws();
            std::string key;
            if (!string(&key)) return false;
            ws();
            if (p >= end || *p != ':') return fail("expected `:`");
            ++p;
            const char *v0 = nullptr, *v1 = nullptr;
            if (!value(&v0, &v1)) return false;
            if (target && key == "target_superbatches") {
                if (*seen) return fail("duplicate field `target_superbatches`");
                *seen = true;
                target->assign(v0, v1);
            }
            ws();
            if (p < end && *p == ',') {
                ++p;
                continue;
            }
            if (p < end && *p == '}') {
                ++p;
                return true;
            }
            return fail("expected `,` or `}`");
        }
    }
};

// Parses control.json text; *has_target = 0 when target_superbatches is
// absent or null.  Returns false with a message for malformed input or a
// value that is not a non-negative integer.
bool parse_control(const std::string& text, bool* has_target, uint64_t* target, std::string* err) {
    JsonReader r{text.data(), text.data() + text.size(), {}};
    *has_target = false;
    r.ws();
    if (r.p >= r.end) {
        *err = "EOF while parsing a value";
        return false;
    }
    if (*r.p != '{') {
        // a valid JSON value of another type is a type error, as serde reports it
        if (!r.value()) {
            *err = r.err;
            return false;
        }
        *err = "invalid type, expected struct ControlFile";
        return false;
    }
    std::string raw;
    bool seen = false;
    if (!r.object(&raw, &seen)) {
        *err = r.err;
        return false;
    }
    r.ws();
    if (r.p != r.end) {
        *err = "trailing characters";
        return false;
    }
    if (!seen || raw == "null") return true;
    if (raw.empty() || raw.find_first_not_of("0123456789") != std::string::npos) {
        *err = "invalid type: " + raw + ", expected usize";
        return false;
    }
    errno = 0;
    char* endp = nullptr;
    const unsigned long long v = std::strtoull(raw.c_str(), &endp, 10);
    if (errno == ERANGE) {
        *err = "number out of range for usize";
        return false;
    }
    *has_target = true;
    *target = (uint64_t)v;
    return true;
}

// format_utc_iso (crates/nnue-train/src/experiment.rs:564-567)
std::string utc_iso_now() {
    const time_t t = time(nullptr);
    struct tm g;
    gmtime_r(&t, &g);
    char buf[32];
    snprintf(buf, sizeof buf, "%04d-%02d-%02dT%02d:%02d:%02dZ", g.tm_year + 1900, g.tm_mon + 1, g.tm_mday, g.tm_hour,
             g.tm_min, g.tm_sec);
    return buf;
}

// std::io::Error's display of an errno value.
std::string os_error(int e) { return std::string(std::strerror(e)) + " (os error " + std::to_string(e) + ")"; }

// apply_control (trainer.rs:670-731).  Returns true with *target when a new
// effective target was applied.
bool apply_control(const std::string& control_path, const std::string& history_path, TataraControlState& st,
                   uint64_t current, uint64_t start, uint64_t configured_end, uint64_t* target) {
    struct stat sst;
    if (stat(control_path.c_str(), &sst) != 0) {
        if (errno == ENOENT) return false;
        fprintf(stderr, "[control] warning: failed to read %s: %s; ignoring\n", control_path.c_str(),
                os_error(errno).c_str());
        return false;
    }
    std::string text;
    {
        if (S_ISDIR(sst.st_mode)) {
            fprintf(stderr, "[control] warning: failed to read %s: %s; ignoring\n", control_path.c_str(),
                    os_error(EISDIR).c_str());
            return false;
        }
        FILE* f = fopen(control_path.c_str(), "rb");
        if (!f) {
            if (errno == ENOENT) return false;
            fprintf(stderr, "[control] warning: failed to read %s: %s; ignoring\n", control_path.c_str(),
                    os_error(errno).c_str());
            return false;
        }
        char buf[4096];
        size_t n;
        while ((n = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
        const bool bad = ferror(f);
        fclose(f);
        if (bad) {
            fprintf(stderr, "[control] warning: failed to read %s: read error; ignoring\n", control_path.c_str());
            return false;
        }
    }
    bool has = false;
    uint64_t requested = 0;
    std::string err;
    if (!parse_control(text, &has, &requested, &err)) {
        fprintf(stderr, "[control] warning: failed to parse %s: %s; ignoring\n", control_path.c_str(), err.c_str());
        return false;
    }
    if (!has) return false;
    if (requested < start) {
        // ControlState::should_warn_stale: once per requested value
        if (!(st.has_ignored_stale && st.ignored_stale_target == requested)) {
            st.has_ignored_stale = 1;
            st.ignored_stale_target = requested;
            fprintf(stderr,
                    "[control] warning: ignoring stale target_superbatches=%llu from %s below run start_superbatch=%llu\n",
                    (unsigned long long)requested, control_path.c_str(), (unsigned long long)start);
        }
        return false;
    }
    st.has_ignored_stale = 0;
    const uint64_t t = std::min(std::max(requested, current), configured_end);
    if (t == st.effective_target) return false;
    st.effective_target = t;
    printf("[control] applied: target_superbatches=%llu (superbatch=%llu)\n", (unsigned long long)t,
           (unsigned long long)current);
    fflush(stdout);
    const std::string line = std::string("{\"type\":\"control\",\"timestamp\":\"") + utc_iso_now() +
                             "\",\"target_superbatches\":" + std::to_string(t) +
                             ",\"superbatch\":" + std::to_string(current) + "}\n";
    FILE* h = fopen(history_path.c_str(), "ab");
    bool ok = h != nullptr;
    const int open_err = errno;
    if (h) {
        ok = fwrite(line.data(), 1, line.size(), h) == line.size();
        ok = (fclose(h) == 0) && ok;
    }
    if (!ok)
        fprintf(stderr, "[control] warning: failed to append %s: %s; training will continue\n", history_path.c_str(),
                h ? "write error" : os_error(open_err).c_str());
    *target = t;
    return true;
}

struct DevBatch {
    int32_t *stm = nullptr, *nstm = nullptr, *nnz = nullptr, *bucket = nullptr;
    float *score = nullptr, *wdl = nullptr;
};

// The driver's buffers; the trainer's stream is drained before they are freed.
struct RunMem {
    hipStream_t stream = nullptr, copy = nullptr;
    std::vector<void*> dev, host;
    std::vector<hipEvent_t> events;
    ~RunMem() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (copy) {
            (void)hipStreamSynchronize(copy);
            (void)hipStreamDestroy(copy);
        }
        for (void* p : dev) (void)hipFree(p);
        for (void* p : host) (void)hipHostFree(p);
        for (hipEvent_t e : events) (void)hipEventDestroy(e);
    }
    template <class T>
    int32_t alloc(T** p, uint64_t n) {
        TATARA_HIP(hipMalloc((void**)p, (n ? n : 1) * sizeof(T)), "hipMalloc (run)");
        dev.push_back(*p);
        return kOk;
    }
    int32_t alloc_pinned(uint8_t** p, uint64_t n) {
        TATARA_HIP(hipHostMalloc((void**)p, n ? n : 1, hipHostMallocDefault), "hipHostMalloc (run)");
        host.push_back(*p);
        return kOk;
    }
    int32_t event(hipEvent_t* e) {
        TATARA_HIP(hipEventCreateWithFlags(e, hipEventDisableTiming), "hipEventCreate (run)");
        events.push_back(*e);
        return kOk;
    }
};

// One in-flight batch: the pinned records, their device copy and the decoded
// arrays.  `uploaded` (copy stream) completes when the records have reached
// the device, after which the pinned buffer may be refilled; `decoded` (copy
// stream) when the arrays are ready for the step; `consumed` (trainer stream)
// when the step that used them has finished, after which the slot may be
// refilled.
struct Slot {
    uint8_t* psv_host = nullptr;
    uint8_t* psv_dev = nullptr;
    hipEvent_t uploaded = nullptr, decoded = nullptr, consumed = nullptr;
    DevBatch d;
};

int32_t run(TataraTrainer* trainer, const TataraRunConfig& c, const TataraLrSchedule& lr,
            const TataraWdlSchedule& wdl, const TataraLoss* loss, TataraRunSuperbatch* report,
            uint64_t report_cap, uint64_t* n_report, float* lr_seen, float* wdl_seen, uint64_t seen_cap) {
    // TrainingConfig::validate (trainer.rs:490-510)
    TATARA_REQUIRE(c.start_superbatch >= 1, "start_superbatch must be >= 1 (1-indexed)");
    TATARA_REQUIRE(c.end_superbatch >= c.start_superbatch,
                   "end_superbatch (" + std::to_string(c.end_superbatch) + ") < start_superbatch (" +
                       std::to_string(c.start_superbatch) + ")");
    TATARA_REQUIRE(c.batches_per_superbatch >= 1, "batches_per_superbatch must be >= 1");
    TATARA_REQUIRE(c.batch_size >= 1 && c.batch_size <= 0x7fffffffull, "batch_size out of range");
    TATARA_REQUIRE(c.save_rate >= 1, "save_rate must be >= 1");
    TATARA_REQUIRE(c.data_path && c.output_dir && c.net_id, "data_path, output_dir and net_id are required");
    if (n_report) *n_report = 0;
    int32_t st;
    int32_t max_active = 0;
    if ((st = tatara_feature_set_info(c.feature_set, nullptr, nullptr, nullptr, &max_active, nullptr))) return st;
    EpochReader reader;
    if ((st = reader.open(c.data_path))) return st;

    FeatureSetShape shape;
    if ((st = feature_set_shape(c.feature_set, shape))) return st;
    const uint64_t B = c.batch_size;
    RunMem mem;
    mem.stream = trainer_stream(trainer);
    TATARA_HIP(hipStreamCreateWithFlags(&mem.copy, hipStreamNonBlocking), "hipStreamCreate (run copy)");
    // Two slots: the host reads batch k + 1 and a second stream uploads and
    // decodes it while the trainer's stream runs step k; step k + 1 waits for
    // that decode on the device, not on the host.
    Slot slots[2];
    for (Slot& sl : slots) {
        DevBatch& d = sl.d;
        if ((st = mem.alloc_pinned(&sl.psv_host, B * kPsvBytes)) || (st = mem.alloc(&sl.psv_dev, B * kPsvBytes)) ||
            (st = mem.event(&sl.uploaded)) || (st = mem.event(&sl.decoded)) || (st = mem.event(&sl.consumed)) || (st = mem.alloc(&d.stm, B * max_active)) ||
            (st = mem.alloc(&d.nstm, B * max_active)) || (st = mem.alloc(&d.nnz, B)) ||
            (st = mem.alloc(&d.bucket, B)) || (st = mem.alloc(&d.score, B)) || (st = mem.alloc(&d.wdl, B)))
            return st;
        // the events start out complete
        TATARA_HIP(hipEventRecord(sl.consumed, mem.stream), "run: record the step");
        TATARA_HIP(hipEventRecord(sl.uploaded, mem.copy), "run: record the upload");
    }
    PsvArgs pa{};
    pa.n = (uint32_t)B;
    pa.piece_inputs = shape.piece_inputs;
    pa.max_active = shape.max_active;
    pa.emit_king = shape.emit_king;
    pa.fold_enemy = shape.fold_enemy;
    pa.mirror = shape.mirror;
    pa.bucket_mode = c.bucket_mode;
    pa.num_buckets = c.num_buckets;
    pa.weights = c.progress_weights;
    pa.progress = nullptr;

    uint64_t horizon = 0;
    const bool has_horizon = lr_horizon(lr, horizon);
    const std::string out_dir = c.output_dir, net_id = c.net_id;
    const uint64_t positions_per_sb = c.batches_per_superbatch * B;
    uint64_t step = 0;
    int cur = 0;
    const std::string control_path = out_dir + "/control.json";
    const std::string history_path = out_dir + "/control_history.jsonl";
    TataraControlState control{};
    control.effective_target = c.end_superbatch;
    TataraExperiment* exp = c.experiment;
    // the run id resume checkpoints carry: the experiment's when there is one
    const std::string run_id = exp ? exp->id : (c.run_id ? c.run_id : "");
    // a failed experiment.json write is reported and the run goes on
    auto write_experiment = [&]() {
        if (!exp) return;
        const std::string err = exp->write();
        if (!err.empty())
            fprintf(stderr, "[train] warning: failed to write experiment log %s: %s\n", exp->path.c_str(),
                    err.c_str());
    };
    write_experiment();  // status "running", before the first superbatch
    const auto run_start = std::chrono::steady_clock::now();
    auto run_seconds = [&]() {
        return std::chrono::duration<double>(std::chrono::steady_clock::now() - run_start).count();
    };
    uint64_t sb = c.start_superbatch;
    for (;; ++sb) {
        uint64_t applied = 0;
        if (apply_control(control_path, history_path, control, sb, c.start_superbatch, c.end_superbatch, &applied) &&
            exp) {
            tatara_experiment_set_target_superbatches(exp, applied);
            write_experiment();
        }
        const auto t0 = std::chrono::steady_clock::now();
        double sb_loss = 0.0;
        uint64_t sb_positions = 0;
        for (uint64_t b = 0; b < c.batches_per_superbatch; ++b, ++step) {
            const float lr_v = lr_at(lr, b, sb);
            const float wdl_v = wdl_at(wdl, b, sb, c.end_superbatch);
            if (lr_seen && step < seen_cap) lr_seen[step] = lr_v;
            if (wdl_seen && step < seen_cap) wdl_seen[step] = wdl_v;
            Slot& sl = slots[cur];
            // the upload that last read this pinned buffer has finished
            TATARA_HIP(hipEventSynchronize(sl.uploaded), "run: wait for the upload");
            bool king_blocked = false;
            if ((st = reader.read(sl.psv_host, B, shape.emit_king && shape.fold_enemy, &king_blocked))) return st;
            TATARA_HIP(hipStreamWaitEvent(mem.copy, sl.consumed, 0), "run: wait for the slot's last step");
            TATARA_HIP(hipMemcpyAsync(sl.psv_dev, sl.psv_host, B * kPsvBytes, hipMemcpyHostToDevice, mem.copy),
                       "PSV upload");
            TATARA_HIP(hipEventRecord(sl.uploaded, mem.copy), "run: record the upload");
            const DevBatch& d = sl.d;
            pa.psv = sl.psv_dev;
            pa.stm = d.stm;
            pa.nstm = d.nstm;
            pa.nnz = d.nnz;
            pa.bucket = d.bucket;
            pa.score = d.score;
            pa.wdl = d.wdl;
            if ((st = launch_psv_to_batch(pa, mem.copy))) return st;
            TATARA_HIP(hipEventRecord(sl.decoded, mem.copy), "run: record the decode");
            TATARA_HIP(hipStreamWaitEvent(mem.stream, sl.decoded, 0), "run: order the step");
            TataraBatch bt{};
            bt.n_pos = (int32_t)B;
            bt.max_active = max_active;
            bt.stm_indices = d.stm;
            bt.nstm_indices = d.nstm;
            bt.nnz = d.nnz;
            bt.bucket_idx = d.bucket;
            bt.score = d.score;
            bt.wdl = d.wdl;
            bt.on_device = king_blocked ? TATARA_BATCH_KING_BLOCKED : 1;
            double lagged = 0.0;
            if ((st = tatara_trainer_train_step(trainer, &bt, lr_v, wdl_v, loss, &lagged))) return st;
            TATARA_HIP(hipEventRecord(sl.consumed, mem.stream), "run: record the step");
            sb_loss += lagged;
            sb_positions += B;
            cur ^= 1;
        }
        double flushed = 0.0;
        if ((st = tatara_trainer_flush_pending_loss(trainer, &flushed))) return st;
        sb_loss += flushed;
        const double secs =
            std::max(1e-9, std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
        const double mean = sb_positions ? sb_loss / (double)sb_positions : NAN;
        const double pps = (double)sb_positions / secs;
        const double eta = pps > 0.0 ? (double)(positions_per_sb * (control.effective_target - sb)) / pps : NAN;
        const float lr_now = lr_at(lr, 0, sb), wdl_now = wdl_at(wdl, 0, sb, c.end_superbatch);
        if (c.print_progress) {
            printf("[train] superbatch %llu/%llu | loss %.6f | %.0f pos/s | lr %s | wdl %.3f | sb %.1fs | ETA %s\n",
                   (unsigned long long)sb, (unsigned long long)control.effective_target, mean, pps,
                   rust_exp4(lr_now).c_str(), (double)wdl_now, secs, format_hms(eta).c_str());
            fflush(stdout);
        }
        const bool saved = sb % c.save_rate == 0 || sb == control.effective_target;
        if (saved) {
            const std::string base = out_dir + "/" + net_id + "-" + std::to_string(sb);
            if ((st = tatara_trainer_export_quantised(trainer, (base + ".bin").c_str(), c.feature_set,
                                                      c.has_fv_scale, c.fv_scale)))
                return st;
            if (c.print_progress) printf("[train] checkpoint saved: %s.bin\n", base.c_str());
            if ((st = tatara_trainer_save_resume(trainer, (base + ".ckpt").c_str(), c.feature_set, c.bucket_mode,
                                                 sb, run_id.c_str(), has_horizon ? horizon : 0)))
                return st;
            if (c.print_progress) printf("[train] resume checkpoint saved: %s.ckpt\n", base.c_str());
            if (c.has_keep_raw) prune_raw(out_dir, net_id, c.keep_raw_checkpoints);
        }
        if (report && n_report && *n_report < report_cap) {
            TataraRunSuperbatch& r = report[(*n_report)++];
            r.superbatch = sb;
            r.positions = sb_positions;
            r.loss_sum = sb_loss;
            r.mean_loss = mean;
            r.seconds = secs;
            r.lr = lr_now;
            r.wdl = wdl_now;
            r.saved = saved ? 1 : 0;
        }
        // after the superbatch's checkpoints exist (trainer.rs:1157-1173)
        if (exp) {
            tatara_experiment_record_superbatch(exp, sb, mean, sb_positions, run_seconds(), nullptr, nullptr);
            if (saved) {
                const std::string base = net_id + "-" + std::to_string(sb);
                exp->checkpoints.push_back(base + ".bin");
                exp->checkpoints.push_back(base + ".ckpt");
            }
            write_experiment();
        }
        if (sb == control.effective_target) break;
    }
    if (c.print_progress) {
        printf("[train] done in %s (%llu superbatches)\n", format_hms(run_seconds()).c_str(),
               (unsigned long long)(sb + 1 - c.start_superbatch));
        fflush(stdout);
    }
    if (exp) {
        tatara_experiment_mark_finished(exp, run_seconds());
        write_experiment();
    }
    return kOk;
}

}  // namespace

}  // namespace tatara

using namespace tatara;

extern "C" int32_t tatara_control_apply(const char* control_path, const char* history_path,
                                        TataraControlState* state, uint64_t current_superbatch,
                                        uint64_t start_superbatch, uint64_t configured_end, int32_t* applied,
                                        uint64_t* target) {
    TATARA_REQUIRE(control_path && history_path && state && applied && target, "control_apply: null argument");
    uint64_t t = 0;
    const bool ok = apply_control(control_path, history_path, *state, current_superbatch, start_superbatch,
                                  configured_end, &t);
    *applied = ok ? 1 : 0;
    *target = ok ? t : 0;
    return kOk;
}

extern "C" int32_t tatara_train_run(TataraTrainer* trainer, const TataraRunConfig* config,
                                    const TataraLrSchedule* lr, const TataraWdlSchedule* wdl,
                                    const TataraLoss* loss, TataraRunSuperbatch* report, uint64_t report_cap,
                                    uint64_t* n_report, float* lr_seen, float* wdl_seen, uint64_t seen_cap) {
    TATARA_REQUIRE(trainer && config && lr && wdl && loss, "train_run: null argument");
    return run(trainer, *config, *lr, *wdl, loss, report, report_cap, n_report, lr_seen, wdl_seen, seen_cap);
}
