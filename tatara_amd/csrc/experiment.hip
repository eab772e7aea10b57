// Structured run log (crates/nnue-train/src/experiment.rs): the document of
// one training run, updated as the run goes and rewritten whole each time
// (temp file + rename), so an interrupted run leaves the last complete
// document.  The layout is serde_json's pretty printer (two-space indent,
// fields in the reference's declaration order, optional fields omitted when
// absent).  Host code only.
#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <new>
#include <string>

#include <sys/stat.h>

#include "common.hpp"
#include "experiment.hpp"

namespace tatara {

// Days since 1970-01-01 to the proleptic Gregorian date: Howard Hinnant's
// published civil_from_days algorithm ("chrono-Compatible Low-Level Date
// Algorithms"), which the reference also names (experiment.rs:577).  It
// works in 400-year eras counted from 0000-03-01 (so the leap day ends each
// era's year): the era,
// the day within it, the year within it, the day of that March-based year,
// and the month from the five-month 153-day pattern of March..July and
// August..December.
Civil civil_from_epoch(uint64_t epoch_secs) {
    const int64_t days = (int64_t)(epoch_secs / 86400);
    const uint64_t rem = epoch_secs % 86400;
    Civil c;
    c.hour = (uint32_t)(rem / 3600);
    c.minute = (uint32_t)(rem % 3600 / 60);
    c.second = (uint32_t)(rem % 60);
    const int64_t z = days + 719468;  // days from 0000-03-01
    const int64_t era = (z >= 0 ? z : z - 146096) / 146097;
    const int64_t doe = z - era * 146097;                                    // [0, 146096]
    const int64_t yoe = (doe - doe / 1460 + doe / 36524 - doe / 146096) / 365;  // [0, 399]
    const int64_t doy = doe - (365 * yoe + yoe / 4 - yoe / 100);             // [0, 365]
    const int64_t mp = (5 * doy + 2) / 153;                                  // [0, 11], 0 = March
    c.day = (uint32_t)(doy - (153 * mp + 2) / 5 + 1);
    c.month = (uint32_t)(mp < 10 ? mp + 3 : mp - 9);
    c.year = yoe + era * 400 + (c.month <= 2 ? 1 : 0);
    return c;
}

std::string format_utc_iso(uint64_t epoch_secs) {
    const Civil c = civil_from_epoch(epoch_secs);
    char buf[64];
    snprintf(buf, sizeof buf, "%04lld-%02u-%02uT%02u:%02u:%02uZ", (long long)c.year, c.month, c.day, c.hour, c.minute,
             c.second);
    return buf;
}

std::string format_utc_compact(uint64_t epoch_secs) {
    const Civil c = civil_from_epoch(epoch_secs);
    char buf[64];
    snprintf(buf, sizeof buf, "%04lld%02u%02ut%02u%02u%02uz", (long long)c.year, c.month, c.day, c.hour, c.minute,
             c.second);
    return buf;
}

uint64_t now_epoch_secs() {
    const time_t t = time(nullptr);
    return t > 0 ? (uint64_t)t : 0;
}

// The fewest significant digits that read back as v (each precision
// correctly rounded by printf, checked with strtod), then one of the ryu
// crate's layouts, by the decimal exponent kk with v = 0.d1d2... x 10^kk:
// integer digits + ".0" (up to 16 integer digits), a decimal point inside
// the digits, "0.000ddd" (kk > -5), else scientific "de-7" / "d.ddde21".
std::string json_f64(double v) {
    if (v == 0.0) return std::signbit(v) ? "-0.0" : "0.0";
    char buf[48];
    for (int prec = 1; prec <= 17; ++prec) {
        snprintf(buf, sizeof buf, "%.*e", prec - 1, v);
        if (strtod(buf, nullptr) == v) break;
    }
    const bool neg = buf[0] == '-';
    const char* p = buf + (neg ? 1 : 0);
    std::string digits(1, *p++);
    if (*p == '.')
        for (++p; *p != 'e'; ++p) digits.push_back(*p);
    const int e10 = atoi(p + 1);
    while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
    const int n = (int)digits.size();
    const int kk = e10 + 1, k = kk - n;
    std::string out = neg ? "-" : "";
    if (k >= 0 && kk <= 16)
        out += digits + std::string((size_t)k, '0') + ".0";
    else if (kk > 0 && kk <= 16)
        out += digits.substr(0, (size_t)kk) + "." + digits.substr((size_t)kk);
    else if (kk > -5 && kk <= 0)
        out += "0." + std::string((size_t)-kk, '0') + digits;
    else if (n == 1)
        out += digits + "e" + std::to_string(kk - 1);
    else
        out += digits.substr(0, 1) + "." + digits.substr(1) + "e" + std::to_string(kk - 1);
    return out;
}

// serde_json's string escapes: \" \\ and the short forms of \b \f \n \r \t,
// \u00XX for the other control characters; everything else as is.
std::string json_string(const std::string& s) {
    std::string out = "\"";
    for (const unsigned char ch : s) {
        switch (ch) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (ch < 0x20) {
                    char u[8];
                    snprintf(u, sizeof u, "\\u%04x", ch);
                    out += u;
                } else {
                    out.push_back((char)ch);
                }
        }
    }
    return out + "\"";
}

namespace {

// One pretty-printed object: "key": value lines at the given indent.
struct Obj {
    std::string ind, body;
    bool first = true;
    explicit Obj(int depth) : ind((size_t)depth * 2, ' ') {}
    void raw(const char* key, const std::string& v) {
        body += first ? "\n" : ",\n";
        first = false;
        body += ind + "  " + json_string(key) + ": " + v;
    }
    void str(const char* key, const std::string& v) { raw(key, json_string(v)); }
    void u64(const char* key, uint64_t v) { raw(key, std::to_string(v)); }
    void f64(const char* key, double v) { raw(key, json_f64(v)); }
    void boolean(const char* key, bool v) { raw(key, v ? "true" : "false"); }
    std::string close() const { return first ? "{}" : "{" + body + "\n" + ind + "}"; }
};

std::string indent_lines(const std::string& text, int depth) {
    std::string out;
    const std::string pad((size_t)depth * 2, ' ');
    for (const char ch : text) {
        out.push_back(ch);
        if (ch == '\n') out += pad;
    }
    return out;
}

std::string trim(const std::string& s) {
    size_t a = 0, b = s.size();
    while (a < b && isspace((unsigned char)s[a])) ++a;
    while (b > a && isspace((unsigned char)s[b - 1])) --b;
    return s.substr(a, b - a);
}

// mkdir -p of the directory part of `path`.
std::string make_parent_dirs(const std::string& path) {
    const size_t slash = path.find_last_of('/');
    if (slash == std::string::npos || slash == 0) return "";
    const std::string dir = path.substr(0, slash);
    for (size_t i = 1; i <= dir.size(); ++i) {
        if (i < dir.size() && dir[i] != '/') continue;
        const std::string part = dir.substr(0, i);
        if (mkdir(part.c_str(), 0777) != 0 && errno != EEXIST)
            return "cannot create " + part + ": " + std::strerror(errno);
    }
    return "";
}

}  // namespace

}  // namespace tatara

using namespace tatara;

void TataraExperiment::touch() { last_updated_at = format_utc_iso(now_epoch_secs()); }

std::string TataraExperiment::to_json() const {
    Obj doc(0);
    doc.u64("schema_version", 2);  // SCHEMA_VERSION (experiment.rs:39)
    {
        Obj g(1);
        g.str("name", "tatara");
        g.str("version", generator_version);
        doc.raw("generator", g.close());
    }
    doc.str("id", id);
    doc.str("name", name);
    doc.str("date", date);
    doc.str("status", status);
    doc.str("last_updated_at", last_updated_at);
    if (has_commit) doc.str("commit", commit);
    doc.str("command", command);
    if (has_lineage) {
        Obj l(1);
        if (lineage_has_parent) l.str("parent_id", lineage_parent_id);
        l.str("resumed_from_checkpoint", lineage_checkpoint);
        l.u64("resumed_from_superbatch", lineage_superbatch);
        doc.raw("lineage", l.close());
    }
    doc.raw("params", indent_lines(params_json, 1));
    {
        Obj d(1);
        d.str("name", data_name);
        d.u64("positions", data_positions);
        d.u64("total_positions", data_total_positions);
        d.f64("dataset_passes", data_dataset_passes);
        doc.raw("data", d.close());
    }
    {
        Obj r(1);
        r.u64("training_time_seconds", training_time_seconds);
        r.raw("fv_scale", has_fv_scale ? std::to_string(fv_scale) : "null");
        if (has_target) r.u64("target_superbatches", target_superbatches);
        if (has_best_loss) {
            r.f64("best_loss", best_loss);
            r.u64("best_loss_superbatch", best_loss_superbatch);
        }
        if (has_best_test_loss) {
            r.f64("best_test_loss", best_test_loss);
            r.u64("best_test_loss_superbatch", best_test_loss_superbatch);
        }
        r.u64("mean_pos_per_sec", mean_pos_per_sec);
        r.boolean("interrupted", interrupted);
        doc.raw("results", r.close());
    }
    std::string hist = history.empty() ? "[]" : "[";
    for (size_t i = 0; i < history.size(); ++i) {
        const Entry& e = history[i];
        Obj h(2);
        h.u64("superbatch", e.superbatch);
        h.f64("loss", e.loss);
        if (e.has_test_loss) h.f64("test_loss", e.test_loss);
        if (e.has_test_accuracy) h.f64("test_accuracy", e.test_accuracy);
        hist += (i ? ",\n    " : "\n    ") + h.close();
    }
    if (!history.empty()) hist += "\n  ]";
    doc.raw("history", hist);
    std::string ck = checkpoints.empty() ? "[]" : "[";
    for (size_t i = 0; i < checkpoints.size(); ++i) ck += (i ? ",\n    " : "\n    ") + json_string(checkpoints[i]);
    if (!checkpoints.empty()) ck += "\n  ]";
    doc.raw("checkpoints", ck);
    return doc.close();
}

std::string TataraExperiment::write() const {
    std::string err = make_parent_dirs(path);
    if (!err.empty()) return err;
    const std::string tmp = path + ".tmp";
    const std::string json = to_json() + "\n";
    FILE* f = fopen(tmp.c_str(), "wb");
    if (!f) return "cannot create " + tmp + ": " + std::strerror(errno);
    const bool ok = fwrite(json.data(), 1, json.size(), f) == json.size();
    const int e = errno;
    if (fclose(f) != 0 || !ok) {
        remove(tmp.c_str());
        return "cannot write " + tmp + ": " + std::strerror(ok ? errno : e);
    }
    if (rename(tmp.c_str(), path.c_str()) != 0) {
        const int re = errno;
        remove(tmp.c_str());
        return "cannot rename " + tmp + " to " + path + ": " + std::strerror(re);
    }
    return "";
}

extern "C" int32_t tatara_experiment_create(const TataraExperimentInit* init, TataraExperiment** out) {
    TATARA_REQUIRE(init && out, "experiment_create: null argument");
    TATARA_REQUIRE(init->path && init->id && init->name && init->command && init->params_json && init->data_name,
                   "experiment_create: path, id, name, command, params_json and data_name are required");
    const std::string params = trim(init->params_json);
    TATARA_REQUIRE(params.size() >= 2 && params.front() == '{' && params.back() == '}',
                   "experiment_create: params_json must be a JSON object");
    TATARA_REQUIRE(!init->has_lineage || init->lineage_checkpoint,
                   "experiment_create: a lineage needs its checkpoint name");
    TataraExperiment* e = new (std::nothrow) TataraExperiment();
    if (!e) {
        set_error("experiment_create: out of host memory");
        return kErrOutOfMemory;
    }
    e->path = init->path;
    e->id = init->id;
    e->name = init->name;
    e->date = format_utc_iso(init->start_epoch_secs);
    e->last_updated_at = e->date;
    e->status = "running";
    e->has_commit = init->commit != nullptr;
    if (e->has_commit) e->commit = init->commit;
    e->command = init->command;
    e->generator_version = init->generator_version ? init->generator_version : tatara_version();
    e->has_lineage = init->has_lineage != 0;
    if (e->has_lineage) {
        e->lineage_has_parent = init->lineage_parent_id != nullptr;
        if (e->lineage_has_parent) e->lineage_parent_id = init->lineage_parent_id;
        e->lineage_checkpoint = init->lineage_checkpoint;
        e->lineage_superbatch = init->lineage_superbatch;
    }
    e->params_json = params;
    e->data_name = init->data_name;
    e->data_positions = init->data_positions;
    e->has_fv_scale = init->has_fv_scale != 0;
    e->fv_scale = init->fv_scale;
    *out = e;
    return kOk;
}

extern "C" int32_t tatara_experiment_destroy(TataraExperiment* e) {
    delete e;
    return kOk;
}

extern "C" int32_t tatara_experiment_set_target_superbatches(TataraExperiment* e, uint64_t target) {
    TATARA_REQUIRE(e, "experiment: null handle");
    e->has_target = true;
    e->target_superbatches = target;
    e->touch();
    return kOk;
}

extern "C" int32_t tatara_experiment_record_superbatch(TataraExperiment* e, uint64_t superbatch, double mean_loss,
                                                       uint64_t sb_positions, double elapsed_seconds,
                                                       const double* test_loss, const double* test_accuracy) {
    TATARA_REQUIRE(e, "experiment: null handle");
    e->positions_trained =
        e->positions_trained > UINT64_MAX - sb_positions ? UINT64_MAX : e->positions_trained + sb_positions;
    const bool finite = std::isfinite(mean_loss);
    if (!finite) {
        const char* shown = std::isnan(mean_loss) ? "NaN" : (mean_loss > 0 ? "inf" : "-inf");
        fprintf(stderr,
                "[train] warning: superbatch %llu loss is non-finite (%s); recording 0.0 in experiment.json\n",
                (unsigned long long)superbatch, shown);
    }
    TataraExperiment::Entry h{};
    h.superbatch = superbatch;
    h.loss = finite ? mean_loss : 0.0;
    h.has_test_loss = test_loss && std::isfinite(*test_loss);
    h.test_loss = h.has_test_loss ? *test_loss : 0.0;
    h.has_test_accuracy = test_accuracy && std::isfinite(*test_accuracy);
    h.test_accuracy = h.has_test_accuracy ? *test_accuracy : 0.0;
    e->history.push_back(h);
    if (finite && (!e->has_best_loss || mean_loss < e->best_loss)) {
        e->has_best_loss = true;
        e->best_loss = mean_loss;
        e->best_loss_superbatch = superbatch;
    }
    if (h.has_test_loss && (!e->has_best_test_loss || h.test_loss < e->best_test_loss)) {
        e->has_best_test_loss = true;
        e->best_test_loss = h.test_loss;
        e->best_test_loss_superbatch = superbatch;
    }
    const double elapsed = std::fmax(elapsed_seconds, 0.0);
    e->training_time_seconds = (uint64_t)std::round(elapsed);
    e->mean_pos_per_sec = elapsed > 0.0 ? (uint64_t)std::round((double)e->positions_trained / elapsed) : 0;
    e->data_total_positions = e->positions_trained;
    e->data_dataset_passes = e->data_positions > 0 ? (double)e->positions_trained / (double)e->data_positions : 0.0;
    e->touch();
    return kOk;
}

extern "C" int32_t tatara_experiment_note_checkpoint(TataraExperiment* e, const char* file_name) {
    TATARA_REQUIRE(e && file_name, "experiment_note_checkpoint: null argument");
    e->checkpoints.emplace_back(file_name);
    return kOk;
}

extern "C" int32_t tatara_experiment_mark_finished(TataraExperiment* e, double elapsed_seconds) {
    TATARA_REQUIRE(e, "experiment: null handle");
    e->status = "completed";
    e->training_time_seconds = (uint64_t)std::round(std::fmax(elapsed_seconds, 0.0));
    e->touch();
    return kOk;
}

extern "C" int32_t tatara_experiment_mark_interrupted(TataraExperiment* e) {
    TATARA_REQUIRE(e, "experiment: null handle");
    e->interrupted = true;
    e->touch();
    return kOk;
}

extern "C" int32_t tatara_experiment_write(TataraExperiment* e) {
    TATARA_REQUIRE(e, "experiment: null handle");
    const std::string err = e->write();
    if (!err.empty()) {
        set_error("io error: experiment.json: " + err);
        return kErrInvalid;
    }
    return kOk;
}

extern "C" int32_t tatara_format_utc_iso(uint64_t epoch_secs, char* out) {
    TATARA_REQUIRE(out, "format_utc_iso: null output");
    const std::string s = format_utc_iso(epoch_secs);
    TATARA_REQUIRE(s.size() <= 20, "format_utc_iso: year beyond 9999");
    memcpy(out, s.c_str(), s.size() + 1);
    return kOk;
}

extern "C" int32_t tatara_format_utc_compact(uint64_t epoch_secs, char* out) {
    TATARA_REQUIRE(out, "format_utc_compact: null output");
    const std::string s = format_utc_compact(epoch_secs);
    TATARA_REQUIRE(s.size() <= 16, "format_utc_compact: year beyond 9999");
    memcpy(out, s.c_str(), s.size() + 1);
    return kOk;
}
