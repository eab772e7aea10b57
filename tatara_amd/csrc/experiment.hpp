// Structured run log: one experiment.json per training run
// (crates/nnue-train/src/experiment.rs).  Host code only.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/tatara_hip.h"

namespace tatara {

// Year, month, day, hour, minute, second (UTC) of a UNIX time in seconds
// (civil_from_epoch, experiment.rs:583-603).
struct Civil {
    int64_t year;
    uint32_t month, day, hour, minute, second;
};
Civil civil_from_epoch(uint64_t epoch_secs);
std::string format_utc_iso(uint64_t epoch_secs);      // YYYY-MM-DDTHH:MM:SSZ
std::string format_utc_compact(uint64_t epoch_secs);  // YYYYMMDDtHHMMSSz
uint64_t now_epoch_secs();

// A finite f64 as serde_json writes it (the shortest digits that read back to
// the same value, laid out as the ryu crate does).
std::string json_f64(double v);
std::string json_string(const std::string& s);

}  // namespace tatara

// ExperimentLogger (experiment.rs:356-540): the document and where it goes.
struct TataraExperiment {
    std::string path;
    // ExperimentDoc (experiment.rs:262-292)
    std::string id, name, date, status, last_updated_at, command, generator_version;
    bool has_commit = false;
    std::string commit;
    bool has_lineage = false, lineage_has_parent = false;
    std::string lineage_parent_id, lineage_checkpoint;
    uint64_t lineage_superbatch = 0;
    std::string params_json;  // the caller's "params" object
    // DataInfo
    std::string data_name;
    uint64_t data_positions = 0, data_total_positions = 0;
    double data_dataset_passes = 0.0;
    // Results
    uint64_t training_time_seconds = 0, mean_pos_per_sec = 0;
    bool has_fv_scale = false;
    int32_t fv_scale = 0;
    bool has_target = false;
    uint64_t target_superbatches = 0;
    bool has_best_loss = false;
    double best_loss = 0.0;
    uint64_t best_loss_superbatch = 0;
    bool has_best_test_loss = false;
    double best_test_loss = 0.0;
    uint64_t best_test_loss_superbatch = 0;
    bool interrupted = false;
    struct Entry {
        uint64_t superbatch;
        double loss;
        bool has_test_loss, has_test_accuracy;
        double test_loss, test_accuracy;
    };
    std::vector<Entry> history;
    std::vector<std::string> checkpoints;
    uint64_t positions_trained = 0;

    void touch();
    std::string to_json() const;
    // Writes <path>.tmp and renames it over <path>; an empty string on success,
    // else the error (the caller reports it and carries on).
    std::string write() const;
};
