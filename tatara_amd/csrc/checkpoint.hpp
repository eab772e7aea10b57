// Raw resume checkpoints (RNRC v8; see checkpoint.hip).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/tatara_hip.h"

namespace tatara {

class TrainerBase;

// RawCkptArch (bins/nnue_train/src/ckpt.rs:213-226): the identity a checkpoint
// header records and a load checks.
struct CkptArch {
    std::string fs_name;
    uint64_t train_ft_in = 0, ft_out = 0, max_active = 0;
    bool factorize = false;
    uint32_t feature_hash = 0;
    std::string arch_kind;
    bool has_bucket_mode = false;
    std::string bucket_mode;  // "" when the architecture has none
    std::vector<uint64_t> topology;
};

// RawCkptHeader (ckpt.rs:247-265); lr_horizon 0 and an empty run id mean none.
struct CkptHeader {
    uint32_t version = 0;
    uint64_t superbatch = 0, step_count = 0, lr_horizon = 0, num_groups = 0;
    std::string run_id;
};

int32_t ckpt_arch_from_c(const TataraCkptArch& c, CkptArch& a);
std::string ckpt_header_bytes(const CkptArch& a, const std::string& run_id, uint64_t superbatch,
                              uint64_t step_count, uint64_t lr_horizon, uint64_t num_groups);
int32_t save_resume_checkpoint(TrainerBase& t, const char* path, const CkptArch& arch,
                               const std::vector<const char*>& groups, uint64_t superbatch, const char* run_id,
                               uint64_t lr_horizon);
int32_t load_resume_checkpoint(TrainerBase& t, const char* path, const CkptArch& arch,
                               const std::vector<const char*>& groups, TataraCkptHeader* out);

}  // namespace tatara
