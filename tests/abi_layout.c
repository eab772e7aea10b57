/* Layout of the C ABI's structs (include/tatara_hip.h) on x86-64 Linux.
 *
 * Compiled with the host C compiler by tests/test_abi_layout.py (no GPU, no
 * HIP): the static assertions pin the size and field offsets a foreign-language
 * binding must reproduce (the Rust #[repr(C)] structs of the integration guide, the
 * ctypes structs of tatara_amd/_lib.py), and main() prints every field's
 * offset and size so the test can compare those bindings field by field. */
#include <assert.h>
#include <stddef.h>
#include <stdio.h>

#include "../include/tatara_hip.h"

#define CHECK(T, f, off) static_assert(offsetof(T, f) == (off), #T "." #f " moved")

static_assert(sizeof(TataraTrainerConfig) == 88, "TataraTrainerConfig size");
CHECK(TataraTrainerConfig, arch, 0);
CHECK(TataraTrainerConfig, optimizer, 40);
CHECK(TataraTrainerConfig, ft_weight_decay, 44);
CHECK(TataraTrainerConfig, bias_lr_mult, 64);
CHECK(TataraTrainerConfig, keep_grads, 68);
CHECK(TataraTrainerConfig, ft_fp16, 72);
CHECK(TataraTrainerConfig, ft_fp16_out, 76);
CHECK(TataraTrainerConfig, fp16_opt_state, 80);
CHECK(TataraTrainerConfig, tf32, 84);

static_assert(sizeof(TataraLoss) == 44, "TataraLoss size");
CHECK(TataraLoss, scale, 4);
CHECK(TataraLoss, weight_boost_w2, 40);

static_assert(sizeof(TataraBatch) == 64, "TataraBatch size");
CHECK(TataraBatch, stm_indices, 8);
CHECK(TataraBatch, bucket_idx, 32);
CHECK(TataraBatch, wdl, 48);
CHECK(TataraBatch, on_device, 56);

static_assert(sizeof(TataraCkptHeader) == 312, "TataraCkptHeader size");
CHECK(TataraCkptHeader, superbatch, 8);
CHECK(TataraCkptHeader, header_bytes, 40);
CHECK(TataraCkptHeader, run_id, 48);

static_assert(sizeof(TataraRunConfig) == 136, "TataraRunConfig size");
CHECK(TataraRunConfig, start_superbatch, 32);
CHECK(TataraRunConfig, has_fv_scale, 72);
CHECK(TataraRunConfig, keep_raw_checkpoints, 88);
CHECK(TataraRunConfig, progress_weights, 112);
CHECK(TataraRunConfig, print_progress, 120);
CHECK(TataraRunConfig, experiment, 128);

static_assert(sizeof(TataraExperimentInit) == 120, "TataraExperimentInit size");
CHECK(TataraExperimentInit, start_epoch_secs, 24);
CHECK(TataraExperimentInit, has_lineage, 56);
CHECK(TataraExperimentInit, lineage_parent_id, 64);
CHECK(TataraExperimentInit, params_json, 88);
CHECK(TataraExperimentInit, has_fv_scale, 112);
CHECK(TataraExperimentInit, fv_scale, 116);

#define F(T, f) printf("%s %s %zu %zu\n", #T, #f, offsetof(T, f), sizeof(((T*)0)->f))
#define S(T) printf("%s sizeof %zu %zu\n", #T, (size_t)0, sizeof(T))

int main(void) {
    S(TataraTrainerConfig);
    F(TataraTrainerConfig, arch); F(TataraTrainerConfig, device); F(TataraTrainerConfig, max_batch);
    F(TataraTrainerConfig, ft_in); F(TataraTrainerConfig, max_active); F(TataraTrainerConfig, piece_inputs);
    F(TataraTrainerConfig, ft_out); F(TataraTrainerConfig, l1_out); F(TataraTrainerConfig, l2_out);
    F(TataraTrainerConfig, num_buckets); F(TataraTrainerConfig, optimizer);
    F(TataraTrainerConfig, ft_weight_decay); F(TataraTrainerConfig, dense_weight_decay);
    F(TataraTrainerConfig, bias_weight_decay); F(TataraTrainerConfig, ft_lr_mult);
    F(TataraTrainerConfig, dense_lr_mult); F(TataraTrainerConfig, bias_lr_mult);
    F(TataraTrainerConfig, keep_grads); F(TataraTrainerConfig, ft_fp16); F(TataraTrainerConfig, ft_fp16_out);
    F(TataraTrainerConfig, fp16_opt_state); F(TataraTrainerConfig, tf32);

    S(TataraLoss);
    F(TataraLoss, kind); F(TataraLoss, scale); F(TataraLoss, nnue2score); F(TataraLoss, in_scaling);
    F(TataraLoss, in_offset); F(TataraLoss, target_offset); F(TataraLoss, target_scaling);
    F(TataraLoss, pow_exp); F(TataraLoss, qp_asymmetry); F(TataraLoss, weight_boost_w1);
    F(TataraLoss, weight_boost_w2);

    S(TataraBatch);
    F(TataraBatch, n_pos); F(TataraBatch, max_active); F(TataraBatch, stm_indices);
    F(TataraBatch, nstm_indices); F(TataraBatch, nnz); F(TataraBatch, bucket_idx); F(TataraBatch, score);
    F(TataraBatch, wdl); F(TataraBatch, on_device);

    S(TataraCkptHeader);
    F(TataraCkptHeader, version); F(TataraCkptHeader, superbatch); F(TataraCkptHeader, step_count);
    F(TataraCkptHeader, lr_horizon); F(TataraCkptHeader, num_groups); F(TataraCkptHeader, header_bytes);
    F(TataraCkptHeader, run_id);

    S(TataraCkptArch);
    F(TataraCkptArch, feature_set); F(TataraCkptArch, ft_factorize); F(TataraCkptArch, arch);
    F(TataraCkptArch, bucket_mode); F(TataraCkptArch, ft_out); F(TataraCkptArch, l1_out);
    F(TataraCkptArch, l2_out); F(TataraCkptArch, num_buckets);

    S(TataraRunConfig);
    F(TataraRunConfig, data_path); F(TataraRunConfig, output_dir); F(TataraRunConfig, net_id);
    F(TataraRunConfig, run_id); F(TataraRunConfig, start_superbatch); F(TataraRunConfig, end_superbatch);
    F(TataraRunConfig, batches_per_superbatch); F(TataraRunConfig, batch_size); F(TataraRunConfig, save_rate);
    F(TataraRunConfig, has_fv_scale); F(TataraRunConfig, fv_scale); F(TataraRunConfig, has_keep_raw);
    F(TataraRunConfig, keep_raw_checkpoints); F(TataraRunConfig, feature_set); F(TataraRunConfig, bucket_mode);
    F(TataraRunConfig, num_buckets); F(TataraRunConfig, progress_weights); F(TataraRunConfig, print_progress);
    F(TataraRunConfig, experiment);

    S(TataraExperimentInit);
    F(TataraExperimentInit, path); F(TataraExperimentInit, id); F(TataraExperimentInit, name);
    F(TataraExperimentInit, start_epoch_secs); F(TataraExperimentInit, commit); F(TataraExperimentInit, command);
    F(TataraExperimentInit, generator_version); F(TataraExperimentInit, has_lineage);
    F(TataraExperimentInit, lineage_parent_id); F(TataraExperimentInit, lineage_checkpoint);
    F(TataraExperimentInit, lineage_superbatch); F(TataraExperimentInit, params_json);
    F(TataraExperimentInit, data_name); F(TataraExperimentInit, data_positions);
    F(TataraExperimentInit, has_fv_scale); F(TataraExperimentInit, fv_scale);

    S(TataraRunSuperbatch);
    F(TataraRunSuperbatch, superbatch); F(TataraRunSuperbatch, positions); F(TataraRunSuperbatch, loss_sum);
    F(TataraRunSuperbatch, mean_loss); F(TataraRunSuperbatch, seconds); F(TataraRunSuperbatch, lr);
    F(TataraRunSuperbatch, wdl); F(TataraRunSuperbatch, saved);

    S(TataraLrSchedule);
    F(TataraLrSchedule, kind); F(TataraLrSchedule, start); F(TataraLrSchedule, gamma); F(TataraLrSchedule, max_lr);
    F(TataraLrSchedule, period); F(TataraLrSchedule, total); F(TataraLrSchedule, warmup_batches);
    F(TataraLrSchedule, next); F(TataraLrSchedule, next_after);

    S(TataraControlState);
    F(TataraControlState, effective_target); F(TataraControlState, ignored_stale_target);
    F(TataraControlState, has_ignored_stale);

    S(TataraWdlSchedule);
    F(TataraWdlSchedule, kind); F(TataraWdlSchedule, start); F(TataraWdlSchedule, end);
    F(TataraWdlSchedule, warmup_batches); F(TataraWdlSchedule, next); F(TataraWdlSchedule, next_after);
    return 0;
}
