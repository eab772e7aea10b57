// Learning-rate and WDL-lambda schedules of the superbatch driver
// (crates/nnue-train/src/schedule.rs).  Host code, f32 arithmetic in the
// reference's operation order.
#pragma once

#include <cstdint>

#include "../../include/tatara_hip.h"

namespace tatara {

// f32::powi as Rust lowers it on x86-64 (llvm.powi.f32 -> compiler-rt
// __powisf2): square-and-multiply over the exponent's bits, the reciprocal
// of the product for a negative exponent.
float powi_f32(float a, int32_t b);

float lr_at(const TataraLrSchedule& s, uint64_t batch, uint64_t superbatch);
// Terminal superbatch of the schedule's curve, or false when it has none.
bool lr_horizon(const TataraLrSchedule& s, uint64_t& horizon);
float wdl_at(const TataraWdlSchedule& s, uint64_t batch, uint64_t superbatch, uint64_t max);

}  // namespace tatara
