// Learning-rate / WDL-lambda schedules: LrSchedulerEnum, WarmupLR and
// SequenceLR; WdlSchedulerEnum, WarmupWDL and SequenceWDL
// (crates/nnue-train/src/schedule.rs:23-570).  Every value is computed in f32
// in the reference's order (this file is built with -ffp-contract=off, as
// Rust does not contract); `usize as f32` is a round-to-nearest conversion,
// cos / powf are the C library's cosf / powf that Rust's f32 methods call on
// linux-gnu.
#include "schedule.hpp"

#include <cmath>

#include "common.hpp"

namespace tatara {

namespace {

constexpr float kPi = 3.14159265358979323846f;  // std::f32::consts::PI

float f32(uint64_t n) { return (float)n; }

// cosine_interp (schedule.rs:256-258): start at p = 0, end at p = 1.
float cosine_interp(float start, float end, float p) {
    return end + 0.5f * (start - end) * (1.0f + cosf(kPi * p));
}

float base_lr(const TataraLrSchedule& s, uint64_t superbatch) {
    switch (s.kind) {
        case TATARA_LR_CONSTANT:
            return s.start;
        case TATARA_LR_DROP:  // DropLR (schedule.rs:64-71)
            return superbatch > s.period ? s.start * s.gamma : s.start;
        case TATARA_LR_STEP: {  // StepLR (schedule.rs:92-97): saturating_sub(1) / step
            const uint64_t steps = (superbatch > 0 ? superbatch - 1 : 0) / (s.period ? s.period : 1);
            return s.start * powi_f32(s.gamma, (int32_t)steps);
        }
        case TATARA_LR_LINEAR: {  // LinearDecayLR (schedule.rs:118-125)
            if (superbatch >= s.period) return s.gamma;
            const float lambda = f32(superbatch) / f32(s.period);
            return s.start + lambda * (s.gamma - s.start);
        }
        case TATARA_LR_COSINE: {  // CosineDecayLR (schedule.rs:150-158)
            if (superbatch >= s.period) return s.gamma;
            const float progress = f32(superbatch) / f32(s.period);
            const float lambda = 1.0f - 0.5f * (1.0f + cosf(kPi * progress));
            return s.start + lambda * (s.gamma - s.start);
        }
        case TATARA_LR_EXPONENTIAL: {  // ExponentialDecayLR (schedule.rs:183-190)
            if (superbatch >= s.period) return s.gamma;
            const float lambda = f32(superbatch) / f32(s.period);
            return s.start * powf(s.gamma / s.start, lambda);
        }
        case TATARA_LR_ONE_CYCLE: {  // OneCycleLR (schedule.rs:260-275)
            if (superbatch <= s.period) {
                const float denom = f32(s.period > 1 ? s.period : 1);
                return cosine_interp(s.start, s.max_lr, f32(superbatch) / denom);
            }
            if (superbatch >= s.total) return s.gamma;
            const uint64_t span = s.total - s.period;
            const float denom = f32(span > 1 ? span : 1);
            return cosine_interp(s.max_lr, s.gamma, f32(superbatch - s.period) / denom);
        }
        default:
            return NAN;
    }
}

// WarmupLR (schedule.rs:303-313) around the base curve, then SequenceLR
// (schedule.rs:339-347) handing over to `next` after next_after superbatches.
float lr_of(const TataraLrSchedule& s, uint64_t batch, uint64_t superbatch) {
    if (s.next && superbatch > s.next_after) return lr_of(*s.next, batch, superbatch - s.next_after);
    const float base = base_lr(s, superbatch);
    if (s.warmup_batches > 0 && superbatch == 1 && batch < s.warmup_batches)
        return base / f32(s.warmup_batches - batch);
    return base;
}

float base_wdl(const TataraWdlSchedule& s, uint64_t superbatch, uint64_t max) {
    switch (s.kind) {
        case TATARA_WDL_CONSTANT:
            return s.start;
        case TATARA_WDL_LINEAR: {  // LinearWDL (schedule.rs:465-469)
            const uint64_t span = max > 1 ? max - 1 : 1;  // (max - 1).max(1)
            const float grad = (s.end - s.start) / f32(span);
            return s.start + grad * f32(superbatch - 1);
        }
        default:
            return NAN;
    }
}

float wdl_of(const TataraWdlSchedule& s, uint64_t batch, uint64_t superbatch, uint64_t max) {
    // SequenceWDL (schedule.rs:515-524): the first part sees max = midpoint,
    // the second its own superbatch count and max - midpoint
    if (s.next) {
        if (superbatch <= s.next_after) {
            TataraWdlSchedule first = s;
            first.next = nullptr;
            return wdl_of(first, batch, superbatch, s.next_after);
        }
        return wdl_of(*s.next, batch, superbatch - s.next_after, max - s.next_after);
    }
    const float base = base_wdl(s, superbatch, max);
    if (s.warmup_batches > 0 && superbatch == 1 && batch < s.warmup_batches)
        return base / f32(s.warmup_batches - batch);  // WarmupWDL (schedule.rs:486-493)
    return base;
}

}  // namespace

float powi_f32(float a, int32_t b) {
    const bool recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

float lr_at(const TataraLrSchedule& s, uint64_t batch, uint64_t superbatch) { return lr_of(s, batch, superbatch); }

bool lr_horizon(const TataraLrSchedule& s, uint64_t& horizon) {
    // LrScheduler::horizon (schedule.rs:32-35): warmup passes it through; a
    // sequence keeps the trait's default, none
    if (s.next) return false;
    switch (s.kind) {
        case TATARA_LR_LINEAR:
        case TATARA_LR_COSINE:
        case TATARA_LR_EXPONENTIAL:
            horizon = s.period;
            return true;
        case TATARA_LR_ONE_CYCLE:
            horizon = s.total;
            return true;
        default:
            return false;
    }
}

float wdl_at(const TataraWdlSchedule& s, uint64_t batch, uint64_t superbatch, uint64_t max) {
    return wdl_of(s, batch, superbatch, max);
}

}  // namespace tatara

using namespace tatara;

extern "C" {

int32_t tatara_lr_schedule_one_cycle(float max_lr, float warmup_pct, float div_factor, float final_div_factor,
                                     uint64_t total_superbatch, TataraLrSchedule* out) {
    TATARA_REQUIRE(out, "one-cycle: out is null");
    // OneCycleLR::new (schedule.rs:233-253)
    TataraLrSchedule s{};
    s.kind = TATARA_LR_ONE_CYCLE;
    s.max_lr = max_lr;
    s.start = max_lr / div_factor;
    s.gamma = s.start / final_div_factor;
    float w = roundf(warmup_pct * (float)total_superbatch);  // round half away from zero
    const float hi = (float)total_superbatch;
    w = w < 0.0f ? 0.0f : (w > hi ? hi : w);
    s.period = w != w ? 0 : (uint64_t)w;  // `as usize` saturates, NaN -> 0
    s.total = total_superbatch;
    *out = s;
    return kOk;
}

int32_t tatara_lr_at(const TataraLrSchedule* s, uint64_t batch, uint64_t superbatch, float* lr) {
    TATARA_REQUIRE(s && lr, "lr_at: null argument");
    *lr = lr_at(*s, batch, superbatch);
    return kOk;
}

int32_t tatara_lr_horizon(const TataraLrSchedule* s, uint64_t* horizon, int32_t* has_horizon) {
    TATARA_REQUIRE(s && horizon && has_horizon, "lr_horizon: null argument");
    uint64_t h = 0;
    *has_horizon = lr_horizon(*s, h) ? 1 : 0;
    *horizon = h;
    return kOk;
}

int32_t tatara_wdl_at(const TataraWdlSchedule* s, uint64_t batch, uint64_t superbatch, uint64_t max, float* wdl) {
    TATARA_REQUIRE(s && wdl, "wdl_at: null argument");
    TATARA_REQUIRE(superbatch >= 1, "wdl_at: superbatch is 1-based");
    *wdl = wdl_at(*s, batch, superbatch, max);
    return kOk;
}

}  // extern "C"
