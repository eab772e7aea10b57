// Seeded weight initialisation, restating crates/nnue-train/src/init.rs:109-209
// (XorShift + sample) and the default specs LayerStackInit::default_uniform /
// SimpleInit::default_uniform (init.rs:211-310).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace tatara {

enum class InitDist { Zeroed, Uniform };

struct LayerInit {
    InitDist dist;
    bool fan_in;  // scale = sqrt(gain / fan_in) instead of an absolute half width
    float value;  // half width or gain
    uint64_t seed;
};

// init::sample for Dist::Zeroed / Dist::Uniform without per-bucket repeat.
inline std::vector<float> init_sample(uint64_t n, uint64_t fan_in, const LayerInit& li) {
    std::vector<float> out(n, 0.0f);
    if (li.dist == InitDist::Zeroed) return out;
    float mag = li.value;
    if (li.fan_in) {
        const float f = (float)(fan_in < 1 ? 1 : fan_in);
        mag = std::sqrt(li.value / f);
    }
    uint64_t s = li.seed > 1 ? li.seed : 1;
    for (uint64_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        const float u = (float)(s >> 11) / (float)(1ULL << 53);
        out[i] = (u * 2.0f - 1.0f) * mag;
    }
    return out;
}

// LayerStackInit::default_uniform (init.rs:252-266): seeds 0x100..0x104.
struct LayerStackInitSpec {
    LayerInit ft_w{InitDist::Uniform, true, 1.0f, 0x100};
    LayerInit ft_b{InitDist::Zeroed, false, 0.0f, 0};
    LayerInit l1_w{InitDist::Uniform, false, 0.01f, 0x101};
    LayerInit l1_b{InitDist::Zeroed, false, 0.0f, 0};
    LayerInit l1s_w{InitDist::Uniform, false, 0.01f, 0x102};
    LayerInit l1s_b{InitDist::Zeroed, false, 0.0f, 0};
    LayerInit l2_w{InitDist::Uniform, false, 0.01f, 0x103};
    LayerInit l2_b{InitDist::Zeroed, false, 0.0f, 0};
    LayerInit l3_w{InitDist::Uniform, false, 0.01f, 0x104};
    LayerInit l3_b{InitDist::Zeroed, false, 0.0f, 0};
};

// SimpleInit::default_uniform (init.rs:290-303): +-0.01, seeds 0x5071e001..8.
struct SimpleInitSpec {
    LayerInit ft_w{InitDist::Uniform, false, 0.01f, 0x5071e001};
    LayerInit ft_b{InitDist::Uniform, false, 0.01f, 0x5071e002};
    LayerInit l1_w{InitDist::Uniform, false, 0.01f, 0x5071e003};
    LayerInit l1_b{InitDist::Uniform, false, 0.01f, 0x5071e004};
    LayerInit l2_w{InitDist::Uniform, false, 0.01f, 0x5071e005};
    LayerInit l2_b{InitDist::Uniform, false, 0.01f, 0x5071e006};
    LayerInit l3_w{InitDist::Uniform, false, 0.01f, 0x5071e007};
    LayerInit l3_b{InitDist::Uniform, false, 0.01f, 0x5071e008};
};

}  // namespace tatara
