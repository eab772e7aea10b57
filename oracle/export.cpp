// CPU oracle for the quantised network export (.bin).
//
// TEST INFRASTRUCTURE ONLY.  The checker for the HIP product path
// (tatara_amd/csrc/export.hip); only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it.
//
// Restates, in the reference's order of operations and with Rust's numeric
// semantics (f64 `round` = half away from zero; `as` casts saturate and send
// NaN to 0):
//   - encode_signed_leb128 / write_leb128_tensor_i16 / decode_single_leb128
//     (crates/nnue-format/src/layerstack_weights.rs:120-223);
//   - pad32 (:105-108);
//   - build_arch_str / features_token (:242-343) without the PSQT, threat and
//     effect-bucket tokens (those feature extensions are not on this path);
//   - compute_fc_hash / ft_hash / network_hash (:351-399);
//   - coalesce_ft_factorized, Base mode (:412-491);
//   - LayerStackWeights::save_quantised (:568-829) and clamp_i8 (:1306-1314);
//   - simple_fv_scale, arch_identity / build_arch_str, compute_fc_hash,
//     ft_hash, network_hash, SimpleWeights::save_quantised and its
//     clamp_round / write_* helpers (crates/nnue-format/src/simple_weights.rs:
//     90-95, :254-340, :374-429, :545-690);
//   - layerstack_export_fv_scale (bins/nnue_train/src/training.rs:72-86).

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

namespace {

// Rust `f64 as iN`: NaN -> 0, saturating at the type's bounds, else truncation.
template <typename T>
T rust_cast(double v) {
    if (std::isnan(v)) return 0;
    const double lo = (double)std::numeric_limits<T>::min();
    const double hi = (double)std::numeric_limits<T>::max();
    if (v <= lo) return std::numeric_limits<T>::min();
    if (v >= hi) return std::numeric_limits<T>::max();
    return (T)v;
}

// f64::clamp(min, max): NaN stays NaN.
double rust_clamp(double v, double lo, double hi) {
    if (std::isnan(v)) return v;
    if (v < lo) return lo;
    if (v > hi) return hi;
    return v;
}

// layerstack_weights.rs clamp_i8
int8_t ls_clamp_i8(double v) {
    if (v < -128.0) return -128;
    if (v > 127.0) return 127;
    return rust_cast<int8_t>(v);
}

// simple_weights.rs clamp_round
double simple_clamp_round(double v, double lo, double hi) {
    const double r = std::round(v);
    if (r < lo) return lo;
    if (r > hi) return hi;
    return r;
}

struct Writer {
    std::vector<uint8_t> b;
    void u8(uint8_t v) { b.push_back(v); }
    void u32(uint32_t v) {
        for (int i = 0; i < 4; ++i) b.push_back((uint8_t)(v >> (8 * i)));
    }
    void i32(int32_t v) { u32((uint32_t)v); }
    void i16(int16_t v) {
        b.push_back((uint8_t)((uint16_t)v & 0xff));
        b.push_back((uint8_t)((uint16_t)v >> 8));
    }
    void bytes(const void* p, size_t n) {
        const uint8_t* c = (const uint8_t*)p;
        b.insert(b.end(), c, c + n);
    }
};

void leb128(int64_t val, std::vector<uint8_t>& out) {
    int64_t value = val;
    for (;;) {
        const uint8_t byte = (uint8_t)(value & 0x7f);
        value >>= 7;  // arithmetic shift
        const bool sign_bit = (byte & 0x40) != 0;
        const bool more = (value != 0 || sign_bit) && (value != -1 || !sign_bit);
        if (more) {
            out.push_back(byte | 0x80);
        } else {
            out.push_back(byte);
            return;
        }
    }
}

void write_leb128_tensor_i16(Writer& w, const std::vector<int16_t>& v) {
    std::vector<uint8_t> c;
    c.reserve(v.size() * 2);
    for (int16_t x : v) leb128(x, c);
    w.bytes("COMPRESSED_LEB128", 17);
    w.u32((uint32_t)c.size());
    w.bytes(c.data(), c.size());
}

uint64_t pad32(uint64_t x) { return (x + 31) / 32 * 32; }

uint32_t fc_hash_chain(uint32_t input_slice, const uint64_t* outs, const bool* relu, int n) {
    uint32_t prev = 0xEC42E90Du;
    prev ^= input_slice;
    for (int i = 0; i < n; ++i) {
        uint32_t h = 0xCC03DAE4u;
        h += (uint32_t)outs[i];
        h ^= prev >> 1;
        h ^= prev << 31;
        if (relu[i]) h += 0x538D24C7u;
        prev = h;
    }
    return prev;
}

uint32_t ls_fc_hash(uint64_t ft_out, uint64_t l2_out) {
    const uint64_t outs[3] = {ft_out, l2_out, 1};
    const bool relu[3] = {true, true, false};
    return fc_hash_chain((uint32_t)(ft_out * 2), outs, relu, 3);
}

uint32_t simple_fc_hash(uint64_t l1_input, uint64_t l1_out, uint64_t l2_out) {
    const uint64_t outs[3] = {l1_out, l2_out, 1};
    const bool relu[3] = {true, true, false};
    return fc_hash_chain((uint32_t)l1_input, outs, relu, 3);
}

uint32_t ft_hash(uint32_t feature_hash, uint64_t ft_out) { return feature_hash ^ (uint32_t)(ft_out * 2); }

std::string ls_arch(const char* name, uint64_t input_size, uint64_t ft_out, uint64_t l1_out,
                    uint64_t l2_in, uint64_t l2_out, bool has_fv, int32_t fv) {
    char buf[1024];
    const unsigned long long F2 = ft_out * 2;
    std::snprintf(buf, sizeof buf,
                  "Features=%s(Friend)[%llu->%llux2],"
                  "Network=AffineTransform[1<-%llu](ClippedReLU[%llu](AffineTransform[%llu<-%llu]("
                  "SqrClippedReLU[%llu](AffineTransform[%llu<-%llu](InputSlice[%llu(0:%llu)])))))",
                  name, (unsigned long long)input_size, (unsigned long long)ft_out,
                  (unsigned long long)l2_out, (unsigned long long)l2_out, (unsigned long long)l2_out,
                  (unsigned long long)l2_in, (unsigned long long)l2_in, (unsigned long long)l1_out, F2,
                  F2, F2);
    std::string s(buf);
    if (has_fv) s += ",fv_scale=" + std::to_string(fv);
    return s;
}

// activation: 0 CReLU, 1 SCReLU, 2 Pairwise
uint64_t simple_combined_dim(uint64_t ft_out, int act) { return 2 * ft_out / (act == 2 ? 2 : 1); }

std::string simple_identity(const char* name, uint64_t ft_in, uint64_t ft_out, uint64_t l1_out,
                            uint64_t l2_out, int act) {
    char blk[128];
    if (act == 2)
        std::snprintf(blk, sizeof blk, "[%llu->%llu/2x2]-Pairwise", (unsigned long long)ft_in,
                      (unsigned long long)ft_out);
    else
        std::snprintf(blk, sizeof blk, "[%llu->%llux2]", (unsigned long long)ft_in, (unsigned long long)ft_out);
    const char* a = act == 1 ? "SqrClippedReLU" : "ClippedReLU";
    const unsigned long long li = simple_combined_dim(ft_out, act);
    char buf[1024];
    std::snprintf(buf, sizeof buf,
                  "Features=%s(Friend)%s,Network=AffineTransform[1<-%llu](%s[%llu](AffineTransform[%llu<-%llu]("
                  "%s[%llu](AffineTransformSparseInput[%llu<-%llu](InputSlice[%llu(0:%llu)])))))",
                  name, blk, (unsigned long long)l2_out, a, (unsigned long long)l2_out,
                  (unsigned long long)l2_out, (unsigned long long)l1_out, a, (unsigned long long)l1_out,
                  (unsigned long long)l1_out, li, li, li);
    return buf;
}

int64_t finish(const Writer& w, uint8_t* out, int64_t cap) {
    const int64_t n = (int64_t)w.b.size();
    if (out && n <= cap) std::memcpy(out, w.b.data(), (size_t)n);
    return n;
}

}  // namespace

extern "C" {

int64_t orc_leb128_encode(const int64_t* v, int64_t n, uint8_t* out) {
    std::vector<uint8_t> c;
    for (int64_t i = 0; i < n; ++i) leb128(v[i], c);
    if (out) std::memcpy(out, c.data(), c.size());
    return (int64_t)c.size();
}

// decode_single_leb128: 0 ok, -1 unexpected end, -2 overflow.
int32_t orc_leb128_decode_one(const uint8_t* data, int64_t len, int64_t* value, int64_t* consumed) {
    int64_t result = 0;
    int shift = 0;
    int64_t pos = 0;
    for (;;) {
        if (pos >= len) return -1;
        const uint8_t b = data[pos++];
        result |= (int64_t)((uint64_t)(b & 0x7f) << shift);
        shift += 7;
        if ((b & 0x80) == 0) {
            if (shift < 64 && (b & 0x40) != 0) result |= (int64_t)(~0ull << shift);
            *value = result;
            *consumed = pos;
            return 0;
        }
        if (shift >= 64) return -2;
    }
}

// Decodes a whole compressed block (no magic/size) into i16 values; returns the count or <0.
int64_t orc_leb128_decode_i16(const uint8_t* data, int64_t len, int16_t* out, int64_t cap) {
    int64_t pos = 0, n = 0;
    while (pos < len) {
        int64_t v, c;
        const int32_t rc = orc_leb128_decode_one(data + pos, len - pos, &v, &c);
        if (rc) return rc;
        if (n < cap) out[n] = (int16_t)v;
        ++n;
        pos += c;
    }
    return n;
}

// Quantisers of the two exporters.  kind: 0 LS FT i16 (round.clamp as i16),
// 1 LS clamp_i8, 2 LS bias (round as i32), 3 Simple i16 clamp_round,
// 4 Simple i8 clamp_round, 5 Simple i32 clamp_round.
void orc_quantise(const float* v, int64_t n, double scale, int32_t kind, int64_t* out) {
    for (int64_t i = 0; i < n; ++i) {
        const double x = scale * (double)v[i];
        int64_t q = 0;
        switch (kind) {
            case 0: q = rust_cast<int16_t>(rust_clamp(std::round(x), -32768.0, 32767.0)); break;
            case 1: q = ls_clamp_i8(std::round(x)); break;
            case 2: q = rust_cast<int32_t>(std::round(x)); break;
            case 3: q = rust_cast<int16_t>(simple_clamp_round(x, -32768.0, 32767.0)); break;
            case 4: q = rust_cast<int8_t>(simple_clamp_round(x, -128.0, 127.0)); break;
            case 5: q = rust_cast<int32_t>(simple_clamp_round(x, -2147483648.0, 2147483647.0)); break;
        }
        out[i] = q;
    }
}

uint64_t orc_pad32(uint64_t x) { return pad32(x); }
uint32_t orc_ls_fc_hash(uint64_t ft_out, uint64_t l2_out) { return ls_fc_hash(ft_out, l2_out); }
uint32_t orc_ls_network_hash(uint32_t feature_hash, uint64_t ft_out, uint64_t l2_out) {
    return ls_fc_hash(ft_out, l2_out) ^ ft_hash(feature_hash, ft_out);
}
uint32_t orc_simple_fc_hash(uint64_t l1_input, uint64_t l1_out, uint64_t l2_out) {
    return simple_fc_hash(l1_input, l1_out, l2_out);
}
uint32_t orc_simple_network_hash(uint32_t feature_hash, uint64_t ft_out, uint64_t l1_out, uint64_t l2_out,
                                 int32_t act) {
    return simple_fc_hash(simple_combined_dim(ft_out, act), l1_out, l2_out) ^ ft_hash(feature_hash, ft_out);
}

int64_t orc_ls_arch_str(const char* name, uint64_t input_size, uint64_t ft_out, uint64_t l1_out, uint64_t l2_in,
                        uint64_t l2_out, int32_t has_fv, int32_t fv, char* out, int64_t cap) {
    const std::string s = ls_arch(name, input_size, ft_out, l1_out, l2_in, l2_out, has_fv != 0, fv);
    if (out && (int64_t)s.size() < cap) std::memcpy(out, s.c_str(), s.size() + 1);
    return (int64_t)s.size();
}

int64_t orc_simple_arch_str(const char* name, uint64_t ft_in, uint64_t ft_out, uint64_t l1_out,
                            uint64_t l2_out, int32_t act, int32_t fv, char* out, int64_t cap) {
    const std::string s = simple_identity(name, ft_in, ft_out, l1_out, l2_out, act) + ",fv_scale=" +
                          std::to_string(fv);
    if (out && (int64_t)s.size() < cap) std::memcpy(out, s.c_str(), s.size() + 1);
    return (int64_t)s.size();
}

// simple_fv_scale: ((127 * 64) as f32 / scale).round() as i32
int32_t orc_simple_fv_scale(float scale) {
    const float q = (float)(127 * 64) / scale;
    return rust_cast<int32_t>((double)std::round(q));
}

// layerstack_export_fv_scale: override, else Sigmoid -> round(8128 / scale) (f32), Wrm -> None.
int32_t orc_ls_export_fv_scale(int32_t has_override, int32_t override_value, int32_t loss_kind,
                               float score_scale, int32_t* value) {
    if (has_override) {
        *value = override_value;
        return 1;
    }
    if (loss_kind == 0) {
        *value = rust_cast<int32_t>((double)std::round((float)(127 * 64) / score_scale));
        return 1;
    }
    return 0;
}

// coalesce_ft_factorized, Base mode: out[f][o] = w[f][o] + w[ft_in + f % pi][o] (f32 add).
void orc_coalesce(const float* w, int64_t ft_in, int64_t pi, int64_t ft_out, float* out) {
    for (int64_t f = 0; f < ft_in; ++f)
        for (int64_t o = 0; o < ft_out; ++o) {
            float x = w[f * ft_out + o];
            if (pi > 0) x += w[(ft_in + f % pi) * ft_out + o];
            out[f * ft_out + o] = x;
        }
}

// LayerStackWeights::save_quantised (no PSQT / threat).  ft_w is the export-shape
// table (already coalesced).  Returns the file size; bytes are copied when out
// is non-null and the size fits cap.
int64_t orc_ls_save_quantised(const char* name, uint32_t feature_hash, uint64_t ft_in, uint64_t ft_out,
                              uint64_t l1_out, uint64_t l2_out, uint64_t nb, const float* ft_w,
                              const float* ft_b, const float* l1_w, const float* l1_b, const float* l1s_w,
                              const float* l1s_b, const float* l2_w, const float* l2_b, const float* l3_w,
                              const float* l3_b, int32_t has_fv, int32_t fv, uint8_t* out, int64_t cap) {
    const uint64_t l2_in = (l1_out - 1) * 2;
    Writer w;
    w.u32(0x7AF32F21u);
    w.u32(ls_fc_hash(ft_out, l2_out) ^ ft_hash(feature_hash, ft_out));
    const std::string arch = ls_arch(name, ft_in, ft_out, l1_out, l2_in, l2_out, has_fv != 0, fv);
    w.u32((uint32_t)arch.size());
    w.bytes(arch.data(), arch.size());
    w.u32((uint32_t)nb);
    w.u32(ft_hash(feature_hash, ft_out));
    const double qa = 127.0;
    {
        std::vector<int16_t> q(ft_out);
        for (uint64_t i = 0; i < ft_out; ++i)
            q[i] = rust_cast<int16_t>(rust_clamp(std::round(qa * (double)ft_b[i]), -32768.0, 32767.0));
        write_leb128_tensor_i16(w, q);
    }
    {
        std::vector<int16_t> q(ft_in * ft_out);
        for (uint64_t i = 0; i < ft_in * ft_out; ++i)
            q[i] = rust_cast<int16_t>(rust_clamp(std::round(qa * (double)ft_w[i]), -32768.0, 32767.0));
        write_leb128_tensor_i16(w, q);
    }
    const double qb = 64.0, bias_scale = 8128.0;
    const uint32_t fch = ls_fc_hash(ft_out, l2_out);
    for (uint64_t b = 0; b < nb; ++b) {
        w.u32(fch);
        for (uint64_t o = 0; o < l1_out; ++o) {
            const float merged = l1_b[b * l1_out + o] + l1s_b[o];
            w.i32(rust_cast<int32_t>(std::round(bias_scale * (double)merged)));
        }
        for (uint64_t o = 0; o < l1_out; ++o)
            for (uint64_t i = 0; i < pad32(ft_out); ++i) {
                int8_t q = 0;
                if (i < ft_out) {
                    const float merged = l1_w[b * l1_out * ft_out + o * ft_out + i] + l1s_w[i * l1_out + o];
                    q = ls_clamp_i8(std::round(qb * (double)merged));
                }
                w.u8((uint8_t)q);
            }
        for (uint64_t o = 0; o < l2_out; ++o)
            w.i32(rust_cast<int32_t>(std::round(127.0 * qb * (double)l2_b[b * l2_out + o])));
        for (uint64_t o = 0; o < l2_out; ++o)
            for (uint64_t i = 0; i < pad32(l2_in); ++i) {
                int8_t q = 0;
                if (i < l2_in) q = ls_clamp_i8(std::round(qb * (double)l2_w[b * l2_out * l2_in + o * l2_in + i]));
                w.u8((uint8_t)q);
            }
        w.i32(rust_cast<int32_t>(std::round(127.0 * qb * (double)l3_b[b])));
        for (uint64_t i = 0; i < pad32(l2_out); ++i) {
            int8_t q = 0;
            if (i < l2_out) q = ls_clamp_i8(std::round(qb * (double)l3_w[b * l2_out + i]));
            w.u8((uint8_t)q);
        }
    }
    return finish(w, out, cap);
}

// SimpleWeights::save_quantised.  l1_w is (l1_out, combined_dim) and l2_w is
// (l2_out, l1_out), both out-major as SimpleWeights holds them.
int64_t orc_simple_save_quantised(const char* name, uint32_t feature_hash, uint64_t ft_in, uint64_t ft_out,
                                  uint64_t l1_out, uint64_t l2_out, int32_t act, int32_t fv,
                                  const float* ft_w, const float* ft_b, const float* l1_w, const float* l1_b,
                                  const float* l2_w, const float* l2_b, const float* l3_w, const float* l3_b,
                                  uint8_t* out, int64_t cap) {
    const uint64_t l1_in = simple_combined_dim(ft_out, act);
    Writer w;
    w.u32(0x7AF32F16u);
    w.u32(simple_fc_hash(l1_in, l1_out, l2_out) ^ ft_hash(feature_hash, ft_out));
    const std::string arch = simple_identity(name, ft_in, ft_out, l1_out, l2_out, act) + ",fv_scale=" +
                             std::to_string(fv);
    w.u32((uint32_t)arch.size());
    w.bytes(arch.data(), arch.size());
    w.u32(ft_hash(feature_hash, ft_out));
    const double qa = act == 1 ? 255.0 : 127.0;
    for (uint64_t i = 0; i < ft_out; ++i)
        w.i16(rust_cast<int16_t>(simple_clamp_round(qa * (double)ft_b[i], -32768.0, 32767.0)));
    for (uint64_t i = 0; i < ft_in * ft_out; ++i)
        w.i16(rust_cast<int16_t>(simple_clamp_round(qa * (double)ft_w[i], -32768.0, 32767.0)));
    w.u32(simple_fc_hash(l1_in, l1_out, l2_out));
    const double bs = 127.0 * 64.0, ws = 64.0;
    auto bias = [&](const float* v, uint64_t n) {
        for (uint64_t i = 0; i < n; ++i)
            w.i32(rust_cast<int32_t>(simple_clamp_round(bs * (double)v[i], -2147483648.0, 2147483647.0)));
    };
    auto weight = [&](const float* v, uint64_t out_dim, uint64_t in_dim) {
        for (uint64_t o = 0; o < out_dim; ++o)
            for (uint64_t i = 0; i < pad32(in_dim); ++i) {
                int8_t q = 0;
                if (i < in_dim) q = rust_cast<int8_t>(simple_clamp_round(ws * (double)v[o * in_dim + i], -128.0, 127.0));
                w.u8((uint8_t)q);
            }
    };
    bias(l1_b, l1_out);
    weight(l1_w, l1_out, l1_in);
    bias(l2_b, l2_out);
    weight(l2_w, l2_out, l1_out);
    bias(l3_b, 1);
    weight(l3_w, 1, l2_out);
    return finish(w, out, cap);
}

}  // extern "C"
