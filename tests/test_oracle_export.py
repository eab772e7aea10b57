"""Export oracle (oracle/export.cpp) pinned against known answers.

Independent pins, not restatements of the oracle's own formulas:
  - signed LEB128 byte strings from the DWARF specification's examples and
    the reference's LEB128 tests (layerstack_weights.rs:1668-1695);
  - pad32 values (layerstack_weights.rs:1697-1707);
  - arch-string substrings (layerstack_weights.rs:2413-2457);
  - the network hash of YaneuraOu's published HalfKP 256x2-32-32 evaluation
    files (0x3E5AA6EE), which the Simple exporter's hash chain must reproduce;
  - the fc_hash dependence test (layerstack_weights.rs:2392-2411);
  - the coalesce known answer (layerstack_weights.rs:1449-1480);
  - rounding/saturation boundaries (layerstack_weights.rs:1628-1661):
    half away from zero, saturating casts, NaN -> 0;
  - whole-file structure: size by formula, every field parsed back, and the
    dequantised values within half a quantum of the weights.
"""
import numpy as np
import pytest

from oracle import export as ox
from oracle import features as of

# DWARF v4, 7.6 (signed LEB128 examples) and the reference's round-trip cases.
DWARF = {2: "02", -2: "7e", 127: "ff00", -127: "817f", 128: "8001", -128: "807f", 129: "8101", -129: "ff7e",
         0: "00", -123456: "c0bb78"}


def test_leb128_known_encodings():
    for v, hexs in DWARF.items():
        assert ox.leb128_encode([v]).hex() == hexs, v


def test_leb128_roundtrip_and_lengths():
    cases = [-65, -64, -1, 0, 1, 63, 64, 127, 128, 32767, -32768, 8191, 8192, -8192, -8193]
    for v in cases:
        b = ox.leb128_encode([v])
        val, used = ox.leb128_decode_one(b)
        assert (val, used) == (v, len(b))
        # length classes of an i16: [-64, 63] one byte, [-8192, 8191] two, else three
        assert len(b) == (1 if -64 <= v <= 63 else 2 if -8192 <= v <= 8191 else 3), v
    vals = np.array([0, 1, -1, 127, -128, 32767, -32768, 100, -100], np.int16)
    assert np.array_equal(ox.leb128_decode_i16(ox.leb128_encode(vals)), vals)
    # every i16 round-trips
    allv = np.arange(-32768, 32768, dtype=np.int64)
    assert np.array_equal(ox.leb128_decode_i16(ox.leb128_encode(allv)), allv.astype(np.int16))
    with pytest.raises(ValueError):
        ox.leb128_decode_one(b"\x80")


def test_pad32():
    assert [ox.pad32(x) for x in (0, 1, 30, 32, 33, 1536)] == [0, 32, 32, 32, 64, 1536]


def test_arch_strings():
    s = ox.ls_arch_str("HalfKaHmMerged", 73305, 1536, 16, 30, 32, 28)
    for sub in ("HalfKaHmMerged", "73305->1536x2", "AffineTransform[1<-32]", "ClippedReLU[32]",
                "AffineTransform[32<-30]", "SqrClippedReLU[30]", "AffineTransform[16<-3072]",
                "InputSlice[3072(0:3072)]", "fv_scale=28"):
        assert sub in s, sub
    assert "PSQT=" not in s and "Threat=" not in s
    s2 = ox.ls_arch_str("HalfKaHmMerged", 73305, 1536, 16, 30, 32, None)
    assert "fv_scale" not in s2 and s == s2 + ",fv_scale=28"
    # Simple: the YaneuraOu halfkp_256x2-32-32 topology (with the sparse-input L1 token)
    s3 = ox.simple_arch_str("HalfKP", 125388, 256, 32, 32, 28)
    assert s3.startswith("Features=HalfKP(Friend)[125388->256x2],Network=AffineTransform[1<-32](")
    assert "AffineTransformSparseInput[32<-512](InputSlice[512(0:512)])" in s3
    assert s3.endswith(")))))" + ",fv_scale=28")
    assert "[125388->256/2x2]-Pairwise" in ox.simple_arch_str("HalfKP", 125388, 256, 32, 32, 28, "pairwise")
    assert "SqrClippedReLU[32]" in ox.simple_arch_str("HalfKP", 125388, 256, 32, 32, 28, "screlu")


def test_hashes():
    halfkp = of.feature_set_info("halfkp")
    assert halfkp["ft_in"] == 125388
    # YaneuraOu's published HalfKP(Friend)[125388->256x2]-32-32 network hash
    assert ox.simple_network_hash(0x5D69D5B8, 256, 32, 32) == 0x3E5AA6EE
    h = ox.ls_fc_hash(1536, 32)
    assert h != 0 and h != ox.ls_fc_hash(3072, 32) and h != ox.ls_fc_hash(1536, 64)
    assert ox.ls_network_hash(0x7F134CB8, 1536, 32) == h ^ 0x7F134CB8 ^ 3072


def test_coalesce_known_answer():
    ft_in, pi, ft_out = 81 * 1548, 1548, 2
    w = np.zeros((ft_in + pi) * ft_out, np.float32)
    f = np.arange(ft_in, dtype=np.float32)[:, None]
    o = np.arange(ft_out, dtype=np.float32)[None, :]
    w[:ft_in * ft_out] = (f + o * 0.5).ravel()
    p = np.arange(pi, dtype=np.float32)[:, None]
    w[ft_in * ft_out:] = (10_000.0 + p + o * 0.25).ravel()
    out = ox.coalesce(w, ft_in, pi, ft_out).reshape(ft_in, ft_out)
    for feat in (0, 1, pi - 1, pi, 2 * pi + 7, ft_in - 1):
        for k in range(ft_out):
            want = np.float32(np.float32(feat + k * 0.5) + np.float32(10_000.0 + feat % pi + k * 0.25))
            assert out[feat, k] == want
    assert np.array_equal(ox.coalesce(w[:ft_in * ft_out], ft_in, 0, ft_out), w[:ft_in * ft_out])


def test_rounding_and_saturation():
    # half away from zero (1.5 * 127 = 190.5 -> 191; banker's rounding would give 190)
    q = ox.quantise([0.5, 1.5, -0.5, -1.5], 127.0, ox.Q_LS_I16)
    assert q.tolist() == [64, 191, -64, -191]
    # i16 saturation after rounding; NaN -> 0; infinities saturate
    q = ox.quantise([32767.4, 32767.5, -32768.4, -32768.5, 300.0 * 127, np.nan, np.inf, -np.inf], 1.0,
                    ox.Q_LS_I16)
    assert q.tolist() == [32767, 32767, -32768, -32768, 32767, 0, 32767, -32768]
    for kind in (ox.Q_LS_I8, ox.Q_SIMPLE_I8):
        q = ox.quantise([-128.49, 127.49, -128.5, 127.5, np.nan, 0.5, -0.5], 1.0, kind)
        assert q.tolist() == [-128, 127, -128, 127, 0, 1, -1]
    assert ox.quantise([3e9, -3e9, np.nan, 2.5], 1.0, ox.Q_LS_I32).tolist() == [2**31 - 1, -2**31, 0, 3]
    assert ox.quantise([3e9, -3e9, np.nan, 2.5], 1.0, ox.Q_SIMPLE_I32).tolist() == [2**31 - 1, -2**31, 0, 3]
    assert ox.quantise([40000.0, np.nan], 1.0, ox.Q_SIMPLE_I16).tolist() == [32767, 0]


def test_fv_scale():
    assert ox.simple_fv_scale(290.0) == 28  # 8128 / 290 = 28.03
    assert ox.simple_fv_scale(600.0) == 14
    assert ox.ls_export_fv_scale(None, 0, 290.0) == 28
    assert ox.ls_export_fv_scale(None, 1, 290.0) is None
    assert ox.ls_export_fv_scale(16, 1, 290.0) == 16


def _ls_weights(rng, ft_in, ft_out, l1, l2, nb, scale=0.05):
    l2_in = 2 * (l1 - 1)
    shapes = dict(ft_w=ft_in * ft_out, ft_b=ft_out, l1_w=nb * l1 * ft_out, l1_b=nb * l1, l1_shared_weight=ft_out * l1,
                  l1_shared_bias=l1, l2_w=nb * l2 * l2_in, l2_b=nb * l2, l3_w=nb * l2, l3_b=nb)
    return {k: rng.normal(0, scale, n).astype(np.float32) for k, n in shapes.items()}


def test_layerstack_file_structure():
    rng = np.random.default_rng(3)
    fs = 4  # halfka-hm-merged
    info = of.feature_set_info(fs)
    ft_in, ft_out, l1, l2, nb = info["ft_in"], 128, 16, 32, 9
    w = _ls_weights(rng, ft_in, ft_out, l1, l2, nb)
    w["ft_w"][:5] = [300.0, -300.0, 1.5, -0.5, np.nan]
    buf = ox.ls_save_quantised(fs, 0x7F134CB8, ft_in, ft_out, l1, l2, nb, w, fv_scale=28)
    d = ox.parse_layerstack(buf, ft_out, l1, l2)
    assert d["trailing"] == 0
    assert d["version"] == 0x7AF32F21 and d["num_buckets"] == nb
    assert d["network_hash"] == ox.ls_network_hash(0x7F134CB8, ft_out, l2)
    assert d["ft_hash"] == 0x7F134CB8 ^ (2 * ft_out)
    assert d["arch"] == ox.ls_arch_str("HalfKaHmMerged", ft_in, ft_out, l1, 2 * (l1 - 1), l2, 28)
    q = d["ft_w"].astype(np.float64)
    assert q.size == ft_in * ft_out
    assert q[:5].tolist() == [32767, -32768, 191, -64, 0]
    ref = w["ft_w"][5:].astype(np.float64)
    assert np.all(np.abs(q[5:] / 127.0 - ref) <= 0.5 / 127.0 + 1e-12)
    assert np.all(np.abs(d["ft_b"] / 127.0 - w["ft_b"]) <= 0.5 / 127.0 + 1e-9)
    fc = ox.ls_fc_hash(ft_out, l2)
    l1w = w["l1_w"].reshape(nb, l1, ft_out)
    l1s = w["l1_shared_weight"].reshape(ft_out, l1)
    for b, s in enumerate(d["stacks"]):
        assert s["fc_hash"] == fc
        merged = (l1w[b] + l1s.T).astype(np.float64)  # f32 add, then f64 scale
        assert np.all(s["l1_w"][:, ft_out:] == 0)
        assert np.all(np.abs(s["l1_w"][:, :ft_out] / 64.0 - merged) <= 0.5 / 64 + 1e-9)
        mb = (w["l1_b"].reshape(nb, l1)[b] + w["l1_shared_bias"]).astype(np.float64)
        assert np.all(np.abs(s["l1_b"] / 8128.0 - mb) <= 0.5 / 8128 + 1e-12)
        assert np.all(s["l2_w"][:, 30:] == 0) and s["l3_w"].size == 32
    # size by formula
    comp = len(ox.leb128_encode(ox.quantise(w["ft_w"], 127.0, 0)))
    compb = len(ox.leb128_encode(ox.quantise(w["ft_b"], 127.0, 0)))
    stack = 4 + 4 * l1 + l1 * ft_out + 4 * l2 + l2 * 32 + 4 + 32
    assert len(buf) == 12 + len(d["arch"]) + 8 + 2 * 21 + comp + compb + nb * stack


def test_zeroed_layerstack_matches_formula():
    info = of.feature_set_info(4)
    ft_in, ft_out, l1, l2, nb = info["ft_in"], 1536, 16, 32, 9
    w = {k: np.zeros_like(v) for k, v in _ls_weights(np.random.default_rng(0), ft_in, 128, l1, l2, nb).items()}
    w["ft_w"] = np.zeros(ft_in * ft_out, np.float32)
    w["ft_b"] = np.zeros(ft_out, np.float32)
    w["l1_w"] = np.zeros(nb * l1 * ft_out, np.float32)
    w["l1_shared_weight"] = np.zeros(ft_out * l1, np.float32)
    buf = ox.ls_save_quantised(4, 0x7F134CB8, ft_in, ft_out, l1, l2, nb, w, fv_scale=28)
    d = ox.parse_layerstack(buf, ft_out, l1, l2)
    # one LEB128 byte per zero value
    assert d["ft_w_bytes"] == ft_in * ft_out and not d["ft_w"].any() and d["trailing"] == 0


def test_simple_file_structure():
    rng = np.random.default_rng(4)
    info = of.feature_set_info(0)
    ft_in, ft_out, l1, l2 = info["ft_in"], 32, 32, 32
    w = dict(ft_w=rng.normal(0, 0.05, ft_in * ft_out), ft_b=rng.normal(0, 0.05, ft_out),
             l1_w=rng.normal(0, 0.5, l1 * 2 * ft_out), l1_b=rng.normal(0, 0.5, l1), l2_w=rng.normal(0, 0.5, l2 * l1),
             l2_b=rng.normal(0, 0.5, l2), l3_w=rng.normal(0, 3, l2), l3_b=rng.normal(0, 0.5, 1))
    buf = ox.simple_save_quantised(0, 0x5D69D5B8, ft_in, ft_out, l1, l2, w, fv_scale=28)
    d = ox.parse_simple(buf, ft_in, ft_out, l1, l2)
    assert d["trailing"] == 0 and d["version"] == 0x7AF32F16
    assert d["network_hash"] == ox.simple_network_hash(0x5D69D5B8, ft_out, l1, l2)
    assert d["fc_hash"] == ox.simple_fc_hash(2 * ft_out, l1, l2)
    assert np.array_equal(d["ft_w"], ox.quantise(w["ft_w"], 127.0, ox.Q_SIMPLE_I16).astype(np.int16))
    assert np.array_equal(d["l1_w"][:, :2 * ft_out],
                          ox.quantise(w["l1_w"], 64.0, ox.Q_SIMPLE_I8).reshape(l1, 2 * ft_out).astype(np.int8))
    # l3 weights ~ N(0, 3): many saturate at +-127/64
    l3 = ox.quantise(w["l3_w"], 64.0, ox.Q_SIMPLE_I8)
    assert np.array_equal(d["l3_w"][:l2], l3.astype(np.int8)) and not d["l3_w"][l2:].any()
    assert l3.max() == 127 and l3.min() == -128  # saturated both ways
    ok = np.abs(w["l3_w"]) * 64 < 127
    assert np.all(np.abs(l3[ok] / 64.0 - w["l3_w"][ok]) <= 0.5 / 64 + 1e-12)
