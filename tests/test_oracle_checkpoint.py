"""Raw resume checkpoint headers (RNRC): the oracle (oracle/checkpoint.py) and
the library's header writer / reader (tatara_amd.checkpoint over the C ABI,
host code) against the reference's format tests
(bins/nnue_train/src/tests/raw_ckpt_format_tests.rs), which build legacy
headers byte by byte and edit v8 headers at documented field offsets.  Every
case runs on both implementations; the library must write the oracle's bytes
and fail with the oracle's message.  No GPU needed.
"""
import struct

import pytest

from oracle import checkpoint as oc
from tatara_amd import checkpoint as pc
from tatara_amd._lib import TataraError

DEFAULT_FT_OUT, DEFAULT_L1_OUT, DEFAULT_L2_OUT, DEFAULT_NUM_BUCKETS = 1536, 16, 32, 9  # arch.rs:18-42


def ls_arch(mode="progress8kpabs", factorize=False):
    return oc.layerstack("halfka-hm-merged", DEFAULT_FT_OUT, DEFAULT_L1_OUT, DEFAULT_L2_OUT,
                         DEFAULT_NUM_BUCKETS, mode, factorize)


def simple_arch():
    return oc.Arch("halfka-hm-merged", "simple", DEFAULT_FT_OUT,
                   (DEFAULT_FT_OUT, DEFAULT_L1_OUT, DEFAULT_L2_OUT), None)


def to_product(a: oc.Arch) -> pc.CkptArch:
    assert a.feature_hash is None
    if a.arch_kind == "layerstack":
        ft_out, l1, l2, nb = a.topology
        assert ft_out == a.ft_out
        return pc.CkptArch(a.feature_set, "layerstack", ft_out, l1, l2, nb, a.bucket_mode, a.factorize)
    ft_out, l1, l2 = a.topology
    return pc.CkptArch(a.feature_set, "simple", ft_out, l1, l2, 0, None, a.factorize)


class Oracle:
    name = "oracle"

    @staticmethod
    def write(a, run_id, sb, steps, horizon, ng):
        return oc.write_header(a, run_id, sb, steps, horizon, ng)

    @staticmethod
    def read(data, a):
        h = oc.read_header(bytes(data), a)
        return h["superbatch"], h["step_count"], h["num_groups"], h["run_id"], h["lr_horizon"], h["version"]

    error = oc.CkptError


class Product:
    name = "library"

    @staticmethod
    def write(a, run_id, sb, steps, horizon, ng):
        return pc.write_header(to_product(a), run_id, sb, steps, horizon, ng)

    @staticmethod
    def read(data, a):
        h = pc.read_header(bytes(data), to_product(a))
        return h.superbatch, h.step_count, h.num_groups, h.producer_run_id, h.lr_horizon, h.version

    error = TataraError


IMPLS = [Oracle, Product]
ids = [i.name for i in IMPLS]


def reject(impl, data, a, match=None):
    with pytest.raises(impl.error) as e:
        impl.read(data, a)
    if match is not None:
        assert match in str(e.value), str(e.value)
    return str(e.value)


# -- helpers restating the reference test's header builders -------------------

def u32(x):
    return struct.pack("<I", x)


def u64(x):
    return struct.pack("<Q", x)


def legacy_header(version, fs, run_id, superbatch, step_count, num_groups):
    """legacy_raw_ckpt_header (raw_ckpt_format_tests.rs:71-100): versions 1..3."""
    kb, pi, ma, _ = oc.FEATURE_SETS[fs]
    b = oc.MAGIC + u32(version)
    if version >= 2:
        b += u32(len(fs)) + fs.encode() + u64(kb * pi) + u64(DEFAULT_FT_OUT) + u64(ma)
    if version >= 3:
        rid = (run_id or "").encode()
        b += u32(len(rid)) + rid
    return b + u64(superbatch) + u64(step_count) + u64(num_groups)


def v4_layerstack_header(superbatch, step_count, num_groups):
    """v4_layerstack_header (raw_ckpt_format_tests.rs:103-130)."""
    fs = "halfka-hm-merged"
    kb, pi, ma, _ = oc.FEATURE_SETS[fs]
    b = oc.MAGIC + u32(4) + u32(len(fs)) + fs.encode() + u64(kb * pi) + u64(DEFAULT_FT_OUT) + u64(ma)
    b += u32(0) + u32(len("layerstack")) + b"layerstack"
    topo = (DEFAULT_FT_OUT, DEFAULT_L1_OUT, DEFAULT_L2_OUT, DEFAULT_NUM_BUCKETS)
    b += u64(len(topo)) + b"".join(u64(d) for d in topo)
    return b + u64(superbatch) + u64(step_count) + u64(num_groups)


def bucket_mode_field_offset(buf, a):
    """raw_ckpt_format_tests.rs:191-197."""
    off = 4 + 4 + 4 + len(a.feature_set) + 8 + 8 + 8 + 1 + 4
    rid = struct.unpack_from("<I", buf, off)[0]
    off += 4 + rid
    an = struct.unpack_from("<I", buf, off)[0]
    return off + 4 + an


def downgrade_v8_to_v7(buf, a):
    """raw_ckpt_format_tests.rs:199-204."""
    buf = bytearray(buf)
    off = bucket_mode_field_offset(buf, a)
    n = struct.unpack_from("<I", buf, off)[0]
    del buf[off:off + 4 + n]
    buf[4:8] = u32(7)
    return buf


def remove_v7_feature_hash(buf, a):
    """raw_ckpt_format_tests.rs:206-212."""
    buf = downgrade_v8_to_v7(buf, a)
    buf[4:8] = u32(6)
    max_active_off = 4 + 4 + 4 + len(a.feature_set) + 8 + 8
    hoff = max_active_off + 8 + 1
    del buf[hoff:hoff + 4]
    return buf


# -- the reference's cases ------------------------------------------------------

def test_constants():
    # raw_ckpt_constants_are_stable
    assert oc.MAGIC == b"RNRC" and oc.VERSION == 8
    assert Product.write(ls_arch(), "", 0, 0, None, 10)[:8] == b"RNRC" + u32(8)


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_v8_bucket_modes_round_trip(impl):
    for a in (ls_arch("progress8kpabs"), ls_arch("kingrank9"), simple_arch()):
        buf = impl.write(a, "bucket-mode-roundtrip", 2, 20, None, 10)
        assert impl.read(buf, a)[:3] == (2, 20, 10)


def test_writers_agree_byte_for_byte():
    cases = [(ls_arch(), "", 0, 0, None, 10), (ls_arch("kingrank9"), "net-20260520-1234", 7, 99, 123, 10),
             (ls_arch(factorize=True), "run-1", 2, 20, None, 10), (simple_arch(), "x", 1, 5, 9, 8),
             (oc.simple("halfkp", 256, 32, 32, True), "simple-run", 3, 192, None, 8),
             (oc.layerstack("halfkp", 768, 8, 32, 9, "kingrank9"), "é-run", 2 ** 40, 2 ** 63, 2 ** 33, 10)]
    for fs in oc.FEATURE_SETS:
        cases.append((oc.layerstack(fs, 512, 16, 32, 8, "progress8kpabs", True), "r", 1, 2, 3, 10))
    for args in cases:
        assert Product.write(*args) == Oracle.write(*args), args


def test_overlong_run_id_is_omitted():
    # save_raw_checkpoint_file omits a run id over MAX_RUN_ID_BYTES
    long_id = "x" * 257
    assert Product.write(ls_arch(), long_id, 1, 0, None, 10) == Oracle.write(ls_arch(), "", 1, 0, None, 10)
    ok_id = "y" * 256
    h = Product.read(Product.write(ls_arch(), ok_id, 1, 0, None, 10), ls_arch())
    assert h[3] == ok_id


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_v8_rejects_cross_bucket_mode_in_both_directions(impl):
    for written, requested in (("progress8kpabs", "kingrank9"), ("kingrank9", "progress8kpabs")):
        buf = Oracle.write(ls_arch(written), "", 1, 0, None, 10)
        reject(impl, buf, ls_arch(requested),
               f"checkpoint bucket mode '{written}' does not match --bucket-mode '{requested}'")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_v7_layerstack_defaults_to_progress8kpabs(impl):
    prog = ls_arch("progress8kpabs")
    buf = downgrade_v8_to_v7(Oracle.write(prog, "legacy-v7", 7, 70, 100, 10), prog)
    assert impl.read(buf, prog)[:3] == (7, 70, 10)
    assert impl.read(buf, prog)[5] == 7
    reject(impl, buf, ls_arch("kingrank9"),
           "checkpoint bucket mode 'progress8kpabs' does not match --bucket-mode 'kingrank9'")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_empty_bucket_mode_does_not_match_layerstack(impl):
    a = ls_arch()
    buf = bytearray(Oracle.write(a, "", 1, 0, None, 10))
    off = bucket_mode_field_offset(buf, a)
    n = struct.unpack_from("<I", buf, off)[0]
    buf[off:off + 4 + n] = u32(0)
    reject(impl, buf, a, "raw checkpoint bucket mode \"\" does not match architecture 'layerstack'")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_ft_factorize_round_trips_and_mismatch_rejects(impl):
    on, off = ls_arch(factorize=True), ls_arch()
    assert impl.read(Oracle.write(on, "run-1", 2, 20, None, 10), on)[:3] == (2, 20, 10)
    reject(impl, Oracle.write(on, "", 1, 0, None, 10), off, "ft-factorize")
    reject(impl, Oracle.write(off, "", 1, 0, None, 10), on, "ft-factorize")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_accepts_legacy_factorized_max_active(impl):
    a = ls_arch(factorize=True)
    buf = remove_v7_feature_hash(Oracle.write(a, "run-legacy", 3, 30, None, 10), a)
    base = a.max_active
    off = 4 + 4 + 4 + len(a.feature_set) + 8 + 8
    assert struct.unpack_from("<Q", buf, off)[0] == base, "fixture must point at the max_active field"
    buf[off:off + 8] = u64(2 * base)
    assert impl.read(buf, a)[:3] == (3, 30, 10)
    # only with the factorizer: a non-factorized 2x base is rejected
    o = ls_arch()
    b2 = remove_v7_feature_hash(Oracle.write(o, "", 1, 0, None, 10), o)
    b2[off:off + 8] = u64(2 * base)
    reject(impl, b2, o, "max_active")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_feature_hash_mismatch_rejects_and_v6_has_none(impl):
    a = ls_arch()
    buf = bytearray(Oracle.write(a, "", 5, 50, None, 10))
    hoff = 4 + 4 + 4 + len(a.feature_set) + 8 + 8 + 8 + 1
    assert struct.unpack_from("<I", buf, hoff)[0] == 0x7F134CB8
    buf[hoff:hoff + 4] = u32(0x7F134CB9)
    reject(impl, buf, a, "raw checkpoint feature hash mismatch: got 0x7f134cb9, want 0x7f134cb8")
    v6 = remove_v7_feature_hash(Oracle.write(a, "", 5, 50, None, 10), a)
    assert impl.read(v6, a)[:3] == (5, 50, 10)


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_v5_lr_horizon_and_run_id(impl):
    a = ls_arch()
    sb, steps, ng, rid, hz, _ = impl.read(Oracle.write(a, "net-20260520-1234", 7, 99, 123, 10), a)
    assert (sb, steps, ng, rid, hz) == (7, 99, 10, "net-20260520-1234", 123)
    assert impl.read(Oracle.write(a, "", 1, 0, None, 10), a)[3:5] == (None, None)


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_reads_legacy_v1_v2_v3_and_v4(impl):
    a = ls_arch()
    h1 = impl.read(legacy_header(1, "halfka-hm-merged", None, 3, 30, 10), a)
    h2 = impl.read(legacy_header(2, "halfka-hm-merged", None, 4, 40, 10), a)
    h3 = impl.read(legacy_header(3, "halfka-hm-merged", "legacy-run", 5, 50, 10), a)
    assert h1[:4] == (3, 30, 10, None) and h2[0] == 4 and h2[3] is None
    assert h3[0] == 5 and h3[3] == "legacy-run"
    assert h1[4] is None and h2[4] is None and h3[4] is None
    h4 = impl.read(v4_layerstack_header(6, 60, 10), a)
    assert h4[:3] == (6, 60, 10) and h4[4] is None
    # version 1 is always halfka-hm-merged
    reject(impl, legacy_header(1, "halfka-hm-merged", None, 3, 30, 10), oc.layerstack("halfkp", 1536, 16, 32, 9),
           "raw checkpoint version 1 is always 'halfka-hm-merged', requested 'halfkp'")
    # legacy layerstack files are progress8kpabs
    reject(impl, v4_layerstack_header(6, 60, 10), ls_arch("kingrank9"),
           "checkpoint bucket mode 'progress8kpabs' does not match --bucket-mode 'kingrank9'")
    reject(impl, legacy_header(3, "halfka-hm-merged", None, 1, 0, 10), ls_arch("kingrank9"),
           "checkpoint bucket mode 'progress8kpabs' does not match --bucket-mode 'kingrank9'")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_rejects_wrong_arch_kind_topology_and_version(impl):
    written = oc.Arch("halfka-hm-merged", "simple", DEFAULT_FT_OUT, ls_arch().topology, None)
    reject(impl, Oracle.write(written, "", 1, 0, None, 10), ls_arch(), "arch kind mismatch")
    wrong = oc.Arch("halfka-hm-merged", "layerstack", DEFAULT_FT_OUT, (1, 2, 3, 4), "progress8kpabs")
    reject(impl, Oracle.write(wrong, "", 1, 0, None, 10), ls_arch(), "topology dim")
    reject(impl, legacy_header(3, "halfka-hm-merged", None, 1, 0, 8), simple_arch(), "predates the arch-kind header")
    buf = bytearray(legacy_header(3, "halfka-hm-merged", None, 1, 0, 10))
    buf[4:8] = u32(99)
    reject(impl, buf, ls_arch(), "version 99 is not supported")
    buf[4:8] = u32(0)
    reject(impl, buf, ls_arch(), "version 0 is not supported")
    reject(impl, b"RNRX" + bytes(buf[4:]), ls_arch(), "magic mismatch")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_identity_mismatches(impl):
    a = ls_arch()
    buf = Oracle.write(a, "", 1, 0, None, 10)
    reject(impl, buf, oc.layerstack("halfka-merged", 1536, 16, 32, 9), "feature set mismatch")
    reject(impl, buf, oc.layerstack("halfka-hm-merged", 768, 16, 32, 9), "ft_out mismatch: got 1536, want 768")
    reject(impl, buf, oc.layerstack("halfka-hm-merged", 1536, 8, 32, 9), "topology dim 1 mismatch: got 16, want 8")
    reject(impl, buf, oc.layerstack("halfka-hm-merged", 1536, 16, 32, 8), "topology dim 3 mismatch")
    sbuf = Oracle.write(simple_arch(), "", 1, 0, None, 8)
    reject(impl, sbuf, ls_arch(), "arch kind mismatch: checkpoint is 'simple', requested 'layerstack'")
    # the same feature set name with another ft_in (a different feature table) is an ft_in mismatch
    edited = bytearray(buf)
    edited[4 + 4 + 4 + len(a.feature_set):4 + 4 + 4 + len(a.feature_set) + 8] = u64(1)
    reject(impl, edited, a, "ft_in mismatch: got 1, want 73305")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_malformed_names(impl):
    a = ls_arch()
    buf = bytearray(Oracle.write(a, "run", 1, 0, None, 10))
    bad = bytearray(buf)
    bad[8:12] = u32(257)
    reject(impl, bad, a, "feature set name length 257 is implausible (max 256)")
    rid_off = 4 + 4 + 4 + len(a.feature_set) + 8 + 8 + 8 + 1 + 4
    bad = bytearray(buf)
    bad[rid_off:rid_off + 4] = u32(300)
    reject(impl, bad, a, "producer run id length 300 is implausible (max 256)")
    bad = bytearray(buf)
    bad[rid_off + 4:rid_off + 7] = b"\xff\xfe\xfd"
    reject(impl, bad, a, "producer run id is not valid UTF-8")
    arch_off = rid_off + 4 + 3
    bad = bytearray(buf)
    bad[arch_off + 4:arch_off + 14] = b"layerstacx"
    reject(impl, bad, a, "unknown arch kind 'layerstacx'")


@pytest.mark.parametrize("impl", IMPLS, ids=ids)
def test_every_truncation_names_its_field(impl):
    for a, hz in ((ls_arch(factorize=True), 77), (simple_arch(), None)):
        buf = Oracle.write(a, "trunc-run", 4, 44, hz, 10)
        assert impl.read(buf, a)[:3] == (4, 44, 10)
        for n in range(len(buf)):
            msg = reject(impl, buf[:n], a, "raw checkpoint truncated while reading ")
            want = reject(Oracle, buf[:n], a)
            assert want in msg, (n, msg, want)


def test_header_size_is_reported():
    a = ls_arch()
    buf = Oracle.write(a, "abc", 1, 2, 3, 10)
    assert pc.read_header(buf + b"\0" * 64, to_product(a)).header_bytes == len(buf)
    assert oc.read_header(buf + b"\0" * 64, a)["header_bytes"] == len(buf)
