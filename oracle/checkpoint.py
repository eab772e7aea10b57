"""Raw resume checkpoint (RNRC) oracle - TEST INFRASTRUCTURE ONLY.

A Python restatement of the reference's raw checkpoint format, used by
tests/ as the checker of the library's writer and reader; nothing in the
product imports it.  It follows bins/nnue_train/src/ckpt.rs:
  - layout and version rules: :18-110 (RAW_CKPT_MAGIC, RAW_CKPT_VERSION = 8);
  - write_raw_ckpt_header: :269-312;
  - read_raw_ckpt_header (versions 1..8, identity checks and messages): :322-612;
  - save_raw_checkpoint_file / load_raw_checkpoint_file / read_raw_ckpt_group:
    :614-757 (group = u64 len + f32 w, m, v, slow);
and the identity inputs of FeatureSetSpec (crates/shogi-features/src/
feature_set.rs:103-185 shapes, :1063-1084 pinned hashes), ArchKind /
BucketMode canonical names (crates/nnue-format/src/arch_kind.rs:23-28,
crates/nnue-train/src/dataloader.rs:313-318) and the trainers' topologies
(ckpt.rs:186-199; trainer_simple.rs:2881-2885).

Parity pinning: tests/test_oracle_checkpoint.py checks this module against
the reference's own format tests (bins/nnue_train/src/tests/
raw_ckpt_format_tests.rs: the byte-built v1..v4 headers, the v8 -> v7 -> v6
downgrades at the documented field offsets, every accept / reject case).
"""
from __future__ import annotations

import io
import os
import struct
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

MAGIC = b"RNRC"
VERSION = 8
MAX_NAME = 256
MAX_RUN_ID = 256

# canonical name -> (king buckets, piece inputs, max_active, feature hash)
FEATURE_SETS = {
    "halfkp": (81, 1548, 38, 0x5D69D5B8),
    "halfka-split": (81, 1710, 40, 0x5F134CB8),
    "halfka-merged": (81, 1629, 40, 0xACD68C97),
    "halfka-hm-split": (45, 1710, 40, 0x2A46AC09),
    "halfka-hm-merged": (45, 1629, 40, 0x7F134CB8),
}
ARCH_KINDS = ("layerstack", "simple")


class CkptError(ValueError):
    """io::ErrorKind::InvalidData of the reference reader."""


@dataclass
class Arch:
    """RawCkptArch: feature set identity + arch kind, bucket mode, ft_out, topology."""

    feature_set: str
    arch_kind: str
    ft_out: int
    topology: tuple
    bucket_mode: Optional[str] = None
    factorize: bool = False
    feature_hash: Optional[int] = None  # default: the feature set's pinned hash

    @property
    def ft_in(self) -> int:
        kb, pi, _, _ = FEATURE_SETS[self.feature_set]
        return kb * pi

    @property
    def piece_inputs(self) -> int:
        return FEATURE_SETS[self.feature_set][1]

    @property
    def train_ft_in(self) -> int:
        return self.ft_in + (self.piece_inputs if self.factorize else 0)

    @property
    def max_active(self) -> int:
        return FEATURE_SETS[self.feature_set][2]

    @property
    def hash(self) -> int:
        return FEATURE_SETS[self.feature_set][3] if self.feature_hash is None else self.feature_hash


def layerstack(feature_set="halfka-hm-merged", ft_out=1536, l1=16, l2=32, nb=9, bucket_mode="progress8kpabs",
               factorize=False) -> Arch:
    return Arch(feature_set, "layerstack", ft_out, (ft_out, l1, l2, nb), bucket_mode, factorize)


def simple(feature_set="halfkp", ft_out=256, l1=32, l2=32, factorize=False) -> Arch:
    return Arch(feature_set, "simple", ft_out, (ft_out, l1, l2), None, factorize)


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<I", len(b)) + b


def write_header(arch: Arch, run_id: str, superbatch: int, step_count: int, lr_horizon: Optional[int],
                 num_groups: int) -> bytes:
    """write_raw_ckpt_header: always version 8."""
    out = bytearray(MAGIC)
    out += struct.pack("<I", VERSION)
    out += _str(arch.feature_set)
    out += struct.pack("<QQQ", arch.train_ft_in, arch.ft_out, arch.max_active)
    out += bytes([1 if arch.factorize else 0])
    out += struct.pack("<I", arch.hash)
    out += _str(run_id)
    out += _str(arch.arch_kind)
    out += _str(arch.bucket_mode or "")
    out += struct.pack("<Q", len(arch.topology))
    for d in arch.topology:
        out += struct.pack("<Q", d)
    out += struct.pack("<QQQQ", superbatch, step_count, lr_horizon or 0, num_groups)
    return bytes(out)


class _R:
    def __init__(self, f):
        self.f = f

    def exact(self, n: int, what: str) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise CkptError(f"raw checkpoint truncated while reading {what}")
        return b

    def u32(self, what):
        return struct.unpack("<I", self.exact(4, what))[0]

    def u64(self, what):
        return struct.unpack("<Q", self.exact(8, what))[0]

    def name(self, what, len_what, limit=MAX_NAME):
        n = self.u32(len_what)
        if n > limit:
            raise CkptError(f"raw checkpoint {what} length {n} is implausible (max {limit})")
        try:
            return self.exact(n, what).decode("utf-8")
        except UnicodeDecodeError:
            raise CkptError(f"raw checkpoint {what} is not valid UTF-8") from None


def read_header(data, want: Arch) -> dict:
    """read_raw_ckpt_header; data is bytes or a binary file object."""
    f = io.BytesIO(data) if isinstance(data, (bytes, bytearray)) else data
    r = _R(f)
    magic = r.exact(4, "magic")
    if magic != MAGIC:
        raise CkptError(f"raw checkpoint magic mismatch: got {magic!r}, want {MAGIC!r}")
    version = r.u32("version")
    if version == 0 or version > VERSION:
        raise CkptError(f"raw checkpoint version {version} is not supported (this build reads 1..={VERSION})")
    if version >= 2:
        fs = r.name("feature set name", "feature set name length")
        ft_in, ft_out, max_active = r.u64("ft_in"), r.u64("ft_out"), r.u64("max_active")
        factorize = r.exact(1, "ft_factorize flag")[0] != 0 if version >= 6 else False
        fhash = r.u32("feature hash") if version >= 7 else None
        if fs != want.feature_set:
            raise CkptError(f"raw checkpoint feature set mismatch: checkpoint is '{fs}', requested "
                            f"'{want.feature_set}' (cannot resume across feature sets)")
        if factorize != want.factorize:
            raise CkptError(f"raw checkpoint ft-factorize mismatch: checkpoint {str(factorize).lower()}, "
                            f"requested {str(want.factorize).lower()} (cannot resume across --ft-factorize on/off)")
        if fhash is not None and fhash != want.hash:
            raise CkptError(f"raw checkpoint feature hash mismatch: got {fhash:#010x}, want {want.hash:#010x}")
        if ft_in != want.train_ft_in:
            raise CkptError(f"raw checkpoint ft_in mismatch: got {ft_in}, want {want.train_ft_in}")
        if ft_out != want.ft_out:
            raise CkptError(f"raw checkpoint ft_out mismatch: got {ft_out}, want {want.ft_out}")
        legacy = want.factorize and max_active == 2 * want.max_active
        if max_active != want.max_active and not legacy:
            raise CkptError(f"raw checkpoint max_active mismatch: got {max_active}, want {want.max_active}")
    elif want.feature_set != "halfka-hm-merged":
        raise CkptError(f"raw checkpoint version 1 is always 'halfka-hm-merged', requested "
                        f"'{want.feature_set}' (cannot resume across feature sets)")
    run_id = None
    if version >= 3:
        rid = r.name("producer run id", "producer run id length", MAX_RUN_ID)
        run_id = rid or None
    if version >= 4:
        arch = r.name("arch kind name", "arch kind name length")
        if arch not in ARCH_KINDS:
            raise CkptError(f"raw checkpoint has unknown arch kind '{arch}'")
        if arch != want.arch_kind:
            raise CkptError(f"raw checkpoint arch kind mismatch: checkpoint is '{arch}', requested "
                            f"'{want.arch_kind}' (cannot resume across architectures)")
        if version >= 8:
            mode = r.name("bucket mode name", "bucket mode name length") or None
        else:
            mode = "progress8kpabs" if arch == "layerstack" else None
        if mode != want.bucket_mode:
            if mode is not None and want.bucket_mode is not None:
                raise CkptError(f"checkpoint bucket mode '{mode}' does not match --bucket-mode '{want.bucket_mode}'")
            raise CkptError(f"raw checkpoint bucket mode \"{mode or ''}\" does not match architecture "
                            f"'{want.arch_kind}'")
        count = r.u64("topology dim count")
        if count != len(want.topology):
            raise CkptError(f"raw checkpoint topology dim count {count} != expected {len(want.topology)}")
        for i, wd in enumerate(want.topology):
            d = r.u64("topology dim")
            if d != wd:
                raise CkptError(f"raw checkpoint topology dim {i} mismatch: got {d}, want {wd} "
                                "(network architecture mismatch)")
    elif want.arch_kind != "layerstack":
        raise CkptError(f"raw checkpoint version {version} predates the arch-kind header and is always "
                        f"'layerstack', requested '{want.arch_kind}' (cannot resume across architectures)")
    elif want.bucket_mode != "progress8kpabs":
        raise CkptError(f"checkpoint bucket mode 'progress8kpabs' does not match --bucket-mode "
                        f"'{want.bucket_mode or ''}'")
    superbatch = r.u64("superbatch")
    step_count = r.u64("step_count")
    horizon = (r.u64("lr_horizon") or None) if version >= 5 else None
    num_groups = r.u64("num_groups")
    return dict(version=version, superbatch=superbatch, step_count=step_count, num_groups=num_groups,
                run_id=run_id, lr_horizon=horizon, header_bytes=f.tell())


@dataclass
class Group:
    name: str
    w: np.ndarray
    m: np.ndarray
    v: np.ndarray
    slow: np.ndarray = field(default=None)


def save_file(path, arch: Arch, run_id: str, superbatch: int, step_count: int, lr_horizon: Optional[int],
              groups: list) -> None:
    """save_raw_checkpoint_file: header, then u64 len + w, m, v, slow (f32 LE) per group."""
    tmp = str(path) + ".tmp"
    with open(tmp, "wb") as f:
        f.write(write_header(arch, run_id if len(run_id.encode()) <= MAX_RUN_ID else "", superbatch, step_count,
                             lr_horizon, len(groups)))
        for g in groups:
            n = g.w.size
            f.write(struct.pack("<Q", n))
            for a in (g.w, g.m, g.v, g.slow):
                assert a.size == n
                f.write(np.ascontiguousarray(a, dtype="<f4").tobytes())
    os.replace(tmp, path)


def load_file(path, want: Arch, expected_groups: list):
    """load_raw_checkpoint_file: header checked against want; expected_groups is
    [(name, len)] in format order.  Returns (header dict, [Group])."""
    with open(path, "rb") as f:
        h = read_header(f, want)
        if h["num_groups"] != len(expected_groups):
            raise CkptError(f"raw checkpoint num_groups {h['num_groups']} != expected {len(expected_groups)}")
        r = _R(f)
        out = []
        for name, n in expected_groups:
            ln = r.u64(f"group {name} len")
            if ln != n:
                raise CkptError(f"raw checkpoint group {name} len mismatch: got {ln}, want {n} "
                                "(network architecture mismatch)")
            arrs = [np.frombuffer(r.exact(4 * n, f"group {name} {k}"), dtype="<f4").astype(np.float32)
                    for k in ("w", "m", "v", "slow")]
            out.append(Group(name, *arrs))
    return h, out


def f16_moment_round_trip(x: np.ndarray, scale: float) -> np.ndarray:
    """The true f32 value an f16 moment holds after a load into an f16-state
    trainer and a save: f16(clamp(x * scale, +-65504)) * (1 / scale)
    (MomentBuf::from_host_f32 / to_host_f32, trainer_common.rs:89-126)."""
    y = np.clip(x.astype(np.float32) * np.float32(scale), np.float32(-65504.0), np.float32(65504.0))
    return y.astype(np.float16).astype(np.float32) * np.float32(1.0 / scale)
