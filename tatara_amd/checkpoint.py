"""Raw resume checkpoints (RNRC version 8) over the C ABI.

The file format, header rules and group order are the reference's
(bins/nnue_train/src/ckpt.rs:18-110, 268-757); LayerStackTrainer /
SimpleTrainer.save_resume_checkpoint and .load_resume_checkpoint write and
read whole files.  The functions here expose the library's header writer and
validating reader on their own (host code, no GPU needed).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

from . import _lib
from ._lib import TataraCkptArch, TataraCkptHeader, check

ARCHS = {"layerstack": 0, "simple": 1}
# feature-set and bucket-mode names as in tatara_amd.dataloader
FEATURE_SETS = {"halfkp": 0, "halfka-split": 1, "halfka-merged": 2, "halfka-hm-split": 3,
                "halfka-hm-merged": 4}
BUCKET_MODES = {None: 0, "kingrank9": 1, "progress8kpabs": 2}


@dataclass
class CkptArch:
    """RawCkptArch (ckpt.rs:213-226)."""

    feature_set: str
    arch: str
    ft_out: int
    l1_out: int
    l2_out: int
    num_buckets: int = 0
    bucket_mode: Optional[str] = None   # LayerStack: "kingrank9" / "progress8kpabs"
    ft_factorize: bool = False

    def to_c(self) -> TataraCkptArch:
        return TataraCkptArch(FEATURE_SETS[self.feature_set], int(self.ft_factorize), ARCHS[self.arch],
                              BUCKET_MODES[self.bucket_mode], self.ft_out, self.l1_out, self.l2_out,
                              self.num_buckets)


@dataclass
class CkptHeader:
    """RawCkptHeader (ckpt.rs:247-265) plus the version read and the header size."""

    version: int
    superbatch: int
    step_count: int
    num_groups: int
    producer_run_id: Optional[str]
    lr_horizon: Optional[int]
    header_bytes: int

    @classmethod
    def from_c(cls, h: TataraCkptHeader) -> "CkptHeader":
        rid = h.run_id.decode()
        return cls(h.version, h.superbatch, h.step_count, h.num_groups, rid or None, h.lr_horizon or None,
                   h.header_bytes)


def write_header(arch: CkptArch, run_id: str, superbatch: int, step_count: int,
                 lr_horizon: Optional[int], num_groups: int) -> bytes:
    """write_raw_ckpt_header (ckpt.rs:269-312), always version 8."""
    lib = _lib.load()
    ca = arch.to_c()
    n = C.c_uint64()
    buf = (C.c_uint8 * 4096)()
    check(lib.tatara_ckpt_write_header(C.byref(ca), run_id.encode(), superbatch, step_count, lr_horizon or 0,
                                       num_groups, buf, len(buf), C.byref(n)))
    return bytes(buf[: n.value])


def read_header(data: bytes, expected: CkptArch) -> CkptHeader:
    """read_raw_ckpt_header (ckpt.rs:322-612); raises TataraError on malformed
    or mismatching input with the reference's message."""
    lib = _lib.load()
    ca = expected.to_c()
    out = TataraCkptHeader()
    buf = (C.c_uint8 * max(1, len(data))).from_buffer_copy(data if data else b"\0")
    check(lib.tatara_ckpt_read_header(buf, len(data), C.byref(ca), C.byref(out)))
    return CkptHeader.from_c(out)
