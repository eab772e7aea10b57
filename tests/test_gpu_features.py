"""GPU dataloader step (tatara_psv_to_batch) vs the CPU feature oracle: bit-exact.

Every output of the HIP decode -- index rows (emission order, -1 padding),
nnz, score, wdl, kingrank9 and KP-absolute progress buckets -- must equal
oracle/features.cpp on the same records: the reference's sample.psv, seeded
synthetic positions (40 pieces, hands, promotions) and
random byte records (corrupt input, invalid kings, over-full boards).  The
glibc-equivalent expf used by the progress bucket is compared with glibc
itself bit for bit.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import features as of
from tatara_amd import psv
from tatara_amd.dataloader import ProgressWeights, device_batch_to_host, psv_to_device_batch
from tatara_amd.trainer import DeviceArray

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
FS = ("halfkp", "halfka-split", "halfka-merged", "halfka-hm-split", "halfka-hm-merged")


def records():
    raw = np.fromfile(GOLDEN / "sample.psv", dtype=np.uint8).reshape(100, 40)
    return np.concatenate([raw, psv.synthetic_psv(8192, seed=11)])


def compare(recs, fs, mode, nb=1, weights=None):
    wobj = ProgressWeights(weights) if weights is not None else None
    db = psv_to_device_batch(recs, fs, {"progress": "progress8kpabs"}.get(mode, mode), nb, wobj)
    got = device_batch_to_host(db)
    want = of.psv_to_batch(recs, fs, mode, nb, None if weights is None else wobj.host)
    for k in ("stm", "nstm", "nnz", "score", "wdl", "bucket"):
        g = got[k].reshape(want[k].shape)
        bad = np.nonzero(g != want[k])[0] if g.ndim == 1 else np.nonzero((g != want[k]).any(1))[0]
        assert bad.size == 0, f"{fs}/{mode}: {k} differs at records {bad[:10]}"
    return got


@pytest.mark.parametrize("fs", FS)
def test_features_bit_exact(gpu, fs):
    compare(records(), fs, "none")


def test_kingrank9_bit_exact(gpu):
    got = compare(records(), "halfka-hm-merged", "kingrank9")
    assert len(np.unique(got["bucket"])) == 9


@pytest.mark.parametrize("std,nb", [(0.01, 8), (0.1, 9), (1.0, 8)])
def test_progress_buckets_bit_exact(gpu, std, nb):
    w = np.random.default_rng(int(std * 100) + nb).normal(0.0, std, 81 * 1548)
    got = compare(records(), "halfka-hm-merged", "progress", nb, w)
    if std >= 0.1:
        assert len(np.unique(got["bucket"])) >= 4


def test_random_byte_records(gpu):
    """Corrupt input: invalid kings, over-full boards, long hands -- same results."""
    rng = np.random.default_rng(5)
    recs = rng.integers(0, 256, (4096, 40), dtype=np.uint8)
    w = rng.normal(0.0, 0.05, 81 * 1548)
    for fs in ("halfkp", "halfka-hm-merged"):
        compare(recs, fs, "kingrank9")
        compare(recs, fs, "progress", 9, w)


def test_empty_and_single(gpu):
    recs = records()[:1]
    compare(recs, "halfka-hm-merged", "kingrank9")


def test_expf_matches_glibc(gpu):
    from tatara_amd import _lib

    rng = np.random.default_rng(1)
    # every 256th bit pattern of the non-negative floats up to 110, both signs,
    # plus 1M random bit patterns (NaN excluded)
    pos = np.arange(0, 0x42DC0000, 256, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rnd = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([pos, -pos, rnd[~np.isnan(rnd)]]).astype(np.float32)
    dx, dy = DeviceArray(x), DeviceArray.empty(x.shape, np.float32)
    _lib.check(_lib.load().tatara_op_expf(dx.ptr, dy.ptr, x.size))
    y = dy.to_host()
    ref = of.expf(x)
    bad = np.nonzero(y.view(np.uint32) != ref.view(np.uint32))[0]
    assert bad.size == 0, (x[bad[:5]], y[bad[:5]], ref[bad[:5]])
