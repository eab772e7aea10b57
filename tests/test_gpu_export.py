"""Quantised export on the GPU (tatara_trainer_export_quantised,
tatara_op_quantise_ft) vs the CPU export oracle: byte-identical files.

The trainers are stepped on GPU-decoded PSV batches so the weights are
non-trivial, then planted with the values where quantisation has edges
(rounding ties, i16/i8 saturation, NaN, infinities), exported, and compared
byte for byte with oracle/export.cpp fed the same f32 weights read back from
the device.  The op-level test covers the FT quantiser alone (raw i16 and
LEB128, with and without factorizer rows, tile-boundary sizes).
"""
import ctypes as C

import numpy as np
import pytest

from oracle import export as ox
from oracle import features as of
from tatara_amd import _lib, psv
from tatara_amd.dataloader import psv_to_device_batch
from tatara_amd.trainer import (DeviceArray, LayerStackConfig, LayerStackTrainer, Sigmoid, SimpleConfig,
                                SimpleTrainer, Wrm, check, simple_fv_scale)

pytestmark = pytest.mark.gpu

EDGES = np.array([300.0, -300.0, 1.5, -0.5, np.nan, np.inf, -np.inf, 258.0, -258.5, 0.5 / 127, -0.5 / 127],
                 np.float32)


def quantise_op(w, rows, cols, pi, leb128):
    n = rows * cols
    dw = DeviceArray(np.ascontiguousarray(w, np.float32)) if w.size else None
    cap = max(3 * n, 1)
    dout = DeviceArray.empty(cap, np.uint8)
    nbytes = C.c_uint64()
    check(_lib.load().tatara_op_quantise_ft(dw.ptr if dw else None, rows, cols, pi, 127.0, int(leb128), dout.ptr,
                                            cap, C.byref(nbytes)))
    return dout.to_host()[:nbytes.value].tobytes()


@pytest.mark.parametrize("rows,cols,pi", [(37, 96, 0), (1000, 256, 100), (4096, 4, 7), (73305, 128, 1629), (0, 8, 0)])
def test_op_quantise_matches_oracle(gpu, rows, cols, pi):
    rng = np.random.default_rng(rows + cols)
    w = rng.normal(0.0, 0.3, (rows + pi) * cols).astype(np.float32)
    if w.size:
        w[:min(w.size, EDGES.size)] = EDGES[:min(w.size, EDGES.size)]
        w[-1] = np.nan
    vals = ox.coalesce(w, rows, pi, cols) if rows else np.zeros(0, np.float32)
    q = ox.quantise(vals, 127.0, ox.Q_LS_I16)
    assert quantise_op(w, rows, cols, pi, False) == q.astype("<i2").tobytes()
    assert quantise_op(w, rows, cols, pi, True) == ox.leb128_encode(q)


def _ls_trainer(pi, l1=16, l2=32):
    info = of.feature_set_info("halfka-hm-merged")  # 45 x 1629 rows
    cfg = LayerStackConfig(ft_in=info["ft_in"], max_active=info["max_active"], piece_inputs=pi, ft_out=128,
                           l1_out=l1, l2_out=l2, num_buckets=9, max_batch=1024, optimizer="ranger")
    return info, LayerStackTrainer(cfg)


def _plant(t, name, idx, values):
    w = t.get(name)
    w[idx] = values
    t.set(name, w)


@pytest.mark.parametrize("factorized,fv,l1,l2", [(True, 28, 16, 32), (False, None, 16, 32), (True, 28, 32, 64),
                                                 (False, 28, 8, 16)])
def test_layerstack_export_bytes(gpu, tmp_path, factorized, fv, l1, l2):
    info, t = _ls_trainer(1629 if factorized else 0, l1, l2)
    ft_in, pi = info["ft_in"], 1629 if factorized else 0
    with t:
        for s in range(3):
            db = psv_to_device_batch(psv.synthetic_psv(1024, seed=40 + s), "halfka-hm-merged", "kingrank9", 9)
            t.train_step(db, None, 2e-3, 0.0, Sigmoid())
        t.flush_pending_loss()
        _plant(t, "ft_w", np.arange(EDGES.size) * 131, EDGES)
        if factorized:
            _plant(t, "ft_w", ft_in * 128 + np.arange(4), [0.25, -3.0, 1e-3, 300.0])  # virtual rows
        _plant(t, "l1_w", [0, 5, 77], [3.0, -3.0, 0.5 / 64])
        _plant(t, "l1_shared_weight", [0, 1], [1.0, -2.5])
        _plant(t, "l2_b", [3], [1e6])
        path = tmp_path / "ls.bin"
        t.save_quantised(path, "halfka-hm-merged", fv_scale=fv)
        got = path.read_bytes()
        w = {g: t.get(g) for g in t.GROUPS}
    w["ft_w"] = ox.coalesce(w["ft_w"], ft_in, pi, 128)
    want = ox.ls_save_quantised(4, info_hash("halfka-hm-merged"), ft_in, 128, l1, l2, 9, w, fv_scale=fv)
    assert len(got) == len(want)
    if got != want:
        bad = np.nonzero(np.frombuffer(got, np.uint8) != np.frombuffer(want, np.uint8))[0]
        raise AssertionError(f"{bad.size} bytes differ, first at {bad[:8]}")
    d = ox.parse_layerstack(got, 128, l1, l2)
    assert d["trailing"] == 0 and ("fv_scale=28" in d["arch"]) == (fv is not None)


def info_hash(fs):
    h = C.c_uint32()
    check(_lib.load().tatara_feature_set_info(of.FEATURE_SETS.index(fs), None, None, None, None, C.byref(h)))
    return h.value


# 256x2-32-32 and the README's 512x2-8-64
@pytest.mark.parametrize("factorized,ft_out,l1,l2", [(True, 256, 32, 32), (False, 256, 32, 32), (True, 512, 8, 64)])
def test_simple_export_bytes(gpu, tmp_path, factorized, ft_out, l1, l2):
    info = of.feature_set_info("halfkp")
    ft_in, pi = info["ft_in"], 1548 if factorized else 0
    cfg = SimpleConfig(ft_in=ft_in, max_active=info["max_active"], piece_inputs=pi, ft_out=ft_out, l1_out=l1,
                       l2_out=l2, max_batch=1024, optimizer="adamw", weight_decay=0.01)
    fv = simple_fv_scale(290.0)
    with SimpleTrainer(cfg) as t:
        for s in range(3):
            db = psv_to_device_batch(psv.synthetic_psv(1024, seed=60 + s), "halfkp", "none", 1)
            t.train_step(db, 2e-3, 0.0, Wrm())
        t.flush_pending_loss()
        _plant(t, "ft_w", np.arange(EDGES.size) * 257, EDGES)
        _plant(t, "l1_w", [0, 31, 32], [2.0, -2.0, 0.5 / 64])
        _plant(t, "l3_b", [0], [-1e7])
        path = tmp_path / "simple.bin"
        t.save_quantised(path, "halfkp", fv_scale=fv)
        got = path.read_bytes()
        w = {g: t.get(g) for g in t.GROUPS}
    w["ft_w"] = ox.coalesce(w["ft_w"], ft_in, pi, ft_out)
    # to_simple_weights: the device's in-major dense tables become out-major
    w["l1_w"] = w["l1_w"].reshape(2 * ft_out, l1).T.copy()
    w["l2_w"] = w["l2_w"].reshape(l1, l2).T.copy()
    want = ox.simple_save_quantised(0, 0x5D69D5B8, ft_in, ft_out, l1, l2, w, fv_scale=fv)
    assert len(got) == len(want)
    if got != want:
        bad = np.nonzero(np.frombuffer(got, np.uint8) != np.frombuffer(want, np.uint8))[0]
        raise AssertionError(f"{bad.size} bytes differ, first at {bad[:8]}")
    d = ox.parse_simple(got, ft_in, ft_out, l1, l2)
    assert d["trailing"] == 0 and d["network_hash"] == ox.simple_network_hash(0x5D69D5B8, ft_out, l1, l2)


def test_export_rejects_wrong_feature_set(gpu, tmp_path):
    _, t = _ls_trainer(1629)
    with t:
        with pytest.raises(Exception, match="ft_in"):
            t.save_quantised(tmp_path / "x.bin", "halfkp", fv_scale=28)
        assert not (tmp_path / "x.bin").exists()
    _, t = _ls_trainer(45)  # 73305 rows folded over 45 pieces: not the feature set's factorizer
    with t:
        with pytest.raises(Exception, match="piece_inputs"):
            t.save_quantised(tmp_path / "x.bin", "halfka-hm-merged", fv_scale=28)
