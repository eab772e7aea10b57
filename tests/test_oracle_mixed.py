"""Mixed-precision oracle (oracle/layerstack.py Precision, orc_ft_grad_fp16)
pinned independently of its own formulas.

  - f16 rounding: IEEE binary16 round-to-nearest-even, overflow to infinity
    (the values __float2half_rn gives), on hand-picked ties and boundaries;
  - the fp16 gradient gather follows the reference kernel's accumulation
    order (four interleaved partial sums, native_kernels.cu:1030-1075): a
    cancellation case whose sequential sum differs tells the orders apart;
    overwrite / add-if-nonzero semantics; the sum equals the exact sum within
    f32 rounding;
  - f16 moments: at step 1 RAdam uses this step's f32 moments, so the weights
    equal the fp32 path's exactly and the stored moments are f16(m 2^28),
    f16(v 2^40) of the fp32 moments; later steps stay within f16 precision;
  - all flags off is the fp32 step, bit for bit; each f16 mode moves the
    step's outputs by no more than f16 precision allows;
  - the TF32-class L1 products (tf32): the L1 outputs, the L1 weight
    gradients and the L1 input gradient equal float64 products of the
    stated operands (forward: f16 combined and f16 weights, the bucket bias
    added after the bucket sum; weight gradients: f16 combined and f32 dl1;
    input gradient: f32 dl1 and f32 weights) within f32 summation error,
    and planted mistakes (an operand rounded where it is not, or left
    unrounded where it is) fall outside that.
"""
import numpy as np
import pytest

from oracle import ffi
from oracle import layerstack as ols
from tatara_amd.synthetic import small_spec, structured_batch

SPEC = small_spec(king_buckets=6, piece_inputs=48, max_active=32)


def test_f16_rounding():
    x = np.array([2049.0, 2051.0, 2050.0, 65504.0, 65519.0, 65520.0, -65520.0, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -24], np.float32)
    want = [2048.0, 2052.0, 2050.0, 65504.0, 65504.0, np.inf, -np.inf, 1.0, 1.0 + 2.0 ** -9, 0.0,
            2.0 ** -24, 2.0 ** -24]
    assert ols.f16(x).tolist() == want


def test_fp16_gather_order_and_semantics():
    # one feature (0) with 5 occurrences at positions 0..4, rows = 1 column
    vals = np.array([1e8, 1.0, -1e8, 1.0, 1.0], np.float32)
    idx = np.zeros((5, 1), np.int32)
    nnz = np.ones(5, np.int32)
    g = np.zeros(2, np.float32)
    ffi.ft_grad_fp16(vals[:, None], idx, nnz, g, 5, 1, 2, 1, 1.0, add=False)
    # s0 = 1e8 + 1 (=1e8), s1 = 1, s2 = -1e8, s3 = 1 -> (1e8 + 1) + (-1e8 + 1) = 0 in f32;
    # a sequential sum would give 2
    assert g[0] == np.float32(np.float32(1e8 + 1) + np.float32(-1e8 + 1)) == 0.0
    assert g[1] == 0.0  # overwrite writes every feature
    g2 = np.full(2, 7.0, np.float32)
    ffi.ft_grad_fp16(vals[:, None], idx, nnz, g2, 5, 1, 2, 1, 1.0, add=True)
    assert g2.tolist() == [7.0, 7.0]  # the sum is 0: nothing added
    rng = np.random.default_rng(1)
    b, rows, cols, ma = 64, 8, 20, 6
    dft = ols.f16(rng.normal(0, 100, (b, rows)))
    idx = rng.integers(-1, cols + 1, (b, ma)).astype(np.int32)  # includes invalid indices
    nnz = rng.integers(0, ma + 1, b).astype(np.int32)
    g = np.zeros(cols * rows, np.float32)
    inv = np.float32(1.0 / 1024)
    ffi.ft_grad_fp16(dft, idx, nnz, g, b, rows, cols, ma, inv, add=False)
    exact = np.zeros((cols, rows))
    for p in range(b):
        for s in range(nnz[p]):
            f = idx[p, s]
            if 0 <= f < cols:
                exact[f] += dft[p].astype(np.float64)
    np.testing.assert_allclose(g.reshape(cols, rows), exact * float(inv), rtol=1e-5, atol=1e-4)


def _setup(seed=0, b=64):
    sh = ols.LsShape(ft_in=SPEC["ft_in"], max_active=SPEC["max_active"], piece_inputs=SPEC["piece_inputs"],
                     ft_out=128, l1=16, l2=32, nb=4)
    batch, bucket = structured_batch(b, SPEC, num_buckets=4, seed=seed, nnz_min=20)
    bd = dict(stm=batch.stm_indices, nstm=batch.nstm_indices, nnz=batch.nnz, bucket=bucket, score=batch.score,
              wdl=batch.wdl)
    return sh, bd


LOSS = {"kind": "sigmoid", "scale": 1.0 / 290.0}


def test_flags_off_is_the_fp32_step():
    sh, bd = _setup()
    opt = ols.OptConfig()
    s1, s2 = ols.default_init(sh), ols.default_init(sh)
    a1, _, _ = ols.train_step(sh, s1, bd, opt, 1e-3, 0.0, LOSS, 1)
    a2, _, _ = ols.train_step(sh, s2, bd, opt, 1e-3, 0.0, LOSS, 1, ols.Precision())
    assert a1 == a2 and all(np.array_equal(s1[k]["w"], s2[k]["w"]) for k in s1)


def test_f16_state_step_one_and_two():
    sh, bd = _setup(2)
    opt = ols.OptConfig()
    ref = ols.default_init(sh)
    half = ols.to_f16_state(ols.default_init(sh))
    prec = ols.Precision(False, False, True)
    ols.train_step(sh, ref, bd, opt, 1e-3, 0.0, LOSS, 1)
    ols.train_step(sh, half, bd, opt, 1e-3, 0.0, LOSS, 1, prec)
    assert np.array_equal(ref["ft_w"]["w"], half["ft_w"]["w"])
    assert np.array_equal(half["ft_w"]["m16"], ols.f16(np.clip(ref["ft_w"]["m"] * ols.M_SCALE, -65504, 65504)))
    assert np.array_equal(half["ft_w"]["v16"], ols.f16(np.minimum(ref["ft_w"]["v"] * ols.V_SCALE, 65504)))
    # step 2 reads the rounded moments: the update differs by at most f16 precision
    ols.train_step(sh, ref, bd, opt, 1e-3, 0.0, LOSS, 2)
    ols.train_step(sh, half, bd, opt, 1e-3, 0.0, LOSS, 2, prec)
    d = np.abs(ref["ft_w"]["w"] - half["ft_w"]["w"])
    assert d.max() > 0.0 and d.max() <= 2e-3 * 2e-3  # lr * (relative moment error); updates are ~lr


@pytest.mark.parametrize("prec", [ols.Precision(True, False, False), ols.Precision(True, True, False),
                                  ols.Precision.all_optim()], ids=["fwd", "fwd_out", "all"])
def test_each_mode_within_f16_precision_of_fp32(prec):
    sh, bd = _setup(4)
    opt = ols.OptConfig()
    ref = ols.default_init(sh)
    mix = ols.to_f16_state(ols.default_init(sh)) if prec.fp16_opt_state else ols.default_init(sh)
    acc_r, a_r, g_r = ols.train_step(sh, ref, bd, opt, 1e-3, 0.0, LOSS, 1)
    acc_m, a_m, g_m = ols.train_step(sh, mix, bd, opt, 1e-3, 0.0, LOSS, 1, prec)
    # FT sums of ~40 f16 rows: relative error ~ 2^-11 per row
    s = np.abs(a_r["ft_stm"]).max()
    assert np.abs(a_m["ft_stm"] - a_r["ft_stm"]).max() <= 40 * 2.0 ** -11 * s
    assert np.array_equal(a_m["ft_stm"], a_r["ft_stm"]) == (not prec.ft_fp16)
    assert abs(acc_m - acc_r) <= 1e-3 * abs(acc_r)
    gm, gr = g_m["ft_w"], g_r["ft_w"]
    assert np.abs(gm - gr).max() <= 1e-2 * np.abs(gr).max()


def test_tf32_l1_products():
    """The oracle's tf32 step against float64 products of the stated operands."""
    sh, bd = _setup(5)
    opt = ols.OptConfig()
    st = ols.default_init(sh)
    prec = ols.Precision(tf32=True)
    a, acc = ols.forward(sh, st, bd, 0.0, LOSS, prec)
    g = ols.backward(sh, st, bd, a, prec)
    b, fo, l1, nb = bd["stm"].shape[0], sh.ft_out, sh.l1, sh.nb
    comb32, _ = ols.forward(sh, ols.default_init(sh), bd, 0.0, LOSS)
    c = ols.f16(comb32["combined"]).reshape(b, fo).astype(np.float64)
    assert np.array_equal(a["combined"], ols.f16(comb32["combined"]))
    w1 = ols.f16(st["l1_w"]["w"]).reshape(nb, l1, fo).astype(np.float64)
    ws = ols.f16(st["l1_shared_weight"]["w"]).reshape(fo, l1).astype(np.float64)
    bk = bd["bucket"]
    valid = (bk >= 0) & (bk < nb)
    exp_b = np.zeros((b, l1))
    exp_b[valid] = np.einsum("rk,rok->ro", c[valid], w1[bk[valid]]) + st["l1_b"]["w"].reshape(nb, l1)[bk[valid]]
    exp_s = c @ ws + st["l1_shared_bias"]["w"]
    mag_b = np.zeros((b, l1))
    mag_b[valid] = np.einsum("rk,rok->ro", np.abs(c[valid]), np.abs(w1[bk[valid]]))
    tol = fo * 2.0 ** -24 * (mag_b + np.abs(c) @ np.abs(ws)) + 1e-12
    assert np.all(np.abs(a["l1_bucket"].reshape(b, l1) - exp_b) <= tol)
    assert np.all(np.abs(a["l1_shared"].reshape(b, l1) - exp_s) <= tol)
    # a planted mistake: the forward with unrounded weights is far outside the bound
    plant = np.einsum("rk,rok->ro", c[valid], st["l1_w"]["w"].reshape(nb, l1, fo)[bk[valid]].astype(np.float64))
    assert np.max(np.abs(plant + st["l1_b"]["w"].reshape(nb, l1)[bk[valid]] - exp_b[valid]) - tol[valid]) > 0
    # weight gradients: f32 dl1 times the f16 combined
    d = a["dl1_total"].reshape(b, l1).astype(np.float64)
    exp_ws = c.T @ d
    tol_ws = b * 2.0 ** -24 * (np.abs(c).T @ np.abs(d)) + 1e-30
    assert np.all(np.abs(g["l1_shared_weight"].reshape(fo, l1) - exp_ws) <= tol_ws)
    # a planted mistake: the f32 combined in the weight gradient
    c32 = comb32["combined"].reshape(b, fo).astype(np.float64)
    assert np.max(np.abs(c32.T @ d - exp_ws) - tol_ws) > 0
    exp_w1 = np.zeros((nb, l1, fo))
    for k in range(nb):
        rows = bk == k
        exp_w1[k] = d[rows].T @ c[rows]
    mag_w1 = np.zeros((nb, l1, fo))
    for k in range(nb):
        rows = bk == k
        mag_w1[k] = np.abs(d[rows]).T @ np.abs(c[rows])
    assert np.all(np.abs(g["l1_w"].reshape(nb, l1, fo) - exp_w1) <= b * 2.0 ** -24 * mag_w1 + 1e-30)
    # the L1 input gradient: f32 dl1 times the f32 weights, bucket + shared
    w1_32 = st["l1_w"]["w"].reshape(nb, l1, fo).astype(np.float64)
    ws_32 = st["l1_shared_weight"]["w"].reshape(fo, l1).astype(np.float64)
    exp_dc = np.zeros((b, fo))
    mag_dc = np.zeros((b, fo))
    exp_dc[valid] = np.einsum("ro,rok->rk", d[valid], w1_32[bk[valid]])
    mag_dc[valid] = np.einsum("ro,rok->rk", np.abs(d[valid]), np.abs(w1_32[bk[valid]]))
    exp_dc += d @ ws_32.T
    mag_dc += np.abs(d) @ np.abs(ws_32).T
    tol_dc = 2 * l1 * 2.0 ** -24 * mag_dc + 1e-30
    assert np.all(np.abs(a["dcombined"].reshape(b, fo) - exp_dc) <= tol_dc)
    # a planted mistake: the f16-rounded weights in the input gradient
    plant_dc = np.zeros((b, fo))
    plant_dc[valid] = np.einsum("ro,rok->rk", d[valid], w1[bk[valid]])
    plant_dc += d @ ws.T
    assert np.max(np.abs(plant_dc - exp_dc) - tol_dc) > 0
    # and the step recomputed with f32 operands agrees only within the
    # f16 rounding
    a32, _ = ols.forward(sh, ols.default_init(sh), bd, 0.0, LOSS, ols.Precision())
    g32 = ols.backward(sh, ols.default_init(sh), bd, a32, ols.Precision())
    assert np.abs(g["ft_b"] - g32["ft_b"]).max() <= 2e-2 * np.abs(g32["ft_b"]).max()
    assert abs(acc - ols.forward(sh, ols.default_init(sh), bd, 0.0, LOSS)[1]) <= 1e-3 * abs(acc)
