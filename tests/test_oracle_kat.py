"""Pins the CPU oracle to the reference's own known-answer tests.

Each test cites the reference test it reproduces; the expected values are
the ones written in those tests.  Where the reference has no stored value,
the check is one the mathematics fixes (closed forms in float64, finite
differences, invariants), chosen so that a dropped term, a wrong sign or a
transposed operand would fail.
"""
import math

import numpy as np
import pytest

from oracle import ffi
from oracle import layerstack as ols

F32 = np.float32


def arr(*v):
    return np.array(v, dtype=np.float32)


# -- sparse_ft_forward.rs:132-195 ----------------------------------------------
def test_sparse_forward_reference_case():
    w = arr(0, 1, 2, 3, 4, 5)
    idx = np.array([0, 1, -1, -1, 2, 2, 1, 0], np.int32)
    out = ffi.sparse_ft_forward(w, idx, [2, 4], 2, 2, 3, 4)
    assert out.tolist() == [2.0, 4.0, 10.0, 14.0]


def test_sparse_forward_padding_oob_duplicates():
    assert ffi.sparse_ft_forward(arr(1, 2, 3, 4), [-1] * 6, [6], 1, 2, 2, 6).tolist() == [0, 0]
    assert ffi.sparse_ft_forward(arr(1, 2, 3, 4), [0, 5, -1], [3], 1, 2, 2, 3).tolist() == [1, 2]
    assert ffi.sparse_ft_forward(arr(1, 10, 2, 20), [0, 0, 1], [3], 1, 2, 2, 3).tolist() == [4, 40]
    assert ffi.sparse_ft_forward(arr(1, 2), np.zeros(0, np.int32), [0], 1, 2, 1, 0).tolist() == [0, 0]


# -- sparse_ft_backward.rs:276-398 ---------------------------------------------
def test_sparse_backward_reference_case():
    g = np.zeros(9, np.float32)
    ffi.sparse_ft_backward(arr(0, 1, 2, 3, 4, 5), [0, 1, -1, -1, 2, 2, 1, 0], g, 2, 3, 3, 4)
    assert g.tolist() == [3, 5, 7, 3, 5, 7, 6, 8, 10]


def test_sparse_backward_edges():
    g = np.zeros(6, np.float32)
    ffi.sparse_ft_backward(arr(1, 2, 3), [-1] * 4, g, 1, 3, 2, 4)
    assert g.tolist() == [0] * 6
    g = np.zeros(4, np.float32)
    ffi.sparse_ft_backward(arr(1, 1), [0, 5, -1], g, 1, 2, 2, 3)
    assert g.tolist() == [1, 1, 0, 0]
    g = np.zeros(4, np.float32)
    ffi.sparse_ft_backward(arr(10, 20), [0, 0, 1], g, 1, 2, 2, 3)
    assert g.tolist() == [20, 40, 10, 20]
    g = arr(1.0)
    ffi.sparse_ft_backward(arr(5), [0], g, 1, 1, 1, 1)
    assert g.tolist() == [6.0]


def test_forward_backward_consistency():
    w = arr(0, 1, 2, 3, 4, 5)
    idx = [0, 1, -1, -1, 2, 2, 1, 0]
    out = ffi.sparse_ft_forward(w, idx, [4, 4], 2, 2, 3, 4)
    g = np.zeros(6, np.float32)
    ffi.sparse_ft_backward(out, idx, g, 2, 2, 3, 4)
    assert g.tolist() == [12, 18, 12, 18, 20, 28]


def test_backward_nnz_variant_equals_padded_backward():
    rng = np.random.default_rng(3)
    b, ma, cols, rows = 7, 6, 11, 8
    idx = rng.integers(-1, cols + 2, size=(b, ma)).astype(np.int32)
    nnz = rng.integers(0, ma + 1, size=b).astype(np.int32)
    padded = idx.copy()
    for i in range(b):
        padded[i, nnz[i]:] = -1
    go = rng.standard_normal(b * rows).astype(np.float32)
    g1 = np.zeros(rows * cols, np.float32)
    g2 = np.zeros(rows * cols, np.float32)
    ffi.sparse_ft_backward(go, padded.ravel(), g1, b, rows, cols, ma)
    ffi.sparse_ft_backward_nnz(go, idx.ravel(), nnz, g2, b, rows, cols, ma)
    assert np.array_equal(g1, g2)


def test_sparse_forward_matches_float64_brute_force():
    rng = np.random.default_rng(0)
    b, ma, cols, rows = 9, 5, 13, 16
    w = rng.standard_normal(rows * cols).astype(np.float32)
    idx = rng.integers(-2, cols + 3, size=(b, ma)).astype(np.int32)
    nnz = rng.integers(0, ma + 1, size=b).astype(np.int32)
    out = ffi.sparse_ft_forward(w, idx.ravel(), nnz, b, rows, cols, ma).reshape(b, rows)
    W = w.reshape(cols, rows)
    for i in range(b):
        acc = np.zeros(rows, np.float32)
        for n in range(nnz[i]):
            v = idx[i, n]
            if 0 <= v < cols:
                acc = acc + W[v]
        assert np.array_equal(out[i], acc)


# -- ft_factorize.rs tests: fold == virtual-index forward, reduce == virtual backward
FT_IN, FT_OUT, PI = 6, 4, 2


def _train_w():
    return np.array([((i * 37 % 101) - 50.0) * 0.013 for i in range((FT_IN + PI) * FT_OUT)], np.float32)


def _real_train_indices():
    real = [0, 4, 5, 2, 3, -1]
    train = []
    for pos in (real[0:3], real[3:6]):
        row = list(pos) + [FT_IN + v % PI if v >= 0 else -1 for v in pos]
        train += row
    return np.array(real, np.int32), np.array(train, np.int32)


def test_fold_matches_virtual_index_forward():
    w = _train_w()
    comb = ffi.ft_fold_virtual(w, FT_IN, FT_OUT, PI)
    real, train = _real_train_indices()
    a = ffi.sparse_ft_forward(comb, real, [3, 3], 2, FT_OUT, FT_IN, 3)
    b = ffi.sparse_ft_forward(w, train, [6, 6], 2, FT_OUT, FT_IN + PI, 6)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-6)


def test_reduce_matches_virtual_index_backward():
    real, train = _real_train_indices()
    go = np.array([(i + 1.0) * 0.25 for i in range(2 * FT_OUT)], np.float32)
    g_new = np.zeros((FT_IN + PI) * FT_OUT, np.float32)
    ffi.sparse_ft_backward(go, real, g_new, 2, FT_OUT, FT_IN, 3)
    ffi.ft_reduce_virtual_grad(g_new, FT_IN, FT_OUT, PI)
    g_virt = np.zeros((FT_IN + PI) * FT_OUT, np.float32)
    ffi.sparse_ft_backward(go, train, g_virt, 2, FT_OUT, FT_IN + PI, 6)
    np.testing.assert_allclose(g_new, g_virt, rtol=1e-6, atol=1e-6)


def test_reduce_is_sequential_sum_over_king_buckets():
    rng = np.random.default_rng(1)
    ft_in, ft_out, pi = 12, 8, 3
    g = rng.standard_normal((ft_in + pi) * ft_out).astype(np.float32)
    ffi.ft_reduce_virtual_grad(g, ft_in, ft_out, pi)
    G = g.reshape(ft_in + pi, ft_out)
    for v in range(pi):
        acc = np.zeros(ft_out, np.float32)
        for f in range(v, ft_in, pi):
            acc = acc + G[f]
        assert np.array_equal(G[ft_in + v], acc)


# -- ft_post_perspective.rs tests ------------------------------------------------
SC = np.float32(127.0 / 128.0)


def test_ft_post_forward_cases():
    c = ffi.ft_post_perspective_fwd(arr(0.5, 0.25, 2.0, -1.0), arr(0.8, 0.1, 0.3, 0.9), np.zeros(4, np.float32), 1, 4, 1.0)
    exp = [F32(0.5) * F32(1.0), F32(0.25) * F32(0.0), F32(0.8) * F32(0.3), F32(0.1) * F32(0.9)]
    assert c.tolist() == [float(e) for e in exp]
    c1 = ffi.ft_post_perspective_fwd(arr(10, -10), arr(0, 0), arr(0.5, 0.5), 1, 2, SC)
    assert c1[0] == 0.0 and c1[1] == F32(0.25) * SC
    c2 = ffi.ft_post_perspective_fwd(arr(0.5, 0.5), arr(0.5, 0.5), arr(0.5, 0.5), 1, 2, SC)
    assert c2.tolist() == [float(SC), float(SC)]
    assert math.isnan(ffi.ft_post_perspective_fwd(arr(np.nan, 0.5), arr(0.5, 0.5), arr(0, 0), 1, 2, 1.0)[0])


def test_ft_post_grad_cases():
    gb = np.zeros(2, np.float32)
    g = ffi.ft_post_perspective_grad(arr(3.0, 999.0), arr(0.5, 0.25), arr(0, 0), gb, 1, 2, 0, 2, 1.0)
    assert g.tolist() == [0.75, 1.5] and gb.tolist() == [0.75, 1.5]
    gb = arr(7.0, 8.0)
    g = ffi.ft_post_perspective_grad(arr(10, 0), arr(-1, 5), arr(0, 0), gb, 1, 2, 0, 2, 1.0)
    assert g.tolist() == [0, 0] and gb.tolist() == [7, 8]
    gb = np.zeros(4, np.float32)
    g = ffi.ft_post_perspective_grad(arr(1, 2, 10, 20), arr(0.5, 0.5, 0.5, 0.5), np.zeros(4, np.float32), gb, 1, 4, 2, 4, 1.0)
    assert g.tolist() == [5, 10, 5, 10] and gb.tolist() == [5, 10, 5, 10]


def test_ft_post_grad_matches_finite_difference():
    rng = np.random.default_rng(5)
    b, d = 3, 8
    ft = rng.uniform(0.05, 0.95, b * d).astype(np.float32)
    bias = rng.uniform(-0.02, 0.02, d).astype(np.float32)
    dcomb = rng.standard_normal(b * d).astype(np.float32)
    gb = np.zeros(d, np.float32)
    g_stm = ffi.ft_post_perspective_grad(dcomb, ft, bias, gb, b, d, 0, d, SC)
    # L = sum_c dcomb[:, c<half] * combined[:, c<half] as a function of ft (stm side)
    def L(x):
        c = ffi.ft_post_perspective_fwd(x, ft, bias, b, d, SC).reshape(b, d).astype(np.float64)
        return float((c[:, : d // 2] * dcomb.reshape(b, d)[:, : d // 2]).sum())
    eps = 1e-3
    for k in [0, 3, 5, 9, 17]:
        xp = ft.copy(); xp[k] += eps
        xm = ft.copy(); xm[k] -= eps
        fd = (L(xp) - L(xm)) / (2 * eps)
        assert abs(fd - g_stm[k]) < 2e-3 * max(1.0, abs(fd))


# -- dense_mm.rs / dense_mm_bucket.rs tests -----------------------------------------
def test_dense_mm_cases():
    assert ffi.dense_mm_fwd(arr(1, 2, 3, 4), arr(5, 6, 7, 8), arr(10, 20), 2, 2, 2).tolist() == [29, 42, 53, 70]
    assert ffi.dense_mm_bwd_input(arr(1, 1, 1, 1), arr(5, 6, 7, 8), 2, 2, 2).tolist() == [11, 15, 11, 15]
    assert ffi.dense_mm_bwd_weight(arr(1, 2, 3, 4), arr(10, 20, 30, 40), 2, 2, 2).tolist() == [100, 140, 140, 200]
    assert ffi.bias_grad(arr(10, 20, 30, 40), arr(1, 2), 2, 2).tolist() == [41, 62]


def test_dense_mm_bucket_cases():
    w = arr(1, 2, 3, 4)
    assert ffi.dense_mm_fwd_bucket(arr(1, 1, 2, 2), w, arr(10, 20), [0, 1], 2, 2, 1, 2).tolist() == [13, 34]
    assert ffi.dense_mm_fwd_bucket(arr(5, 5), w, arr(10, 20), [-1], 1, 2, 1, 2).tolist() == [0]
    assert ffi.dense_mm_fwd_bucket(arr(5, 5), w, arr(10, 20), [2], 1, 2, 1, 2).tolist() == [0]
    assert ffi.dense_mm_bwd_input_bucket(arr(1, 1), w, [0, 1], 2, 2, 1, 2).tolist() == [1, 2, 3, 4]
    assert ffi.dense_mm_bwd_input_bucket(arr(1), w, [-5], 1, 2, 1, 2).tolist() == [0, 0]
    assert ffi.dense_mm_bwd_weight_bucket(arr(1, 1, 2, 2, 3, 3), arr(10, 20, 30), [0, 0, 1], 3, 2, 1, 2).tolist() == [50, 50, 90, 90]
    assert ffi.dense_mm_bwd_weight_bucket(arr(1, 1, 100, 100), arr(10, 10), [0, -1], 2, 2, 1, 2).tolist() == [10, 10, 0, 0]
    assert ffi.bias_grad_bucket(arr(1, 2, 3, 4, 5, 6), [0, 1, 0], arr(10, 20, 30, 40), 3, 2, 2).tolist() == [16, 28, 33, 44]


def test_dense_mm_bucket_is_transpose_consistent():
    # <dy, W x> == <W^T dy, x> per row, for each bucket (closed form check)
    rng = np.random.default_rng(7)
    b, i, o, nb = 6, 5, 3, 3
    x = rng.standard_normal(b * i).astype(np.float32)
    w = rng.standard_normal(nb * o * i).astype(np.float32)
    bk = np.array([0, 2, 1, 1, 0, 2], np.int32)
    dy = rng.standard_normal(b * o).astype(np.float32)
    y = ffi.dense_mm_fwd_bucket(x, w, np.zeros(nb * o, np.float32), bk, b, i, o, nb)
    dx = ffi.dense_mm_bwd_input_bucket(dy, w, bk, b, i, o, nb)
    lhs = (y.astype(np.float64) * dy).reshape(b, o).sum(1)
    rhs = (dx.astype(np.float64) * x).reshape(b, i).sum(1)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-5, atol=1e-5)


# -- pointwise glue -------------------------------------------------------------------
def test_crelu_cases():
    assert ffi.crelu_fwd(arr(-2, -0.5, 0, 0.3, 1, 1.5, 7)).tolist() == [0, 0, 0, float(F32(0.3)), 1, 1, 1]
    assert ffi.crelu_grad(arr(-1, 0, 0.0001, 0.5, 0.9999, 1, 2), arr(*[3] * 7)).tolist() == [0, 0, 3, 3, 3, 0, 0]
    assert ffi.crelu_grad(arr(np.nan), arr(5))[0] == 0.0


def test_abs_pow2_scale_cases():
    y = ffi.abs_pow2_scale_fwd(arr(-3, 0, 0.5, 2), SC)
    assert y[0] == F32(9.0) * SC and y[1] == 0.0
    dx = ffi.abs_pow2_scale_grad(arr(1, -2, 0, 4), arr(0.5, 1, 3, -1), 2.0)
    assert dx.tolist() == [2.0, -8.0, 0.0, -16.0]


def test_concat_slice_elementwise():
    out = ffi.concat_l1sqr_main_fwd(arr(1, 2, 3, 4), arr(5, 6, 7, 8), 2, 2, 2)
    assert out.tolist() == [1, 2, 5, 6, 3, 4, 7, 8]
    da, db = ffi.concat_l1sqr_main_grad(out, 2, 2)
    assert da.tolist() == [1, 2, 3, 4] and db.tolist() == [5, 6, 7, 8]
    assert ffi.slice_extract_2d(arr(1, 2, 3, 4, 5, 6), 2, 3, 1, 2).tolist() == [2, 3, 5, 6]
    dst = np.zeros(6, np.float32)
    ffi.slice_scatter_2d(arr(7, 8), dst, 2, 1, 3, 2)
    assert dst.tolist() == [0, 0, 7, 0, 0, 8]
    assert ffi.elementwise_add(arr(1, 2), arr(3, 4)).tolist() == [4, 6]


# -- losses (loss_wdl.rs:102-300, loss_wrm.rs:255-987) ------------------------------------
def _sig64(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def test_loss_wdl_closed_form_and_grad():
    out = arr(0.5, -0.3, 1.0)
    score = arr(0, 0, 0.5)
    d, acc = ffi.loss_wdl(out, score, arr(1, 1, 1), arr(1, 1, 1), 0.0, 1.0)
    p, ys = _sig64(out), _sig64(score)
    assert abs(acc - ((p - ys) ** 2).sum()) < 1e-6
    np.testing.assert_allclose(d, 2 * (p - ys) * p * (1 - p), rtol=1e-5, atol=1e-7)
    d, acc = ffi.loss_wdl(arr(0), arr(999), arr(0.5), arr(1), 1.0, 1.0)
    assert d[0] == 0.0 and acc == 0.0
    d, acc = ffi.loss_wdl(arr(100, -100, 0), arr(1, -1, 0.5), arr(1, 0, 0.5), arr(1, 1, 1), 0.5, 0.0)
    assert d.tolist() == [0, 0, 0]
    d_a, acc_a = ffi.loss_wdl(arr(1, 1), arr(0, 0), arr(1, 1), arr(1, 1), 0.0, 1.0)
    d_b, acc_b = ffi.loss_wdl(arr(1, 1), arr(0, 0), arr(1, 1), arr(0.5, 0.5), 0.0, 1.0)
    assert acc_a == acc_b and np.allclose(d_b, d_a * 0.5, atol=1e-7)


WRM = dict(nnue2score=600.0, in_scaling=340.0, in_offset=270.0, target_offset=270.0,
           target_scaling=380.0)


def _wrm(out, score, wdl, norm, lam, pow_exp=2.0, asym=0.0, w1=0.0, w2=0.5, ext=False):
    return ffi.loss_wrm(out, score, wdl, norm, lam, WRM["nnue2score"], WRM["in_scaling"],
                        WRM["in_offset"], WRM["target_offset"], WRM["target_scaling"], pow_exp,
                        asym, w1, w2, ext)


def _wrm64(out, score, wdl, lam):
    s = np.asarray(score, np.float64)
    t = 0.5 * (1 + _sig64((s - 270) / 380) - _sig64((-s - 270) / 380))
    target = lam * np.asarray(wdl, np.float64) + (1 - lam) * t
    sn = np.asarray(out, np.float64) * 600
    q, qm = _sig64((sn - 270) / 340), _sig64((-sn - 270) / 340)
    err = 0.5 * (1 + q - qm) - target
    return err, q, qm


def test_loss_wrm_zero_and_formula():
    d, acc = _wrm(arr(0), arr(0), arr(0.5), arr(1), 0.0)
    assert acc == 0.0 and d[0] == 0.0
    d, acc = _wrm(arr(0), arr(999), arr(0.5), arr(1), 1.0)
    assert acc == 0.0 and d[0] == 0.0
    rng = np.random.default_rng(2)
    out = rng.uniform(-2, 2, 16).astype(np.float32)
    score = rng.uniform(-1500, 1500, 16).astype(np.float32)
    wdl = rng.choice([0.0, 0.5, 1.0], 16).astype(np.float32)
    d, acc = _wrm(out, score, wdl, np.ones(16, np.float32), 0.3)
    err, q, qm = _wrm64(out, score, wdl, 0.3)
    assert abs(acc - (err ** 2).sum()) < 1e-5
    np.testing.assert_allclose(d, err * (600 / 340) * (q * (1 - q) + qm * (1 - qm)), rtol=2e-4, atol=1e-7)


def test_loss_wrm_grad_matches_finite_difference():
    out = arr(-0.7, -0.1, 0.05, 0.4, 1.3)
    score = arr(-800, 100, 0, 350, 1200)
    wdl = arr(0, 0.5, 0.5, 1, 1)
    for ext, kw in ((False, {}), (True, dict(pow_exp=2.5, asym=0.3, w1=1.0, w2=0.5))):
        d, _ = _wrm(out, score, wdl, np.ones(5, np.float32), 0.2, ext=ext, **kw)
        eps = 1e-3
        for k in range(5):
            op, om = out.copy(), out.copy()
            op[k] += eps
            om[k] -= eps
            # squared form: d(err^2)/dout = 2 err dqf/dout and dqf/dout carries a
            # factor 1/2, so the gradient is exactly d(loss)/dout (norm = 1);
            # extended form: the loss carries n * (1/sum w), the gradient 1/sum w
            _, lp = _wrm(op, score, wdl, np.ones(5, np.float32), 0.2, ext=ext, **kw)
            _, lm = _wrm(om, score, wdl, np.ones(5, np.float32), 0.2, ext=ext, **kw)
            fd = (lp - lm) / (2 * eps)
            factor = 1.0 if not ext else 1.0 / 5.0
            assert abs(fd * factor - d[k]) < 2e-3 * max(1e-3, abs(fd * factor)), (ext, k, fd, d[k])


# -- optimizer (radam_step.rs:162-200+, optimizer.rs:196-242, ranger_step.rs:111+) ----------
def test_radam_step_size_denom_closed_forms():
    ss, dn = ffi.radam_step_size_denom(1, 0.9, 0.999, 5.0)
    assert dn == 0 and abs(ss - 1.0 / (1.0 - 0.9)) < 1e-5
    ss, dn = ffi.radam_step_size_denom(1000, 0.9, 0.999, 5.0)
    b2t = 0.999 ** 1000
    nmax = 2 / 0.001 - 1
    n = nmax - 2 * 1000 * b2t / (1 - b2t)
    exp = math.sqrt((1 - b2t) * (n - 4) / (nmax - 4) * (n - 2) / n * nmax / (nmax - 2)) / (1 - 0.9 ** 1000)
    assert dn == 1 and abs(ss - exp) < 1e-5 * exp


def test_radam_one_step_cases():
    w, m, v, g = arr(1.0), arr(0.0), arr(0.0), arr(0.1)
    ffi.radam_step(w, m, v, g, 0.1, 10.0, 0, 0.0, 0.9, 0.999, 1e-8, ols.F32_MIN, ols.F32_MAX)
    assert abs(w[0] - 0.99) < 1e-6 and abs(m[0] - 0.01) < 1e-7 and abs(v[0] - 1e-5) < 1e-9 and g[0] == 0.0
    w, m, v, g = arr(1.0), arr(0.01), arr(1e-5), arr(0.1)
    ffi.radam_step(w, m, v, g, 0.1, 1.0, 1, 0.0, 0.9, 0.999, 1e-8, ols.F32_MIN, ols.F32_MAX)
    mi, vi = 0.9 * 0.01 + 0.1 * 0.1, 0.999 * 1e-5 + 0.001 * 0.01
    assert abs(w[0] - (1.0 - 0.1 * mi / (math.sqrt(vi) + 1e-8))) < 1e-5
    # decay and clamp
    w, m, v, g = arr(2.0, -2.0), arr(0, 0), arr(0, 0), arr(0, 0)
    ffi.radam_step(w, m, v, g, 0.5, 1.0, 1, 0.1, 0.9, 0.999, 1e-8, -1.5, 1.5)
    assert w.tolist() == [1.5, -1.5]
    w, m, v, g = arr(1.0), arr(0), arr(0), arr(0)
    ffi.radam_step(w, m, v, g, 0.5, 1.0, 1, 0.1, 0.9, 0.999, 1e-8, ols.F32_MIN, ols.F32_MAX)
    assert w[0] == F32(1.0) * (F32(1.0) - F32(0.1) * F32(0.5))


def test_ranger_lerp_cases():
    w, s = arr(1, 2, 3), arr(10, 20, 30)
    ffi.ranger_lookahead_lerp(w, s, 1.0)
    assert w.tolist() == [1, 2, 3] and s.tolist() == [1, 2, 3]
    w, s = arr(1, 2, 3), arr(10, 20, 30)
    ffi.ranger_lookahead_lerp(w, s, 0.0)
    assert w.tolist() == [10, 20, 30] and s.tolist() == [10, 20, 30]
    w, s = arr(2, -4, 0), arr(4, 4, 10)
    ffi.ranger_lookahead_lerp(w, s, 0.5)
    assert w.tolist() == [3, 0, 5] and s.tolist() == [3, 0, 5]


# -- init (init.rs:439-480) ---------------------------------------------------------------
def _xorshift_py(seed, n, scale):
    s = max(seed, 1)
    out = []
    mask = (1 << 64) - 1
    for _ in range(n):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        u = np.float32(s >> 11) / np.float32(1 << 53)
        out.append((u * np.float32(2.0) - np.float32(1.0)) * np.float32(scale))
    return np.array(out, np.float32)


def test_init_uniform_is_bit_identical_to_xorshift():
    for seed, n in ((0x100, 37), (0x5071E003, 1024), (1, 9), (0, 5)):
        got = ffi.init_sample(n, 99, "uniform", "abs", 0.01, seed)
        assert np.array_equal(got, _xorshift_py(seed, n, 0.01)), hex(seed)


def test_init_fanin_bound():
    fan_in = 73305
    v = ffi.init_sample(200_000, fan_in, "uniform", "fanin", 1.0, 0xABCD)
    bound = np.float32(math.sqrt(1.0 / fan_in))
    assert v.max() <= bound and v.max() > bound * 0.98
    assert v.min() >= -bound and v.min() < -bound * 0.98


def test_init_per_bucket_repeat_and_zero():
    v = ffi.init_sample(12, 4, "uniform", "abs", 0.5, 7, num_buckets=3, per_bucket_repeat=True)
    assert np.array_equal(v[:4], v[4:8]) and np.array_equal(v[:4], v[8:])
    assert not np.any(ffi.init_sample(8, 4, "zero"))


# -- the oracle step: properties fixed by the mathematics ----------------------------------
def test_oracle_step_linear_gradients_match_finite_difference():
    """Finite-difference check of d(loss)/d(l3_b) and d(loss)/d(l1_shared_bias[last]).

    The sigmoid-MSE gradient the reference emits is dL/dout * (1/b) / 2
    (loss = sum err^2, grad = 2 err p (1-p) scale / b) so the directional
    derivative of sum(err^2)/(2b)... is compared to the bias gradients.
    """
    sh = ols.LsShape(ft_in=40, max_active=6, piece_inputs=8, ft_out=16, l1=16, l2=32, nb=3)
    st = ols.default_init(sh)
    rng = np.random.default_rng(11)
    b = 32
    stm = rng.integers(0, 40, (b, 6)).astype(np.int32)
    nstm = rng.integers(0, 40, (b, 6)).astype(np.int32)
    batch = dict(stm=stm, nstm=nstm, nnz=np.full(b, 6, np.int32),
                 bucket=rng.integers(0, 3, b).astype(np.int32),
                 score=rng.uniform(-600, 600, b).astype(np.float32),
                 wdl=rng.choice([0, 0.5, 1], b).astype(np.float32))
    # make activations non-trivial
    st["ft_w"]["w"][:] = rng.uniform(0.0, 0.08, st["ft_w"]["w"].size).astype(np.float32)
    loss = {"kind": "sigmoid", "scale": 1.0 / 290.0}
    a, acc = ols.forward(sh, st, batch, 0.0, loss)
    g = ols.backward(sh, st, batch, a)

    def L(name, k, eps):
        s2 = {kk: {q: vv.copy() for q, vv in v.items()} for kk, v in st.items()}
        s2[name]["w"][k] += eps
        _, acc2 = ols.forward(sh, s2, batch, 0.0, loss)
        return acc2

    # parameters the loss depends on linearly up to the sigmoid (scale 1/290
    # keeps it near-linear), so a wide central difference is accurate and
    # stays far above the float32 noise of the summed loss
    for name, k in (("l3_b", 1), ("l1_shared_bias", 15), ("l3_w", 3 * 32 // 3)):
        eps = 1.0
        fd = (L(name, k, eps) - L(name, k, -eps)) / (2 * eps)
        # d(sum err^2)/dθ = 2 sum err dp/dθ ; reference grad = that / b
        assert abs(fd / b - g[name][k]) < 5e-3 * max(abs(fd / b), 1e-6), (name, fd / b, g[name][k])
