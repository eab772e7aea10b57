"""NaN and infinity propagation through the HIP path vs the CPU oracle (GPU).

The reference's equivalence suite plants NaN in the inputs of its element-wise
kernels and in one gradient cell of the optimizer fixture, and asserts NaN
wherever the CPU result is NaN and the usual bar elsewhere
(gpu_cpu_equivalence_tests.rs:137-160 assert_close, :178-232 crelu/screlu,
:5019 radam_fixture grad[n/2] = NaN).  Here the same is asserted for:

  - the FT gather and the pairwise FT forward with a NaN weight row, a NaN
    cell and +-Inf cells: bit-exact with NaN in the same places
    (np.array_equal(..., equal_nan=True));
  - every FT weight-gradient kernel with NaN / +-Inf planted in dft rows: the
    sequential kernels bit-exact with NaN in the same places; the
    matrix-core kernel NaN in exactly the oracle's cells, bit-exact in every
    (king block, 128-column half) whose rows hold a non-finite value (it
    takes the sequential sums there, so a NaN reaches only its own row's
    features), and within its summation bound elsewhere;
  - the RAdam step with the reference's fixture (NaN gradient cell, weights
    past the clamp) and the lookahead lerp with a NaN weight;
  - one LayerStack training step with a NaN FT weight cell, f32 and mixed
    precision (the matrix-core backward): NaN in the same cells as the
    oracle's step for every activation, gradient and post-step tensor, and
    the usual tolerances elsewhere.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import ffi
from oracle import layerstack as ols
from tatara_amd._lib import check
from tatara_amd.trainer import GROUPS, DeviceArray, LayerStackTrainer, Sigmoid

from test_gpu_ops import _blocked_grad, _exact_grad, _oracle_grad, dev, ragged_indices
from test_gpu_trainer import as_dict, batch_for, close, loss_dict, make

pytestmark = pytest.mark.gpu

SC = np.float32(127.0 / 128.0)


def same(got, exp, what=""):
    """Bit-exact, NaN where the oracle has NaN (and nowhere else)."""
    got, exp = np.asarray(got), np.asarray(exp)
    gn, en = np.isnan(got), np.isnan(exp)
    assert np.array_equal(gn, en), f"{what}: NaN at {np.flatnonzero(gn != en)[:8]} differs"
    assert np.array_equal(got, exp, equal_nan=True), f"{what}: {np.count_nonzero(got[~en] != exp[~en])} cells differ"


def close_nan(got, exp, rtol, what="", **kw):
    """NaN in exactly the oracle's cells; the finite cells within tolerance."""
    got = np.asarray(got, np.float64).ravel()
    exp = np.asarray(exp, np.float64).ravel()
    gn, en = np.isnan(got), np.isnan(exp)
    assert np.array_equal(gn, en), (f"{what}: NaN masks differ in {np.count_nonzero(gn != en)} cells "
                                    f"(gpu {gn.sum()}, oracle {en.sum()})")
    fin = ~en
    for k in ("atol",):
        if isinstance(kw.get(k), np.ndarray):
            kw[k] = np.asarray(kw[k], np.float64).ravel()[fin]
    if "atol_frac" in kw:
        kw["atol"] = kw.get("atol", 0.0) + kw.pop("atol_frac") * (np.abs(exp[fin]).max() if fin.any() else 0.0)
    close(got[fin], exp[fin], rtol, what=what, **kw)
    return int(en.sum())


def plant_weights(w, rows):
    """A NaN cell, a whole NaN row, +Inf and -Inf cells (the last two in the
    same column, so that a row holding both features sums to NaN)."""
    cols_ = w.shape[1]
    w[3, 5] = np.nan
    w[7, :] = np.nan
    w[11, cols_ - 1] = np.inf
    w[12, cols_ - 1] = -np.inf
    return w


@pytest.mark.parametrize("rows", [64, 1536])
def test_sparse_forward_nan(gpu, rows):
    rng = np.random.default_rng(rows)
    b, ma, cols = 64, 30, 40  # few columns: most rows hold a planted feature
    w = plant_weights(rng.standard_normal((cols, rows)).astype(np.float32), rows)
    idx, nnz = ragged_indices(rng, b, ma, cols)
    exp = ffi.sparse_ft_forward(w, idx, nnz, b, rows, cols, ma)
    assert np.isnan(exp).any() and np.isinf(exp).any()
    W, I, N = dev(w), dev(idx), dev(nnz)
    out = DeviceArray.empty((b, rows), np.float32)
    check(gpu.tatara_op_sparse_ft_forward(W.ptr, I.ptr, N.ptr, out.ptr, b, rows, cols, ma))
    same(out.to_host().ravel(), exp, "sparse forward")


@pytest.mark.parametrize("ft_out", [256, 1536])
def test_ft_forward_pairwise_nan(gpu, ft_out):
    """CReLU passes NaN through (x < 0 and x > 1 both false), and the
    pairwise product of a NaN with a clipped 0 is NaN, as in the oracle."""
    rng = np.random.default_rng(ft_out)
    b, ma, cols = 64, 30, 60
    w = plant_weights((rng.standard_normal((cols, ft_out)) * 0.05 + 0.02).astype(np.float32), ft_out)
    bias = (rng.standard_normal(ft_out) * 0.1 + 0.2).astype(np.float32)
    bias[9] = np.nan
    si, nnz = ragged_indices(rng, b, ma, cols)
    ni, _ = ragged_indices(rng, b, ma, cols)
    s_exp = ffi.sparse_ft_forward(w, si, nnz, b, ft_out, cols, ma)
    n_exp = ffi.sparse_ft_forward(w, ni, nnz, b, ft_out, cols, ma)
    c_exp = ffi.ft_post_perspective_fwd(s_exp, n_exp, bias, b, ft_out, SC)
    W, S, Nn, N, B = dev(w), dev(si), dev(ni), dev(nnz), dev(bias)
    so = DeviceArray.empty((b, ft_out), np.float32)
    no = DeviceArray.empty((b, ft_out), np.float32)
    co = DeviceArray.empty((b, ft_out), np.float32)
    check(gpu.tatara_op_ft_forward_pairwise(W.ptr, S.ptr, Nn.ptr, N.ptr, B.ptr, so.ptr, no.ptr, co.ptr,
                                            b, ft_out, cols, ma, 0, float(SC)))
    same(so.to_host().ravel(), s_exp, "stm raw sums")
    same(no.to_host().ravel(), n_exp, "nstm raw sums")
    same(co.to_host().ravel(), c_exp, "combined")
    assert np.isnan(c_exp).any()


def plant_dft(dft, b):
    """NaN in one cell and in a whole row, +Inf and -Inf in one column of two
    rows (rows 20 and 21: where they share a feature the sum is NaN)."""
    dft[0, 4, 17] = np.nan
    dft[1, 9, :] = np.nan
    dft[0, 20, dft.shape[2] - 3] = np.inf
    dft[0, 21, dft.shape[2] - 3] = -np.inf
    return dft


def _king_batch(spec, b, ma, seed):
    from tatara_amd.synthetic import structured_batch
    batch, _ = structured_batch(b, spec, num_buckets=1, seed=seed, nnz_min=ma // 2)
    return batch.stm_indices, batch.nstm_indices, batch.nnz


def test_ft_weight_grad_nan_sequential_kernels(gpu):
    """The occurrence-list kernel (f32), the f32 block scan and its fallback,
    and the f16 block scan and its fallback: bit-exact with NaN."""
    from tatara_amd.synthetic import small_spec
    spec = small_spec(king_buckets=8, piece_inputs=200, max_active=30)
    b, ma, ft_out, cols, pi = 128, 30, 512, spec["ft_in"], spec["piece_inputs"]
    rng = np.random.default_rng(31)
    si, ni, nnz = _king_batch(spec, b, ma, 6)
    dft = plant_dft(rng.standard_normal((2, b, ft_out)).astype(np.float32), b)
    exp = _oracle_grad(dft, si, ni, nnz, b, ft_out, cols, ma)
    assert np.isnan(exp).any() and np.isinf(exp).any()
    # occurrence lists (the plain kernel)
    D, S, Nn, N = dev(dft), dev(si), dev(ni), dev(nnz)
    g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
    check(gpu.tatara_op_ft_weight_grad(D.ptr, S.ptr, Nn.ptr, N.ptr, g.ptr, b, ft_out, cols, ma))
    same(g.to_host(), exp, "occurrence lists f32")
    # f32 block scan, then a row across blocks (its fallback)
    got, used = _blocked_grad(gpu, dft, si, ni, nnz, b, ft_out, cols, ma, pi)
    assert used == 1
    same(got, exp, "block scan f32")
    si2 = si.copy()
    si2[0, 0] = (si[0, 0] + pi) % cols
    got, used = _blocked_grad(gpu, dft, si2, ni, nnz, b, ft_out, cols, ma, pi)
    assert used == 0
    same(got, _oracle_grad(dft, si2, ni, nnz, b, ft_out, cols, ma), "occurrence fallback f32")
    # f16 dft, both paths
    d16 = plant_dft((rng.standard_normal((2, b, ft_out)) * 3000.0).astype(np.float16), b)
    inv = np.float32(1.0 / (16384.0 * b))
    for idx, want in ((si, 1), (si2, 0)):
        D, S = dev(d16.view(np.uint16)), dev(idx)
        g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
        used = C.c_uint32(99)
        check(gpu.tatara_op_ft_weight_grad_blocked_f16(D.ptr, C.c_float(inv), S.ptr, Nn.ptr, N.ptr, g.ptr, b,
                                                       ft_out, cols, ma, pi, C.byref(used)))
        assert used.value == want
        exp16 = (_oracle_grad(d16.astype(np.float32), idx, ni, nnz, b, ft_out, cols, ma) * inv).astype(np.float32)
        same(g.to_host(), exp16, f"f16 {'block scan' if want else 'occurrence lists'}")


@pytest.mark.parametrize("kb,pi,ma,b,ft_out", [(10, 64, 40, 256, 512), (45, 1629, 40, 1024, 512),
                                               (7, 300, 12, 48, 1024)])
def test_ft_weight_grad_mfma_f16_nan(gpu, kb, pi, ma, b, ft_out):
    """The matrix-core backward with non-finite dft values: NaN in exactly
    the oracle's cells.  A (king block, 128-column half) whose rows hold a
    non-finite value in its columns is summed sequentially: bit-exact with
    the oracle there; the other cells keep the matrix-core bound."""
    from tatara_amd.synthetic import small_spec, HALFKA_HM_MERGED
    spec = HALFKA_HM_MERGED if pi == 1629 else small_spec(king_buckets=kb, piece_inputs=pi, max_active=ma)
    cols = spec["ft_in"]
    si, ni, nnz = _king_batch(spec, b, ma, pi + b + 2)
    rng = np.random.default_rng(pi + 1)
    mag = np.exp2(rng.uniform(-24.0, 15.9, (2, b, ft_out)))
    vals = (np.sign(rng.standard_normal((2, b, ft_out))) * mag).astype(np.float16)
    vals = plant_dft(vals, b)
    inv = np.float32(1.0 / (16384.0 * b))
    D, S, Nn, N = dev(vals.view(np.uint16)), dev(si), dev(ni), dev(nnz)
    g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
    used = C.c_uint32(99)
    check(gpu.tatara_op_ft_weight_grad_mfma_f16(D.ptr, C.c_float(inv), S.ptr, Nn.ptr, N.ptr, g.ptr, b, ft_out,
                                                cols, ma, pi, C.byref(used)))
    assert used.value == 1
    got = g.to_host().reshape(cols, ft_out)
    seq = (_oracle_grad(vals.astype(np.float32), si, ni, nnz, b, ft_out, cols, ma) * inv).astype(np.float32)
    seq = seq.reshape(cols, ft_out)
    assert np.isnan(seq).any()
    assert np.array_equal(np.isnan(got), np.isnan(seq)), "NaN cells differ from the oracle's"
    # (block, half) regions with a non-finite value in one of their rows
    seqr = np.zeros((cols, ft_out), bool)
    for p, idx in ((0, si), (1, ni)):
        for r, c in zip(*np.nonzero(~np.isfinite(vals[p].astype(np.float32)))):
            f = idx[r, :nnz[r]]
            f = f[(f >= 0) & (f < cols)]
            if f.size:
                k = int(f[0]) // pi
                h = (c // 128) * 128
                seqr[k * pi:(k + 1) * pi, h:h + 128] = True
    assert seqr.any()
    assert np.array_equal(got[seqr], seq[seqr], equal_nan=True), "sequential region not bit-exact"
    # elsewhere: the matrix-core summation bound (finite cells only)
    fin = np.isfinite(vals.astype(np.float32))
    exact, absum, h = _exact_grad(np.where(fin, vals, np.float16(0)), si, ni, nnz, cols)
    n_stages = -(-2 * b // 32)
    bound = ((h[:, None] + n_stages) * 2.0 ** -23 * absum + 2.0 ** -24 * np.abs(exact)) * float(inv)
    rest = ~seqr
    err = np.abs(got[rest].astype(np.float64) - exact[rest] * float(inv))
    assert np.all(err <= bound[rest]), f"worst {np.max(err / np.maximum(bound[rest], 1e-300)):.3g} of the bound"


@pytest.mark.parametrize("denom", [0, 1])
def test_radam_and_lerp_nan(gpu, denom):
    """radam_fixture of the reference: weights 0 and 1 past the clamp, the
    middle gradient cell NaN (its weight, m and v become NaN; its gradient
    is reset to 0 like the others); the lerp with a NaN fast weight."""
    n = 259
    rng = np.random.default_rng(denom + 7)
    w = rng.uniform(-1, 1, n).astype(np.float32)
    w[0], w[1] = 5.0, -5.0
    m = (-0.02 + 0.0003 * (np.arange(n) % 97)).astype(np.float32)
    v = (1e-6 + 1e-7 * (np.arange(n) % 89)).astype(np.float32)
    g = rng.uniform(-1, 1, n).astype(np.float32)
    g[n // 2] = np.nan
    args = (8.75e-4, 12.5, denom, 0.01, 0.99, 0.999, 1e-8, -1.984375, 1.984375)
    ew, em, ev, eg = w.copy(), m.copy(), v.copy(), g.copy()
    ffi.radam_step(ew, em, ev, eg, *args)
    assert np.isnan(ew[n // 2]) and ew[0] == 1.984375 and ew[1] == -1.984375
    W, M, V, G = dev(w), dev(m), dev(v), dev(g)
    check(gpu.tatara_op_radam_step(W.ptr, M.ptr, V.ptr, G.ptr, *args, n))
    for d, e, k in ((W, ew, "w"), (M, em, "m"), (V, ev, "v"), (G, eg, "grad")):
        same(d.to_host(), e, k)
    s = rng.standard_normal(n).astype(np.float32)
    s[3] = np.nan
    S = dev(s)
    check(gpu.tatara_op_ranger_lookahead_lerp(W.ptr, S.ptr, 0.5, n))
    ffi.ranger_lookahead_lerp(ew, s, 0.5)
    same(W.to_host(), ew, "lerp w")
    same(S.to_host(), s, "lerp slow")


MODES = {"f32": ols.Precision(), "all_optim": ols.Precision.all_optim()}


@pytest.mark.parametrize("mode,ft_out", [("f32", 256), ("f32", 512), ("all_optim", 512)])
def test_train_step_with_a_nan_ft_weight(gpu, mode, ft_out):
    """One step with ft_w[f, c] = NaN for a feature f of a few rows: the FT
    sums, combined, the net output, the dft and every gradient and post-step
    tensor hold NaN in exactly the oracle's cells (all_optim at ft_out 512:
    the matrix-core FT backward, whose blocks with NaN rows are summed
    sequentially); finite cells within the one-step bars."""
    import dataclasses
    prec = MODES[mode]
    sh, cfg = make(ft_out=ft_out)
    cfg = dataclasses.replace(cfg, ft_fp16=prec.ft_fp16, ft_fp16_out=prec.ft_fp16_out,
                              fp16_opt_state=prec.fp16_opt_state, tf32=prec.tf32)
    b = cfg.max_batch
    batch, bucket = batch_for(21, b, sh.nb)
    st = ols.default_init(sh)
    # the least frequent feature among the first rows' stm features
    feats, counts = np.unique(batch.stm_indices[:, :8][batch.stm_indices[:, :8] >= 0], return_counts=True)
    f = int(feats[np.argmin(counts)])
    w = st["ft_w"]["w"].reshape(-1, sh.ft_out)
    w[f, 5] = np.nan
    if prec.fp16_opt_state:
        st = ols.to_f16_state(st)
    opt = ols.OptConfig(optimizer="ranger", weight_decay=0.01)
    loss = Sigmoid()
    with LayerStackTrainer(cfg) as t:
        t.set("ft_w", st["ft_w"]["w"])
        t.train_step(batch, bucket, 8.75e-4, 0.25, loss)
        acc, a, g = ols.train_step(sh, st, as_dict(batch, bucket), opt, 8.75e-4, 0.25, loss_dict(loss), 1, prec)
        bf = b * sh.ft_out
        same(t.activation("ft_stm_out", bf), a["ft_stm"], "ft_stm_out")
        same(t.activation("ft_nstm_out", bf), a["ft_nstm"], "ft_nstm_out")
        same(t.activation("combined", bf), a["combined"], "combined")
        nan_rows = close_nan(t.activation("net_output", b), a["net"], 1e-5, atol=1e-6, what="net_output")
        assert 0 < nan_rows < b
        for k in ("dft_stm", "dft_nstm"):
            if prec.ft_fp16_out:
                close_nan(t.activation(k, bf), a[k + "16"], 2e-3, atol=2.0 ** -24, what=k + " (f16)")
            else:
                close_nan(t.activation(k, bf), a[k], 1e-4, atol_frac=1e-5, what=k)
        for name in GROUPS:
            close_nan(t.get(name, "w"), st[name]["w"], 1e-5, atol=1e-6, what=f"{name}.w")
            for k in ("m", "v"):
                got_nan = np.isnan(t.get(name, k))
                assert np.array_equal(got_nan, np.isnan(np.asarray(st[name][k], np.float32)).ravel()), \
                    f"{name}.{k}: NaN cells differ"
        assert np.isnan(t.get("ft_w", "w")).any()
        assert np.isnan(t.flush_pending_loss()) and np.isnan(acc)
