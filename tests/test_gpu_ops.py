"""Kernel-level parity of the HIP ops against the CPU oracle (GPU).

Bar: bit-exact for the sparse gather, the FT post activation, the
deterministic FT weight gradient, the factorizer fold/reduce and the
optimizer element update (the reference itself asserts tolerance 0.0 for the
gather, gpu_cpu_equivalence_tests.rs:3836-3844).
"""
import ctypes as C

import numpy as np
import pytest

from oracle import ffi
from tatara_amd.trainer import DeviceArray
from tatara_amd._lib import check

pytestmark = pytest.mark.gpu

SC = np.float32(127.0 / 128.0)


def dev(a):
    return DeviceArray(np.ascontiguousarray(a))


def ragged_indices(rng, b, ma, cols, oob=True):
    idx = rng.integers(0, cols, (b, ma)).astype(np.int32)
    nnz = rng.integers(0, ma + 1, b).astype(np.int32)
    if oob:
        m = rng.random((b, ma))
        idx[m < 0.05] = -1
        idx[(m >= 0.05) & (m < 0.08)] = cols + 3  # out of range: skipped
    # slots past nnz hold garbage that must be ignored
    for i in range(b):
        idx[i, nnz[i]:] = rng.integers(-5, cols, ma - nnz[i])
    nnz[0] = ma
    if b > 1:
        nnz[1] = 0
    # duplicate index inside one row
    if ma >= 3 and b > 2:
        idx[2, 1] = idx[2, 0]
        nnz[2] = max(nnz[2], 3)
    return idx, nnz


def test_sparse_forward_reference_fixture(gpu):
    # sparse_ft_forward.rs:132 fixture (rows=2) embedded in rows=8 columns
    rows, cols = 8, 3
    w = np.zeros((cols, rows), np.float32)
    w[:, :2] = np.array([[0, 1], [2, 3], [4, 5]], np.float32)
    idx = np.array([[0, 1, -1, -1], [2, 2, 1, 0]], np.int32)
    nnz = np.array([2, 4], np.int32)
    W, I, N = dev(w), dev(idx), dev(nnz)
    out = DeviceArray.empty((2, rows), np.float32)
    check(gpu.tatara_op_sparse_ft_forward(W.ptr, I.ptr, N.ptr, out.ptr, 2, rows, cols, 4))
    got = out.to_host()
    assert got[:, :2].ravel().tolist() == [2.0, 4.0, 10.0, 14.0]
    assert not got[:, 2:].any()


@pytest.mark.parametrize("b,ma,cols,rows", [(37, 40, 300, 64), (256, 38, 2000, 256), (64, 40, 500, 1536)])
def test_sparse_forward_bit_exact(gpu, b, ma, cols, rows):
    rng = np.random.default_rng(b + rows)
    w = rng.standard_normal((cols, rows)).astype(np.float32)
    idx, nnz = ragged_indices(rng, b, ma, cols)
    exp = ffi.sparse_ft_forward(w, idx, nnz, b, rows, cols, ma)
    W, I, N = dev(w), dev(idx), dev(nnz)
    out = DeviceArray.empty((b, rows), np.float32)
    check(gpu.tatara_op_sparse_ft_forward(W.ptr, I.ptr, N.ptr, out.ptr, b, rows, cols, ma))
    assert np.array_equal(out.to_host().ravel(), exp)


@pytest.mark.parametrize("pi", [0, 50])
@pytest.mark.parametrize("ft_out", [256, 768, 1536])
def test_ft_forward_pairwise_bit_exact(gpu, pi, ft_out):
    rng = np.random.default_rng(ft_out + pi)
    b, ma, cols = 96, 40, 600
    w = (rng.standard_normal((cols, ft_out)) * 0.05 + 0.02).astype(np.float32)
    bias = (rng.standard_normal(ft_out) * 0.1 + 0.2).astype(np.float32)
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
                                            b, ft_out, cols, ma, pi, float(SC)))
    assert np.array_equal(so.to_host().ravel(), s_exp)
    assert np.array_equal(no.to_host().ravel(), n_exp)
    assert np.array_equal(co.to_host().ravel(), c_exp)


@pytest.mark.parametrize("b,ma,cols,ft_out", [(48, 40, 200, 256), (200, 38, 3000, 1536), (16, 4, 7, 64)])
def test_ft_weight_grad_bit_exact(gpu, b, ma, cols, ft_out):
    rng = np.random.default_rng(cols)
    si, nnz = ragged_indices(rng, b, ma, cols)
    ni, _ = ragged_indices(rng, b, ma, cols)
    dft = rng.standard_normal((2, b, ft_out)).astype(np.float32)
    exp = np.zeros(cols * ft_out, np.float32)
    ffi.sparse_ft_backward_nnz(dft[0].ravel(), si, nnz, exp, b, ft_out, cols, ma)
    ffi.sparse_ft_backward_nnz(dft[1].ravel(), ni, nnz, exp, b, ft_out, cols, ma)
    D, S, Nn, N = dev(dft), dev(si), dev(ni), dev(nnz)
    g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
    check(gpu.tatara_op_ft_weight_grad(D.ptr, S.ptr, Nn.ptr, N.ptr, g.ptr, b, ft_out, cols, ma))
    assert np.array_equal(g.to_host(), exp)


def _blocked_grad(gpu, dft, si, ni, nnz, b, ft_out, cols, ma, pi):
    D, S, Nn, N = dev(dft), dev(si), dev(ni), dev(nnz)
    g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
    used = C.c_uint32(99)
    check(gpu.tatara_op_ft_weight_grad_blocked(D.ptr, S.ptr, Nn.ptr, N.ptr, g.ptr, b, ft_out, cols, ma, pi,
                                               C.byref(used)))
    return g.to_host(), used.value


def _oracle_grad(dft, si, ni, nnz, b, ft_out, cols, ma):
    exp = np.zeros(cols * ft_out, np.float32)
    ffi.sparse_ft_backward_nnz(dft[0].ravel(), si, nnz, exp, b, ft_out, cols, ma)
    ffi.sparse_ft_backward_nnz(dft[1].ravel(), ni, nnz, exp, b, ft_out, cols, ma)
    return exp


@pytest.mark.parametrize("kb,pi,ma,b,ft_out", [(10, 64, 40, 256, 256), (45, 1629, 40, 1024, 512),
                                               (81, 1548, 38, 512, 256), (7, 300, 12, 48, 200),
                                               (3, 40, 8, 16, 64)])
def test_ft_weight_grad_block_scan_bit_exact(gpu, kb, pi, ma, b, ft_out):
    """King-bucketed rows: the block scan runs and every cell equals the
    oracle's sequential stm-then-nstm sum."""
    from tatara_amd.synthetic import small_spec, structured_batch, HALFKA_HM_MERGED, HALFKP
    spec = {1629: HALFKA_HM_MERGED, 1548: HALFKP}.get(pi) or small_spec(king_buckets=kb, piece_inputs=pi,
                                                                        max_active=ma)
    batch, _ = structured_batch(b, spec, num_buckets=1, seed=pi + b, nnz_min=ma // 2)
    cols = spec["ft_in"]
    rng = np.random.default_rng(b)
    dft = rng.standard_normal((2, b, ft_out)).astype(np.float32)
    got, used = _blocked_grad(gpu, dft, batch.stm_indices, batch.nstm_indices, batch.nnz, b, ft_out, cols, ma,
                              spec["piece_inputs"])
    assert used == 1
    exp = _oracle_grad(dft, batch.stm_indices, batch.nstm_indices, batch.nnz, b, ft_out, cols, ma)
    assert np.array_equal(got, exp)


def test_ft_weight_grad_block_scan_duplicates_and_ragged(gpu):
    """A feature twice (or three times) in one row hands the batch to the
    occurrence-list path; invalid and out-of-range slots and empty rows do
    not.  Bit-exact either way."""
    from tatara_amd.synthetic import small_spec, structured_batch
    spec = small_spec(king_buckets=6, piece_inputs=96, max_active=24)
    b, ma, ft_out = 96, 24, 256
    batch, _ = structured_batch(b, spec, num_buckets=1, seed=5, nnz_min=4)
    si, ni, nnz = batch.stm_indices.copy(), batch.nstm_indices.copy(), batch.nnz.copy()
    nnz[:8] = ma
    si[0, 5] = si[0, 0]               # twice
    si[1, 3] = si[1, 9] = si[1, 2]    # three times
    ni[2, 7] = ni[2, 1]
    si[3, 4] = -1                     # skipped slot inside nnz
    ni[4, 6] = spec["ft_in"] + 5      # out of range: skipped
    nnz[5] = 0                        # empty row
    cols = spec["ft_in"]
    rng = np.random.default_rng(11)
    dft = rng.standard_normal((2, b, ft_out)).astype(np.float32)
    got, used = _blocked_grad(gpu, dft, si, ni, nnz, b, ft_out, cols, ma, spec["piece_inputs"])
    assert used == 0
    assert np.array_equal(got, _oracle_grad(dft, si, ni, nnz, b, ft_out, cols, ma))
    # without the repeated features: the block scan
    si[0, 5], si[1, 3], si[1, 9], ni[2, 7] = -1, -1, -1, -1
    got, used = _blocked_grad(gpu, dft, si, ni, nnz, b, ft_out, cols, ma, spec["piece_inputs"])
    assert used == 1
    assert np.array_equal(got, _oracle_grad(dft, si, ni, nnz, b, ft_out, cols, ma))


def test_ft_weight_grad_block_scan_falls_back(gpu):
    """Rows whose features span king blocks take the occurrence-list path,
    with the same bit-exact result."""
    rng = np.random.default_rng(3)
    b, ma, cols, ft_out, pi = 64, 20, 640, 256, 64
    si, nnz = ragged_indices(rng, b, ma, cols)
    ni, _ = ragged_indices(rng, b, ma, cols)
    dft = rng.standard_normal((2, b, ft_out)).astype(np.float32)
    got, used = _blocked_grad(gpu, dft, si, ni, nnz, b, ft_out, cols, ma, pi)
    assert used == 0
    assert np.array_equal(got, _oracle_grad(dft, si, ni, nnz, b, ft_out, cols, ma))


@pytest.mark.parametrize("bucketed", [True, False], ids=["block_scan", "occurrence_lists"])
def test_ft_weight_grad_blocked_f16_bit_exact(gpu, bucketed):
    """f16 dft: each cell is the sequential f32 sum of the f16 values
    (converted exactly, so the f32 oracle of the converted values gives the
    sum bit for bit), times the inverse scale."""
    from tatara_amd.synthetic import small_spec, structured_batch
    spec = small_spec(king_buckets=8, piece_inputs=200, max_active=30)
    b, ma, ft_out, cols = 128, 30, 512, spec["ft_in"]
    rng = np.random.default_rng(17)
    if bucketed:
        batch, _ = structured_batch(b, spec, num_buckets=1, seed=4, nnz_min=10)
        si, ni, nnz = batch.stm_indices, batch.nstm_indices, batch.nnz
    else:
        si, nnz = ragged_indices(rng, b, ma, cols)
        ni, _ = ragged_indices(rng, b, ma, cols)
    dft16 = (rng.standard_normal((2, b, ft_out)) * 3000.0).astype(np.float16)
    inv = np.float32(1.0 / (16384.0 * b))
    D, S, Nn, N = dev(dft16.view(np.uint16)), dev(si), dev(ni), dev(nnz)
    g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
    used = C.c_uint32(99)
    check(gpu.tatara_op_ft_weight_grad_blocked_f16(D.ptr, C.c_float(inv), S.ptr, Nn.ptr, N.ptr, g.ptr, b, ft_out,
                                                   cols, ma, spec["piece_inputs"], C.byref(used)))
    assert used.value == (1 if bucketed else 0)
    exp = _oracle_grad(dft16.astype(np.float32), si, ni, nnz, b, ft_out, cols, ma) * inv
    assert np.array_equal(g.to_host(), exp.astype(np.float32))


def _exact_grad(vals, si, ni, nnz, cols):
    """float64 sums of f16 values, with the sums of their magnitudes and the
    occurrence counts.  Exact: binary16 values lie in [2^-24, 65504], so a
    sum of a few thousand of them needs fewer than 53 significand bits."""
    b, ft_out = vals.shape[1], vals.shape[2]
    g = np.zeros((cols, ft_out))
    a = np.zeros((cols, ft_out))
    h = np.zeros(cols, np.int64)
    for p, idx in ((0, si), (1, ni)):
        for r in range(b):
            f = idx[r, :nnz[r]]
            f = f[(f >= 0) & (f < cols)]
            np.add.at(g, f, vals[p, r].astype(np.float64))
            np.add.at(a, f, np.abs(vals[p, r].astype(np.float64)))
            np.add.at(h, f, 1)
    return g, a, h


@pytest.mark.parametrize("kb,pi,ma,b,ft_out", [(10, 64, 40, 256, 256), (45, 1629, 40, 1024, 512),
                                               (81, 1548, 38, 512, 256), (7, 300, 12, 48, 200),
                                               (3, 40, 8, 16, 64)])
def test_ft_weight_grad_mfma_f16_within_summation_bound(gpu, kb, pi, ma, b, ft_out):
    """The matrix-core gradient from an f16 dft: every cell is the f32 sum of
    the same f16 values as the sequential sum, in the matrix core's order.
    Bound per cell, against the exact (float64) sum S of its h values with
    magnitude sum A:  |g - S inv| <= ((h + n_stages) 2^-23 A + 2^-24 |S|) inv,
    n_stages = ceil(2b / 32) (one rounded f32 add per value and per 32-row
    MFMA step, then the product with inv).  Values span the f16 range:
    subnormals, +-65504 and zeros; the cells match the sequential f32 sum
    within the same bound, and a planted mistake (one occurrence dropped)
    breaks it."""
    from tatara_amd.synthetic import small_spec, structured_batch, HALFKA_HM_MERGED, HALFKP
    spec = {1629: HALFKA_HM_MERGED, 1548: HALFKP}.get(pi) or small_spec(king_buckets=kb, piece_inputs=pi,
                                                                        max_active=ma)
    batch, _ = structured_batch(b, spec, num_buckets=1, seed=pi + b + 1, nnz_min=ma // 2)
    si, ni, nnz = batch.stm_indices, batch.nstm_indices, batch.nnz
    cols = spec["ft_in"]
    rng = np.random.default_rng(pi)
    mag = np.exp2(rng.uniform(-24.0, 15.9, (2, b, ft_out)))
    vals = (np.sign(rng.standard_normal((2, b, ft_out))) * mag).astype(np.float16)
    vals[0, 0, :8] = np.float16(65504.0)
    vals[1, 0, :8] = np.float16(-65504.0)
    vals[0, 1, 8:16] = np.float16(2.0 ** -24)
    vals[:, 2, :] = 0
    inv = np.float32(1.0 / (16384.0 * b))
    D, S, Nn, N = dev(vals.view(np.uint16)), dev(si), dev(ni), dev(nnz)
    g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
    used = C.c_uint32(99)
    check(gpu.tatara_op_ft_weight_grad_mfma_f16(D.ptr, C.c_float(inv), S.ptr, Nn.ptr, N.ptr, g.ptr, b, ft_out,
                                                cols, ma, spec["piece_inputs"], C.byref(used)))
    assert used.value == 1
    got = g.to_host().reshape(cols, ft_out).astype(np.float64)
    exact, absum, h = _exact_grad(vals, si, ni, nnz, cols)
    n_stages = -(-2 * b // 32)
    bound = ((h[:, None] + n_stages) * 2.0 ** -23 * absum + 2.0 ** -24 * np.abs(exact)) * float(inv)
    err = np.abs(got - exact * float(inv))
    assert np.all(err <= bound), f"worst {np.max(err / np.maximum(bound, 1e-300)):.3g} of the bound"
    seq = _oracle_grad(vals.astype(np.float32), si, ni, nnz, b, ft_out, cols, ma).reshape(cols, ft_out)
    seq = (seq * inv).astype(np.float64)
    assert np.all(np.abs(got - seq) <= 2 * bound)
    # a dropped occurrence is far outside the bound
    f = int(si[3, 0])
    assert np.any(np.abs(got[f] - (exact[f] - vals[0, 3].astype(np.float64)) * float(inv)) > 2 * bound[f])


def test_ft_weight_grad_mfma_f16_falls_back_on_repeated_features(gpu):
    """A feature twice in one row: the batch goes to the occurrence lists
    (sequential sums, bit-exact with the oracle)."""
    from tatara_amd.synthetic import small_spec, structured_batch
    spec = small_spec(king_buckets=6, piece_inputs=96, max_active=24)
    b, ma, ft_out = 96, 24, 512
    batch, _ = structured_batch(b, spec, num_buckets=1, seed=5, nnz_min=4)
    si, ni, nnz = batch.stm_indices.copy(), batch.nstm_indices.copy(), batch.nnz.copy()
    nnz[:4] = ma
    si[0, 5] = si[0, 0]
    cols = spec["ft_in"]
    rng = np.random.default_rng(12)
    vals = (rng.standard_normal((2, b, ft_out)) * 3000.0).astype(np.float16)
    inv = np.float32(1.0 / (16384.0 * b))
    D, S, Nn, N = dev(vals.view(np.uint16)), dev(si), dev(ni), dev(nnz)
    g = DeviceArray(np.full(cols * ft_out, 7.0, np.float32))
    used = C.c_uint32(99)
    check(gpu.tatara_op_ft_weight_grad_mfma_f16(D.ptr, C.c_float(inv), S.ptr, Nn.ptr, N.ptr, g.ptr, b, ft_out,
                                                cols, ma, spec["piece_inputs"], C.byref(used)))
    assert used.value == 0
    exp = _oracle_grad(vals.astype(np.float32), si, ni, nnz, b, ft_out, cols, ma) * inv
    assert np.array_equal(g.to_host(), exp.astype(np.float32))


def test_fold_reduce_bit_exact(gpu):
    rng = np.random.default_rng(9)
    ft_in, ft_out, pi = 45 * 12, 256, 12
    w = rng.standard_normal((ft_in + pi) * ft_out).astype(np.float32)
    W = dev(w)
    comb = DeviceArray.empty(ft_in * ft_out, np.float32)
    check(gpu.tatara_op_ft_fold_virtual(W.ptr, comb.ptr, ft_in, ft_out, pi))
    assert np.array_equal(comb.to_host(), ffi.ft_fold_virtual(w, ft_in, ft_out, pi))
    g = rng.standard_normal((ft_in + pi) * ft_out).astype(np.float32)
    G = dev(g)
    check(gpu.tatara_op_ft_reduce_virtual_grad(G.ptr, ft_in, ft_out, pi))
    exp = g.copy()
    ffi.ft_reduce_virtual_grad(exp, ft_in, ft_out, pi)
    assert np.array_equal(G.to_host(), exp)


@pytest.mark.parametrize("denom", [0, 1])
def test_radam_and_lerp_bit_exact(gpu, denom):
    rng = np.random.default_rng(denom)
    n = 10_007
    w = rng.standard_normal(n).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    v = (rng.random(n) * 1e-5).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    args = (1e-3, 12.5, denom, 0.01, 0.99, 0.999, 1e-8, -1.984375, 1.984375)
    ew, em, ev, eg = w.copy(), m.copy(), v.copy(), g.copy()
    ffi.radam_step(ew, em, ev, eg, *args)
    W, M, V, G = dev(w), dev(m), dev(v), dev(g)
    check(gpu.tatara_op_radam_step(W.ptr, M.ptr, V.ptr, G.ptr, *args, n))
    for d, e in ((W, ew), (M, em), (V, ev), (G, eg)):
        assert np.array_equal(d.to_host(), e)
    s = rng.standard_normal(n).astype(np.float32)
    S = dev(s)
    check(gpu.tatara_op_ranger_lookahead_lerp(W.ptr, S.ptr, 0.5, n))
    ffi.ranger_lookahead_lerp(ew, s, 0.5)
    assert np.array_equal(W.to_host(), ew) and np.array_equal(S.to_host(), s)
