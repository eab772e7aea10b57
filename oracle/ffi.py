"""ctypes binding of the CPU oracle (oracle/oracle.cpp -> oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product never uses it.
Every wrapper takes/returns numpy arrays and calls the C restatement of the
reference CPU function named in oracle.cpp.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

_f = C.POINTER(C.c_float)
_i = C.POINTER(C.c_int32)
_d = C.POINTER(C.c_double)
_I64 = C.c_int64
_lib = None


def build() -> Path:
    """Compiles the oracle with its Makefile (g++, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
    return _lib


def set_threads(n: int) -> int:
    fn = lib().orc_set_threads
    fn.restype = C.c_int
    return fn(C.c_int(n))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def P(a: np.ndarray):
    if a.dtype == np.float32:
        return a.ctypes.data_as(_f)
    if a.dtype == np.int32:
        return a.ctypes.data_as(_i)
    if a.dtype == np.float64:
        return a.ctypes.data_as(_d)
    raise TypeError(a.dtype)


# -- sparse FT ----------------------------------------------------------------
def sparse_ft_forward(weight, indices, nnz, batch, rows, cols, max_active):
    w, idx, n = f32(weight), i32(indices), i32(nnz)
    out = np.zeros(batch * rows, dtype=np.float32)
    lib().orc_sparse_ft_forward(P(w), P(idx), P(n), P(out), _I64(batch), _I64(rows), _I64(cols),
                                _I64(max_active))
    return out


def sparse_ft_backward(grad_out, indices, grad_weight, batch, rows, cols, nnz):
    """Accumulates into grad_weight (modified in place and returned)."""
    g, idx = f32(grad_out), i32(indices)
    assert grad_weight.dtype == np.float32 and grad_weight.flags.c_contiguous
    lib().orc_sparse_ft_backward(P(g), P(idx), P(grad_weight), _I64(batch), _I64(rows), _I64(cols),
                                 _I64(nnz))
    return grad_weight


def sparse_ft_backward_nnz(grad_out, indices, nnz, grad_weight, batch, rows, cols, max_active):
    g, idx, n = f32(grad_out), i32(indices), i32(nnz)
    assert grad_weight.dtype == np.float32 and grad_weight.flags.c_contiguous
    lib().orc_sparse_ft_backward_nnz(P(g), P(idx), P(n), P(grad_weight), _I64(batch), _I64(rows),
                                     _I64(cols), _I64(max_active))
    return grad_weight


def ft_grad_fp16(dft16, indices, nnz, grad_weight, batch, rows, cols, max_active, inv_scale, add):
    """gather_and_sum_per_feature_{overwrite,add}_fp16 (in place on grad_weight)."""
    g, idx, n = f32(dft16), i32(indices), i32(nnz)
    assert grad_weight.dtype == np.float32 and grad_weight.flags.c_contiguous
    lib().orc_ft_grad_fp16(P(g), P(idx), P(n), P(grad_weight), _I64(batch), _I64(rows), _I64(cols),
                           _I64(max_active), C.c_float(inv_scale), C.c_int32(int(add)))
    return grad_weight


def ft_fold_virtual(w, ft_in, ft_out, piece_inputs):
    w = f32(w)
    comb = np.zeros(ft_in * ft_out, dtype=np.float32)
    lib().orc_ft_fold_virtual(P(w), P(comb), _I64(ft_in), _I64(ft_out), _I64(piece_inputs))
    return comb


def ft_reduce_virtual_grad(grad, ft_in, ft_out, piece_inputs):
    assert grad.dtype == np.float32 and grad.flags.c_contiguous
    lib().orc_ft_reduce_virtual_grad(P(grad), _I64(ft_in), _I64(ft_out), _I64(piece_inputs))
    return grad


# -- FT post ------------------------------------------------------------------
def ft_post_perspective_fwd(stm, nstm, bias, batch, ft_dim, scale):
    s, n, b = f32(stm), f32(nstm), f32(bias)
    out = np.zeros(batch * ft_dim, dtype=np.float32)
    lib().orc_ft_post_perspective_fwd(P(s), P(n), P(b), P(out), _I64(batch), _I64(ft_dim),
                                      C.c_float(scale))
    return out


def ft_post_perspective_grad(d_combined, ft_out, bias, grad_bias, batch, ft_dim, d_off, d_stride,
                             scale):
    """Returns grad_ft_out; grad_bias is accumulated in place."""
    d, f, b = f32(d_combined), f32(ft_out), f32(bias)
    g = np.zeros(batch * ft_dim, dtype=np.float32)
    assert grad_bias.dtype == np.float32
    lib().orc_ft_post_perspective_grad(P(d), P(f), P(b), P(g), P(grad_bias), _I64(batch),
                                       _I64(ft_dim), _I64(d_off), _I64(d_stride), C.c_float(scale))
    return g


# -- dense ----------------------------------------------------------------------
def dense_mm_fwd(x, w, bias, batch, in_dim, out_dim):
    x, w, b = f32(x), f32(w), f32(bias)
    y = np.zeros(batch * out_dim, dtype=np.float32)
    lib().orc_dense_mm_fwd(P(x), P(w), P(b), P(y), _I64(batch), _I64(in_dim), _I64(out_dim))
    return y


def dense_mm_bwd_input(dy, w, batch, in_dim, out_dim):
    dy, w = f32(dy), f32(w)
    dx = np.zeros(batch * in_dim, dtype=np.float32)
    lib().orc_dense_mm_bwd_input(P(dy), P(w), P(dx), _I64(batch), _I64(in_dim), _I64(out_dim))
    return dx


def dense_mm_bwd_weight(x, dy, batch, in_dim, out_dim):
    x, dy = f32(x), f32(dy)
    gw = np.zeros(in_dim * out_dim, dtype=np.float32)
    lib().orc_dense_mm_bwd_weight(P(x), P(dy), P(gw), _I64(batch), _I64(in_dim), _I64(out_dim))
    return gw


def bias_grad(dy, grad_bias, batch, out_dim):
    dy = f32(dy)
    lib().orc_bias_grad(P(dy), P(grad_bias), _I64(batch), _I64(out_dim))
    return grad_bias


def dense_mm_fwd_bucket(x, w, bias, bucket, batch, in_dim, out_dim, nb):
    x, w, b, bk = f32(x), f32(w), f32(bias), i32(bucket)
    y = np.zeros(batch * out_dim, dtype=np.float32)
    lib().orc_dense_mm_fwd_bucket(P(x), P(w), P(b), P(bk), P(y), _I64(batch), _I64(in_dim),
                                  _I64(out_dim), _I64(nb))
    return y


def dense_mm_bwd_input_bucket(dy, w, bucket, batch, in_dim, out_dim, nb):
    dy, w, bk = f32(dy), f32(w), i32(bucket)
    dx = np.zeros(batch * in_dim, dtype=np.float32)
    lib().orc_dense_mm_bwd_input_bucket(P(dy), P(w), P(bk), P(dx), _I64(batch), _I64(in_dim),
                                        _I64(out_dim), _I64(nb))
    return dx


def dense_mm_bwd_weight_bucket(x, dy, bucket, batch, in_dim, out_dim, nb):
    x, dy, bk = f32(x), f32(dy), i32(bucket)
    gw = np.zeros(nb * out_dim * in_dim, dtype=np.float32)
    lib().orc_dense_mm_bwd_weight_bucket(P(x), P(dy), P(bk), P(gw), _I64(batch), _I64(in_dim),
                                         _I64(out_dim), _I64(nb))
    return gw


def bias_grad_bucket(dy, bucket, grad_bias, batch, out_dim, nb):
    dy, bk = f32(dy), i32(bucket)
    lib().orc_bias_grad_bucket(P(dy), P(bk), P(grad_bias), _I64(batch), _I64(out_dim), _I64(nb))
    return grad_bias


# -- pointwise ------------------------------------------------------------------
def _unary(name, x, *scal):
    x = f32(x)
    y = np.zeros_like(x)
    getattr(lib(), name)(P(x), P(y), *scal, _I64(x.size))
    return y


def crelu_fwd(x):
    return _unary("orc_crelu_fwd", x)


def crelu_grad(x, dy):
    x, dy = f32(x), f32(dy)
    dx = np.zeros_like(x)
    lib().orc_crelu_grad(P(x), P(dy), P(dx), _I64(x.size))
    return dx


def abs_pow2_scale_fwd(x, scale):
    return _unary("orc_abs_pow2_scale_fwd", x, C.c_float(scale))


def abs_pow2_scale_grad(x, dy, scale):
    x, dy = f32(x), f32(dy)
    dx = np.zeros_like(x)
    lib().orc_abs_pow2_scale_grad(P(x), P(dy), P(dx), C.c_float(scale), _I64(x.size))
    return dx


def concat_l1sqr_main_fwd(a, b, batch, a_dim, b_dim):
    a, b = f32(a), f32(b)
    out = np.zeros(batch * (a_dim + b_dim), dtype=np.float32)
    lib().orc_concat_l1sqr_main_fwd(P(a), P(b), P(out), _I64(batch), _I64(a_dim), _I64(b_dim))
    return out


def concat_l1sqr_main_grad(dout, batch, dim):
    dout = f32(dout)
    da = np.zeros(batch * dim, dtype=np.float32)
    db = np.zeros(batch * dim, dtype=np.float32)
    lib().orc_concat_l1sqr_main_grad(P(dout), P(da), P(db), _I64(batch), _I64(dim))
    return da, db


def elementwise_add(a, b):
    a, b = f32(a), f32(b)
    c = np.zeros_like(a)
    lib().orc_elementwise_add(P(a), P(b), P(c), _I64(a.size))
    return c


def slice_extract_2d(src, batch, src_stride, src_offset, out_dim):
    src = f32(src)
    dst = np.zeros(batch * out_dim, dtype=np.float32)
    lib().orc_slice_extract_2d(P(src), P(dst), _I64(batch), _I64(src_stride), _I64(src_offset),
                               _I64(out_dim))
    return dst


def slice_scatter_2d(src, dst, batch, in_dim, dst_stride, dst_offset):
    src = f32(src)
    lib().orc_slice_scatter_2d(P(src), P(dst), _I64(batch), _I64(in_dim), _I64(dst_stride),
                               _I64(dst_offset))
    return dst


# -- losses ------------------------------------------------------------------------
def loss_wdl(out, score, wdl, per_pos_norm, lam, scale):
    out, score, wdl, norm = f32(out), f32(score), f32(wdl), f32(per_pos_norm)
    d = np.zeros_like(out)
    acc = np.zeros(1, dtype=np.float64)
    lib().orc_loss_wdl(P(out), P(score), P(wdl), P(norm), P(d), P(acc), C.c_float(lam),
                       C.c_float(scale), _I64(out.size))
    return d, float(acc[0])


def loss_wrm(out, score, wdl, per_pos_norm, lam, nnue2score, in_scaling, in_offset, target_offset,
             target_scaling, pow_exp, qp_asymmetry, w1, w2, extended):
    out, score, wdl, norm = f32(out), f32(score), f32(wdl), f32(per_pos_norm)
    d = np.zeros_like(out)
    acc = np.zeros(1, dtype=np.float64)
    F = C.c_float
    lib().orc_loss_wrm(P(out), P(score), P(wdl), P(norm), P(d), P(acc), F(lam), F(nnue2score),
                       F(in_scaling), F(in_offset), F(target_offset), F(target_scaling), F(pow_exp),
                       F(qp_asymmetry), F(w1), F(w2), C.c_int32(1 if extended else 0),
                       _I64(out.size))
    return d, float(acc[0])


# -- optimizer -----------------------------------------------------------------------
def radam_step_size_denom(step, beta1, beta2, n_sma_threshold):
    ss = C.c_float()
    dn = C.c_int32()
    lib().orc_radam_step_size_denom(C.c_uint64(step), C.c_float(beta1), C.c_float(beta2),
                                    C.c_float(n_sma_threshold), C.byref(ss), C.byref(dn))
    return ss.value, dn.value


def radam_step(w, m, v, g, lr, step_size, denom, decay, beta1, beta2, eps, min_w, max_w):
    """In place on float32 arrays w, m, v, g."""
    for a in (w, m, v, g):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    F = C.c_float
    lib().orc_radam_step(P(w), P(m), P(v), P(g), F(lr), F(step_size), C.c_int32(denom), F(decay),
                         F(beta1), F(beta2), F(eps), F(min_w), F(max_w), _I64(w.size))


def ranger_lookahead_lerp(w, slow, alpha):
    lib().orc_ranger_lookahead_lerp(P(w), P(slow), C.c_float(alpha), _I64(w.size))


# -- init ---------------------------------------------------------------------------
def init_sample(n, fan_in, dist="uniform", scale_kind="abs", value=0.01, seed=1, num_buckets=1,
                per_bucket_repeat=False):
    out = np.zeros(n, dtype=np.float32)
    d = {"zero": 0, "uniform": 1, "normal": 2}[dist]
    sk = {"abs": 0, "fanin": 1}[scale_kind]
    lib().orc_init_sample(_I64(n), _I64(num_buckets), _I64(fan_in), C.c_int32(d), C.c_int32(sk),
                          C.c_float(value), C.c_int32(1 if per_bucket_repeat else 0),
                          C.c_uint64(seed), P(out))
    return out
