"""Pins the Simple-architecture oracle step (oracle/simple.py) without the reference.

The reference's Simple GPU trainer has no stored golden values, so the
composition is checked against what the mathematics fixes: the gradient of
the summed squared error, taken by float64 reverse-mode autodiff over an
independent restatement of the forward (matrix form, torch on the CPU),
divided by the batch size (the reference scales dy by per_pos_norm = 1/b).
A transposed layer (all of l1/l2 are square-adjacent at these shapes), a
dropped bias, a missing CReLU mask or a mis-routed factorizer row fails
it.  Initialisation and the optimizer composition are checked against
SimpleInit::default_uniform (crates/nnue-train/src/init.rs:290-303) and
radam_step_cpu.
"""
import numpy as np
import pytest

from oracle import ffi
from oracle import simple as osi

torch = pytest.importorskip("torch")

SH = osi.SimpleShape(ft_in=40, max_active=6, piece_inputs=8, ft_out=16, l1=32, l2=32)


def _batch(b=48, seed=3):
    rng = np.random.default_rng(seed)
    stm = rng.integers(0, SH.ft_in, (b, SH.max_active)).astype(np.int32)
    nstm = rng.integers(0, SH.ft_in, (b, SH.max_active)).astype(np.int32)
    nnz = rng.integers(2, SH.max_active + 1, b).astype(np.int32)
    for i in range(b):
        stm[i, nnz[i]:] = -1
        nstm[i, nnz[i]:] = -1
    return dict(stm=stm, nstm=nstm, nnz=nnz, bucket=None,
                score=rng.uniform(-900, 900, b).astype(np.float32),
                wdl=rng.choice([0.0, 0.5, 1.0], b).astype(np.float32))


def _state(seed=5):
    st = osi.default_init(SH)
    rng = np.random.default_rng(seed)
    # spread the activations over the linear part of every CReLU
    st["ft_w"]["w"][:] = rng.uniform(-0.05, 0.12, st["ft_w"]["w"].size).astype(np.float32)
    st["l1_w"]["w"][:] = rng.uniform(-0.08, 0.1, st["l1_w"]["w"].size).astype(np.float32)
    st["l1_b"]["w"][:] = rng.uniform(0.1, 0.4, st["l1_b"]["w"].size).astype(np.float32)
    st["l2_w"]["w"][:] = rng.uniform(-0.1, 0.12, st["l2_w"]["w"].size).astype(np.float32)
    st["l2_b"]["w"][:] = rng.uniform(0.1, 0.4, st["l2_b"]["w"].size).astype(np.float32)
    st["l3_w"]["w"][:] = rng.uniform(-1.0, 1.0, st["l3_w"]["w"].size).astype(np.float32)
    return st


def _torch_loss(st, batch, lam, loss):
    """Sum of squared errors in float64, forward written in matrix form."""
    T = {k: torch.tensor(v["w"].astype(np.float64), requires_grad=True) for k, v in st.items()}
    fi, fo, pi = SH.ft_in, SH.ft_out, SH.piece_inputs
    W = T["ft_w"].reshape(SH.train_ft_in, fo)

    def persp(idx):
        rows = []
        for i in range(idx.shape[0]):
            f = [int(x) for x in idx[i, : batch["nnz"][i]] if 0 <= x < fi]
            acc = torch.zeros(fo, dtype=torch.float64)
            for x in f:  # comb[f] = W[f] + W[ft_in + f mod PI]
                acc = acc + W[x] + W[fi + x % pi]
            rows.append(acc)
        return torch.stack(rows) + T["ft_b"]

    x = torch.cat([persp(batch["stm"]).clamp(0, 1), persp(batch["nstm"]).clamp(0, 1)], dim=1)
    h1 = (x @ T["l1_w"].reshape(2 * fo, SH.l1) + T["l1_b"]).clamp(0, 1)
    h2 = (h1 @ T["l2_w"].reshape(SH.l1, SH.l2) + T["l2_b"]).clamp(0, 1)
    net = h2 @ T["l3_w"] + T["l3_b"]
    score = torch.tensor(batch["score"].astype(np.float64))
    wdl = torch.tensor(batch["wdl"].astype(np.float64))
    if loss["kind"] == "sigmoid":
        s = loss["scale"]
        y = lam * wdl + (1 - lam) * torch.sigmoid(score * s)
        err = torch.sigmoid(net * s) - y
    else:
        to, ts = loss["target_offset"], loss["target_scaling"]
        t = 0.5 * (1 + torch.sigmoid((score - to) / ts) - torch.sigmoid((-score - to) / ts))
        y = lam * wdl + (1 - lam) * t
        sn = net * loss["nnue2score"]
        io, isc = loss["in_offset"], loss["in_scaling"]
        pred = 0.5 * (1 + torch.sigmoid((sn - io) / isc) - torch.sigmoid((-sn - io) / isc))
        err = pred - y
    L = (err ** 2).sum()
    L.backward()
    return float(L.detach()), {k: v.grad.numpy() for k, v in T.items()}


WRM = {"kind": "wrm", "nnue2score": 600.0, "in_scaling": 340.0, "in_offset": 270.0,
       "target_offset": 270.0, "target_scaling": 380.0, "pow_exp": 2.0, "qp_asymmetry": 0.0,
       "w1": 0.0, "w2": 0.5}


@pytest.mark.parametrize("loss", [WRM, {"kind": "sigmoid", "scale": 1.0 / 290.0}], ids=["wrm", "sigmoid"])
def test_gradients_match_float64_autodiff(loss):
    batch = _batch()
    st = _state()
    b = batch["stm"].shape[0]
    a, acc = osi.forward(SH, st, batch, 0.25, loss)
    g = osi.backward(SH, st, batch, a)
    L64, g64 = _torch_loss(st, batch, 0.25, loss)
    assert abs(acc - L64) <= 1e-5 * abs(L64)
    for name, _ in osi.GROUPS:
        ref = g64[name] / b
        scale = np.abs(ref).max()
        assert scale > 0, name
        np.testing.assert_allclose(g[name], ref, rtol=2e-3, atol=2e-5 * scale, err_msg=name)


def test_default_init_matches_simple_init():
    st = osi.default_init(SH)
    assert np.array_equal(st["ft_w"]["w"][: SH.ft_in * SH.ft_out],
                          ffi.init_sample(SH.ft_in * SH.ft_out, SH.ft_in, "uniform", "abs", 0.01, 0x5071E001))
    assert not st["ft_w"]["w"][SH.ft_in * SH.ft_out:].any()  # factorizer rows start at zero
    for k, (name, _) in enumerate(osi.GROUPS):
        w = st[name]["w"]
        assert w.size == SH.sizes()[name]
        assert np.array_equal(st[name]["slow"], w)  # slow_param <- param
        assert not st[name]["m"].any() and not st[name]["v"].any()
        if name != "ft_w":
            assert np.all(np.abs(w) <= 0.01) and np.any(w != 0)
    assert np.array_equal(st["l3_b"]["w"], ffi.init_sample(1, SH.l2, "uniform", "abs", 0.01, 0x5071E008))


def test_adamw_step_is_radam_with_unit_step_size_and_clamps():
    batch = _batch(16, 9)
    st = _state(2)
    st["l1_w"]["w"][0] = np.float32(127.0 / 64.0)  # at the quantised bound
    opt = osi.OptConfig("adamw", 0.01)
    before = {k: v["w"].copy() for k, v in st.items()}
    _, _, g = osi.train_step(SH, st, batch, opt, 1e-3, 0.0, WRM, 1)
    for name, quant in osi.GROUPS:
        w, m, v = before[name].copy(), np.zeros_like(before[name]), np.zeros_like(before[name])
        lo, hi = (-127 / 64, 127 / 64) if quant else (np.finfo(np.float32).min, np.finfo(np.float32).max)
        ffi.radam_step(w, m, v, g[name].copy(), np.float32(1e-3), 1.0, 1, 0.01, 0.9, 0.999, 1e-8, lo, hi)
        assert np.array_equal(st[name]["w"], w), name
    assert st["l1_w"]["w"][0] <= np.float32(127.0 / 64.0)
