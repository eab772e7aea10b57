"""Pins the composed LayerStack oracle step (oracle/layerstack.py) without the reference.

The reference's LayerStack trainer has no stored golden values, so the
composition of the restated CPU kernels is checked against what the
mathematics fixes: the gradient of the loss, taken by float64 reverse-mode
autodiff (torch on the CPU) over an independent restatement of the forward
in matrix form, following the reference's wiring
(bins/nnue_train/src/trainer_layerstack.rs:2113-2720):

  FT      raw[b] = sum of comb rows of the valid slots, comb[f] = W[f] +
          W[ft_in + f mod PI] (factorizer); pairwise post per perspective:
          crelu(raw[c] + beta[c]) * crelu(raw[c + h] + beta[c + h]) * 127/128,
          stm filling columns [0, h), nstm [h, ft_out)
          (ft_post_perspective_fwd, native_kernels.cu:1499-1527)
  L1      per-bucket W1[g] [l1][ft_out] + b1[g], plus shared x Ws [ft_out][l1]
          + bs; rows with an out-of-range bucket get 0 from every per-bucket
          layer (dense_mm_fwd_bucket, native_kernels.cu:2355-2392)
  tail    main = l1[:, :l1-1], skip = l1[:, l1-1]; l2_pre = [main^2 * 127/128,
          main]; l2_in = crelu(l2_pre)
  L2, L3  per-bucket affine, crelu between; net = l3 + skip
  loss    sigmoid-MSE, WRM and the extended WRM of loss_wdl.rs / loss_wrm.rs

For sigmoid and plain WRM the reference's dy is dL/dnet / b for L = sum of
squared errors (per_pos_norm = 1/b); for the extended WRM it is dL/dnet for
L = sum(asym |err|^p w) / sum(w) (loss_wrm.rs, the weight-normalised form).
All ten parameter groups' gradients are compared.  Planted wiring mistakes
(the concat halves swapped in the backward, a wrong bucket row in a bias
gradient, the L2 weight gradient taken from l2_pre instead of l2_input, the
FT-post gradient of one half routed to the other) must fail the comparison.
"""
import numpy as np
import pytest

from oracle import ffi
from oracle import layerstack as ols

torch = pytest.importorskip("torch")

SIGMOID = {"kind": "sigmoid", "scale": 1.0 / 290.0}
WRM = {"kind": "wrm", "nnue2score": 600.0, "in_scaling": 340.0, "in_offset": 270.0, "target_offset": 270.0,
       "target_scaling": 380.0, "pow_exp": 2.0, "qp_asymmetry": 0.0, "w1": 0.0, "w2": 0.5}
WRM_EXT = dict(WRM, pow_exp=2.5, qp_asymmetry=0.2, w1=1.0, w2=0.5)
LOSSES = {"sigmoid": SIGMOID, "wrm": WRM, "wrm_ext": WRM_EXT}


def _shape(l1=16, nb=3):
    return ols.LsShape(ft_in=40, max_active=6, piece_inputs=8, ft_out=16, l1=l1, l2=32, nb=nb)


def _batch(sh, b=48, seed=3):
    rng = np.random.default_rng(seed)
    ma = sh.max_active
    stm = rng.integers(0, sh.ft_in, (b, ma)).astype(np.int32)
    nstm = rng.integers(0, sh.ft_in, (b, ma)).astype(np.int32)
    nnz = rng.integers(2, ma + 1, b).astype(np.int32)
    stm[np.arange(ma)[None, :] >= nnz[:, None]] = -1
    nstm[np.arange(ma)[None, :] >= nnz[:, None]] = -1
    stm[4, 0] = sh.ft_in + 3  # out of range: skipped by the gather
    bucket = rng.integers(0, sh.nb, b).astype(np.int32)
    bucket[5] = -1      # no per-bucket layers
    bucket[9] = sh.nb   # out of range
    return dict(stm=stm, nstm=nstm, nnz=nnz, bucket=bucket,
                score=rng.uniform(-900, 900, b).astype(np.float32),
                wdl=rng.choice([0.0, 0.5, 1.0], b).astype(np.float32))


def _state(sh, seed=5):
    """Weights that put a good share of every CReLU's inputs in its linear part."""
    st = ols.default_init(sh)
    rng = np.random.default_rng(seed)

    def fill(name, lo, hi):
        st[name]["w"][:] = rng.uniform(lo, hi, st[name]["w"].size).astype(np.float32)

    fill("ft_w", -0.08, 0.2)
    fill("ft_b", -0.2, 0.4)
    fill("l1_w", -0.3, 0.4)
    fill("l1_b", -0.4, 0.7)
    fill("l1_shared_weight", -0.3, 0.4)
    fill("l1_shared_bias", -0.3, 0.3)
    fill("l2_w", -0.3, 0.4)
    fill("l2_b", 0.1, 0.4)
    fill("l3_w", -1.0, 1.0)
    fill("l3_b", -0.2, 0.2)
    return st


def _torch_loss(sh, st, batch, lam, loss):
    """Float64 loss as the reference defines it (see the module docstring) and the
    autodiff gradient of every group."""
    T = {k: torch.tensor(v["w"].astype(np.float64), requires_grad=True) for k, v in st.items()}
    fi, fo, pi, nb, l1, l2 = sh.ft_in, sh.ft_out, sh.piece_inputs, sh.nb, sh.l1, sh.l2
    l1e, h = l1 - 1, fo // 2
    b = batch["stm"].shape[0]
    W = T["ft_w"].reshape(sh.train_ft_in, fo)

    def raw(idx):
        rows = []
        for i in range(b):
            acc = torch.zeros(fo, dtype=torch.float64)
            for x in idx[i, : batch["nnz"][i]]:
                if 0 <= x < fi:
                    acc = acc + W[int(x)] + W[fi + int(x) % pi]
            rows.append(acc)
        return torch.stack(rows)

    def post(r):
        a = (r[:, :h] + T["ft_b"][:h]).clamp(0, 1)
        c = (r[:, h:] + T["ft_b"][h:]).clamp(0, 1)
        return a * c * (127.0 / 128.0)

    x = torch.cat([post(raw(batch["stm"])), post(raw(batch["nstm"]))], dim=1)
    bk = torch.tensor(batch["bucket"].astype(np.int64))
    valid = ((bk >= 0) & (bk < nb)).to(torch.float64)[:, None]
    g = bk.clamp(0, nb - 1)

    def per_bucket(inp, w, bias, n_out):
        Wg = w.reshape(nb, n_out, -1)[g]            # [b][out][in]
        y = torch.einsum("bi,boi->bo", inp, Wg) + bias.reshape(nb, n_out)[g]
        return y * valid

    l1_total = per_bucket(x, T["l1_w"], T["l1_b"], l1) + x @ T["l1_shared_weight"].reshape(fo, l1) \
        + T["l1_shared_bias"]
    main, skip = l1_total[:, :l1e], l1_total[:, l1e]
    l2_in = torch.cat([main * main * (127.0 / 128.0), main], dim=1).clamp(0, 1)
    l2_act = per_bucket(l2_in, T["l2_w"], T["l2_b"], l2).clamp(0, 1)
    net = per_bucket(l2_act, T["l3_w"], T["l3_b"], 1)[:, 0] + skip

    score = torch.tensor(batch["score"].astype(np.float64))
    wdl = torch.tensor(batch["wdl"].astype(np.float64))
    if loss["kind"] == "sigmoid":
        s = loss["scale"]
        err = torch.sigmoid(net * s) - (lam * wdl + (1 - lam) * torch.sigmoid(score * s))
        L, norm = (err ** 2).sum(), 1.0 / b
    else:
        to, ts = loss["target_offset"], loss["target_scaling"]
        pf = 0.5 * (1 + torch.sigmoid((score - to) / ts) - torch.sigmoid((-score - to) / ts))
        target = lam * wdl + (1 - lam) * pf
        sn = net * loss["nnue2score"]
        io, isc = loss["in_offset"], loss["in_scaling"]
        qf = 0.5 * (1 + torch.sigmoid((sn - io) / isc) - torch.sigmoid((-sn - io) / isc))
        err = qf - target
        extended = loss["pow_exp"] != 2.0 or loss["qp_asymmetry"] != 0.0 or loss["w1"] != 0.0
        if not extended:
            L, norm = (err ** 2).sum(), 1.0 / b
        else:
            w = 1 + (2.0 ** loss["w1"] - 1) * ((pf - 0.5) ** 2 * pf * (1 - pf)) ** loss["w2"]
            asym = torch.where(qf > target, 1 + loss["qp_asymmetry"], 1.0).detach()
            L, norm = (asym * err.abs() ** loss["pow_exp"] * w).sum() / w.sum(), 1.0
    L.backward()
    return float(L.detach()), {k: v.grad.numpy() * norm for k, v in T.items()}


def _check(sh, st, batch, lam, loss):
    a, _ = ols.forward(sh, st, batch, lam, loss)
    g = ols.backward(sh, st, batch, a)
    _, ref = _torch_loss(sh, st, batch, lam, loss)
    for name in ref:
        scale = np.abs(ref[name]).max()
        assert scale > 0, f"{name}: the test batch leaves this group without gradient"
        np.testing.assert_allclose(g[name], ref[name], rtol=2e-3, atol=2e-5 * scale, err_msg=name)


@pytest.mark.parametrize("loss", list(LOSSES))
@pytest.mark.parametrize("l1,nb", [(16, 3), (8, 4)], ids=["l1_16", "l1_8"])
def test_gradients_match_float64_autodiff(loss, l1, nb):
    sh = _shape(l1, nb)
    _check(sh, _state(sh), _batch(sh), 0.25, LOSSES[loss])


def test_activations_reach_every_crelu_region():
    """The batch and weights above put inputs below 0, above 1 and in between
    at every CReLU (FT post, L2 input, L2 output), so a missing mask or clamp
    cannot hide."""
    for l1, nb in ((16, 3), (8, 4)):
        sh = _shape(l1, nb)
        st = _state(sh)
        a, _ = ols.forward(sh, st, _batch(sh), 0.25, SIGMOID)
        ft_pre = (a["ft_stm"].reshape(-1, sh.ft_out) + st["ft_b"]["w"]).ravel()
        for k, v in (("ft_pre", ft_pre), ("l2_pre", a["l2_pre"]), ("l2_out", a["l2_out"])):
            assert (v < 0).mean() > 0.01 and (v > 1).mean() > 0.01 and ((v > 0) & (v < 1)).mean() > 0.3, (l1, k)


def _planted(monkeypatch, what):
    if what == "concat_halves_swapped":
        real = ffi.concat_l1sqr_main_grad
        monkeypatch.setattr(ffi, "concat_l1sqr_main_grad", lambda *a: tuple(reversed(real(*a))))
    elif what == "bias_grad_wrong_bucket_row":
        real = ffi.bias_grad_bucket
        monkeypatch.setattr(ffi, "bias_grad_bucket",
                            lambda dy, bucket, gb, b, n, nb: real(dy, np.where(bucket >= 0, (bucket + 1) % nb, bucket),
                                                                  gb, b, n, nb))
    elif what == "l2_weight_grad_from_l2_pre":
        real = ffi.dense_mm_bwd_weight_bucket
        state = {}

        def fake(x, dy, bucket, b, i, o, nb):
            if i == state.get("l2_in") and "pre" in state:
                x = state["pre"]
            return real(x, dy, bucket, b, i, o, nb)

        monkeypatch.setattr(ffi, "dense_mm_bwd_weight_bucket", fake)
        return state
    elif what == "ft_post_grad_halves_routed_wrong":
        real = ffi.ft_post_perspective_grad
        monkeypatch.setattr(ffi, "ft_post_perspective_grad",
                            lambda d, ft, bias, gb, b, dim, off, stride, s: real(d, ft, bias, gb, b, dim,
                                                                                 dim // 2 - off, stride, s))
    return None


@pytest.mark.parametrize("what", ["concat_halves_swapped", "bias_grad_wrong_bucket_row", "l2_weight_grad_from_l2_pre",
                                  "ft_post_grad_halves_routed_wrong"])
def test_planted_wiring_mistakes_fail(monkeypatch, what):
    sh = _shape()
    st, batch = _state(sh), _batch(sh)
    state = _planted(monkeypatch, what)
    if state is not None:
        a, _ = ols.forward(sh, st, batch, 0.25, SIGMOID)
        state["l2_in"], state["pre"] = sh.l2_in, a["l2_pre"]
    with pytest.raises(AssertionError):
        _check(sh, st, batch, 0.25, SIGMOID)
