"""Learning-rate / WDL schedules: the oracle against the reference's own
schedule tests, and the library's schedules (C ABI, host code) against the
oracle bit for bit.

Pins: every assertion of crates/nnue-train/src/schedule.rs:575-899 (the
reference's unit tests, same inputs, same tolerances), run on both the
oracle and the library; the compiler-rt powi restatement against exact
powers of two and a float64 power; and the library equal to the oracle on a
grid of batches and superbatches for every kind.
"""
import numpy as np
import pytest

import oracle.schedule as osch
import tatara_amd.run as psch

F = np.float32
EPS = 1e-6


@pytest.fixture(params=["oracle", "library"])
def S(request):
    return osch if request.param == "oracle" else psch


def test_constant_lr_is_invariant(S):
    lr = S.ConstantLR(1e-3)
    assert lr.lr(0, 1) == F(1e-3)
    assert lr.lr(100, 50) == F(1e-3)


def test_drop_lr_steps_once_after_drop_superbatch(S):
    lr = S.DropLR(1.0, 0.1, 10)
    assert lr.lr(0, 5) == 1.0
    assert lr.lr(0, 10) == 1.0
    assert abs(lr.lr(0, 11) - 0.1) < EPS
    assert abs(lr.lr(0, 100) - 0.1) < EPS


def test_step_lr_multiplicative_every_step(S):
    lr = S.StepLR(1.0, 0.5, 3)
    assert lr.lr(0, 0) == 1.0
    assert lr.lr(0, 3) == 1.0
    assert abs(lr.lr(0, 4) - 0.5) < EPS
    assert abs(lr.lr(0, 7) - 0.25) < EPS


def test_linear_decay_lr_interpolates(S):
    lr = S.LinearDecayLR(1.0, 0.0, 10)
    assert abs(lr.lr(0, 0) - 1.0) < EPS
    assert abs(lr.lr(0, 5) - 0.5) < EPS
    assert abs(lr.lr(0, 10) - 0.0) < EPS
    assert abs(lr.lr(0, 100) - 0.0) < EPS


def test_cosine_decay_lr_midpoint(S):
    lr = S.CosineDecayLR(1.0, 0.0, 10)
    assert abs(lr.lr(0, 0) - 1.0) < EPS
    assert abs(lr.lr(0, 5) - 0.5) < EPS
    assert abs(lr.lr(0, 10) - 0.0) < EPS


def test_exponential_decay_lr_factor(S):
    lr = S.ExponentialDecayLR(1.0, 0.01, 10)
    assert abs(lr.lr(0, 5) - 0.1) < 1e-5
    assert abs(lr.lr(0, 10) - 0.01) < EPS


def test_warmup_lr_only_in_first_superbatch(S):
    w = S.WarmupLR(S.ConstantLR(1.0), 4)
    assert abs(w.lr(0, 1) - 0.25) < EPS
    assert abs(w.lr(1, 1) - 1.0 / 3.0) < EPS
    assert abs(w.lr(2, 1) - 0.5) < EPS
    assert abs(w.lr(3, 1) - 1.0) < EPS
    assert abs(w.lr(4, 1) - 1.0) < EPS
    assert abs(w.lr(0, 2) - 1.0) < EPS


def test_sequence_lr_switches_at_midpoint(S):
    seq = S.SequenceLR(S.ConstantLR(1.0), S.ConstantLR(2.0), 5)
    assert seq.lr(0, 1) == 1.0
    assert seq.lr(0, 5) == 1.0
    assert seq.lr(0, 6) == 2.0
    assert seq.lr(0, 100) == 2.0


def test_one_cycle_lr_warmup_then_anneal(S):
    lr = S.OneCycleLR(1.0, 0.2, 25.0, 100.0, 10)
    assert lr.initial_lr == F(0.04)
    assert lr.warmup_superbatch == 2
    assert abs(lr.final_lr - 0.0004) < EPS
    assert abs(lr.lr(0, 0) - 0.04) < EPS
    assert abs(lr.lr(0, 2) - 1.0) < EPS
    assert abs(lr.lr(0, 1) - (0.04 + 0.5 * (1.0 - 0.04))) < EPS
    assert abs(lr.lr(0, 6) - (0.0004 + 0.5 * (1.0 - 0.0004))) < EPS
    assert abs(lr.lr(0, 10) - 0.0004) < EPS
    assert abs(lr.lr(0, 100) - 0.0004) < EPS


def test_one_cycle_lr_zero_warmup_pct_has_no_division_by_zero(S):
    lr = S.OneCycleLR(1.0, 0.0, 25.0, 100.0, 10)
    assert lr.warmup_superbatch == 0
    assert np.isfinite(lr.lr(0, 0))
    assert np.isfinite(lr.lr(0, 1))


def test_horizon_reports_terminal_superbatch(S):
    assert S.LinearDecayLR(1.0, 0.0, 42).horizon() == 42
    assert S.CosineDecayLR(1.0, 0.0, 7).horizon() == 7
    assert S.ExponentialDecayLR(1.0, 0.01, 9).horizon() == 9
    assert S.OneCycleLR(1.0, 0.2, 25.0, 100.0, 100).horizon() == 100
    assert S.ConstantLR(1e-3).horizon() is None
    assert S.StepLR(1.0, 0.5, 3).horizon() is None
    assert S.DropLR(1.0, 0.1, 10).horizon() is None
    oc = S.OneCycleLR(1.0, 0.2, 25.0, 100.0, 50)
    assert S.WarmupLR(oc, 4).horizon() == 50
    assert S.WarmupLR(S.ConstantLR(1.0), 4).horizon() is None


def test_constant_wdl_is_invariant(S):
    w = S.ConstantWDL(0.5)
    assert w.blend(0, 1, 10) == 0.5
    assert w.blend(100, 5, 10) == 0.5


def test_linear_wdl_interpolates_with_max(S):
    w = S.LinearWDL(0.0, 1.0)
    assert abs(w.blend(0, 1, 10) - 0.0) < EPS
    assert abs(w.blend(0, 10, 10) - 1.0) < EPS
    assert abs(w.blend(0, 5, 10) - 4.0 / 9.0) < EPS
    assert np.isfinite(w.blend(0, 1, 1))


def test_warmup_wdl_only_in_first_superbatch(S):
    w = S.WarmupWDL(S.ConstantWDL(0.5), 2)
    assert abs(w.blend(0, 1, 10) - 0.25) < EPS
    assert abs(w.blend(1, 1, 10) - 0.5) < EPS
    assert abs(w.blend(2, 1, 10) - 0.5) < EPS
    assert abs(w.blend(0, 2, 10) - 0.5) < EPS


def test_sequence_wdl_propagates_normalised_max(S):
    seq = S.SequenceWDL(S.LinearWDL(0.0, 1.0), S.LinearWDL(1.0, 2.0), 5)
    assert abs(seq.blend(0, 1, 10) - 0.0) < EPS
    assert abs(seq.blend(0, 5, 10) - 1.0) < EPS
    assert abs(seq.blend(0, 6, 10) - 1.0) < EPS
    assert abs(seq.blend(0, 10, 10) - 2.0) < EPS


def test_powi_square_and_multiply():
    for k in range(0, 40):
        assert osch.powi(F(0.5), k) == F(2.0 ** -k)
        assert osch.powi(F(2.0), -k) == F(2.0 ** -k)
    rng = np.random.default_rng(0)
    for _ in range(500):
        a = F(rng.uniform(0.05, 1.5))
        k = int(rng.integers(0, 60))
        exact = float(a) ** k
        got = float(osch.powi(a, k))
        if exact > 1e-30:
            assert abs(got - exact) <= 8 * k * np.spacing(F(exact)) + 1e-45, (a, k)


def _lr_cases(S):
    return [
        S.ConstantLR(8.75e-4),
        S.StepLR(8.75e-4, 0.992, 1),
        S.StepLR(1e-3, 0.3, 7),
        S.DropLR(1e-3, 0.1, 40),
        S.LinearDecayLR(1e-3, 3e-5, 37),
        S.CosineDecayLR(2e-3, 1e-5, 41),
        S.ExponentialDecayLR(1e-3, 1e-5, 29),
        S.OneCycleLR(3e-3, 0.3, 25.0, 1e4, 50),
        S.OneCycleLR(1e-3, 0.0, 10.0, 100.0, 13),
        S.WarmupLR(S.CosineDecayLR(2e-3, 1e-5, 41), 7),
        S.SequenceLR(S.WarmupLR(S.ConstantLR(1e-3), 5), S.StepLR(5e-4, 0.9, 3), 11),
    ]


def _wdl_cases(S):
    return [
        S.ConstantWDL(0.3),
        S.LinearWDL(0.0, 1.0),
        S.LinearWDL(0.75, 0.125),
        S.WarmupWDL(S.LinearWDL(0.2, 0.9), 3),
        S.SequenceWDL(S.LinearWDL(0.0, 0.5), S.WarmupWDL(S.LinearWDL(0.5, 1.0), 2), 9),
    ]


def test_library_equals_oracle_bit_for_bit():
    for lo, lp in zip(_lr_cases(osch), _lr_cases(psch)):
        assert lo.horizon() == lp.horizon()
        for sb in range(0, 64):
            for b in (0, 1, 2, 4, 6, 9):
                x, y = F(lo.lr(b, sb)), F(lp.lr(b, sb))
                assert x.tobytes() == y.tobytes(), (type(lo).__name__, b, sb, x, y)
    for mx in (1, 2, 10, 33):
        for wo, wp in zip(_wdl_cases(osch), _wdl_cases(psch)):
            for sb in range(1, 40):
                for b in (0, 1, 2, 5):
                    if isinstance(wo, osch.SequenceWDL) and mx <= wo.mid:
                        continue  # the second part would see max - midpoint < 1
                    x, y = F(wo.blend(b, sb, mx)), F(wp.blend(b, sb, mx))
                    assert x.tobytes() == y.tobytes(), (type(wo).__name__, b, sb, mx, x, y)


def test_library_rejects_superbatch_zero_for_wdl():
    from tatara_amd._lib import TataraError
    with pytest.raises(TataraError):
        psch.ConstantWDL(0.5).blend(0, 0, 10)
