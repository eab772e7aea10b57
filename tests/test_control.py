"""control.json handling of the superbatch driver (host code, CPU only).

tatara_control_apply is the function tatara_train_run calls at the start of
every superbatch (apply_control, crates/nnue-train/src/trainer.rs:670-731).
The cases are the reference's own control tests (trainer.rs:1805-2180):
clamping to the current superbatch, the deduplicated stale warning, missing /
unreadable / malformed files, targets at or beyond the configured end, a
failing history append, unknown fields; plus the serde_json typing rules of
`target_superbatches: Option<usize>` (null, floats, negatives, strings,
duplicate fields, trailing characters).  The run-level cases (a run stopping
at the target, resume offsets) are in tests/test_gpu_run.py.
"""
import ctypes as C
import json

import pytest

from tatara_amd import _lib
from tatara_amd._lib import TataraControlState


def apply(tmp_path, text, state, current, start, end, history=None):
    control = tmp_path / "control.json"
    if text is not None:
        control.write_text(text)
    hist = history if history is not None else tmp_path / "control_history.jsonl"
    applied, target = C.c_int32(), C.c_uint64()
    _lib.check(_lib.load().tatara_control_apply(str(control).encode(), str(hist).encode(), C.byref(state),
                                                current, start, end, C.byref(applied), C.byref(target)))
    return (target.value if applied.value else None), hist


def state(effective):
    return TataraControlState(effective_target=effective, ignored_stale_target=0, has_ignored_stale=0)


def test_target_below_current_clamps_to_current_and_is_recorded(tmp_path, capfd):
    st = state(8)
    got, hist = apply(tmp_path, '{"target_superbatches": 3}', st, 5, 1, 8)
    assert got == 5 and st.effective_target == 5
    rec = json.loads(hist.read_text().splitlines()[0])
    assert rec["type"] == "control" and rec["target_superbatches"] == 5 and rec["superbatch"] == 5
    assert rec["timestamp"].endswith("Z") and len(rec["timestamp"]) == 20
    assert "[control] applied: target_superbatches=5 (superbatch=5)" in capfd.readouterr().out


def test_stop_after_current_superbatch(tmp_path):
    st = state(3)
    got, hist = apply(tmp_path, '{"target_superbatches": 1}', st, 1, 1, 3)
    assert got == 1 and st.effective_target == 1
    assert len(hist.read_text().splitlines()) == 1
    # the same request again changes nothing and records nothing
    got, _ = apply(tmp_path, '{"target_superbatches": 1}', st, 1, 1, 3)
    assert got is None and len(hist.read_text().splitlines()) == 1


def test_stale_target_warning_is_deduplicated(tmp_path, capfd):
    st = state(5)
    warn = "ignoring stale target_superbatches="
    for text, expect in (('{"target_superbatches": 2}', 1), ('{"target_superbatches": 2}', 0),
                         ('{"target_superbatches": 1}', 1)):
        got, hist = apply(tmp_path, text, st, 3, 3, 5)
        assert got is None and st.effective_target == 5
        assert capfd.readouterr().err.count(warn) == expect
    assert not hist.exists()
    # a valid request clears the remembered stale value
    got, _ = apply(tmp_path, '{"target_superbatches": 4}', st, 3, 3, 5)
    assert got == 4
    capfd.readouterr()
    apply(tmp_path, '{"target_superbatches": 2}', st, 3, 3, 5)
    assert capfd.readouterr().err.count(warn) == 1


@pytest.mark.parametrize("case", ["missing", "unreadable", "malformed"])
def test_missing_unreadable_and_malformed_control_change_nothing(tmp_path, capfd, case):
    st = state(3)
    if case == "unreadable":
        (tmp_path / "control.json").mkdir()
        text = None
    else:
        text = None if case == "missing" else "{ not json"
    got, hist = apply(tmp_path, text, st, 1, 1, 3)
    assert got is None and st.effective_target == 3 and not hist.exists()
    err = capfd.readouterr().err
    if case == "missing":
        assert err == ""
    elif case == "unreadable":
        assert "[control] warning: failed to read" in err and "; ignoring" in err
    else:
        assert "[control] warning: failed to parse" in err and "; ignoring" in err


def test_target_at_or_above_configured_end_is_a_noop(tmp_path):
    for target in (3, 99):
        st = state(3)
        got, hist = apply(tmp_path, json.dumps({"target_superbatches": target}), st, 1, 1, 3)
        assert got is None and st.effective_target == 3 and not hist.exists()


def test_history_append_failure_still_applies(tmp_path, capfd):
    hist = tmp_path / "control_history.jsonl"
    hist.mkdir()
    st = state(3)
    got, _ = apply(tmp_path, '{"target_superbatches": 2}', st, 1, 1, 3, history=hist)
    assert got == 2 and st.effective_target == 2
    assert "[control] warning: failed to append" in capfd.readouterr().err


def test_unknown_fields_are_ignored(tmp_path):
    st = state(4)
    got, _ = apply(tmp_path, '{"target_superbatches": 2, "unknown_field": true, "nested": {"a": [1, 2.5, null]}}',
                   st, 1, 1, 4)
    assert got == 2


@pytest.mark.parametrize("text,applied", [
    ('{"target_superbatches": null}', False),
    ("{}", False),
    ('  {"target_superbatches" : 2 }  \n', True),
    ('{"target_superbatches": 2.0}', "error"),
    ('{"target_superbatches": 2e0}', "error"),
    ('{"target_superbatches": -1}', "error"),
    ('{"target_superbatches": "2"}', "error"),
    ('{"target_superbatches": 2, "target_superbatches": 2}', "error"),
    ('{"target_superbatches": 2} x', "error"),
    ("[2]", "error"),
    ("", "error"),
])
def test_target_superbatches_typing(tmp_path, capfd, text, applied):
    st = state(5)
    got, _ = apply(tmp_path, text, st, 1, 1, 5)
    err = capfd.readouterr().err
    if applied is True:
        assert got == 2
    else:
        assert got is None and st.effective_target == 5
        assert ("failed to parse" in err) == (applied == "error")
