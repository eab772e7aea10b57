"""bench.py's contract on the CPU: the single-GPU guard and the isolation of
the secondary workload figures (no GPU work is started here)."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_exits_with_a_message(n):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(n)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and f"--gpus {n}" in r.stderr
    assert r.stdout == ""


def test_a_failing_secondary_workload_is_reported_not_raised(monkeypatch):
    def fake(name, b, steps, warmup, n_batches):
        if name == "ls768":
            raise RuntimeError("out of memory")
        return {"value": 1.0, "unit": "pos/s"}

    monkeypatch.setattr(bench, "one_workload", fake)
    out = bench.other_workloads(["ls1536_mixed", "ls768", "simple"], 65536, 20, 3)
    assert out["ls1536_mixed"]["value"] == 1.0 and out["simple"]["value"] == 1.0
    assert out["ls768"]["value"] is None and "out of memory" in out["ls768"]["error"]


def test_every_other_workload_is_a_baseline_config():
    assert set(bench.WORKLOADS) == {"ls1536", "ls1536_mixed", "ls768", "simple"}
    for w in bench.WORKLOADS.values():
        assert w["ref"] > 0 and w["ref_src"].startswith("README.md:")
