"""bench.py's command-line contract on the CPU: one GPU only (a request for
more exits with a message and a non-zero status, before touching a GPU)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_extra_legs_report_a_failing_child(monkeypatch):
    """The default run's child legs: a child that fails is reported in the
    line (exit status and message), not raised."""
    sys.path.insert(0, ROOT)
    import bench

    monkeypatch.setattr(bench, "EXTRA_LEGS", [("refused", ["--gpus", "2"], {}, ["value"])])
    out = bench.extra_legs(timeout_s=300)
    assert set(out) == {"refused"}
    assert out["refused"]["error"].startswith("exit 2")
    assert "one GPU" in out["refused"]["error"]
