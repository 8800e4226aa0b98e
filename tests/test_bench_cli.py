"""bench.py's command line: the requests it refuses before touching a GPU."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_unknown_secondary_measurement_is_refused():
    r = run_bench("--extra", "c4,nope")
    assert r.returncode == 2
    assert "nope" in r.stderr and "h3_qkv_lora" in r.stderr and r.stdout == ""


def test_secondary_measurements_are_listed_in_run_order():
    sys.path.insert(0, str(ROOT))
    try:
        import bench
    finally:
        sys.path.remove(str(ROOT))
    assert list(bench.EXTRAS) == ["c3", "c4", "c5", "f1", "f4", "a6", "h3_qkv_lora", "ceilings"]
