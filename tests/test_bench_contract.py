"""bench.py's command-line contract on the CPU: this build measures one GPU,
so any larger --gpus count stops with a message instead of running."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode != 0
    text = r.stdout + r.stderr
    assert "one GPU" in text and "--gpus 2" in text
