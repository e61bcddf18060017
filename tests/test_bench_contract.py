"""CPU checks of bench.py's driver contract: the metric string is the one
the baseline names, and a multi-GPU request ends with a message and exit
status 2 before any GPU work (this build runs on one GPU)."""
import json
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_metric_matches_baseline():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        metric = json.load(f)["metric"]
    with open(os.path.join(ROOT, "bench.py")) as f:
        src = f.read()
    found = re.findall(r'"metric":\s*"([^"]*)"', src)
    assert found == [metric]


def test_multi_gpu_request_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert line and "one GPU" in json.loads(line[-1])["error"]
    assert "only --gpus 1" in r.stderr
