"""bench.py's host-side contract, on the CPU: it refuses more than one GPU before touching a device,
and every `roofline.traffic` figure it reports has its rocprof summary under profiles/."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("argv, env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(argv, env):
    run = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv], capture_output=True, text=True,
                         env={**os.environ, **env}, timeout=120)
    assert run.returncode == 2
    assert run.stdout == ""                       # no JSON line
    assert "one GPU only" in run.stderr


def test_every_reported_traffic_figure_has_its_profile():
    sys.path.insert(0, str(ROOT))
    import bench

    source = (ROOT / "bench.py").read_text()
    names = [part.split('")', 1)[0] for part in source.split('read_traffic("')[1:]]
    assert len(names) == 12
    for name in names:
        traffic = bench.read_traffic(name)
        assert isinstance(traffic, int) and traffic > 0, name
        text = (ROOT / "profiles" / f"{name}.traffic.txt").read_text()
        algorithmic = int(text.split("algorithmic_bytes:", 1)[1].split()[0])
        assert 0.5 < traffic / algorithmic < 20, name
        assert "command: rocprofv3 --pmc" in text, name
