"""Host-side pieces of bench.py that run without a GPU: the one-GPU guard and
the board power / clock reader behind the sustained-load figures."""

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

# The shape of `amd-smi metric -p -c` on the MI355X boxes (fields trimmed).
SAMPLE = """GPU: 0
    POWER:
        SOCKET_POWER: 1354 W
        GFX_VOLTAGE: N/A
    CLOCK:
        GFX_0:
            CLK: 1939 MHz
            MIN_CLK: 500 MHz
            MAX_CLK: 2400 MHz
        GFX_1:
            CLK: 1940 MHz
"""


def _fake_run(stdout):
    def run(*args, **kwargs):
        return subprocess.CompletedProcess(args[0], 0, stdout=stdout, stderr="")
    return run


def test_read_power_parses_socket_power_and_gfx0_clock(monkeypatch):
    monkeypatch.setattr(subprocess, "run", _fake_run(SAMPLE))
    assert bench._read_power() == (1354.0, 1939.0)


@pytest.mark.parametrize("stdout", ["", "GPU: 0\n    POWER:\n        SOCKET_POWER: N/A\n"])
def test_read_power_without_fields_is_none(monkeypatch, stdout):
    monkeypatch.setattr(subprocess, "run", _fake_run(stdout))
    assert bench._read_power() is None


def test_read_power_without_the_tool_is_none(monkeypatch):
    def missing(*args, **kwargs):
        raise FileNotFoundError("amd-smi")
    monkeypatch.setattr(subprocess, "run", missing)
    assert bench._read_power() is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
