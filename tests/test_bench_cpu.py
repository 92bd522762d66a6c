"""bench.py's host-side helpers that need no GPU: the amd-smi sample parser of `--power` and the
single-GPU guard."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402


def _metric(power, clocks):
    return [{"gpu": 0, "power": {"socket_power": {"value": power, "unit": "W"}},
             "clock": {**{f"gfx_{i}": {"clk": {"value": c, "unit": "MHz"}} for i, c in enumerate(clocks)},
                       "mem_0": {"clk": {"value": 2000, "unit": "MHz"}}, "vclk_0": {"clk": "N/A"}}}]


def _fake_run(payload, returncode=0):
    def run(cmd, **kw):
        assert cmd[0] == "amd-smi"
        return subprocess.CompletedProcess(cmd, returncode, stdout=payload, stderr="")
    return run


def test_board_sample_reads_power_and_mean_gfx_clock(monkeypatch):
    monkeypatch.setattr(subprocess, "run", _fake_run(json.dumps(_metric(1374, [2160, 2164, 2100, 2200]))))
    assert bench._board_sample() == (1374.0, 2156.0)


def test_board_sample_accepts_the_gpu_data_wrapper(monkeypatch):
    monkeypatch.setattr(subprocess, "run", _fake_run(json.dumps({"gpu_data": _metric(300, [2400])})))
    assert bench._board_sample() == (300.0, 2400.0)


@pytest.mark.parametrize("payload", ["", "not json", json.dumps([{"gpu": 0}]), json.dumps(_metric("N/A", [])),
                                     json.dumps(_metric(500, []))])
def test_board_sample_returns_none_on_unusable_output(monkeypatch, payload):
    monkeypatch.setattr(subprocess, "run", _fake_run(payload))
    assert bench._board_sample() is None


def test_board_sample_returns_none_without_amd_smi(monkeypatch):
    def missing(cmd, **kw):
        raise FileNotFoundError(cmd[0])
    monkeypatch.setattr(subprocess, "run", missing)
    assert bench._board_sample() is None


def test_more_than_one_gpu_is_refused(monkeypatch, capsys):
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "2"])
    assert bench.main() == 2
    assert "single GPU" in capsys.readouterr().err
