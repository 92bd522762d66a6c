"""Shared pytest setup.

* Puts the package (kernel-forge_amd/) and the repo root (for oracle/) on sys.path.
* Registers the ``gpu`` marker.  Tests marked ``gpu`` need a HIP GPU and call
  the gfx950 library; they are skipped (with a reason) only where no GPU is
  visible, so a GPU box always runs them.
* ``error_log`` collects per-case error statistics like the reference's
  ErrorLog (tests/conftest.py:22-51) and writes them as JSON to
  $KF_RESULTS_DIR when that variable is set.
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "kernel-forge_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libkf_int4.so")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    import torch

    if not torch.cuda.is_available():
        skip = pytest.mark.skip(reason="HIP GPU required")
        for it in gpu_items:
            it.add_marker(skip)


class ErrorLog:
    def __init__(self):
        self.records: dict[str, list[dict]] = {}

    def add(self, suite: str, **record):
        self.records.setdefault(suite, []).append(record)

    def dump(self):
        out_dir = os.environ.get("KF_RESULTS_DIR")
        if not out_dir or not self.records:
            return
        Path(out_dir).mkdir(parents=True, exist_ok=True)
        for suite, recs in self.records.items():
            summary = {
                "suite": suite,
                "total_cases": len(recs),
                "passed_cases": sum(bool(r["passed"]) for r in recs),
                "worst_max_rel_err": max(r["max_rel_err"] for r in recs),
                "rel_err_definition": "max|out - ref| / max|ref| over the whole output tensor",
                "cases": recs,
            }
            (Path(out_dir) / f"correctness_{suite}.json").write_text(json.dumps(summary, indent=1))


@pytest.fixture(scope="session")
def error_log():
    log = ErrorLog()
    yield log
    log.dump()
