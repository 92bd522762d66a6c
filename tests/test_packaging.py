"""kernel-forge_amd/setup.py, the pip entry that mirrors the reference's setup.py: its metadata, and
that its build step is the one that compiles libkf_int4.so into the package (no build here)."""

from __future__ import annotations

import os
from pathlib import Path

import setuptools  # noqa: F401  (first, so that distutils below is setuptools' copy)
from distutils.core import run_setup  # noqa: E402

SETUP = Path(__file__).resolve().parents[1] / "kernel-forge_amd" / "setup.py"


def test_setup_declares_the_package_and_its_library():
    cwd = os.getcwd()
    try:
        os.chdir(SETUP.parent)  # pip runs setup.py from the project directory
        dist = run_setup(str(SETUP), stop_after="init")
    finally:
        os.chdir(cwd)
    assert dist.get_name() == "kernelforge-mi355x"
    import kernelforge
    assert dist.get_version() == kernelforge.__version__
    assert dist.packages == ["kernelforge"]
    assert dist.package_data == {"kernelforge": ["libkf_int4.so"]}
    assert dist.cmdclass["build_py"].__name__ == "BuildWithLibrary"
    assert dist.cmdclass["develop"].__name__ == "DevelopWithLibrary"
