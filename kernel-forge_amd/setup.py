"""Setuptools entry of the MI355X INT4 linear package, the counterpart of the reference's setup.py
for ``kernelforge._C``:

    pip install -e kernel-forge_amd --no-build-isolation     # from the repository root

Its build step compiles ``libkf_int4.so`` for gfx950 with hipcc (``kernelforge/build.py``, the same
build ``__graft_entry__.build()`` runs) into ``kernelforge/``, where ``kernelforge._lib`` loads it;
a non-editable install ships that file inside the package.  The sources it compiles are
``csrc/*.hip`` beside this file and the C-ABI header in ``../include``, so installs run from a
checkout of the whole repository.  The import name is ``kernelforge``, the reference's: uninstall
the reference's package first.
"""

import importlib.util
import re
from pathlib import Path

from setuptools import find_packages, setup
from setuptools.command.build_py import build_py
from setuptools.command.develop import develop

HERE = Path(__file__).resolve().parent
VERSION = re.search(r'^__version__ = "([^"]+)"', (HERE / "kernelforge" / "__init__.py").read_text(), re.M).group(1)


def _build_library() -> None:
    spec = importlib.util.spec_from_file_location("kf_build", HERE / "kernelforge" / "build.py")
    builder = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(builder)
    print(f"built {builder.build_library()}")


class BuildWithLibrary(build_py):
    """build_py (wheels, and editable installs on setuptools >= 64) that first builds
    libkf_int4.so in the source tree."""

    def run(self):
        _build_library()
        super().run()


class DevelopWithLibrary(develop):
    """The legacy editable install (``setup.py develop``, which pip falls back to on older
    setuptools) runs no build_py: build the library here as well."""

    def run(self):
        _build_library()
        super().run()


setup(
    name="kernelforge-mi355x",
    version=VERSION,
    description="KernelForge's INT4 weight-only linear (ops.int4_linear) as gfx950 HIP kernels behind a C ABI",
    packages=find_packages(include=["kernelforge"]),
    package_data={"kernelforge": ["libkf_int4.so"]},
    python_requires=">=3.10",
    install_requires=["torch", "numpy"],
    cmdclass={"build_py": BuildWithLibrary, "develop": DevelopWithLibrary},
)
