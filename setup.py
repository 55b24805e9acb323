"""The `popcorn-amd` distribution: the MI355X kernel backend for Popcorn, installable offline.

    pip install --no-build-isolation .          # compiles libpopcorn_amd.so for gfx950, then installs
    POPCORN_AMD_PREBUILT=1 pip install ...      # ships the library already built in-tree instead

Popcorn's version gate (core/sources.py:50-73) checks `importlib.metadata.version("popcorn-amd")`
against the range `popcorn_amd.backend.register` declares, so the backend is eligible wherever
this distribution's metadata is visible: after an install, or in the source tree once
`python -m popcorn_amd.build` (or `__graft_entry__.build()`) has written it there (it runs this
file's `egg_info`).
"""

from __future__ import annotations

import os
import re
import sys
from pathlib import Path

from setuptools import setup
from setuptools.command.build_py import build_py

ROOT = Path(__file__).resolve().parent
VERSION = re.search(r'^__version__ = "([^"]+)"', (ROOT / "popcorn_amd" / "__init__.py").read_text(), re.M).group(1)


class BuildWithKernels(build_py):
    """Compile the HIP kernel library (hipcc, gfx950) before the package files are collected."""

    def run(self) -> None:
        library = ROOT / "popcorn_amd" / "libpopcorn_amd.so"
        if os.environ.get("POPCORN_AMD_PREBUILT"):
            if not library.exists():
                raise SystemExit(f"POPCORN_AMD_PREBUILT is set but {library} has not been built")
        else:
            sys.path.insert(0, str(ROOT))
            from popcorn_amd import build

            build.build(verbose=True)
        super().run()


setup(
    name="popcorn-amd",
    version=VERSION,
    description="MI355X (gfx950) HIP kernel backend for Popcorn's transformer-block ops",
    python_requires=">=3.10",
    packages=["popcorn_amd", "popcorn_amd.compat"],
    package_data={"popcorn_amd": ["libpopcorn_amd.so", "csrc/*.hip", "csrc/*.h"]},
    install_requires=["torch", "numpy", "packaging", "pyarrow"],
    cmdclass={"build_py": BuildWithKernels},
    zip_safe=False,
)
