"""The `popcorn-amd` distribution installs offline and satisfies Popcorn's version gate on its own.

Popcorn's gate (core/sources.py:50-73) needs `importlib.metadata.version` of
the declared distribution to resolve; here it must resolve from an installed
copy with the source tree off `sys.path`. The install ships the kernel library
built in-tree (POPCORN_AMD_PREBUILT), so the test needs no hipcc run; loading
the library and querying its ABI version needs no GPU.
"""

from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

import popcorn_amd
from popcorn_amd import _lib

ROOT = Path(__file__).resolve().parents[1]

PROBE = """
import importlib.metadata, json, sys
sys.path = [p for p in sys.path if p and not p.startswith({root!r})]
import popcorn_amd
from popcorn_amd import _lib, backend, compat
from popcorn_amd.compat.backends import unavailable_reason
backend.register(compat)
print(json.dumps({{
    "version": importlib.metadata.version("popcorn-amd"),
    "package": popcorn_amd.__file__,
    "abi": _lib.load().pk_version(),
    "gate": unavailable_reason(backend.BACKEND),
    "rms_norm": compat.KERNELS["rms_norm"].available_backends(),
}}))
"""


def test_the_distribution_installs_offline_and_its_gate_resolves(tmp_path):
    if not _lib.LIBRARY.exists():
        pytest.fail(f"{_lib.LIBRARY} is not built; run __graft_entry__.build()")
    target = tmp_path / "site"
    # installed from a copy of the distribution's files, so setuptools' build directory lands there and
    # not in the source tree
    src = tmp_path / "src"
    src.mkdir()
    for name in ("setup.py", "README.md"):
        shutil.copy2(ROOT / name, src / name)
    shutil.copytree(ROOT / "popcorn_amd", src / "popcorn_amd",
                    ignore=shutil.ignore_patterns("__pycache__", "_build", "*.pyc"))
    env = {**os.environ, "POPCORN_AMD_PREBUILT": "1", "PIP_NO_INDEX": "1", "PIP_DISABLE_PIP_VERSION_CHECK": "1"}
    install = subprocess.run([sys.executable, "-m", "pip", "install", "--no-deps", "--no-build-isolation",
                              "--target", str(target), str(src)], env=env, capture_output=True, text=True,
                             timeout=600)
    assert install.returncode == 0, install.stdout[-2000:] + install.stderr[-2000:]
    assert (target / "popcorn_amd" / "libpopcorn_amd.so").exists()
    assert list(target.glob("popcorn_amd-*.dist-info"))

    run_env = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    run_env["PYTHONPATH"] = str(target)
    probe = subprocess.run([sys.executable, "-c", PROBE.format(root=str(ROOT))], cwd=tmp_path, env=run_env,
                           capture_output=True, text=True, timeout=600)
    assert probe.returncode == 0, probe.stderr[-3000:]
    seen = json.loads(probe.stdout.strip().splitlines()[-1])
    assert seen["version"] == popcorn_amd.__version__
    assert seen["package"].startswith(str(target))
    assert seen["abi"] == _lib.ABI_VERSION
    assert seen["gate"] is None
    assert seen["rms_norm"] == ["mi355x", "torch"]
