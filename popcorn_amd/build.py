"""Build recipe for the HIP kernel library: hipcc for gfx950, in-tree output.

`python -m popcorn_amd.build` compiles every `csrc/*.hip` to an object in
`popcorn_amd/_build/` (in parallel) and links `popcorn_amd/libpopcorn_amd.so`.
The library is always rebuilt: the call is the "does it build" check. Asked
to (`python -m popcorn_amd.build` and `__graft_entry__.build()` ask), it then
writes the `popcorn-amd` distribution metadata beside the package in a source
tree (setup.py's `egg_info`, as an editable install would), so Popcorn's
version gate sees the backend when the tree itself is on `sys.path`. setup.py's
own build step does not ask: an install writes its metadata itself.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libpopcorn_amd.so"
INCLUDE = PACKAGE.parent / "include"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # The kernels reproduce torch's rounding sequence (separate products and
    # sums); contraction would fuse them. FMAs are written out where wanted.
    "-ffp-contract=off",
    # Packed fp32 VALU ops are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the popcorn_amd kernels need ROCm's hipcc")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(source: Path) -> Path:
    obj = BUILD / (source.stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False, write_metadata: bool = False) -> Path:
    """Compile all kernels and link the shared library; returns its path.

    With `write_metadata`, also write the distribution metadata into the source tree (see
    `write_source_metadata`).
    """
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")), 16) or 1
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", file=sys.stderr)
    if write_metadata:
        write_source_metadata()
    return LIBRARY


def write_source_metadata() -> None:
    """Run setup.py's `egg_info` in a source tree (no-op for an installed package, which has its metadata)."""
    setup_py = PACKAGE.parent / "setup.py"
    if not setup_py.exists():
        return
    proc = subprocess.run([sys.executable, str(setup_py), "-q", "egg_info", "--egg-base", str(PACKAGE.parent)],
                          cwd=PACKAGE.parent, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"writing the popcorn-amd metadata failed:\n{proc.stderr}")


if __name__ == "__main__":
    build(verbose=True, write_metadata=True)
