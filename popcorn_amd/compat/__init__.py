"""A self-contained counterpart of Popcorn's registration / validation / selection surface.

Popcorn itself (tilde-research/popcorn) does not run in this environment, so
this package provides the parts of it that make a backend a drop-in, under
Popcorn's public names: ops and `register` (ops), backend declarations, the
version gate and the `kernel` proxy (backends), grading against a float64
truth and recording rows (harness), report files (store) and the
evidence-driven choice of implementation (selection).
`popcorn_amd.backend.register(popcorn)` works against this package or against
the real `popcorn` module alike.
"""

from popcorn_amd.compat.backends import declare_backend, kernel
from popcorn_amd.compat.errors import BackendUnavailableError, BackendVersionError, DispatchError, PopcornError
from popcorn_amd.compat.harness import compare, compare_inputs, report
from popcorn_amd.compat.ops import KERNELS, Dispatcher, Implementation, register_kernel
from popcorn_amd.compat.records import Case, Record
from popcorn_amd.compat.selection import Policy, Range
from popcorn_amd.compat.shapes import BFloat16, Float, Float16, Float32, Float64, Int32
from popcorn_amd.compat import harness, references, store  # noqa: E402
from popcorn_amd.compat import kernels  # noqa: E402  registers the transformer-block ops

__all__ = [
    "KERNELS", "Dispatcher", "Implementation", "register_kernel", "BackendUnavailableError", "BackendVersionError",
    "DispatchError", "PopcornError", "compare", "compare_inputs", "report", "Case", "Record", "Policy", "Range",
    "BFloat16", "Float", "Float16", "Float32", "Float64", "Int32", "declare_backend", "kernel", "kernels", "harness",
    "references", "store",
]
