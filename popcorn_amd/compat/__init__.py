"""A self-contained counterpart of Popcorn's registration / validation / selection surface.

Popcorn itself (tilde-research/popcorn) does not run in this environment, so
this package restates the parts of it that make a backend a drop-in: op
objects and `register` (dispatcher), backend declarations and the `kernel`
proxy (sources), the float64-truth comparison and record production
(harness), the report store (store) and the record-driven selector
(selection). `popcorn_amd.backend.register(popcorn)` works against this
package or against the real `popcorn` module alike.
"""

from popcorn_amd.compat.dispatcher import KERNELS, Dispatcher, Implementation, register_kernel
from popcorn_amd.compat.errors import BackendUnavailableError, BackendVersionError, DispatchError, PopcornError
from popcorn_amd.compat.harness import compare_inputs, report
from popcorn_amd.compat.records import Case, Record
from popcorn_amd.compat.selection import Range
from popcorn_amd.compat.shapes import BFloat16, Float, Float16, Float32, Float64, Int32
from popcorn_amd.compat.sources import declare_backend, kernel
from popcorn_amd.compat import harness, store  # noqa: E402
from popcorn_amd.compat import kernels  # noqa: E402  registers the four ops

__all__ = [
    "KERNELS", "Dispatcher", "Implementation", "register_kernel", "BackendUnavailableError", "BackendVersionError",
    "DispatchError", "PopcornError", "compare_inputs", "report", "Case", "Record", "Range", "BFloat16", "Float",
    "Float16", "Float32", "Float64", "Int32", "declare_backend", "kernel", "kernels", "harness", "store",
]
