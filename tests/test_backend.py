"""Registration of the MI355X backend through Popcorn's API (compat counterpart), on the CPU."""

from __future__ import annotations

import importlib.metadata

import torch

import popcorn_amd
from popcorn_amd import backend, compat
from popcorn_amd.compat.backends import installed_version, unavailable_reason
from popcorn_amd.compat.ops import describe


def test_distribution_metadata_resolves_at_the_package_version():
    assert importlib.metadata.version(backend.DISTRIBUTION) == popcorn_amd.__version__


def test_register_declares_gate_and_adds_one_backend_per_op():
    backend.register(compat)
    backend.register(compat)  # idempotent
    assert unavailable_reason(backend.BACKEND) is None
    assert installed_version(backend.BACKEND) == popcorn_amd.__version__
    for name, source, _, forward_only in backend.REGISTRATIONS:
        op = compat.KERNELS[name]
        assert op.available_backends() == (backend.BACKEND, "torch")
        impl = op[backend.BACKEND]
        assert impl.source == source and impl.forward_only == forward_only
        assert impl.fingerprint is not None  # covers the module and its csrc/ kernels


def test_sources_conform_to_reference_signatures():
    backend.register(compat)
    for name, *_ in backend.REGISTRATIONS:
        impl = compat.KERNELS[name][backend.BACKEND]
        impl._ready = False
        impl._prepare()  # resolves the source and checks its leading parameters
        assert impl.source_fn is not None


def test_cpu_tensors_are_declined_and_torch_serves():
    backend.register(compat)
    x, w = torch.randn(4, 8), torch.ones(8)
    op = compat.KERNELS["rms_norm"]
    assert op[backend.BACKEND].refusal(describe(op, (x, w), {}))
    torch.testing.assert_close(op(x, w), compat.references.rms_norm(x, w))
