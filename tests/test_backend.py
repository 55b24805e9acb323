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


def test_predicates_cover_the_mixed_dtype_pairs(monkeypatch):
    """Mixed pairs the kernels implement are accepted; the rest are declined (placement aside, on meta tensors)."""
    monkeypatch.setattr(backend, "_on_hip", lambda *tensors: True)
    bf, f16, f32 = torch.bfloat16, torch.float16, torch.float32

    def t(*shape, dtype):
        return torch.empty(shape, dtype=dtype, device="meta")

    x = t(4, 64, dtype=bf)
    assert backend.rms_norm_supported(x, t(64, dtype=f32), None, 1e-6)
    assert backend.rms_norm_supported(x, t(64, dtype=f32), t(64, dtype=f32), 1e-6)
    assert not backend.rms_norm_supported(x, t(64, dtype=f32), t(64, dtype=bf), 1e-6)
    assert not backend.rms_norm_supported(t(4, 64, dtype=f32), t(64, dtype=bf), None, 1e-6)
    assert not backend.rms_norm_supported(x, t(64, dtype=f16), None, 1e-6)
    assert backend.add_rms_norm_supported(x, x, t(64, dtype=f32), 1e-6, 0.0)
    assert not backend.add_rms_norm_supported(x, t(4, 64, dtype=f32), t(64, dtype=f32), 1e-6, 0.0)
    assert not backend.add_rms_norm_supported(t(4, 64, dtype=f32), t(4, 64, dtype=f32), t(64, dtype=bf), 1e-6, 0.0)

    q, k = t(2, 4, 8, 64, dtype=bf), t(2, 2, 8, 64, dtype=bf)
    for table in (bf, f16, f32):
        cs = t(1, 8, 64, dtype=table)
        assert backend.rope_supported(q, k, cs, cs)
        w = t(64, dtype=bf)
        assert backend.qk_norm_rope_supported(q, k, w, w, cs, cs, 1e-6)
    assert not backend.rope_supported(q, t(2, 2, 8, 64, dtype=f16), t(1, 8, 64, dtype=f32), t(1, 8, 64, dtype=f32))
    assert not backend.rope_supported(q, k, t(1, 8, 64, dtype=f32), t(1, 8, 64, dtype=bf))
    w32, c32 = t(64, dtype=f32), t(1, 8, 64, dtype=f32)
    assert backend.qk_norm_rope_supported(q, k, w32, w32, c32, c32, 1e-6)  # autocast's fp32 norm weights
    assert not backend.qk_norm_rope_supported(q, k, w32, t(64, dtype=bf), c32, c32, 1e-6)
    q32, k32 = t(2, 4, 8, 64, dtype=f32), t(2, 2, 8, 64, dtype=f32)
    assert not backend.qk_norm_rope_supported(q32, k32, t(64, dtype=bf), t(64, dtype=bf), c32, c32, 1e-6)


def test_attention_predicates_cover_the_head_dims(monkeypatch):
    """Forward and backward at every head_dim that is a multiple of 8 up to 256 (Popcorn's grid,
    core/dims.py:74); other widths declined."""
    monkeypatch.setattr(backend, "_on_hip", lambda *tensors: True)

    def qkv(d, grad=False):
        q = torch.empty(1, 16, 8, d, dtype=torch.bfloat16, device="meta")
        k = torch.empty(1, 16, 2, d, dtype=torch.bfloat16, device="meta")
        return [t.requires_grad_(grad) for t in (q, k, k.clone())]

    for d in (16, 32, 48, 64, 80, 96, 128, 192, 256):
        assert backend.attn_supported(*qkv(d), True, None)
        assert backend.attn_supported(*qkv(d, grad=True), True, None)
    for d in (8 * 33, 72 + 4, 100, 4):
        assert not backend.attn_supported(*qkv(d), True, None)
    q, k, v = (t[0] for t in qkv(96))
    assert backend.attn_varlen_supported(q, k, v, torch.zeros(2, dtype=torch.int32), True, None)


def test_attention_predicates_take_fp32(monkeypatch):
    """fp32 attention runs the fp32 kernels, head_dim up to 256, with or without gradients to record."""
    monkeypatch.setattr(backend, "_on_hip", lambda *tensors: True)

    def qkv(d, grad=False):
        q = torch.empty(1, 16, 8, d, dtype=torch.float32, device="meta")
        k = torch.empty(1, 16, 2, d, dtype=torch.float32, device="meta")
        return [t.requires_grad_(grad) for t in (q, k, k.clone())]

    for d in (16, 32, 64, 96, 128, 192, 256):
        assert backend.attn_supported(*qkv(d), True, None)
        assert backend.attn_supported(*qkv(d, grad=True), True, None)
        q, k, v = (t[0] for t in qkv(d, grad=True))
        assert backend.attn_varlen_supported(q, k, v, torch.zeros(2, dtype=torch.int32), False, None)
    for d in (264, 100, 4):
        assert not backend.attn_supported(*qkv(d), True, None)
        assert not backend.attn_supported(*qkv(d, grad=True), True, None)


def test_attention_with_gradients_past_the_kernels_is_refused_before_any_work():
    from popcorn_amd import impls

    for q in (torch.randn(1, 4, 2, 264, requires_grad=True), torch.randn(1, 4, 2, 264).bfloat16().requires_grad_()):
        what = "head_dim=264 is past the attention kernels' 256"
        # CPU tensors: the refusal comes first
        for call in (lambda: impls.attn(q, q, q, True),
                     lambda: impls.attn_varlen(q[0], q[0], q[0], torch.tensor([0, 4]))):
            try:
                call()
            except ValueError as e:
                assert what in str(e), str(e)
            else:
                raise AssertionError(f"{what} with gradients was not refused")
