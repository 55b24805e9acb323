"""The drop-in ops captured in a HIP graph: every replay matches the eager call bit for bit.

Each case captures one call (forward, or forward plus the gradients of every input) with
torch.cuda.graph, after warm-up calls on a side stream as torch requires. It then writes fresh
seeded data into the captured inputs three times, replays, synchronises, runs the same call
eagerly on the same inputs and compares every output with torch.equal. The kernels are
deterministic and take the same launch shapes either way, so a replay that read stale memory,
lost a launch or wrote outside its outputs shows up as a mismatch. No entry point issues a memset,
allocation or synchronisation of its own: scratch comes from torch's allocator (the graph's pool
while capturing) and every launch goes to torch's current stream.

`attn_varlen` is left out: like Popcorn's reference it reads `cu_seqlens` on the host, which
capture does not allow.
"""

import pytest
import torch

from popcorn_amd import impls

# leaves made on the default stream and differentiated under capture on torch's side stream
pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")]
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _refill(tensors, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    with torch.no_grad():
        for t in tensors:
            t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(t.dtype))


def _replays_match_eager(call, inputs, what):
    """Capture `call(*inputs)` (a tuple of tensors), replay it on fresh inputs, compare with eager."""
    _refill(inputs, 10)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            call(*inputs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = call(*inputs)
    for seed in (11, 12, 13):
        _refill(inputs, seed)
        graph.replay()
        torch.cuda.synchronize()
        eager = call(*inputs)
        torch.cuda.synchronize()
        assert len(captured) == len(eager)
        for i, (got, want) in enumerate(zip(captured, eager)):
            assert got.shape == want.shape and got.dtype == want.dtype, f"{what} output {i}"
            assert torch.equal(got, want), f"{what} output {i}, replay with seed {seed}"


def _fwd_bwd(fn, leaves, rest, cotangents):
    """fn's outputs, then the gradients of `leaves` for cotangents cast to the outputs' dtypes."""
    outs = fn(*leaves, *rest)
    outs = outs if isinstance(outs, tuple) else (outs,)
    grads = torch.autograd.grad(outs, leaves, [c.to(o.dtype) for c, o in zip(cotangents, outs)])
    return (*outs, *grads)


def _leaves(*shapes_dtypes):
    return [torch.empty(shape, dtype=dtype, device=DEV).requires_grad_() for shape, dtype in shapes_dtypes]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_rms_norm_graph(dtype):
    x, w = _leaves(((512, 2048), dtype), ((2048,), dtype))
    gy = torch.empty(512, 2048, dtype=dtype, device=DEV)

    def call(x, w, gy):
        return _fwd_bwd(lambda a, b: impls.rms_norm(a, b, None, 1e-6), [x, w], [], [gy])

    _replays_match_eager(call, [x, w, gy], f"rms_norm {dtype}")


def test_rms_norm_forward_only_graph():
    x = torch.empty(4096, 4096, device=DEV)
    w = torch.empty(4096, device=DEV)
    _replays_match_eager(lambda x, w: (impls.rms_norm(x, w, None, 1e-6),), [x, w], "rms_norm forward")


def test_add_rms_norm_graph():
    x, r, w = _leaves(((300, 1024), torch.bfloat16), ((300, 1024), torch.bfloat16), ((1024,), torch.float32))
    gy = torch.empty(300, 1024, dtype=torch.float32, device=DEV)
    gs = torch.empty(300, 1024, dtype=torch.bfloat16, device=DEV)

    def call(x, r, w, gy, gs):
        return _fwd_bwd(lambda a, b, c: impls.add_rms_norm(a, b, c, 1e-6, 1.0), [x, r, w], [], [gy, gs])

    _replays_match_eager(call, [x, r, w, gy, gs], "add_rms_norm")


def test_swiglu_graph():
    a, b = _leaves(((1000, 1408), torch.bfloat16), ((1000, 1408), torch.bfloat16))
    gy = torch.empty(1000, 1408, dtype=torch.bfloat16, device=DEV)
    _replays_match_eager(lambda a, b, gy: _fwd_bwd(impls.swiglu, [a, b], [], [gy]), [a, b, gy], "swiglu")


@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "gptj"])
def test_rotary_graph(interleaved):
    (x,) = _leaves(((2, 256, 8, 128), torch.bfloat16))
    cos = torch.empty(256, 64, device=DEV)
    sin = torch.empty(256, 64, device=DEV)
    gy = torch.empty(2, 256, 8, 128, dtype=torch.float32, device=DEV)

    def call(x, cos, sin, gy):
        return _fwd_bwd(lambda t: impls.rotary_embedding(t, cos, sin, interleaved), [x], [], [gy])

    _replays_match_eager(call, [x, cos, sin, gy], f"rotary interleaved={interleaved}")


def test_rope_graph():
    q, k = _leaves(((2, 8, 256, 128), torch.bfloat16), ((2, 2, 256, 128), torch.bfloat16))
    cos = torch.empty(1, 256, 128, device=DEV)
    sin = torch.empty(1, 256, 128, device=DEV)
    gq = torch.empty(2, 8, 256, 128, device=DEV)
    gk = torch.empty(2, 2, 256, 128, device=DEV)

    def call(q, k, cos, sin, gq, gk):
        return _fwd_bwd(lambda a, b: impls.rope(a, b, cos, sin), [q, k], [], [gq, gk])

    _replays_match_eager(call, [q, k, cos, sin, gq, gk], "rope")


def test_qk_norm_rope_graph():
    q, k, qw, kw = _leaves(((2, 8, 128, 128), torch.bfloat16), ((2, 2, 128, 128), torch.bfloat16),
                           ((128,), torch.bfloat16), ((128,), torch.bfloat16))
    cos = torch.empty(1, 128, 128, dtype=torch.bfloat16, device=DEV)
    sin = torch.empty(1, 128, 128, dtype=torch.bfloat16, device=DEV)
    gq = torch.empty(2, 8, 128, 128, dtype=torch.bfloat16, device=DEV)
    gk = torch.empty(2, 2, 128, 128, dtype=torch.bfloat16, device=DEV)

    def call(q, k, qw, kw, cos, sin, gq, gk):
        return _fwd_bwd(lambda a, b, c, d: impls.qk_norm_rope(a, b, c, d, cos, sin, 1e-6), [q, k, qw, kw], [],
                        [gq, gk])

    _replays_match_eager(call, [q, k, qw, kw, cos, sin, gq, gk], "qk_norm_rope")


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attn_graph(causal, d):
    q, k, v = _leaves(((2, 384, 8, d), torch.bfloat16), ((2, 384, 2, d), torch.bfloat16),
                      ((2, 384, 2, d), torch.bfloat16))
    go = torch.empty(2, 384, 8, d, dtype=torch.bfloat16, device=DEV)

    def call(q, k, v, go):
        return _fwd_bwd(lambda a, b, c: impls.attn(a, b, c, causal), [q, k, v], [], [go])

    _replays_match_eager(call, [q, k, v, go], f"attn causal={causal} d={d}")


def test_attn_forward_graph_at_c5_shape():
    """The C5 forward (B=4, S=8192, 32 q heads over 8 kv heads), no gradient."""
    q = torch.empty(4, 8192, 32, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(4, 8192, 8, 128, dtype=torch.bfloat16, device=DEV)
    v = torch.empty(4, 8192, 8, 128, dtype=torch.bfloat16, device=DEV)
    _replays_match_eager(lambda q, k, v: (impls.attn(q, k, v, True),), [q, k, v], "attn C5 forward")
