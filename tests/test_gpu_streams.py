"""Calls that overlap: on two streams at once, and from two host threads.

The entry points keep no state between calls except read-only tables filled once per process
(occupancy queries, the CU count), and every scratch buffer is the caller's workspace (torch's
allocator in `impls`, which keeps each block on its stream). So two calls running at the same time
on different streams, or issued from different host threads, must give exactly what each gives
alone. Each case runs an op forward and backward on two input sets alone on the default stream,
then both at once, and compares bit for bit.
"""

import threading

import pytest
import torch

from popcorn_amd import impls

# leaves made on the default stream and differentiated on side streams
pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore:The AccumulateGrad node's stream")]
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def _inputs(specs, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return [torch.randn(shape, generator=g, device=DEV).to(dtype).requires_grad_(grad) for shape, dtype, grad in specs]


def _fwd_bwd(fn, leaves, cot_seed):
    outs = fn(*leaves)
    outs = outs if isinstance(outs, tuple) else (outs,)
    g = torch.Generator(device=DEV).manual_seed(cot_seed)
    cots = [torch.randn(o.shape, generator=g, device=DEV).to(o.dtype) for o in outs]
    grads = torch.autograd.grad(outs, [t for t in leaves if t.requires_grad], cots)
    return [o.detach() for o in outs] + list(grads)


BF = torch.bfloat16
CASES = {
    "rms_norm": (lambda x, w: impls.rms_norm(x, w, None, 1e-6), [((4096, 4096), BF, True), ((4096,), BF, True)]),
    "add_rms_norm": (lambda x, r, w: impls.add_rms_norm(x, r, w, 1e-6, 0.0),
                     [((2048, 4096), BF, True), ((2048, 4096), BF, True), ((4096,), torch.float32, True)]),
    "swiglu": (impls.swiglu, [((4096, 2048), BF, True), ((4096, 2048), BF, True)]),
    "qk_norm_rope": (lambda q, k, qw, kw, c, s: impls.qk_norm_rope(q, k, qw, kw, c, s, 1e-6),
                     [((2, 16, 512, 128), BF, True), ((2, 4, 512, 128), BF, True), ((128,), BF, True),
                      ((128,), BF, True), ((1, 512, 128), BF, False), ((1, 512, 128), BF, False)]),
    "attn": (lambda q, k, v: impls.attn(q, k, v, True),
             [((2, 1024, 16, 128), BF, True), ((2, 1024, 4, 128), BF, True), ((2, 1024, 4, 128), BF, True)]),
}


@pytest.mark.parametrize("name", list(CASES))
def test_two_streams_at_once_match_each_call_alone(name):
    fn, specs = CASES[name]
    a, b = _inputs(specs, 1), _inputs(specs, 2)
    want_a, want_b = _fwd_bwd(fn, a, 11), _fwd_bwd(fn, b, 12)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        s1.wait_stream(torch.cuda.current_stream())
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s1):
            got_a = _fwd_bwd(fn, a, 11)
        with torch.cuda.stream(s2):
            got_b = _fwd_bwd(fn, b, 12)
        torch.cuda.synchronize()
        for i, (x, y) in enumerate(zip(got_a + got_b, want_a + want_b)):
            assert torch.equal(x, y), f"{name}: output {i} differs when the two calls overlap"


@pytest.mark.parametrize("name", ["rms_norm", "attn"])
def test_two_host_threads_match_each_call_alone(name):
    """Each thread runs its call on its own stream; the library's once-per-process tables and the
    per-thread error text are shared or kept apart as the header says."""
    fn, specs = CASES[name]
    sets = [_inputs(specs, 3), _inputs(specs, 4)]
    want = [_fwd_bwd(fn, s, 20 + i) for i, s in enumerate(sets)]
    torch.cuda.synchronize()
    got, errors = [None, None], []

    def work(i):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                outs = [_fwd_bwd(fn, sets[i], 20 + i) for _ in range(3)]
            stream.synchronize()
            got[i] = outs
        except Exception as e:  # reported below, on the test's thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for i in range(2):
        for rep in got[i]:
            for j, (x, y) in enumerate(zip(rep, want[i])):
                assert torch.equal(x, y), f"{name}: thread {i} output {j} differs"
