"""pk_probe_mfma, the matrix-core rate probe the bench uses for the power-capped ceiling.

It runs one wave per SIMD of back-to-back bf16 32x32x16 products (32 cycles of
a SIMD's matrix core each), so the cycles it reports per product cannot fall
below 32, and with nothing else competing for the SIMD they stay close to it;
the real-time ticks give the clock, which lies within the board's range.
"""

from __future__ import annotations

import pytest
import torch

from popcorn_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return _lib.load()


@pytest.mark.parametrize("softmax", [0, 1])
def test_probe_reports_product_rate_and_clock(lib, softmax):
    blocks = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 256
    out = torch.zeros(2 * 4 * blocks, dtype=torch.int64, device=DEV)
    print(f"[probe] softmax={softmax} blocks={blocks} iters={iters}", flush=True)
    _lib.check(lib.pk_probe_mfma(softmax, iters, blocks, out.data_ptr(), _lib.stream_handle(torch.device(DEV))), lib)
    torch.cuda.synchronize()
    cycles, ticks = out.view(-1, 2).double().cpu().unbind(1)
    assert bool((cycles > 0).all()) and bool((ticks > 0).all()), "a wave reported no time"
    per_product = float(cycles.mean()) / (iters * 8)
    assert 31.5 <= per_product <= 48.0, per_product
    clock_mhz = float((cycles / ticks).mean()) * 100.0
    assert 300.0 <= clock_mhz <= 2600.0, clock_mhz


def test_probe_refuses_bad_arguments(lib):
    out = torch.zeros(8, dtype=torch.int64, device=DEV)
    stream = _lib.stream_handle(torch.device(DEV))
    assert lib.pk_probe_mfma(0, 0, 1, out.data_ptr(), stream) == _lib.ERR_INVALID
    assert lib.pk_probe_mfma(0, 4, 0, out.data_ptr(), stream) == _lib.ERR_INVALID
    assert lib.pk_probe_mfma(0, 4, 1, None, stream) == _lib.ERR_INVALID
    assert "null pointer" in lib.pk_last_error().decode()


@pytest.mark.parametrize("reads", [1, 2])
def test_stream_probe_copies_or_combines(lib, reads):
    nbytes = (3 << 20) + 48  # not a whole number of blocks: the last block is partial
    gen = torch.Generator(device=DEV).manual_seed(3)
    a = torch.empty(nbytes, dtype=torch.uint8, device=DEV).random_(generator=gen)
    b = torch.empty(nbytes, dtype=torch.uint8, device=DEV).random_(generator=gen)
    y = torch.full((nbytes + 16,), 0x5A, dtype=torch.uint8, device=DEV)  # one guard vector past the end
    print(f"[probe] stream reads={reads} bytes={nbytes}", flush=True)
    _lib.check(lib.pk_probe_stream(a.data_ptr(), b.data_ptr() if reads == 2 else None, y.data_ptr(), nbytes, reads,
                                   _lib.stream_handle(torch.device(DEV))), lib)
    torch.cuda.synchronize()
    want = a if reads == 1 else torch.bitwise_xor(a, b)
    assert torch.equal(y[:nbytes], want)
    assert bool((y[nbytes:] == 0x5A).all()), "the probe wrote past the end"


def test_stream_probe_refuses_bad_arguments(lib):
    a = torch.zeros(64, dtype=torch.uint8, device=DEV)
    stream = _lib.stream_handle(torch.device(DEV))
    assert lib.pk_probe_stream(a.data_ptr(), None, a.data_ptr(), 40, 1, stream) == _lib.ERR_INVALID  # not 16-byte units
    assert lib.pk_probe_stream(a.data_ptr(), None, a.data_ptr(), 32, 3, stream) == _lib.ERR_INVALID
    assert lib.pk_probe_stream(a.data_ptr(), None, a.data_ptr(), 32, 2, stream) == _lib.ERR_INVALID  # b missing
    assert lib.pk_probe_stream(a.data_ptr() + 8, None, a.data_ptr(), 32, 1, stream) == _lib.ERR_INVALID
    assert lib.pk_probe_stream(a.data_ptr(), None, a.data_ptr(), 0, 1, stream) == _lib.OK
