"""Benchmark of the MI355X transformer-block kernels on one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2] [--head-dim D] [--power]
                    [--no-cpu] [--no-others]

A step is one pass of a workload's drop-in call (the `popcorn_amd.impls`
function Popcorn dispatches to) over one batch of synthetic input already
resident in HBM. The default workload is BASELINE config 2 (SwiGLU forward,
bf16, a, b [16384, 14336]); `--workload` picks any of c1..c5, `add_rmsnorm`
(residual add + RMSNorm at C4's shape), `rope` and `qk_norm_rope` (forward +
backward), `attn_bwd` (attention forward + backward at C5's shape), `c5_f32`
and `attn_bwd_f32` (the same two in fp32), the ceilings `mfma_ceiling`,
`mfma_ceiling_softmax` (matrix-core rate under the power limit) and
`stream_<reads>r_<MiB>m` (streaming rate at a
pattern and size), or `copy`, a plain device copy of known size used to
calibrate HBM byte counters. `--head-dim` sets the attention workloads' head_dim;
`--power` adds an `amd-smi` sample of socket power and clocks during a 6 s run.

Rank 0 prints ONE JSON line. `value` is the workload's achieved algorithmic
throughput (TB/s of HBM bytes for c1-c4, TFLOP/s for c5). `roofline` is the
dominant kernel's figure, timed with HIP events on the stream it is launched
on (torch's current stream). `torch_gpu` times Popcorn's PyTorch reference
(the `torch` implementation its dispatcher always holds, restated in
popcorn_amd.compat.references) on the same GPU and inputs: the competitor the
record-driven selector compares against. `cpu_baseline` times that reference
on the host's cores, on the full workload where it takes seconds and on a
stated sample otherwise. `others` holds the same figures for the remaining
configs, and `roofline_fractions` the dominant kernels' fractions of peak for
C1-C5. In the default run each `roofline` also carries `ceiling`: the probe of
the same pattern (reads per write and bytes, or the matrix-core rate with the
attention forward's vector work) timed on the same box after every workload,
and the kernel's rate as a share of it.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from dataclasses import dataclass, field
from typing import Callable

import torch

HBM_PEAK_TBS = 8.0  # MI355X HBM3E, TB/s
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA, TFLOP/s
METRIC = "achieved HBM TB/s (norm/rope/swiglu) + attn-fwd bf16 TFLOP/s, % of peak"
# A workload small enough to sit in the 256 MiB MALL (Infinity Cache) rotates through copies of its
# inputs until the inputs alone span this many bytes, twice the MALL, so each launch reads from HBM.
FLUSH_BYTES = 512 << 20

# HBM bytes per launch of each workload's dominant kernel, from rocprofv3
# FETCH_SIZE / WRITE_SIZE runs scaled by the same counters' reading for a plain
# device copy of known size (FETCH_SIZE reads half the bytes a copy moves,
# WRITE_SIZE all of them): 2 * FETCH_SIZE + WRITE_SIZE, in bytes
# (profiles/hbm_traffic.md). Keyed by workload; re-measure after changing a
# kernel's traffic.
MEASURED_TRAFFIC: dict[str, int | None] = {
    "c1": 134_494_510,
    "c2": 1_409_309_330,
    "c3": 539_013_266,
    "c4": 3_240_305_664,
    "c5": 816_589_355,
    "add_rmsnorm": 4_314_051_694,
    "rope": 337_726_126,
    "qk_norm_rope": 510_771_483,
    "attn_bwd": 6_167_044_055,  # the dq and dk/dv kernels of one pk_attn_bwd call
    "copy": 1_073_766_308,
}


@dataclass
class Workload:
    name: str
    description: str
    dtype: str
    unit: str  # "TB/s" or "TFLOP/s"
    work: float  # algorithmic bytes (TB/s units) or FLOPs per step
    step: Callable[[int], None]  # step(i): one pass of the drop-in call on input copy i
    kernel: str  # dominant kernel's name (as rocprofv3 reports it, prefix)
    kernel_work: float  # algorithmic bytes / FLOPs of one launch of that kernel
    launch: Callable[[int], None]  # one call of the C entry point that runs the dominant kernel, on input copy i
    config: dict = field(default_factory=dict)
    cpu: Callable[[], tuple[float, str]] | None = None  # -> (throughput in unit, sample description)
    torch_step: Callable[[int], None] | None = None  # Popcorn's torch reference on the GPU, same inputs
    # every kernel one `launch` runs, when it is more than the dominant one (the launch's time then
    # covers them all, so the achieved rate of the dominant kernel is understated, never overstated)
    launch_kernels: tuple[str, ...] = ()
    # figures the workload reports beside its rate, read after the timed calls
    extra: Callable[[], dict] | None = None
    peak: float | None = None  # the dominant kernel's peak in `unit` when it is not bf16 MFMA or HBM


def _copies(nbytes: int) -> int:
    """Copies to rotate of inputs of `nbytes` per launch so that one sweep over them spans FLUSH_BYTES."""
    return max(1, math.ceil(FLUSH_BYTES / max(nbytes, 1)))


def _randn(shape, dtype, gen, dev):
    return torch.randn(shape, generator=gen, device=dev, dtype=torch.float32).to(dtype)


def make_workload(name: str, dev: torch.device, head_dim: int = 128) -> Workload:
    from popcorn_amd import _lib, impls
    from popcorn_amd.compat import references as R

    gen = torch.Generator(device=dev).manual_seed(0)
    lib = _lib.load()
    stream = lambda: _lib.stream_handle(dev)  # noqa: E731

    if name == "c1":
        rows, cols = 4096, 4096
        nbytes = rows * cols * 4 * 2 + cols * 4
        # 8 copies of x (512 MiB of x alone, twice the MALL) and of y, so every launch reads its x
        # from HBM and writes a y no recent launch wrote
        n = _copies(rows * cols * 4)
        xs = [_randn((rows, cols), torch.float32, gen, dev) for _ in range(n)]
        w = 1 + 0.1 * _randn((cols,), torch.float32, gen, dev)
        ys = [torch.empty_like(xs[0]) for _ in range(n)]
        held = [None] * n  # the drop-in call's outputs, held so that they rotate like ys

        def step(i):
            held[i % n] = None
            held[i % n] = impls.rms_norm(xs[i % n], w, None, 1e-6)

        def launch(i):
            _lib.check(lib.pk_rmsnorm_fwd(xs[i % n].data_ptr(), w.data_ptr(), None, ys[i % n].data_ptr(), None, rows,
                                          cols, 1e-6, _lib.F32, _lib.F32, stream()))

        def cpu():
            xc = torch.randn(rows, cols)
            wc = 1 + 0.1 * torch.randn(cols)
            t, reps = _time_cpu(lambda: R.rms_norm(xc, wc, None, 1e-6))
            return nbytes / t / 1e12, f"full C1 x [{rows}, {cols}] fp32, median of {reps} reps"

        def torch_step(i):
            R.rms_norm(xs[i % n], w, None, 1e-6)

        return Workload("c1", "RMSNorm forward fp32 x [4096, 4096]", "f32", "TB/s", nbytes, step,
                        "rmsnorm_fwd_grid", nbytes, launch,
                        {"rows": rows, "cols": cols, "eps": 1e-6, "dtype": "fp32"}, cpu, torch_step)

    if name == "c2":
        rows, cols = 16384, 14336
        numel = rows * cols
        nbytes = 3 * numel * 2
        a = _randn((rows, cols), torch.bfloat16, gen, dev)
        b = _randn((rows, cols), torch.bfloat16, gen, dev)
        y = torch.empty_like(a)

        def step(i):
            impls.swiglu(a, b)

        def launch(i):
            _lib.check(lib.pk_swiglu_fwd(a.data_ptr(), b.data_ptr(), y.data_ptr(), numel, _lib.BF16, stream()))

        def cpu():
            ac = torch.randn(rows, cols).bfloat16()
            bc = torch.randn(rows, cols).bfloat16()
            t, reps = _time_cpu(lambda: R.swiglu(ac, bc))
            return nbytes / t / 1e12, f"full C2 a, b [{rows}, {cols}] bf16, median of {reps} reps"

        def torch_step(i):
            R.swiglu(a, b)

        return Workload("c2", "SwiGLU forward bf16 a, b [16384, 14336]", "bf16", "TB/s", nbytes, step,
                        "swiglu_fwd_vec", nbytes, launch, {"rows": rows, "cols": cols, "dtype": "bf16"}, cpu,
                        torch_step)

    if name == "c3":
        B, S, HQ, HKV, D, half = 8, 4096, 32, 8, 128, 64
        q = _randn((B, S, HQ, D), torch.bfloat16, gen, dev)
        k = _randn((B, S, HKV, D), torch.bfloat16, gen, dev)
        pos = torch.arange(S, dtype=torch.float64)[:, None]
        inv_freq = 500000.0 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
        ang = pos * inv_freq[None, :]
        cos, sin = ang.cos().float().to(dev), ang.sin().float().to(dev)
        qb, kb = q.numel() * 2, k.numel() * 2
        table = 2 * S * half * 4
        nbytes = 2 * qb + 2 * kb + 2 * table
        yq, yk = torch.empty_like(q), torch.empty_like(k)

        def step(i):
            impls.rotary_embedding(q, cos, sin)
            impls.rotary_embedding(k, cos, sin)

        def rot(x, y):
            strides = (_lib._i64 * 6)(x.stride(0), x.stride(1), x.stride(2), y.stride(0), y.stride(1), y.stride(2))
            _lib.check(lib.pk_rotary(x.data_ptr(), cos.data_ptr(), sin.data_ptr(), y.data_ptr(), strides, B, S,
                                     x.shape[2], D, half, _lib.BF16, _lib.F32, 0, 0, stream()))

        def launch(i):
            rot(q, yq)

        def cpu():
            qc = torch.randn(B, S, HQ, D).bfloat16()
            kc = torch.randn(B, S, HKV, D).bfloat16()
            cc, sc = cos.cpu(), sin.cpu()
            t, reps = _time_cpu(lambda: (R.rotary_embedding(qc, cc, sc), R.rotary_embedding(kc, cc, sc)))
            return nbytes / t / 1e12, f"full C3 (q and k calls, fp32 tables), median of {reps} reps"

        def torch_step(i):
            R.rotary_embedding(q, cos, sin)
            R.rotary_embedding(k, cos, sin)

        return Workload("c3", "Rotary NeoX bf16 q [8,4096,32,128] + k [8,4096,8,128], fp32 cos/sin [4096,64]",
                        "bf16", "TB/s", nbytes, step, "rotary_kernel", 2 * qb + table, launch,
                        {"batch": B, "seq": S, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "theta": 500000.0,
                         "dtype": "bf16", "tables": "fp32"}, cpu, torch_step)

    if name == "rope":
        # not a BASELINE config: paired q/k rope at the shape of the notebook's fused qk-norm+rope example
        B, HQ, HKV, S, D = 4, 32, 8, 4096, 128
        inv_freq = 500000.0 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
        ang = torch.arange(S, dtype=torch.float64)[:, None] * inv_freq[None, :]
        ang = torch.cat([ang, ang], -1)[None]
        cos, sin = ang.cos().bfloat16().to(dev), ang.sin().bfloat16().to(dev)
        qb, kb = B * HQ * S * D * 2, B * HKV * S * D * 2
        launch_bytes = 2 * (qb + kb) + 2 * S * D * 2
        n = _copies(launch_bytes)
        qs = [_randn((B, HQ, S, D), torch.bfloat16, gen, dev) for _ in range(n)]
        ks = [_randn((B, HKV, S, D), torch.bfloat16, gen, dev) for _ in range(n)]
        gq, gk = _randn((B, HQ, S, D), torch.bfloat16, gen, dev), _randn((B, HKV, S, D), torch.bfloat16, gen, dev)
        leaves = [(q.requires_grad_(), k.requires_grad_()) for q, k in zip(qs, ks)]
        yq, yk = torch.empty_like(qs[0]), torch.empty_like(ks[0])
        strides = (_lib._i64 * 12)(*(x for t in (qs[0], ks[0], yq, yk) for x in t.stride()[:3]))

        def step(i):
            q, k = leaves[i % n]
            oq, ok = impls.rope(q, k, cos, sin)
            torch.autograd.grad((oq, ok), (q, k), (gq, gk))

        def launch(i):
            q, k = qs[i % n], ks[i % n]
            _lib.check(lib.pk_rope(q.data_ptr(), k.data_ptr(), cos.data_ptr(), sin.data_ptr(), yq.data_ptr(),
                                   yk.data_ptr(), strides, B, HQ, HKV, S, D, 1, _lib.BF16, _lib.BF16, _lib.BF16, 0,
                                   stream()))

        def cpu():
            qc = torch.randn(B, HQ, S, D).bfloat16().requires_grad_()
            kc = torch.randn(B, HKV, S, D).bfloat16().requires_grad_()
            cc, sc = cos.cpu(), sin.cpu()
            gqc, gkc = torch.randn(B, HQ, S, D).bfloat16(), torch.randn(B, HKV, S, D).bfloat16()

            def one():
                oq, ok = R.rope(qc, kc, cc, sc)
                torch.autograd.grad((oq, ok), (qc, kc), (gqc, gkc))

            t, reps = _time_cpu(one)
            return 2 * launch_bytes / t / 1e12, f"full shape, fwd+bwd, median of {reps} reps"

        def torch_step(i):
            q, k = leaves[i % n]
            oq, ok = R.rope(q, k, cos, sin)
            torch.autograd.grad((oq, ok), (q, k), (gq, gk))

        return Workload("rope", "rope fwd+bwd bf16 q [4,32,4096,128], k [4,8,4096,128], bf16 cos/sin [1,4096,128]",
                        "bf16", "TB/s", 2 * launch_bytes, step, "rope_kernel", launch_bytes, launch,
                        {"batch": B, "q_heads": HQ, "kv_heads": HKV, "seq": S, "head_dim": D, "cos_batch": 1,
                         "theta": 500000.0, "dtype": "bf16"}, cpu, torch_step)

    if name == "qk_norm_rope":
        # not a BASELINE config: the kernel-writing notebook's fused op at its benchmark shape
        B, HQ, HKV, S, D = 4, 32, 8, 4096, 128
        q = _randn((B, HQ, S, D), torch.bfloat16, gen, dev)
        k = _randn((B, HKV, S, D), torch.bfloat16, gen, dev)
        qw, kw = _randn((D,), torch.bfloat16, gen, dev), _randn((D,), torch.bfloat16, gen, dev)
        half = _randn((1, S, D // 2), torch.bfloat16, gen, dev)
        cos, sin = torch.cos(half).repeat(1, 1, 2), torch.sin(half).repeat(1, 1, 2)
        gq, gk = _randn((B, HQ, S, D), torch.bfloat16, gen, dev), _randn((B, HKV, S, D), torch.bfloat16, gen, dev)
        qkb = (q.numel() + k.numel()) * 2
        side = 2 * S * D * 2 + 2 * D * 2 + 4 * B * (HQ + HKV) * S  # tables, weights, rstd
        fwd_bytes = 2 * qkb + side
        bwd_bytes = 3 * qkb + side
        leaves = [t.requires_grad_() for t in (q, k, qw, kw)]
        dq, dk = torch.empty_like(q), torch.empty_like(k)
        dw = torch.empty((2, D), dtype=torch.bfloat16, device=dev)
        rq = torch.empty((B, HQ, S), dtype=torch.float32, device=dev)
        rk = torch.empty((B, HKV, S), dtype=torch.float32, device=dev)
        yq, yk = torch.empty_like(q), torch.empty_like(k)
        st12 = (_lib._i64 * 12)(*(x for t in (q, k, yq, yk) for x in t.stride()[:3]))
        _lib.check(lib.pk_qk_norm_rope_fwd(q.data_ptr(), k.data_ptr(), qw.data_ptr(), kw.data_ptr(), cos.data_ptr(),
                                           sin.data_ptr(), yq.data_ptr(), yk.data_ptr(), rq.data_ptr(), rk.data_ptr(),
                                           st12, B, HQ, HKV, S, D, 1, 1e-6, _lib.BF16, _lib.BF16, _lib.BF16,
                                           _lib.BF16, stream()))
        ws_bytes = lib.pk_qk_norm_rope_bwd_workspace(B, HQ, HKV, S, D, _lib.BF16)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        st18 = (_lib._i64 * 18)(*(x for t in (q, k, gq, gk, dq, dk) for x in t.stride()[:3]))

        def step(i):
            oq, ok = impls.qk_norm_rope(*leaves, cos, sin, 1e-6)
            torch.autograd.grad((oq, ok), leaves, (gq, gk))

        def launch(i):
            _lib.check(lib.pk_qk_norm_rope_bwd(q.data_ptr(), k.data_ptr(), qw.data_ptr(), kw.data_ptr(),
                                               cos.data_ptr(), sin.data_ptr(), rq.data_ptr(), rk.data_ptr(),
                                               gq.data_ptr(), gk.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                                               dw.data_ptr(), ws.data_ptr(), ws_bytes, st18, B, HQ, HKV, S, D, 1,
                                               _lib.BF16, _lib.BF16, _lib.BF16, _lib.BF16, stream()))

        def cpu():
            qc = torch.randn(B, HQ, S, D).bfloat16().requires_grad_()
            kc = torch.randn(B, HKV, S, D).bfloat16().requires_grad_()
            wq, wk = (torch.randn(D).bfloat16().requires_grad_() for _ in range(2))
            cc, sc = cos.cpu(), sin.cpu()
            gqc, gkc = torch.randn(B, HQ, S, D).bfloat16(), torch.randn(B, HKV, S, D).bfloat16()

            def one():
                oq, ok = R.qk_norm_rope(qc, kc, wq, wk, cc, sc, 1e-6)
                torch.autograd.grad((oq, ok), (qc, kc, wq, wk), (gqc, gkc))

            t, reps = _time_cpu(one)
            return (fwd_bytes + bwd_bytes) / t / 1e12, f"full shape, fwd+bwd, median of {reps} reps"

        def torch_step(i):
            oq, ok = R.qk_norm_rope(*leaves, cos, sin, 1e-6)
            torch.autograd.grad((oq, ok), leaves, (gq, gk))

        return Workload("qk_norm_rope", "qk_norm_rope fwd+bwd bf16 q [4,32,4096,128], k [4,8,4096,128], "
                        "weights [128], bf16 cos/sin [1,4096,128]", "bf16", "TB/s", fwd_bytes + bwd_bytes, step,
                        "qk_norm_rope_bwd_kernel", bwd_bytes, launch,
                        {"batch": B, "q_heads": HQ, "kv_heads": HKV, "seq": S, "head_dim": D, "cos_batch": 1,
                         "eps": 1e-6, "dtype": "bf16"}, cpu, torch_step,
                        launch_kernels=("qk_norm_rope_bwd_kernel", "column_sum_stage", "column_sum_final"))

    if name == "c4":
        rows, cols = 65536, 8192
        x = _randn((rows, cols), torch.bfloat16, gen, dev)
        w = (1 + 0.1 * _randn((cols,), torch.float32, gen, dev)).bfloat16()
        dy = _randn((rows, cols), torch.bfloat16, gen, dev)
        elems = rows * cols
        fwd_bytes = 2 * elems * 2 + cols * 2
        bwd_bytes = 3 * elems * 2 + cols * 2 + cols * 4
        xg = x.detach().requires_grad_()
        wg = w.detach().requires_grad_()
        y = torch.empty_like(x)
        dx = torch.empty_like(x)
        dw = torch.empty_like(w)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        _lib.check(lib.pk_rmsnorm_fwd(x.data_ptr(), w.data_ptr(), None, y.data_ptr(), rstd.data_ptr(), rows, cols,
                                      1e-6, _lib.BF16, _lib.BF16, stream()))
        ws_bytes = lib.pk_rmsnorm_bwd_workspace(rows, cols, _lib.BF16)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

        def step(i):
            yy = impls.rms_norm(xg, wg, None, 1e-6)
            torch.autograd.grad(yy, (xg, wg), dy)

        def launch(i):
            _lib.check(lib.pk_rmsnorm_bwd(x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), dx.data_ptr(),
                                          dw.data_ptr(), None, ws.data_ptr(), ws_bytes, rows, cols, _lib.BF16,
                                          _lib.BF16, stream()))

        def cpu():
            sample = rows
            xc = torch.randn(sample, cols).bfloat16().requires_grad_()
            wc = (1 + 0.1 * torch.randn(cols)).bfloat16().requires_grad_()
            gc = torch.randn(sample, cols).bfloat16()

            def one():
                yc = R.rms_norm(xc, wc, None, 1e-6)
                torch.autograd.grad(yc, (xc, wc), gc)

            t, reps = _time_cpu(one)
            return (fwd_bytes + bwd_bytes) / t / 1e12, f"full C4 [{rows}, {cols}] bf16 fwd+bwd, median of {reps} reps"

        def torch_step(i):
            yy = R.rms_norm(xg, wg, None, 1e-6)
            torch.autograd.grad(yy, (xg, wg), dy)

        return Workload("c4", "RMSNorm fwd+bwd bf16 x, dy [65536, 8192]", "bf16", "TB/s", fwd_bytes + bwd_bytes,
                        step, "rmsnorm_bwd_vec", bwd_bytes, launch,
                        {"rows": rows, "cols": cols, "eps": 1e-6, "dtype": "bf16"}, cpu, torch_step,
                        launch_kernels=("rmsnorm_bwd_vec", "column_sum_stage", "column_sum_final"))

    if name == "add_rmsnorm":
        # not a BASELINE config: the next op on the norm path (residual add + RMSNorm) at C4's shape
        rows, cols = 65536, 8192
        x = _randn((rows, cols), torch.bfloat16, gen, dev)
        res = _randn((rows, cols), torch.bfloat16, gen, dev)
        w = (1 + 0.1 * _randn((cols,), torch.float32, gen, dev)).bfloat16()
        dy = _randn((rows, cols), torch.bfloat16, gen, dev)
        ds = _randn((rows, cols), torch.bfloat16, gen, dev)
        elems = rows * cols
        fwd_bytes = 4 * elems * 2 + cols * 2  # read x, residual; write y, s
        bwd_bytes = 4 * elems * 2 + cols * 2 + cols * 4  # read s, dy, ds; write dx; w; dw
        xg, rg, wg = (t.detach().requires_grad_() for t in (x, res, w))
        y, sm, dsum = torch.empty_like(x), torch.empty_like(x), torch.empty_like(x)
        dw = torch.empty_like(w)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        _lib.check(lib.pk_add_rmsnorm_fwd(x.data_ptr(), res.data_ptr(), w.data_ptr(), y.data_ptr(), sm.data_ptr(),
                                          rstd.data_ptr(), rows, cols, 1e-6, 1.0, _lib.BF16, _lib.BF16, stream()))
        ws_bytes = lib.pk_rmsnorm_bwd_workspace(rows, cols, _lib.BF16)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

        def step(i):
            yy, ss = impls.add_rms_norm(xg, rg, wg, 1e-6, 1.0)
            torch.autograd.grad((yy, ss), (xg, rg, wg), (dy, ds))

        def launch(i):
            _lib.check(lib.pk_add_rmsnorm_bwd(sm.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(),
                                              ds.data_ptr(), dsum.data_ptr(), dw.data_ptr(), ws.data_ptr(), ws_bytes,
                                              rows, cols, 1.0, _lib.BF16, _lib.BF16, stream()))

        def cpu():
            sample = rows
            xc, rc = (torch.randn(sample, cols).bfloat16().requires_grad_() for _ in range(2))
            wc = (1 + 0.1 * torch.randn(cols)).bfloat16().requires_grad_()
            gc, sc = torch.randn(sample, cols).bfloat16(), torch.randn(sample, cols).bfloat16()

            def one():
                yc, s_c = R.add_rms_norm(xc, rc, wc, 1e-6, 1.0)
                torch.autograd.grad((yc, s_c), (xc, rc, wc), (gc, sc))

            t, reps = _time_cpu(one)
            return (fwd_bytes + bwd_bytes) / t / 1e12, f"full [{rows}, {cols}] bf16 fwd+bwd, median of {reps} reps"

        def torch_step(i):
            yy, ss = R.add_rms_norm(xg, rg, wg, 1e-6, 1.0)
            torch.autograd.grad((yy, ss), (xg, rg, wg), (dy, ds))

        return Workload("add_rmsnorm", "add_rms_norm fwd+bwd bf16 x, residual, dy, ds [65536, 8192], offset 1",
                        "bf16", "TB/s", fwd_bytes + bwd_bytes, step, "rmsnorm_bwd_vec", bwd_bytes, launch,
                        {"rows": rows, "cols": cols, "eps": 1e-6, "offset": 1.0, "dtype": "bf16"}, cpu, torch_step,
                        launch_kernels=("rmsnorm_bwd_vec", "column_sum_stage", "column_sum_final"))

    if name in ("attn_bwd", "attn_bwd_f32"):
        # not a BASELINE config: attention forward + backward at C5's shape (causal), bf16 or, for
        # attn_bwd_f32, fp32 on the fp32 matrix-core kernels
        fp32 = name == "attn_bwd_f32"
        dt, code, tag = (torch.float32, _lib.F32, "fp32") if fp32 else (torch.bfloat16, _lib.BF16, "bf16")
        B, S, HQ, HKV, D = 4, 8192, 32, 8, head_dim
        q = _randn((B, S, HQ, D), dt, gen, dev)
        k = _randn((B, S, HKV, D), dt, gen, dev)
        v = _randn((B, S, HKV, D), dt, gen, dev)
        do = _randn((B, S, HQ, D), dt, gen, dev)
        fwd_flops = 4.0 * B * HQ * D * S * S / 2
        bwd_flops = 2.5 * fwd_flops  # the customary count: dQ, dK, dV, dP and S recomputed once (5 products)
        qg, kg, vg = (t.detach().requires_grad_() for t in (q, k, v))
        o, lse = impls.attn_with_lse(q, k, v, True)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws = torch.empty(lib.pk_attn_bwd_workspace(B, S, HQ, HKV, D), dtype=torch.uint8, device=dev)
        strides = (_lib._i64 * 24)(*(s for t in (q, k, v, o, do, dq, dk, dv) for s in t.stride()[:3]))

        def step(i):
            out = impls.attn(qg, kg, vg, True)
            torch.autograd.grad(out, (qg, kg, vg), do)

        def launch(i):
            _lib.check(lib.pk_attn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                                       lse.data_ptr(), ws.data_ptr(), ws.numel(), dq.data_ptr(), dk.data_ptr(),
                                       dv.data_ptr(),
                                       strides, B, S, HQ, HKV, D, D**-0.5, 1, code, stream()))

        def cpu():
            sq = 1024  # one (batch, kv group) of 1024 tokens; work scaled to that
            qc = torch.randn(1, sq, 4, D).to(dt).requires_grad_()
            kc, vc = (torch.randn(1, sq, 1, D).to(dt).requires_grad_() for _ in range(2))
            gc = torch.randn(1, sq, 4, D).to(dt)

            def one():
                oc = R.attn(qc, kc, vc, True)
                torch.autograd.grad(oc, (qc, kc, vc), gc)

            t, reps = _time_cpu(one)
            work = 3.5 * 4.0 * 4 * D * sq * sq / 2
            return work / t / 1e12, f"B=1, S={sq}, Hq=4, Hkv=1 causal fwd+bwd {tag}, median of {reps} reps"

        def torch_step(i):
            out = R.attn(qg, kg, vg, True)
            torch.autograd.grad(out, (qg, kg, vg), do)

        kernels = ("attn_bwd_f32_dq_kernel", "attn_bwd_f32_dkdv_kernel") if fp32 else \
            ("attn_bwd_dq_kernel", "attn_bwd_dkdv_kernel")
        return Workload(name if D == 128 else f"{name}_d{D}",
                        f"Causal GQA attention fwd+bwd {tag} B=4 S=8192 Hq=32 Hkv=8 D={D}", "f32" if fp32 else "bf16",
                        "TFLOP/s", fwd_flops + bwd_flops, step, "attn_bwd", bwd_flops, launch,
                        {"batch": B, "seq": S, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "causal": True,
                         "dtype": tag}, cpu, torch_step, launch_kernels=kernels,
                        peak=FP32_PEAK_TFLOPS if fp32 else None)

    if name in ("c5", "c5_f32"):
        # c5_f32 (not a BASELINE config): C5's shape in fp32, on the fp32 matrix-core kernel
        fp32 = name == "c5_f32"
        dt, code = (torch.float32, _lib.F32) if fp32 else (torch.bfloat16, _lib.BF16)
        B, S, HQ, HKV, D = 4, 8192, 32, 8, head_dim
        q = _randn((B, S, HQ, D), dt, gen, dev)
        k = _randn((B, S, HKV, D), dt, gen, dev)
        v = _randn((B, S, HKV, D), dt, gen, dev)
        flops = 4.0 * B * HQ * D * S * S / 2
        o = torch.empty_like(q)
        lse = torch.empty((B, HQ, S), dtype=torch.float32, device=dev)
        strides = (_lib._i64 * 12)(*(s for t in (q, k, v, o) for s in t.stride()[:3]))

        def step(i):
            with torch.no_grad():
                impls.attn_with_lse(q, k, v, True)

        def launch(i):
            _lib.check(lib.pk_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                       strides, B, S, HQ, HKV, D, D**-0.5, 1, code, stream()))

        def cpu():
            # The largest of (B, S) = (1, 2048), (1, 4096), (1, 8192), (4, 8192) -- the last is C5
            # itself -- whose warmup plus two timed reps fit about 30 s on this host, estimated
            # from (1, 2048).
            def sample(b_cpu, s_cpu):
                qc = torch.randn(b_cpu, s_cpu, HQ, D).to(dt)
                kc, vc = (torch.randn(b_cpu, s_cpu, HKV, D).to(dt) for _ in range(2))
                return lambda: R.attn(qc, kc, vc, True)

            probe = sample(1, 2048)
            probe()
            t0 = time.perf_counter()
            probe()
            unit = time.perf_counter() - t0
            fits = [(b_, s_) for b_, s_ in ((1, 2048), (1, 4096), (1, 8192), (4, 8192))
                    if 3 * unit * b_ * (s_ / 2048) ** 2 <= 30.0]
            b_cpu, s_cpu = fits[-1] if fits else (1, 2048)
            t, reps = _time_cpu(sample(b_cpu, s_cpu), budget_s=0.0, min_reps=2, max_reps=2)
            work = 4.0 * b_cpu * HQ * D * s_cpu * s_cpu / 2
            what = "full C5" if (b_cpu, s_cpu) == (B, S) else f"B={b_cpu}, S={s_cpu} of C5's B=4, S=8192"
            return work / t / 1e12, f"{what}, causal {'fp32' if fp32 else 'bf16'}, 1 warmup + median of {reps} reps"

        def torch_step(i):
            with torch.no_grad():
                R.attn(q, k, v, True)

        tag = "fp32" if fp32 else "bf16"
        return Workload(name if D == 128 else f"{name}_d{D}", f"Causal GQA attention fwd {tag} B=4 S=8192 Hq=32 Hkv=8 D={D}",
                        "f32" if fp32 else "bf16", "TFLOP/s",
                        flops, step, "attn_fwd_f32_kernel" if fp32 else "attn_fwd_kernel", flops, launch,
                        {"batch": B, "seq": S, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "causal": True,
                         "dtype": tag}, cpu, torch_step, peak=FP32_PEAK_TFLOPS if fp32 else None)

    if name in ("mfma_ceiling", "mfma_ceiling_softmax"):
        # not a BASELINE config: the matrix-core rate this board sustains under its power limit,
        # random bf16 operands toggling like real data (pk_probe_mfma), one wave per SIMD on every CU
        softmax = int(name.endswith("softmax"))
        blocks = torch.cuda.get_device_properties(dev).multi_processor_count
        iters = 2048  # 2048 x 8 products of 32 cycles: about 0.3 ms per launch at 1.8 GHz
        out = torch.zeros(2 * 4 * blocks, dtype=torch.int64, device=dev)
        flops = 4.0 * blocks * iters * 8 * (2 * 32 * 32 * 16)

        def step(i):
            _lib.check(lib.pk_probe_mfma(softmax, iters, blocks, out.data_ptr(), stream()))

        def extra():
            cycles, ticks = out.view(-1, 2).double().cpu().unbind(1)
            return {"cycles_per_product": round(float(cycles.mean()) / (iters * 8), 3),
                    "clock_mhz": round(float((cycles / ticks).mean()) * 100.0, 1)}  # ticks run at 100 MHz

        what = "bf16 32x32x16 products" + (" with the attention forward's per-score vector work" if softmax else "")
        return Workload(name, f"matrix-core probe: {what}, {blocks} CUs x 4 waves", "bf16", "TFLOP/s", flops, step,
                        "mfma_probe_kernel", flops, step,
                        {"blocks": blocks, "waves_per_simd": 1, "products_per_wave": iters * 8,
                         "softmax": bool(softmax)}, extra=extra)

    if name.startswith("stream_"):
        # not a BASELINE config: the streaming ceiling at a config's pattern and size, e.g. stream_1r_64m
        # (C1: one read and one write of 64 MiB) or stream_2r_160m (qk_norm_rope's backward: two reads
        # and one write of 160 MiB); pk_probe_stream, inputs and outputs rotated like C1's
        try:
            reads, mib = name[len("stream_"):].split("_")
            reads, nbytes = int(reads.rstrip("r")), int(mib.rstrip("m")) << 20
        except ValueError:
            raise SystemExit(f"bench.py: stream workload {name!r} is not stream_<1|2>r_<MiB>m")
        if reads not in (1, 2) or nbytes <= 0:
            raise SystemExit(f"bench.py: stream workload {name!r} is not stream_<1|2>r_<MiB>m")
        n = _copies(reads * nbytes)
        ins = [[torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(generator=gen) for _ in range(reads)]
               for _ in range(n)]
        outs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(n)]
        moved = (reads + 1) * nbytes

        def step(i):
            a = ins[i % n]
            _lib.check(lib.pk_probe_stream(a[0].data_ptr(), a[-1].data_ptr() if reads == 2 else None,
                                           outs[i % n].data_ptr(), nbytes, reads, stream()))

        return Workload(name, f"streaming probe: {reads} read(s) + 1 write of {nbytes >> 20} MiB each, {n} copies "
                        "rotated", "u8", "TB/s", moved, step, "stream_probe_kernel", moved, step,
                        {"reads": reads, "bytes_each": nbytes, "copies": n})

    if name == "copy":
        numel = 256 << 20  # 512 MiB of bf16 each way
        src = torch.empty(numel, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        nbytes = 2 * numel * 2

        def step(i):
            dst.copy_(src)

        return Workload("copy", "plain device copy, 512 MiB -> 512 MiB", "bf16", "TB/s", nbytes, step, "copy",
                        nbytes, step, {"bytes_each_way": numel * 2})

    raise SystemExit(f"bench.py: unknown workload {name!r} (c1..c5, add_rmsnorm, rope, qk_norm_rope, attn_bwd, "
                     "mfma_ceiling, mfma_ceiling_softmax, copy)")


def _amd_smi_power() -> dict | None:
    """One `amd-smi metric -p -c` sample of GPU 0: socket power and the graphics clock of each XCD."""
    import re
    import subprocess
    try:
        text = subprocess.run(["amd-smi", "metric", "-p", "-c", "-g", "0"], capture_output=True, text=True,
                              timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    power = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", text)
    clocks = [int(m) for m in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*([0-9]+)\s*MHz", text)]
    if power is None and not clocks:
        return None
    return {"socket_power_w": float(power.group(1)) if power else None, "gfx_clock_mhz": clocks}


def _power_sample(fn: Callable[[int], None], seconds: float) -> dict | None:
    """Run `fn` back to back for `seconds` and sample board power and clocks two thirds of the way in.

    The sample comes from `amd-smi` in a thread while the calls keep the GPU busy; the clock it
    reports is what the power manager allows this workload.
    """
    import threading
    box: dict = {}
    sampler = threading.Timer(seconds * 2 / 3, lambda: box.update(sample=_amd_smi_power()))
    calls, t0 = 0, time.perf_counter()
    sampler.start()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn(calls)
            calls += 1
        torch.cuda.synchronize()
    sampler.join()
    sample = box.get("sample")
    if sample is None:
        return None
    return {**sample, "seconds": seconds, "calls": calls, "ms_per_call": round((time.perf_counter() - t0) * 1e3 / calls, 4)}


def _time_cpu(fn, budget_s: float = 5.0, min_reps: int = 2, max_reps: int = 20) -> tuple[float, int]:
    """Median wall time of fn on the CPU after one warmup, over reps filling about budget_s."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    reps = int(min(max_reps, max(min_reps, budget_s / max(first, 1e-6))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], reps


def _time_gpu(fn: Callable[[int], None], steps: int, warmup: int) -> float:
    """Total ms of `steps` back-to-back calls, between two HIP events on torch's current stream.

    The calls run with nothing between them: an event recorded between two
    launches costs the GPU several microseconds of idle time, which would be
    charged to kernels of a few tens of microseconds.
    """
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def _reps(fn: Callable[[int], None], floor: int, target_ms: float = 20.0) -> int:
    """Calls that fill about `target_ms` of GPU time (at least `floor`), from a three-call estimate."""
    est = _time_gpu(fn, 3, 1) / 3
    return max(floor, min(2000, math.ceil(target_ms / max(est, 1e-3))))


def _rate(work: float, ms: float, unit: str) -> float:
    return work / (ms * 1e-3) / 1e12


def _roofline(wl: Workload, steps: int, warmup: int) -> dict:
    """The dominant kernel's average launch: `steps` back-to-back launches between two events.

    A launch is one call of the C entry point; where that runs more kernels than the dominant one
    (`launch_covers`), their time is charged to it too.
    """
    avg = _time_gpu(wl.launch, steps, warmup) / steps
    achieved = _rate(wl.kernel_work, avg, wl.unit)
    hbm = wl.unit == "TB/s"
    peak = wl.peak if wl.peak is not None else (HBM_PEAK_TBS if hbm else BF16_PEAK_TFLOPS)
    return {
        "kernel": wl.kernel,
        "bound": "hbm" if hbm else "mfma",
        "achieved": round(achieved * (1000 if hbm else 1), 2),
        "peak": peak * (1000 if hbm else 1),
        "unit": "GB/s" if hbm else "TFLOP/s",
        "frac": round(achieved / peak, 4),
        "avg_launch_us": round(avg * 1e3, 2),
        "work_per_launch": wl.kernel_work,
        "traffic": MEASURED_TRAFFIC.get(wl.name),
        **({"launch_covers": list(wl.launch_kernels)} if wl.launch_kernels else {}),
    }


# The ceiling each dominant kernel is compared against in the same run: the streaming probe with
# the kernel's reads per write and bytes (pk_probe_stream, rotated like C1), or the matrix-core probe
# with the forward's per-score vector work (pk_probe_mfma). add_rmsnorm's backward reads three
# streams, a pattern the probe does not have; the attention backward's vector work differs from the
# forward's, so it gets none either.
CEILINGS = {
    "c1": "stream_1r_64m",      # x [4096, 4096] fp32 in, y out
    "c2": "stream_2r_448m",     # a, b [16384, 14336] bf16 in, y out
    "c3": "stream_1r_256m",     # the q call: q [8, 4096, 32, 128] bf16 in and out
    "c4": "stream_2r_1024m",    # the backward call: x, dy [65536, 8192] bf16 in, dx out
    "c5": "mfma_ceiling_softmax",
    "rope": "stream_1r_160m",   # q and k in, their rotations out
    "qk_norm_rope": "stream_2r_160m",  # the backward: q/k and their cotangents in, gradients out
}


def _ceiling(name: str, dev: torch.device, kernel_rate: float, steps: int) -> dict | None:
    """The same-run ceiling of workload `name`'s dominant kernel: the probe's launch time and rate, and
    the kernel's rate as a share of it (the kernel's distance from what its pattern can reach on this
    box, as opposed to the published peak)."""
    probe = CEILINGS.get(name)
    if probe is None:
        return None
    torch.cuda.empty_cache()
    wl = make_workload(probe, dev)
    reps = _reps(wl.launch, max(5, steps))
    avg = _time_gpu(wl.launch, reps, _reps(wl.launch, 2, target_ms=60.0)) / reps
    rate = _rate(wl.kernel_work, avg, wl.unit)
    hbm = wl.unit == "TB/s"
    out = {"probe": probe, "avg_launch_us": round(avg * 1e3, 2), "achieved": round(rate * (1000 if hbm else 1), 2),
           "unit": "GB/s" if hbm else "TFLOP/s", "kernel_share": round(kernel_rate / rate, 4)}
    del wl
    torch.cuda.empty_cache()
    return out


def _cpu_threads() -> tuple[int, int]:
    """(threads to use, cores this process may run on): every core of the affinity mask, within the
    host's CPU share for this GPU when one is set (OMP_NUM_THREADS on the GPU boxes)."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return (min(affinity, share) if share > 0 else affinity), affinity


def _cpu_baseline(wl: Workload) -> dict | None:
    if wl.cpu is None:
        return None
    threads, affinity = _cpu_threads()
    torch.set_num_threads(threads)
    value, sample = wl.cpu()
    return {"value": round(value, 6), "unit": wl.unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"popcorn reference (torch, CPU): {sample}; {torch.get_num_threads()} threads, affinity "
                      f"{affinity} cores, os.cpu_count()={os.cpu_count()}"}


def _torch_on_gpu(wl: Workload, ours_ms: float, steps: int, warmup: int) -> dict | None:
    """Popcorn's torch reference timed on the same device and inputs: the implementation the selector
    compares against."""
    if wl.torch_step is None:
        return None
    total = _time_gpu(wl.torch_step, steps, warmup)
    per = total / steps
    return {"ms_per_step": round(per, 4), "value": round(_rate(wl.work, per, wl.unit), 4),
            "speedup": round(per / ours_ms, 3)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    named = ["c1", "c2", "c3", "c4", "c5", "add_rmsnorm", "rope", "qk_norm_rope", "attn_bwd", "c5_f32", "attn_bwd_f32",
             "mfma_ceiling", "mfma_ceiling_softmax", "copy"]

    def workload_name(text: str) -> str:
        if text in named or text.startswith("stream_"):
            return text
        raise argparse.ArgumentTypeError(f"{text!r} is none of {', '.join(named)} or stream_<1|2>r_<MiB>m")

    ap.add_argument("--workload", default="c2", type=workload_name,
                    help=f"one of {', '.join(named)}, or stream_<1|2>r_<MiB>m (the streaming ceiling)")
    ap.add_argument("--head-dim", type=int, default=128,
                    help="head_dim of the c5 and attn_bwd workloads (128 is the BASELINE config)")
    ap.add_argument("--power", action="store_true",
                    help="also run the workload for a few seconds and report amd-smi socket power and clocks")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU reference timing")
    ap.add_argument("--no-others", action="store_true", help="skip the other configs' kernel figures")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; every config's kernels run on a single MI355X "
              "(multi-GPU sharding is described, not run). Use --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    print(f"bench: workload {args.workload}, {args.warmup} warmup + {args.steps} steps", file=sys.stderr, flush=True)
    wl = make_workload(args.workload, dev, args.head_dim)
    torch.cuda.synchronize()
    total_ms = _time_gpu(wl.step, args.steps, args.warmup)
    ms_per_step = total_ms / args.steps
    value = _rate(wl.work, ms_per_step, wl.unit)
    print(f"bench: {wl.name} {ms_per_step:.4f} ms/step, {value:.3f} {wl.unit}", file=sys.stderr, flush=True)
    roof = _roofline(wl, args.steps, args.warmup)
    print(f"bench: {wl.kernel} {roof['avg_launch_us']} us/launch, frac {roof['frac']}", file=sys.stderr, flush=True)

    extra = wl.extra() if wl.extra is not None else None
    power = _power_sample(wl.step, 6.0) if args.power else None
    if power:
        print(f"bench: power {power}", file=sys.stderr, flush=True)
    torch_gpu = _torch_on_gpu(wl, ms_per_step, args.steps, args.warmup)
    if torch_gpu:
        print(f"bench: torch on the GPU {torch_gpu['ms_per_step']} ms/step ({torch_gpu['speedup']}x)", file=sys.stderr,
              flush=True)
    head_unit, head_dtype, head_config = wl.unit, wl.dtype, {"workload": wl.description, **wl.config}
    head_default = args.head_dim == 128  # the ceilings are taken at the BASELINE head_dim
    others = {}
    if not args.no_others and args.workload in ("c1", "c2", "c3", "c4", "c5", "attn_bwd", "add_rmsnorm", "rope",
                                                 "qk_norm_rope"):
        del wl
        for name in ("c1", "c2", "c3", "c4", "c5", "attn_bwd", "add_rmsnorm", "rope", "qk_norm_rope"):
            if name == args.workload:
                continue
            torch.cuda.empty_cache()
            wl_o = make_workload(name, dev)
            reps = _reps(wl_o.step, max(5, args.steps // 2))
            # untimed calls filling about 60 ms of GPU time first: under the attention kernels the
            # clock settles over the first ~40 ms (dispatches fall from 2.3 to 1.9 ms at C5)
            tot = _time_gpu(wl_o.step, reps, _reps(wl_o.step, 2, target_ms=60.0))
            per = tot / reps
            entry = {"workload": wl_o.description, "steps": reps, "ms_per_step": round(per, 4),
                     "value": round(_rate(wl_o.work, per, wl_o.unit), 4), "unit": wl_o.unit,
                     "roofline": _roofline(wl_o, _reps(wl_o.launch, reps), 2),
                     "torch_gpu": _torch_on_gpu(wl_o, per, reps, 2)}
            others[name] = entry
            print(f"bench: {name} {per:.4f} ms/step; {entry['roofline']['kernel']} frac {entry['roofline']['frac']}"
                  + (f"; torch {entry['torch_gpu']['ms_per_step']} ms" if entry["torch_gpu"] else ""),
                  file=sys.stderr, flush=True)
            del wl_o
        torch.cuda.empty_cache()
        # the ceilings run after every workload's own figures, so no workload is timed right after a probe
        for name, rf in [(args.workload, roof if head_default else None),
                         *((n, o["roofline"]) for n, o in others.items())]:
            if rf is None:
                continue
            rate = rf["achieved"] / (1000 if rf["unit"] == "GB/s" else 1)
            ceiling = _ceiling(name, dev, rate, args.steps)
            if ceiling is not None:
                rf["ceiling"] = ceiling
                print(f"bench: {name} ceiling {ceiling['probe']} {ceiling['avg_launch_us']} us, kernel at "
                      f"{ceiling['kernel_share']} of it", file=sys.stderr, flush=True)
    else:
        del wl
    # The CPU baselines run after every GPU figure is taken, so the host threads they leave busy
    # cannot slow the launches of a GPU step timed after them.
    cpu = None
    if not args.no_cpu:
        for name in (args.workload, *others):
            torch.cuda.empty_cache()
            wl_c = make_workload(name, dev, args.head_dim if name == args.workload else 128)
            result = _cpu_baseline(wl_c)
            if name == args.workload:
                cpu = result
            else:
                others[name]["cpu_baseline"] = result
            del wl_c
        torch.cuda.empty_cache()

    fractions = {args.workload: roof["frac"], **{name: o["roofline"]["frac"] for name, o in others.items()}}
    line = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": head_unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head_dtype,
        "data": "synthetic N(0,1) inputs, seeded device generator, resident in HBM",
        "config": head_config,
        "roofline": roof,
        "cpu_baseline": cpu,
        "torch_gpu": torch_gpu,
        "roofline_fractions": {name: fractions[name] for name in ("c1", "c2", "c3", "c4", "c5") if name in fractions},
        "others": others,
    }
    if extra is not None:
        line["probe"] = extra
    if power is not None:
        line["power"] = power
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
