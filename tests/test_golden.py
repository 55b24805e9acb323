"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py).

CPU: the float64 oracle still reproduces every stored output from the stored
inputs. GPU: the HIP kernels reproduce them within the north star's
tolerances: fp32 to 1e-5 of max(1, max|truth|), 16-bit attention to 2e-2 of
that scale, and log-sum-exp to 1e-3 absolute.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import reference as O

GOLDEN = Path(__file__).resolve().parent / "golden"
DEV = "cuda"


def fixture(name):
    with np.load(GOLDEN / f"{name}.npz") as f:
        return {k: (f[k].astype(np.float64) if f[k].dtype != np.int32 else f[k]) for k in f.files}


def same(got, want):
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ oracle (CPU)


def test_oracle_reproduces_rms_norm_and_add_rms_norm():
    f = fixture("rms_norm")
    same(O.rms_norm(f["x"], f["weight"], None, float(f["eps"])), f["y"])
    same(O.rms_norm(f["x"], f["weight"], f["bias"], float(f["eps"])), f["y_bias"])
    for got, key in zip(O.rms_norm_bwd(f["x"], f["weight"], f["dy"], float(f["eps"])), ("dx", "dweight", "dbias")):
        same(got, f[key])
    a = fixture("add_rms_norm")
    y, s = O.add_rms_norm(a["x"], a["residual"], a["weight"], float(a["eps"]), float(a["offset"]))
    same(y, a["y"])
    same(s, a["s"])
    grads = O.add_rms_norm_bwd(a["x"], a["residual"], a["weight"], a["dy"], a["ds"], float(a["eps"]), float(a["offset"]))
    for got, key in zip(grads, ("dx", "dresidual", "dweight")):
        same(got, a[key])


def test_oracle_reproduces_swiglu_and_rotations():
    f = fixture("swiglu")
    same(O.swiglu(f["a"], f["b"]), f["y"])
    for got, key in zip(O.swiglu_bwd(f["dy"], f["a"], f["b"]), ("da", "db")):
        same(got, f[key])
    r = fixture("rotary_embedding")
    for il, sfx in ((False, ""), (True, "_interleaved")):
        same(O.rotary_embedding(r["x"], r["cos"], r["sin"], il), r["y" + sfx])
        same(O.rotary_embedding_bwd(r["dy"], r["cos"], r["sin"], il), r["dx" + sfx])
    p = fixture("rope")
    for got, key in zip((*O.rope(p["q"], p["k"], p["cos"], p["sin"]), *O.rope_bwd(p["dyq"], p["dyk"], p["cos"], p["sin"])),
                        ("yq", "yk", "dq", "dk")):
        same(got, p[key])
    n = fixture("qk_norm_rope")
    args = (n["q"], n["k"], n["q_weight"], n["k_weight"], n["cos"], n["sin"])
    outs = (*O.qk_norm_rope(*args, float(n["eps"])), *O.qk_norm_rope_bwd(*args, n["dyq"], n["dyk"], float(n["eps"])))
    for got, key in zip(outs, ("yq", "yk", "dq", "dk", "dq_weight", "dk_weight")):
        same(got, n[key])


def test_oracle_reproduces_attention():
    f = fixture("attn")
    for causal, tag in ((False, "full"), (True, "causal")):
        o, lse = O.attention(f["q"], f["k"], f["v"], causal, None)
        same(o, f[f"o_{tag}"])
        same(lse, f[f"lse_{tag}"])
        for got, key in zip(O.attention_bwd(f["q"], f["k"], f["v"], f["do"], causal, None), ("dq", "dk", "dv")):
            same(got, f[f"{key}_{tag}"])
    v = fixture("attn_varlen")
    o, lse = O.attention_varlen(v["q"], v["k"], v["v"], v["cu_seqlens"], True, float(v["softmax_scale"]))
    same(o, v["o"])
    same(lse, v["lse"])


# ------------------------------------------------------------------ HIP kernels (GPU)


def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from popcorn_amd import impls

    return impls


def _t(a, dtype=torch.float32, grad=False):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)
    return t.requires_grad_() if grad else t


def close(got, want, rel, what):
    g = got.detach().double().cpu().numpy()
    err = float(np.abs(g - want).max())
    scale = max(1.0, float(np.abs(want).max()))
    assert err <= rel * scale, f"{what}: err {err:.3e} > {rel:.0e} * {scale:.2f}"


@pytest.mark.gpu
def test_hip_rms_norm_family_matches_golden_fp32():
    impls = _gpu()
    f = fixture("rms_norm")
    x, w, b = _t(f["x"], grad=True), _t(f["weight"], grad=True), _t(f["bias"], grad=True)
    y = impls.rms_norm(x, w, None, float(f["eps"]))
    close(y, f["y"], 1e-5, "rms_norm y")
    dx, dw = torch.autograd.grad(y, (x, w), _t(f["dy"]))
    close(dx, f["dx"], 1e-5, "rms_norm dx")
    close(dw, f["dweight"], 1e-5, "rms_norm dw")
    yb = impls.rms_norm(x, w, b, float(f["eps"]))
    close(yb, f["y_bias"], 1e-5, "rms_norm y (bias)")
    (db,) = torch.autograd.grad(yb, (b,), _t(f["dy"]))
    close(db, f["dbias"], 1e-5, "rms_norm dbias")
    a = fixture("add_rms_norm")
    xa, ra, wa = (_t(a[k], grad=True) for k in ("x", "residual", "weight"))
    y, s = impls.add_rms_norm(xa, ra, wa, float(a["eps"]), float(a["offset"]))
    close(y, a["y"], 1e-5, "add_rms_norm y")
    close(s, a["s"], 1e-5, "add_rms_norm s")
    for got, key in zip(torch.autograd.grad((y, s), (xa, ra, wa), (_t(a["dy"]), _t(a["ds"]))),
                        ("dx", "dresidual", "dweight")):
        close(got, a[key], 1e-5, f"add_rms_norm {key}")


@pytest.mark.gpu
def test_hip_swiglu_and_rotations_match_golden_fp32():
    impls = _gpu()
    f = fixture("swiglu")
    a, b = _t(f["a"], grad=True), _t(f["b"], grad=True)
    y = impls.swiglu(a, b)
    close(y, f["y"], 1e-5, "swiglu y")
    for got, key in zip(torch.autograd.grad(y, (a, b), _t(f["dy"])), ("da", "db")):
        close(got, f[key], 1e-5, f"swiglu {key}")
    r = fixture("rotary_embedding")
    for il, sfx in ((False, ""), (True, "_interleaved")):
        x = _t(r["x"], grad=True)
        y = impls.rotary_embedding(x, _t(r["cos"]), _t(r["sin"]), il)
        close(y, r["y" + sfx], 1e-5, "rotary y" + sfx)
        (dx,) = torch.autograd.grad(y, (x,), _t(r["dy"]))
        close(dx, r["dx" + sfx], 1e-5, "rotary dx" + sfx)
    p = fixture("rope")
    q, k = _t(p["q"], grad=True), _t(p["k"], grad=True)
    yq, yk = impls.rope(q, k, _t(p["cos"]), _t(p["sin"]))
    grads = torch.autograd.grad((yq, yk), (q, k), (_t(p["dyq"]), _t(p["dyk"])))
    for got, key in zip((yq, yk, *grads), ("yq", "yk", "dq", "dk")):
        close(got, p[key], 1e-5, f"rope {key}")
    n = fixture("qk_norm_rope")
    leaves = [_t(n[key], grad=True) for key in ("q", "k", "q_weight", "k_weight")]
    yq, yk = impls.qk_norm_rope(*leaves, _t(n["cos"]), _t(n["sin"]), float(n["eps"]))
    grads = torch.autograd.grad((yq, yk), leaves, (_t(n["dyq"]), _t(n["dyk"])))
    for got, key in zip((yq, yk, *grads), ("yq", "yk", "dq", "dk", "dq_weight", "dk_weight")):
        close(got, n[key], 1e-5, f"qk_norm_rope {key}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_hip_attention_matches_golden(dtype):
    impls = _gpu()
    f = fixture("attn")
    for causal, tag in ((False, "full"), (True, "causal")):
        q, k, v = (_t(f[key], dtype, grad=True) for key in ("q", "k", "v"))
        o, lse = impls.attn_with_lse(q.detach(), k.detach(), v.detach(), causal)
        close(o, f[f"o_{tag}"], 2e-2, f"attn o ({tag})")
        np.testing.assert_allclose(lse.double().cpu().numpy(), f[f"lse_{tag}"], rtol=0, atol=1e-3)
        grads = torch.autograd.grad(impls.attn(q, k, v, causal), (q, k, v), _t(f["do"], dtype))
        for got, key in zip(grads, ("dq", "dk", "dv")):
            close(got, f[f"{key}_{tag}"], 2e-2, f"attn {key} ({tag})")
    p = fixture("attn_varlen")
    cu = torch.from_numpy(p["cu_seqlens"]).to(DEV)
    o, lse = impls.attn_varlen_with_lse(_t(p["q"], dtype), _t(p["k"], dtype), _t(p["v"], dtype), cu, True,
                                        float(p["softmax_scale"]))
    close(o, p["o"], 2e-2, "attn_varlen o")
    np.testing.assert_allclose(lse.double().cpu().numpy(), p["lse"], rtol=0, atol=1e-3)
