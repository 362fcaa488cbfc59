"""Pins for the fused Mamba inner-function oracle (oracle/inner_ref.py, the restatement of
MambaInnerFn.forward, selective_scan_interface.py:458-553, and mamba_inner_ref, :659-694):

* a float64 nested-loop brute force (explicit index arithmetic for the conv, the projections, the
  (b l) <-> (b, d, l) layouts, the B/C/delta column split, the RMSNorms and the scan as a closed sum)
  agrees with the tensor restatement, with and without the optional biases and RMSNorms;
* a closed form: with the B rows of x_proj_weight zero, the state stays 0 and the block reduces to
  out_proj((D * conv_out) * silu(z)) + out_proj_bias, independent of the scan;
* RMSNorm known answers (a constant row maps to the weight; [3, 4] to [3, 4] / sqrt(12.5)) and scale
  invariance;
* float64 gradcheck of the restatement's autograd gradients (the gradients the GPU backward is
  compared with) against finite differences;
* the step-by-step restatement of MambaInnerFn.backward (mamba_inner_bwd_ref, the expected values
  when RMSNorm weights are given): without the norms it equals autograd of mamba_inner_ref at both
  checkpoint levels, projected and given B/C; with them at checkpoint_lvl 0 it equals autograd
  through straight-through norms (the norm's value, an identity gradient); at checkpoint_lvl 1 with
  unit weights and eps 0 (where normalising twice changes nothing) it equals checkpoint_lvl 0.

CPU only.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.inner_ref as inner_mod
from oracle.inner_ref import mamba_inner_brute, mamba_inner_bwd_ref, mamba_inner_ref, rms_norm_ref


def _params(seed, batch=2, d_inner=3, L=6, d_state=2, rank=2, d_model=2, W=4, dtype=torch.float64, biases=True):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(dtype)   # noqa: E731
    p = dict(
        xz=r(batch, 2 * d_inner, L),
        conv1d_weight=r(d_inner, 1, W, sc=0.5),
        conv1d_bias=r(d_inner, sc=0.1) if biases else None,
        x_proj_weight=r(rank + 2 * d_state, d_inner, sc=0.5),
        delta_proj_weight=r(d_inner, rank, sc=0.5),
        out_proj_weight=r(d_model, d_inner, sc=0.5),
        out_proj_bias=r(d_model, sc=0.1) if biases else None,
        A=-torch.rand(d_inner, d_state, generator=g).to(dtype) - 0.5,
        D=r(d_inner),
        delta_bias=r(d_inner, sc=0.1),
    )
    return p


def _call(p, **kw):
    return mamba_inner_ref(p["xz"], p["conv1d_weight"], p["conv1d_bias"], p["x_proj_weight"], p["delta_proj_weight"],
                           p["out_proj_weight"], p["out_proj_bias"], p["A"], None, None, p["D"], p["delta_bias"],
                           round_to=None, compute_dtype=torch.float64, **kw)


@pytest.mark.parametrize("biases", [False, True])
@pytest.mark.parametrize("rms", [False, True])
def test_vs_brute(biases, rms):
    p = _params(11 + biases + 2 * rms, biases=biases)
    g = torch.Generator().manual_seed(99)
    extra = {}
    if biases:
        extra.update(B_proj_bias=torch.randn(2, generator=g).double(), C_proj_bias=torch.randn(2, generator=g).double())
    if rms:
        extra.update(b_rms_weight=torch.rand(2, generator=g).double() + 0.5,
                     c_rms_weight=torch.rand(2, generator=g).double() + 0.5,
                     dt_rms_weight=torch.rand(3, generator=g).double() + 0.5)
    got = _call(p, **extra)
    kw = {k: v for k, v in extra.items() if k.endswith("proj_bias") or k.endswith("rms_weight")}
    ref = mamba_inner_brute(p["xz"], p["conv1d_weight"], p["conv1d_bias"], p["x_proj_weight"], p["delta_proj_weight"],
                            p["out_proj_weight"], p["out_proj_bias"], p["A"], p["D"], p["delta_bias"], **kw)
    np.testing.assert_allclose(got.numpy(), np.array(ref), rtol=1e-9, atol=1e-11)


def test_closed_form_without_state_input():
    p = _params(21)
    p["x_proj_weight"][2:4] = 0.0                   # B rows: B = 0, so h = 0 and y = D u
    got = _call(p)
    x, z = p["xz"].chunk(2, dim=1)
    u = F.silu(F.conv1d(x, p["conv1d_weight"], p["conv1d_bias"], padding=3, groups=3)[..., :6])
    gated = p["D"][:, None] * u * F.silu(z)
    want = gated.transpose(1, 2) @ p["out_proj_weight"].t() + p["out_proj_bias"]
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_rms_norm_known_answers_and_scale_invariance():
    w = torch.tensor([2.0, -1.0, 0.5])
    x = torch.full((1, 3, 1), 7.0)
    torch.testing.assert_close(rms_norm_ref(x, w, eps=0.0, dim=1)[0, :, 0], w)
    y = rms_norm_ref(torch.tensor([[3.0, 4.0]]), torch.ones(2), eps=0.0, dim=-1)
    torch.testing.assert_close(y, torch.tensor([[3.0, 4.0]]) / math.sqrt(12.5))
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 16, 8, generator=g, dtype=torch.float64)
    w = torch.rand(16, generator=g, dtype=torch.float64)
    torch.testing.assert_close(rms_norm_ref(x, w, 0.0, 1, torch.float64), rms_norm_ref(37.0 * x, w, 0.0, 1, torch.float64))
    assert rms_norm_ref(x.float().to(torch.bfloat16), w, dim=1).dtype == torch.bfloat16


def test_gradcheck():
    p = _params(31, batch=1, d_inner=2, L=5, d_state=2, rank=1, d_model=2)
    names = ["xz", "conv1d_weight", "conv1d_bias", "x_proj_weight", "delta_proj_weight", "out_proj_weight",
             "out_proj_bias", "A", "D", "delta_bias"]
    args = [p[n].clone().requires_grad_(True) for n in names]

    def f(*a):
        q = dict(zip(names, a))
        return _call(q)
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-6, rtol=1e-5)


NAMES = ["xz", "conv1d_weight", "conv1d_bias", "x_proj_weight", "delta_proj_weight", "out_proj_weight",
         "out_proj_bias", "A", "B", "C", "D", "delta_bias", "B_proj_bias", "C_proj_bias"]


def _bwd_case(seed, given):
    p = _params(seed, batch=2, d_inner=3, L=7, d_state=2, rank=2, d_model=2)
    g = torch.Generator().manual_seed(seed + 1)
    if given:
        p["B"] = torch.randn(2, 1, 2, 7, generator=g, dtype=torch.float64)
        p["C"] = torch.randn(3, 2, generator=g, dtype=torch.float64) if given == "mixed" else \
            torch.randn(2, 1, 2, 7, generator=g, dtype=torch.float64)
    else:
        p["B_proj_bias"] = torch.randn(2, generator=g, dtype=torch.float64) * 0.1
        p["C_proj_bias"] = torch.randn(2, generator=g, dtype=torch.float64) * 0.1
    dout = torch.randn(2, 7, 2, generator=g, dtype=torch.float64)
    return p, dout


def _autograd(p, dout, **kw):
    leaves = {k: (v.clone().requires_grad_(True) if torch.is_tensor(v) else v) for k, v in p.items()}
    y = mamba_inner_ref(*[leaves.get(k) for k in NAMES], round_to=None, compute_dtype=torch.float64, **kw)
    y.backward(dout)
    return {k: v.grad for k, v in leaves.items() if torch.is_tensor(v)}


def _restated(p, dout, **kw):
    args = {k: p.get(k) for k in NAMES}
    return mamba_inner_bwd_ref(*[args[k] for k in NAMES[:8]], dout, B=args["B"], C=args["C"], D=args["D"],
                               delta_bias=args["delta_bias"], B_proj_bias=args["B_proj_bias"],
                               C_proj_bias=args["C_proj_bias"], compute_dtype=torch.float64, **kw)


def _same(got, want, names, rtol=1e-10, atol=1e-12):
    for k in names:
        assert got[k] is not None, k
        torch.testing.assert_close(got[k], want[k], rtol=rtol, atol=atol, msg=lambda m: f"d{k}: {m}")


@pytest.mark.parametrize("lvl", [0, 1])
@pytest.mark.parametrize("given", [None, "variable", "mixed"])
def test_bwd_restatement_is_the_gradient_without_norms(lvl, given):
    p, dout = _bwd_case(41 + lvl, given)
    want = _autograd(p, dout)
    got = _restated(p, dout, checkpoint_lvl=lvl)
    _same(got, want, [k for k in want])


def test_bwd_restatement_with_norms_passes_them_unchanged(monkeypatch):
    """checkpoint_lvl 0 (no second normalisation): the reference's gradients are those of the block
    with each RMSNorm replaced by its value and an identity gradient."""
    p, dout = _bwd_case(51, None)
    g = torch.Generator().manual_seed(52)
    rw = dict(b_rms_weight=torch.rand(2, generator=g, dtype=torch.float64) + 0.5,
              c_rms_weight=torch.rand(2, generator=g, dtype=torch.float64) + 0.5,
              dt_rms_weight=torch.rand(3, generator=g, dtype=torch.float64) + 0.5)
    got = _restated(p, dout, checkpoint_lvl=0, **rw)
    orig = inner_mod.rms_norm_ref

    def straight_through(x, weight, eps=1e-6, dim=-1, compute_dtype=torch.float32):
        y = orig(x.detach(), weight.detach(), eps, dim, compute_dtype)
        return x + (y - x).detach()
    monkeypatch.setattr(inner_mod, "rms_norm_ref", straight_through)
    want = _autograd(p, dout, **rw)
    _same(got, want, [k for k in want])


def test_bwd_restatement_second_normalisation():
    """checkpoint_lvl 1 normalises the saved, normalised B and C again: with unit weights and eps 0
    that changes nothing (x / rms(x) has rms 1), so the gradients equal checkpoint_lvl 0's; with
    other weights they differ (the reference's behaviour, reproduced)."""
    p, dout = _bwd_case(61, None)
    unit = dict(b_rms_weight=torch.ones(2, dtype=torch.float64), c_rms_weight=torch.ones(2, dtype=torch.float64),
                b_c_dt_rms_eps=0.0)
    g0 = _restated(p, dout, checkpoint_lvl=0, **unit)
    g1 = _restated(p, dout, checkpoint_lvl=1, **unit)
    _same(g1, g0, [k for k in g0 if g0[k] is not None], rtol=1e-9, atol=1e-11)
    w = dict(b_rms_weight=torch.tensor([0.5, 2.0], dtype=torch.float64),
             c_rms_weight=torch.tensor([1.5, 0.7], dtype=torch.float64))
    g0 = _restated(p, dout, checkpoint_lvl=0, **w)
    g1 = _restated(p, dout, checkpoint_lvl=1, **w)
    assert (g1["A"] - g0["A"]).abs().max() > 1e-6 * g0["A"].abs().max()
