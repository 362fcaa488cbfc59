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
  compared with) against finite differences.

CPU only.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.inner_ref import mamba_inner_brute, mamba_inner_ref, rms_norm_ref


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
