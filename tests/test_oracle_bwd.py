"""Pins for the backward oracle ``selective_scan_bwd_ref`` (autograd through the restatement of
ssi.py:353-451; the function the reference's selective_scan_cuda.bwd computes,
selective_scan.cpp:415-612, selective_scan_bwd_kernel.cuh:405-880):

* finite differences in float64 (torch.autograd.gradcheck) on tiny shapes pin the autograd path;
* the explicit float64 adjoint recurrence ``brute.scan_bwd_brute`` (reverse scan of the state
  adjoint and the per-step contributions, written without autograd) agrees with it to 1e-9 on every
  B/C layout and flag combination -- the recurrence the GPU kernels implement;
* the L = 1 closed form (out = dt u <B, C> + D u) gives every gradient by hand.

CPU only; no GPU needed.
"""
import math

import numpy as np
import pytest
import torch

from oracle import brute
from oracle.ssm_ref import selective_scan_bwd_ref, selective_scan_ref


def _case(seed, batch=2, dim=4, L=6, N=3, bkind="3d", ckind="3d", G=2, with_D=True, with_z=True,
          with_bias=True, softplus=True, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, L, generator=g, dtype=torch.float64)
    delta = torch.randn(batch, dim, L, generator=g, dtype=torch.float64) * 0.5
    z = torch.randn(batch, dim, L, generator=g, dtype=torch.float64) if with_z else None
    A = -torch.rand(dim, N, generator=g, dtype=torch.float64) * 2 - 0.1
    shapes = {"3d": (batch, N, L), "4d": (batch, G, N, L), "const": (dim, N)}
    B = torch.randn(*shapes[bkind], generator=g, dtype=torch.float64)
    C = torch.randn(*shapes[ckind], generator=g, dtype=torch.float64)
    D = torch.randn(dim, generator=g, dtype=torch.float64) if with_D else None
    bias = (torch.rand(dim, generator=g, dtype=torch.float64) - 0.5) if with_bias else None
    if not softplus:
        delta = delta.abs()
    dout = torch.randn(batch, dim, L, generator=g, dtype=torch.float64)
    c = dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=bias, delta_softplus=softplus)
    return {k: (v.to(dtype) if torch.is_tensor(v) and k not in ("A", "D", "delta_bias") else v)
            for k, v in c.items()}, dout


def _l(t):
    return None if t is None else t.double().tolist()


@pytest.mark.parametrize("bkind,ckind,G", [("3d", "3d", 1), ("4d", "4d", 2), ("const", "const", 1),
                                           ("3d", "const", 1), ("const", "4d", 2)])
@pytest.mark.parametrize("flags", [dict(), dict(with_z=False), dict(with_D=False, with_bias=False),
                                   dict(softplus=False)])
def test_bwd_oracle_matches_explicit_adjoint(bkind, ckind, G, flags):
    case, dout = _case(500 + G + len(str(flags)), bkind=bkind, ckind=ckind, G=G, **flags)
    got = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    ref = brute.scan_bwd_brute(_l(case["u"]), _l(case["delta"]), _l(case["A"]), _l(case["B"]), _l(case["C"]),
                               _l(dout), _l(case["D"]), _l(case["z"]), _l(case["delta_bias"]),
                               case["delta_softplus"], bkind, ckind)
    for k in ("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"):
        if ref[k] is None:
            assert got[k] is None, k
            continue
        np.testing.assert_allclose(got[k].numpy(), np.array(ref[k]), rtol=1e-9, atol=1e-11, err_msg=k)


@pytest.mark.parametrize("bkind,G", [("3d", 1), ("4d", 2), ("4d", 1)])
@pytest.mark.parametrize("flags", [dict(), dict(with_z=False), dict(with_D=False, with_bias=False),
                                   dict(softplus=False)])
@pytest.mark.parametrize("L", [1, 37])
def test_c_adjoint_matches_explicit_adjoint(bkind, G, flags, L):
    """The float64 C adjoint (oracle/scan_f64.c, mm_oracle_scan_bwd_rows_f64: the full-size
    checker of the GPU backward) equals the explicit adjoint brute.scan_bwd_brute, every gradient,
    on each variable-B/C layout and flag combination; softplus past its threshold of 20 is
    included (delta + bias > 20 on some steps)."""
    from oracle import cscan
    case, dout = _case(540 + G + L + len(str(flags)), batch=2, dim=4, L=L, N=3, bkind=bkind, ckind=bkind, G=G,
                       **flags)
    if flags.get("softplus", True):
        case["delta"] = case["delta"].clone()
        case["delta"][0, 1, ::3] = 25.0        # the softplus threshold: ddelta = ddt' there
    ref = brute.scan_bwd_brute(_l(case["u"]), _l(case["delta"]), _l(case["A"]), _l(case["B"]), _l(case["C"]),
                               _l(dout), _l(case["D"]), _l(case["z"]), _l(case["delta_bias"]),
                               case["delta_softplus"], bkind, bkind)
    got = cscan.scan_bwd_all_rows(case["u"], case["delta"], case["A"], case["B"], case["C"], dout, D=case["D"],
                                  z=case["z"], delta_bias=case["delta_bias"], delta_softplus=case["delta_softplus"])
    for k in ("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"):
        if ref[k] is None:
            assert got[k] is None, k
            continue
        np.testing.assert_allclose(got[k], np.array(ref[k]), rtol=1e-10, atol=1e-12, err_msg=k)


def test_bwd_oracle_finite_differences():
    case, dout = _case(520, batch=1, dim=2, L=5, N=2, bkind="4d", ckind="4d", G=2)
    names = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias"]
    tensors = [case[n].detach().clone().requires_grad_(True) for n in names]

    def f(*ts):
        kw = dict(zip(names, ts))
        return (selective_scan_ref(**kw, delta_softplus=True, compute_dtype=torch.float64) * dout).sum()

    assert torch.autograd.gradcheck(f, tensors, eps=1e-6, atol=1e-7, rtol=1e-5)


def test_bwd_oracle_single_step_closed_form():
    """L = 1, no z: out = dt u <B, C> + D u with dt = softplus(delta + bias)."""
    case, dout = _case(530, batch=2, dim=3, L=1, N=4, with_z=False)
    got = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    u, B, C, D, A = case["u"][..., 0], case["B"][..., 0], case["C"][..., 0], case["D"], case["A"]
    raw = case["delta"][..., 0] + case["delta_bias"]
    dt = torch.nn.functional.softplus(raw)
    g = dout[..., 0]
    bc = (B * C).sum(-1)                                   # (batch,)
    np.testing.assert_allclose(got["du"][..., 0], g * (dt * bc[:, None] + D), rtol=1e-12)
    np.testing.assert_allclose(got["ddelta"][..., 0], g * u * bc[:, None] * torch.sigmoid(raw), rtol=1e-12)
    np.testing.assert_allclose(got["dD"], (g * u).sum(0), rtol=1e-12)
    np.testing.assert_allclose(got["dB"][..., 0], ((g * dt * u)[..., None] * C[:, None, :]).sum(1), rtol=1e-12)
    np.testing.assert_allclose(got["dC"][..., 0], ((g * dt * u)[..., None] * B[:, None, :]).sum(1), rtol=1e-12)
    np.testing.assert_allclose(got["dA"], torch.zeros_like(A), atol=0)   # h_{-1} = 0: A is not reached


def test_bwd_oracle_output_dtypes_follow_the_reference():
    case, dout = _case(540, dtype=torch.bfloat16)
    case = {k: (v.to(torch.bfloat16) if k in ("u", "delta", "z", "B", "C") else v) for k, v in case.items()}
    case["A"], case["D"], case["delta_bias"] = case["A"].float(), case["D"].float(), case["delta_bias"].float()
    got = selective_scan_bwd_ref(**case, dout=dout.to(torch.bfloat16))
    assert got["du"].dtype == got["ddelta"].dtype == got["dz"].dtype == torch.bfloat16
    assert got["dB"].dtype == got["dC"].dtype == torch.bfloat16
    assert got["dA"].dtype == got["dD"].dtype == got["ddelta_bias"].dtype == torch.float32
