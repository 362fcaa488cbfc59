"""Pins for the low-rank coupled (MotifMamba P/Q) oracle ``selective_scan_pq_ref``, which restates
``selective_scan_full_matrix_cuda`` (reference mamba_ssm/ops/selective_scan_interface.py:262-350).

Every check compares against something computed another way: the float64 transition-matrix brute
force (``brute.scan_pq_brute``: products of the dense N x N matrices diag(exp(dt A)) + dt P Q), the C
float64 restatement (W = P Q formed first), the P = 0 reduction to the pinned diagonal oracle, a
scalar closed form (N = R = 1, constant dt: a geometric filter with ratio exp(dt A) + dt p q,
checked against numpy.convolve), the gauge invariance P -> P M, Q -> M^-1 Q, per-channel P/Q with
equal slices against shared P/Q, and channel-permutation equivariance. Planted mistakes
(transposed coupling, flipped sign, shared-instead-of-per-channel, dropped coupling) must fail
the brute-force check.

CPU only; no GPU needed.
"""
import math

import numpy as np
import pytest
import torch

from oracle import brute, cscan
from oracle.ssm_ref import selective_scan_pq_ref, selective_scan_ref


def _pq_case(seed, batch=2, dim=3, L=6, N=3, R=2, bkind="3d", ckind="3d", G=1, per_dim=False,
             with_D=True, with_z=True, with_bias=True, softplus=True, pq_std=0.5):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, L, generator=g)
    delta = torch.randn(batch, dim, L, generator=g) * 0.5
    z = torch.randn(batch, dim, L, generator=g) if with_z else None
    A = -torch.rand(dim, N, generator=g) * 2 - 0.1
    shapes = {"3d": (batch, N, L), "4d": (batch, G, N, L), "const": (dim, N)}
    B = torch.randn(*shapes[bkind], generator=g)
    C = torch.randn(*shapes[ckind], generator=g)
    D = torch.randn(dim, generator=g) if with_D else None
    bias = torch.rand(dim, generator=g) - 0.5 if with_bias else None
    if per_dim:
        P = torch.randn(dim, N, R, generator=g) * pq_std
        Q = torch.randn(dim, R, N, generator=g) * pq_std
    else:
        P = torch.randn(N, R, generator=g) * pq_std
        Q = torch.randn(R, N, generator=g) * pq_std
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=bias, delta_softplus=softplus,
                P=P, Q=Q)


def _l(t):
    return None if t is None else t.double().tolist()


def _brute(case, bkind, ckind):
    return brute.scan_pq_brute(_l(case["u"]), _l(case["delta"]), _l(case["A"]), _l(case["B"]),
                               _l(case["C"]), _l(case["P"]), _l(case["Q"]), _l(case["D"]),
                               _l(case["z"]), _l(case["delta_bias"]), case["delta_softplus"],
                               bkind, ckind)


def _check_vs_brute(fn, case, bkind, ckind, tol=2e-5):
    out, last = fn(**case, return_last_state=True)
    ref_out, ref_outz, ref_last = _brute(case, bkind, ckind)
    expect = np.array(ref_outz if case["z"] is not None else ref_out)
    np.testing.assert_allclose(out.double().numpy(), expect, rtol=tol, atol=tol)
    np.testing.assert_allclose(last.double().numpy(), np.array(ref_last), rtol=tol, atol=tol)


@pytest.mark.parametrize("bkind,ckind,G", [("3d", "3d", 1), ("4d", "4d", 3), ("const", "const", 1),
                                           ("3d", "const", 1), ("const", "4d", 3)])
@pytest.mark.parametrize("per_dim", [False, True])
def test_pq_oracle_vs_transition_matrix_brute(bkind, ckind, G, per_dim):
    case = _pq_case(100 + 7 * G + per_dim, bkind=bkind, ckind=ckind, G=G, per_dim=per_dim)
    _check_vs_brute(selective_scan_pq_ref, case, bkind, ckind)


@pytest.mark.parametrize("flags", [dict(with_D=False), dict(with_z=False), dict(with_bias=False),
                                   dict(softplus=False), dict(R=1), dict(R=4, N=4)])
def test_pq_oracle_optional_inputs(flags):
    case = _pq_case(130 + len(str(flags)), **flags)
    _check_vs_brute(selective_scan_pq_ref, case, "3d", "3d")


def test_pq_oracle_c_f64_matches_brute():
    for per_dim, seed in ((False, 140), (True, 141)):
        case = _pq_case(seed, per_dim=per_dim, bkind="4d", ckind="4d", G=3)
        ref_out, ref_outz, ref_last = _brute(case, "4d", "4d")
        r = cscan.scan_rows(case["u"], case["delta"], case["A"], case["B"], case["C"], case["D"],
                            case["z"], case["delta_bias"], True, P=case["P"], Q=case["Q"])
        b, d, L = case["u"].shape
        np.testing.assert_allclose(r["out"].reshape(b, d, L), np.array(ref_out), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(r["out_z"].reshape(b, d, L), np.array(ref_outz), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(r["last_state"].reshape(b, d, -1), np.array(ref_last), rtol=1e-10, atol=1e-12)


def test_pq_all_rows_wrapper_matches_brute():
    """cscan.scan_all_rows with P/Q (one call per (batch, group), B/C shared with a row stride of 0,
    per-channel P/Q sliced by group) against the transition-matrix brute force."""
    for per_dim, seed in ((False, 145), (True, 146)):
        case = _pq_case(seed, dim=6, per_dim=per_dim, bkind="4d", ckind="4d", G=3)
        ref_out, ref_outz, ref_last = _brute(case, "4d", "4d")
        y, last = cscan.scan_all_rows(case["u"], case["delta"], case["A"], case["B"], case["C"], case["D"],
                                      case["z"], case["delta_bias"], True, P=case["P"], Q=case["Q"])
        np.testing.assert_allclose(y, np.array(ref_outz), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(last, np.array(ref_last), rtol=1e-10, atol=1e-12)


def test_pq_zero_coupling_is_the_diagonal_scan():
    case = _pq_case(150, dim=5, L=40, N=16, bkind="4d", ckind="4d", G=5)
    case["P"] = torch.zeros_like(case["P"])
    out, last = selective_scan_pq_ref(**case, return_last_state=True)
    kw = {k: v for k, v in case.items() if k not in ("P", "Q")}
    ref, ref_last = selective_scan_ref(**kw, return_last_state=True)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(last, ref_last, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dt", [0.3, 1.7])
def test_pq_scalar_closed_form(dt):
    """N = R = 1, constant dt, B = C = 1, no softplus: h_t = rho h_{t-1} + dt u_t with
    rho = exp(dt A) + dt p q, so out = (rho^k) * (dt u) as a causal convolution."""
    L = 30
    g = torch.Generator().manual_seed(160)
    u = torch.randn(1, 1, L, generator=g, dtype=torch.float64)
    A, p, q = -0.8, 0.6, -0.45
    rho = math.exp(dt * A) + dt * p * q
    kern = rho ** np.arange(L)
    expect = np.convolve(dt * u[0, 0].numpy(), kern)[:L]
    out, last = selective_scan_pq_ref(u.float(), torch.full((1, 1, L), dt), torch.tensor([[A]]),
                                      torch.ones(1, 1, L), torch.ones(1, 1, L), return_last_state=True,
                                      P=torch.tensor([[p]]), Q=torch.tensor([[q]]))
    np.testing.assert_allclose(out[0, 0].double().numpy(), expect, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(last[0, 0, 0].item(), expect[-1], rtol=2e-5, atol=2e-6)


def test_pq_gauge_invariance():
    """Only the product P Q enters: P -> P M, Q -> M^-1 Q leaves the outputs unchanged."""
    case = _pq_case(170, dim=4, L=50, N=8, R=3, bkind="3d", ckind="3d")
    g = torch.Generator().manual_seed(171)
    M = torch.eye(3) + 0.3 * torch.randn(3, 3, generator=g)
    out, last = selective_scan_pq_ref(**case, return_last_state=True)
    out2, last2 = selective_scan_pq_ref(**{**case, "P": case["P"] @ M, "Q": torch.linalg.solve(M, case["Q"])},
                                        return_last_state=True)
    torch.testing.assert_close(out, out2, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(last, last2, rtol=1e-4, atol=1e-5)


def test_pq_per_dim_equal_slices_is_shared_and_permutes_with_channels():
    case = _pq_case(180, dim=6, L=30, N=4, R=2)
    shared, s_last = selective_scan_pq_ref(**case, return_last_state=True)
    P3 = case["P"].unsqueeze(0).expand(6, -1, -1).contiguous()
    Q3 = case["Q"].unsqueeze(0).expand(6, -1, -1).contiguous()
    per, p_last = selective_scan_pq_ref(**{**case, "P": P3, "Q": Q3}, return_last_state=True)
    torch.testing.assert_close(per, shared, rtol=0, atol=0)
    torch.testing.assert_close(p_last, s_last, rtol=0, atol=0)
    # per-channel P/Q travel with their channel
    c2 = _pq_case(181, dim=6, L=30, N=4, R=2, per_dim=True)
    perm = torch.tensor([3, 0, 5, 1, 4, 2])
    out, last = selective_scan_pq_ref(**c2, return_last_state=True)
    cp = dict(c2)
    for k in ("u", "delta", "z"):
        cp[k] = c2[k][:, perm]
    for k in ("A", "D", "delta_bias", "P", "Q"):
        cp[k] = c2[k][perm]
    out_p, last_p = selective_scan_pq_ref(**cp, return_last_state=True)
    torch.testing.assert_close(out_p, out[:, perm], rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(last_p, last[:, perm], rtol=1e-6, atol=1e-6)


def test_pq_oracle_argument_errors():
    case = _pq_case(190)
    with pytest.raises(ValueError, match="both be provided"):
        selective_scan_pq_ref(**{**case, "Q": None})
    with pytest.raises(ValueError, match="both be 2D or both be 3D"):
        selective_scan_pq_ref(**{**case, "P": case["P"].unsqueeze(0)})
    with pytest.raises(ValueError, match=r"Expected P\(n, r\)"):
        selective_scan_pq_ref(**{**case, "P": torch.randn(4, 2)})
    with pytest.raises(ValueError, match=r"Expected P\(dim, n, r\)"):
        selective_scan_pq_ref(**{**case, "P": torch.randn(2, 3, 2), "Q": torch.randn(2, 2, 3)})


# ---------------------------------------------------------------------------------------------
# Planted mistakes must fail the brute-force pin.
# ---------------------------------------------------------------------------------------------
def _fails(check):
    try:
        check()
    except AssertionError:
        return True
    return False


def test_pq_mutants_are_caught():
    case = _pq_case(200, N=4, R=2)
    case_pd = _pq_case(201, N=4, R=2, per_dim=True)

    def transposed(**kw):   # W^T = Q^T P^T instead of W = P Q
        return selective_scan_pq_ref(**{**kw, "P": kw["Q"].transpose(-1, -2), "Q": kw["P"].transpose(-1, -2)})

    def flipped(**kw):
        return selective_scan_pq_ref(**{**kw, "P": -kw["P"]})

    def dropped(**kw):
        return selective_scan_pq_ref(**{**kw, "P": torch.zeros_like(kw["P"])})

    def shared_instead_of_per_dim(**kw):
        return selective_scan_pq_ref(**{**kw, "P": kw["P"][0], "Q": kw["Q"][0]})

    assert _fails(lambda: _check_vs_brute(transposed, case, "3d", "3d"))
    assert _fails(lambda: _check_vs_brute(flipped, case, "3d", "3d"))
    assert _fails(lambda: _check_vs_brute(dropped, case, "3d", "3d"))
    assert _fails(lambda: _check_vs_brute(shared_instead_of_per_dim, case_pd, "3d", "3d"))
    _check_vs_brute(selective_scan_pq_ref, case, "3d", "3d")
    _check_vs_brute(selective_scan_pq_ref, case_pd, "3d", "3d")
