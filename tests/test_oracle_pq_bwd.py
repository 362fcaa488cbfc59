"""Pins for the gradient oracle of the low-rank coupled (MotifMamba P/Q) scan,
``selective_scan_pq_bwd_ref``: torch autograd through ``selective_scan_pq_ref`` (the restatement of
reference mamba_ssm/ops/selective_scan_interface.py:262-350), which is what the reference returns in
its default gradient mode (ssi.py:152-205).

Every check computes the gradient another way: the float64 explicit adjoint
``brute.scan_pq_bwd_brute`` (reverse scan through the transposed dense transition matrices
diag(exp(dt A)) + dt P Q, with dP = dW Q^T and dQ = P^T dW), central finite differences of the
forward, the P = 0 reduction to the pinned diagonal gradient oracle, and the gauge transform
P -> P M, Q -> M^-1 Q (dP -> dP M^-T, dQ -> M^T dQ, every other gradient unchanged). Planted
mistakes (transposed coupling, coupling dropped from the adjoint) must fail the adjoint check.

CPU only; no GPU needed.
"""
import numpy as np
import pytest
import torch

from oracle import brute
from oracle.ssm_ref import selective_scan_bwd_ref, selective_scan_pq_bwd_ref, selective_scan_pq_ref
from tests.test_oracle_pq import _pq_case

NAMES = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias", "P", "Q"]


def _l(t):
    return None if t is None else t.double().tolist()


def _dout(seed, shape):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


def _brute(case, dout, bkind, ckind):
    return brute.scan_pq_bwd_brute(_l(case["u"]), _l(case["delta"]), _l(case["A"]), _l(case["B"]),
                                   _l(case["C"]), _l(case["P"]), _l(case["Q"]), _l(dout), _l(case["D"]),
                                   _l(case["z"]), _l(case["delta_bias"]), case["delta_softplus"], bkind, ckind)


def _agree(got, ref, rtol=1e-9, atol=1e-10):
    for n in NAMES:
        g, r = got["d" + n], ref["d" + n]
        if r is None:
            assert g is None, n
            continue
        np.testing.assert_allclose(g.numpy(), np.array(r), rtol=rtol, atol=atol, err_msg="d" + n)


@pytest.mark.parametrize("bkind,ckind,G", [("3d", "3d", 1), ("4d", "4d", 3), ("const", "const", 1),
                                           ("3d", "const", 1), ("const", "4d", 3)])
@pytest.mark.parametrize("per_dim", [False, True])
def test_pq_bwd_oracle_matches_explicit_adjoint(bkind, ckind, G, per_dim):
    case = _pq_case(300 + 7 * G + per_dim, bkind=bkind, ckind=ckind, G=G, per_dim=per_dim)
    dout = _dout(301, case["u"].shape)
    got = selective_scan_pq_bwd_ref(**case, dout=dout)
    _agree(got, _brute(case, dout, bkind, ckind))


@pytest.mark.parametrize("flags", [dict(with_D=False), dict(with_z=False), dict(with_bias=False),
                                   dict(softplus=False), dict(R=1), dict(R=4, N=4)])
def test_pq_bwd_oracle_optional_inputs(flags):
    case = _pq_case(320 + len(str(flags)), **flags)
    dout = _dout(321, case["u"].shape)
    _agree(selective_scan_pq_bwd_ref(**case, dout=dout), _brute(case, dout, "3d", "3d"))


def test_pq_bwd_oracle_finite_differences():
    """<grad, E> against (f(x + eps E) - f(x - eps E)) / 2 eps of the float64 forward, for a random
    direction E in every input."""
    case = {k: (v.double() if torch.is_tensor(v) else v)
            for k, v in _pq_case(330, batch=1, dim=2, L=5, N=3, R=2, per_dim=True).items()}
    dout = _dout(331, case["u"].shape).double()
    grads = selective_scan_pq_bwd_ref(**case, dout=dout)
    gen = torch.Generator().manual_seed(332)
    eps = 1e-6
    for n in NAMES:
        E = torch.randn(case[n].shape, generator=gen, dtype=torch.float64)
        plus = dict(case, **{n: case[n] + eps * E})
        minus = dict(case, **{n: case[n] - eps * E})
        fp = (selective_scan_pq_ref(**plus, compute_dtype=torch.float64) * dout).sum().item()
        fm = (selective_scan_pq_ref(**minus, compute_dtype=torch.float64) * dout).sum().item()
        fd = (fp - fm) / (2 * eps)
        an = (grads["d" + n] * E).sum().item()
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (n, fd, an)


def test_pq_bwd_zero_coupling_is_the_diagonal_gradient():
    """P = 0: the recurrence is the diagonal scan, so every gradient but dP/dQ is the pinned
    diagonal oracle's; dQ = P^T dW = 0 and dP = dW Q^T with dW = sum_t dt_t lam_t h_{t-1}^T."""
    case = _pq_case(340, dim=4, L=20, N=6, R=2, bkind="4d", ckind="4d", G=2)
    case["P"] = torch.zeros_like(case["P"])
    dout = _dout(341, case["u"].shape)
    got = selective_scan_pq_bwd_ref(**case, dout=dout)
    kw = {k: v for k, v in case.items() if k not in ("P", "Q")}
    diag = selective_scan_bwd_ref(**kw, dout=dout, dtype=torch.float64)
    for n in ["u", "delta", "A", "B", "C", "D", "z", "delta_bias"]:
        torch.testing.assert_close(got["d" + n], diag["d" + n], rtol=1e-10, atol=1e-12)
    assert float(got["dQ"].abs().max()) == 0.0
    assert float(got["dP"].abs().max()) > 1e-3


def test_pq_bwd_gauge_transform():
    case = _pq_case(350, dim=3, L=16, N=5, R=3)
    dout = _dout(351, case["u"].shape)
    g = torch.Generator().manual_seed(352)
    M = (torch.eye(3) + 0.3 * torch.randn(3, 3, generator=g)).double()
    base = selective_scan_pq_bwd_ref(**case, dout=dout)
    P2 = case["P"].double() @ M
    Q2 = torch.linalg.solve(M, case["Q"].double())
    moved = selective_scan_pq_bwd_ref(**dict(case, P=P2, Q=Q2), dout=dout)
    for n in ["u", "delta", "A", "B", "C", "D", "z", "delta_bias"]:
        torch.testing.assert_close(moved["d" + n], base["d" + n], rtol=1e-8, atol=1e-10)
    torch.testing.assert_close(moved["dP"], base["dP"] @ torch.linalg.inv(M).T, rtol=1e-8, atol=1e-10)
    torch.testing.assert_close(moved["dQ"], M.T @ base["dQ"], rtol=1e-8, atol=1e-10)


def test_pq_bwd_planted_mistakes_fail():
    """A transposed coupling (W^T for W) and an adjoint without the coupling term both move the
    gradients far beyond the tolerance of the adjoint check."""
    case = _pq_case(360, dim=2, L=8, N=4, R=2)
    dout = _dout(361, case["u"].shape)
    ref = _brute(case, dout, "3d", "3d")
    transposed = selective_scan_pq_bwd_ref(**dict(case, P=case["Q"].T.contiguous(), Q=case["P"].T.contiguous()),
                                           dout=dout)
    with pytest.raises(AssertionError):
        _agree(transposed, ref)
    # Dropping the coupling from the adjoint = the diagonal adjoint of the coupled forward's inputs.
    kw = {k: v for k, v in case.items() if k not in ("P", "Q")}
    diag = selective_scan_bwd_ref(**kw, dout=dout, dtype=torch.float64)
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(diag["du"].numpy(), np.array(ref["du"]), rtol=1e-6, atol=1e-8)
