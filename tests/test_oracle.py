"""Pins for the CPU oracle (oracle/): every restated function is checked against something that a
plausible mistake would break -- a hand-worked known answer, the float64 closed-sum brute force,
closed forms, invariants and the C float64 restatement -- and the mutation tests at the bottom
show that those checks do fail for planted mistakes (dropped D, swapped B/C, wrong group
interleave, missing softplus, sigmoid gate).

CPU only; no GPU needed.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from einops import repeat

from oracle import brute, cscan
from oracle.ssm_ref import (chunk_states_ref, selective_scan_ref, selective_scan_ref_chunked,
                            selective_state_update_ref)


def _rand_case(seed, batch=2, dim=4, L=6, N=3, bkind="3d", ckind="3d", G=2, with_D=True,
               with_z=True, with_bias=True, softplus=True):
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
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=bias, delta_softplus=softplus)


def _to_list(t):
    return None if t is None else t.double().tolist()


def _brute(case, bkind, ckind):
    return brute.scan_brute(_to_list(case["u"]), _to_list(case["delta"]), _to_list(case["A"]),
                            _to_list(case["B"]), _to_list(case["C"]), _to_list(case["D"]),
                            _to_list(case["z"]), _to_list(case["delta_bias"]),
                            case["delta_softplus"], bkind, ckind)


def _check_vs_brute(fn, case, bkind, ckind, tol=2e-5):
    out, last = fn(**case, return_last_state=True)
    ref_out, ref_outz, ref_last = _brute(case, bkind, ckind)
    expect = np.array(ref_outz if case["z"] is not None else ref_out)
    np.testing.assert_allclose(out.double().numpy(), expect, rtol=tol, atol=tol)
    np.testing.assert_allclose(last.double().numpy(), np.array(ref_last), rtol=tol, atol=tol)


# ---------------------------------------------------------------------------------------------
# Hand-worked known answer (A = -ln 2 so that exp(delta*A) = 1/2 at delta = 1).
# h0 = 1, h1 = 0.5*1 + 2 = 2.5, h2 = 0.5*2.5 + 4 = 5.25; y = h*C = (1, 5, 15.75); out = y + 0.5 u.
# ---------------------------------------------------------------------------------------------
KNOWN_OUT = [1.5, 6.0, 17.75]
KNOWN_LAST = 5.25


@pytest.mark.parametrize("softplus", [False, True])
def test_known_answer(softplus):
    raw = 1.0 if not softplus else math.log(math.e - 1.0)   # softplus(log(e-1)) = 1
    u = torch.tensor([[[1.0, 2.0, 4.0]]])
    delta = torch.full((1, 1, 3), raw)
    A = torch.tensor([[-math.log(2.0)]])
    B = torch.ones(1, 1, 3)
    C = torch.tensor([[[1.0, 2.0, 3.0]]])
    D = torch.tensor([0.5])
    out, last = selective_scan_ref(u, delta, A, B, C, D, delta_softplus=softplus, return_last_state=True)
    np.testing.assert_allclose(out[0, 0].numpy(), KNOWN_OUT, rtol=1e-6)
    np.testing.assert_allclose(last[0, 0, 0].item(), KNOWN_LAST, rtol=1e-6)
    # the same case through the two float64 restatements
    bo, _, bl = brute.scan_brute(u.tolist(), delta.tolist(), A.tolist(), B.tolist(), C.tolist(),
                                 D.tolist(), None, None, softplus, "3d", "3d")
    np.testing.assert_allclose(bo[0][0], KNOWN_OUT, rtol=1e-7)  # A is -ln2 rounded to f32
    r = cscan.scan_rows(u, delta, A, B, C, D, delta_softplus=softplus)
    np.testing.assert_allclose(r["out"][0], KNOWN_OUT, rtol=1e-7)
    np.testing.assert_allclose(r["last_state"][0, 0], KNOWN_LAST, rtol=1e-7)


@pytest.mark.parametrize("bkind,ckind", [("3d", "3d"), ("4d", "4d"), ("const", "const"),
                                         ("3d", "const"), ("const", "4d")])
@pytest.mark.parametrize("flags", [dict(), dict(with_D=False), dict(with_z=False),
                                   dict(with_bias=False, softplus=False)])
def test_oracle_vs_brute_force(bkind, ckind, flags):
    case = _rand_case(11, bkind=bkind, ckind=ckind, **flags)
    _check_vs_brute(selective_scan_ref, case, bkind, ckind)


@pytest.mark.parametrize("seed,G", [(3, 1), (4, 2), (5, 4)])
def test_c_oracle_matches_torch_oracle(seed, G):
    case = _rand_case(seed, batch=2, dim=8, L=300, N=16, bkind="4d", ckind="4d", G=G)
    out, last = selective_scan_ref(**case, return_last_state=True)
    r = cscan.scan_rows(**case, chunk=128)
    np.testing.assert_allclose(r["out_z"].reshape(out.shape), out.double().numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(r["last_state"].reshape(last.shape), last.double().numpy(), rtol=1e-4, atol=1e-5)
    # state at each chunk end == last_state of the scan over the prefix
    for c, end in enumerate((128, 256, 300)):
        sub = {k: (v[..., :end] if torch.is_tensor(v) and v.dim() >= 3 else v) for k, v in case.items()}
        _, lst = selective_scan_ref(**sub, return_last_state=True)
        np.testing.assert_allclose(r["h_chunks"][:, c, :].reshape(lst.shape), lst.double().numpy(),
                                   rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------------------------
# Closed forms
# ---------------------------------------------------------------------------------------------
def _sp64(x):
    x = np.asarray(x, dtype=np.float64)
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))


def test_closed_form_single_step():
    case = _rand_case(21, batch=3, dim=5, L=1, N=7, bkind="3d", ckind="3d", with_z=False)
    out = selective_scan_ref(**case)
    dt = _sp64(case["delta"].double().numpy() + case["delta_bias"].double().numpy()[None, :, None])
    u = case["u"].double().numpy()
    bc = np.einsum("bnl,bnl->bl", case["B"].double().numpy(), case["C"].double().numpy())
    expect = dt * u * bc[:, None, :] + case["D"].double().numpy()[None, :, None] * u
    np.testing.assert_allclose(out.double().numpy(), expect, rtol=1e-5, atol=1e-6)


def test_closed_form_zero_delta():
    case = _rand_case(22, batch=2, dim=6, L=40, N=4, with_z=False, with_bias=False, softplus=False)
    case["delta"] = torch.zeros_like(case["delta"])
    out, last = selective_scan_ref(**case, return_last_state=True)
    expect = case["D"][None, :, None] * case["u"]
    assert torch.equal(out, expect)
    assert torch.count_nonzero(last) == 0


def test_closed_form_memoryless():
    case = _rand_case(23, batch=2, dim=3, L=30, N=5, with_z=False, with_D=False, with_bias=False)
    case["A"] = torch.full_like(case["A"], -1e4)
    out = selective_scan_ref(**case)
    dt = _sp64(case["delta"].double().numpy())
    bc = np.einsum("bnl,bnl->bl", case["B"].double().numpy(), case["C"].double().numpy())
    expect = dt * case["u"].double().numpy() * bc[:, None, :]
    np.testing.assert_allclose(out.double().numpy(), expect, rtol=1e-5, atol=1e-6)


def test_closed_form_geometric_filter():
    """N = 1 with constant delta: h is the causal filter of b_t = delta u_t B_t with taps a^k."""
    L = 64
    g = torch.Generator().manual_seed(24)
    u = torch.randn(1, 1, L, generator=g)
    Bv = torch.randn(1, 1, L, generator=g)
    Cv = torch.randn(1, 1, L, generator=g)
    dval, Aval = 0.3, -0.7
    out = selective_scan_ref(u, torch.full((1, 1, L), dval), torch.tensor([[Aval]]), Bv, Cv)
    a = math.exp(dval * Aval)
    b = dval * u[0, 0].double().numpy() * Bv[0, 0].double().numpy()
    h = np.convolve(b, a ** np.arange(L))[:L]
    np.testing.assert_allclose(out[0, 0].double().numpy(), h * Cv[0, 0].double().numpy(), rtol=1e-5, atol=1e-6)


def test_closed_form_gate_composition():
    case = _rand_case(25, batch=2, dim=4, L=50, N=8)
    gated = selective_scan_ref(**case)
    plain = selective_scan_ref(**{**case, "z": None})
    z = case["z"].double().numpy()
    expect = plain.double().numpy() * z / (1.0 + np.exp(-z))
    np.testing.assert_allclose(gated.double().numpy(), expect, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------------------------
# Invariants
# ---------------------------------------------------------------------------------------------
def test_linearity_in_u():
    case = _rand_case(31, batch=2, dim=4, L=80, N=16, with_z=False)
    u2 = torch.randn(case["u"].shape, generator=torch.Generator().manual_seed(32))
    f = lambda uu: selective_scan_ref(**{**case, "u": uu}).double()
    lhs = f(2.0 * case["u"] - 3.0 * u2)
    rhs = 2.0 * f(case["u"]) - 3.0 * f(u2)
    np.testing.assert_allclose(lhs.numpy(), rhs.numpy(), rtol=1e-4, atol=1e-4)


def test_group_split():
    """G = 4 over dim channels equals four G = 1 scans over consecutive channel blocks."""
    G, dim = 4, 8
    case = _rand_case(33, batch=2, dim=dim, L=60, N=6, bkind="4d", ckind="4d", G=G)
    full, last = selective_scan_ref(**case, return_last_state=True)
    h = dim // G
    for gi in range(G):
        sl = slice(gi * h, (gi + 1) * h)
        sub = dict(case)
        for k in ("u", "delta", "z"):
            sub[k] = case[k][:, sl]
        for k in ("A",):
            sub[k] = case[k][sl]
        for k in ("D", "delta_bias"):
            sub[k] = case[k][sl]
        sub["B"] = case["B"][:, gi]
        sub["C"] = case["C"][:, gi]
        part, plast = selective_scan_ref(**sub, return_last_state=True)
        torch.testing.assert_close(part, full[:, sl], rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(plast, last[:, sl], rtol=1e-6, atol=1e-6)


def test_chunked_oracle_equals_oracle():
    case = _rand_case(34, batch=2, dim=4, L=70, N=16, bkind="4d", ckind="4d")
    a, la = selective_scan_ref(**case, return_last_state=True)
    b, lb = selective_scan_ref_chunked(**case, return_last_state=True, chunk=16)
    torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(la, lb, rtol=1e-6, atol=1e-6)


def test_decode_steps_equal_scan():
    """L decode steps from a zero state reproduce the scan's outputs and final state."""
    case = _rand_case(35, batch=2, dim=6, L=25, N=16, bkind="3d", ckind="3d")
    out, last = selective_scan_ref(**case, return_last_state=True)
    state = torch.zeros(2, 6, 16)
    for t in range(25):
        y = selective_state_update_ref(state, case["u"][:, :, t], case["delta"][:, :, t], case["A"],
                                       case["B"][:, :, t], case["C"][:, :, t], D=case["D"],
                                       z=case["z"][:, :, t], dt_bias=case["delta_bias"], dt_softplus=True)
        torch.testing.assert_close(y, out[:, :, t], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(state, last, rtol=1e-4, atol=1e-5)


def test_decode_grouped_equals_per_group():
    g = torch.Generator().manual_seed(36)
    batch, dim, N, G = 3, 8, 4, 2
    state = torch.randn(batch, dim, N, generator=g)
    x, dt, z = (torch.randn(batch, dim, generator=g) for _ in range(3))
    A = -torch.rand(dim, N, generator=g)
    B = torch.randn(batch, G, N, generator=g)
    C = torch.randn(batch, G, N, generator=g)
    s_full = state.clone()
    y_full = selective_state_update_ref(s_full, x, dt, A, B, C, dt_softplus=True)
    for gi in range(G):
        sl = slice(gi * dim // G, (gi + 1) * dim // G)
        s = state[:, sl].clone()
        y = selective_state_update_ref(s, x[:, sl], dt[:, sl], A[sl], B[:, gi], C[:, gi], dt_softplus=True)
        torch.testing.assert_close(y, y_full[:, sl])
        torch.testing.assert_close(s, s_full[:, sl])


@pytest.mark.parametrize("state_dtype", [torch.bfloat16, torch.float16])
def test_decode_16bit_state_known_answer(state_dtype):
    """Hand-worked step of a 16-bit state (the upstream kernel: widen, update in float32, store with
    round-to-nearest-even, read y from the float32 state). A = 0 makes the decay 1, so the new state
    is exactly s + dt' B x. With s = 1 and an increment of a quarter ulp, half an ulp and three
    quarters of an ulp, RNE stores 1, 1 (tie to even) and 1 + ulp; y = C . state reads the unrounded
    float32 sums (a y from the rounded state, or truncation instead of RNE, fails here)."""
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[state_dtype]
    incs = torch.tensor([0.25 * ulp, 0.5 * ulp, 0.75 * ulp, 1.5 * ulp])      # 1.5 ulp: tie from odd
    state = torch.ones(1, 4, 1, dtype=state_dtype)
    state[0, 3, 0] = 1.0 + ulp                                               # odd last bit
    x = incs[None, :].clone()                                                # dt' B x = inc
    dt = torch.ones(1, 4)
    A = torch.zeros(4, 1)
    B = torch.ones(1, 1)
    C = torch.ones(1, 1)
    y = selective_state_update_ref(state, x, dt, A, B, C, dt_softplus=False)
    exact = torch.tensor([1 + 0.25 * ulp, 1 + 0.5 * ulp, 1 + 0.75 * ulp, 1 + 2.5 * ulp])
    assert torch.equal(y[0].double(), exact.double())
    stored = torch.tensor([1.0, 1.0, 1.0 + ulp, 1.0 + 2 * ulp], dtype=torch.float64)
    assert torch.equal(state[0, :, 0].double(), stored)
    assert state.dtype == state_dtype


def test_decode_16bit_state_steps_track_float32_state():
    """Steps of a bf16 state stay within the accumulated rounding of a float32 run: each step
    rounds once (at most half an ulp of the largest state seen), and the decay (|a| <= 1) never
    amplifies earlier errors, so after k steps the difference is at most k/2 such ulps."""
    g = torch.Generator().manual_seed(38)
    batch, dim, N, steps = 2, 8, 4, 12
    s32 = torch.randn(batch, dim, N, generator=g)
    s16 = s32.to(torch.bfloat16)
    s32 = s16.float()
    A = -torch.rand(dim, N, generator=g)
    peak = s32.abs().max().item()
    for _ in range(steps):
        x, dt = (torch.randn(batch, dim, generator=g) for _ in range(2))
        B, C = (torch.randn(batch, N, generator=g) for _ in range(2))
        selective_state_update_ref(s32, x, dt, A, B, C, dt_softplus=True)
        selective_state_update_ref(s16, x, dt, A, B, C, dt_softplus=True)
        peak = max(peak, s32.abs().max().item(), s16.float().abs().max().item())
    err = (s16.float() - s32).abs().max().item()
    assert 0 < err <= steps * 2.0 ** -8 * peak * 1.01


def test_chunk_states_prod_a():
    case = _rand_case(37, batch=1, dim=3, L=10, N=2)
    pa = chunk_states_ref(case["delta"], case["A"], case["delta_bias"], True, chunk=4)
    dt = _sp64(case["delta"].double().numpy() + case["delta_bias"].double().numpy()[None, :, None])
    A = case["A"].double().numpy()
    for c, end in enumerate((4, 8, 10)):
        expect = np.ones((1, 3, 2))
        for t in range(end):
            expect *= np.exp(dt[:, :, t:t + 1] * A[None])
        np.testing.assert_allclose(pa[:, :, c].numpy(), expect, rtol=1e-12)


# ---------------------------------------------------------------------------------------------
# Mutation tests: planted mistakes in the oracle must fail the pins above.
# ---------------------------------------------------------------------------------------------
def _fails(check):
    try:
        check()
    except AssertionError:
        return True
    return False


def test_mutants_are_caught():
    case4 = _rand_case(41, bkind="4d", ckind="4d", G=2)
    case3 = _rand_case(42)

    def drop_D(**kw):
        return selective_scan_ref(**{**kw, "D": None})

    def swap_BC(**kw):
        return selective_scan_ref(**{**kw, "B": kw["C"], "C": kw["B"]})

    def no_softplus(**kw):
        return selective_scan_ref(**{**kw, "delta_softplus": False})

    def wrong_group_interleave(**kw):
        dim = kw["u"].shape[1]
        G = kw["B"].shape[1]
        B = repeat(kw["B"], "B G N L -> B (H G) N L", H=dim // G)
        C = repeat(kw["C"], "B G N L -> B (H G) N L", H=dim // G)
        return selective_scan_ref(**{**kw, "B": B, "C": C})

    def sigmoid_gate(**kw):
        out, last = selective_scan_ref(**{**kw, "z": None, "return_last_state": True})
        return out * torch.sigmoid(kw["z"]), last

    assert _fails(lambda: _check_vs_brute(drop_D, case3, "3d", "3d"))
    assert _fails(lambda: _check_vs_brute(swap_BC, case3, "3d", "3d"))
    assert _fails(lambda: _check_vs_brute(no_softplus, case3, "3d", "3d"))
    assert _fails(lambda: _check_vs_brute(wrong_group_interleave, case4, "4d", "4d"))
    assert _fails(lambda: _check_vs_brute(sigmoid_gate, case3, "3d", "3d"))
    # and the unmutated oracle passes the same checks
    _check_vs_brute(selective_scan_ref, case3, "3d", "3d")
    _check_vs_brute(selective_scan_ref, case4, "4d", "4d")
