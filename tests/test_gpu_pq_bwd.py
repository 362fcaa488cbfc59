"""GPU parity of the low-rank coupled (MotifMamba P/Q) backward (MI355X only).

``selective_scan_fn(..., P=P, Q=Q)`` with gradients runs the forward of mm_scan_pq.hip and the
backward of mm_scan_pq_bwd.hip through the C ABI. The gradients (dP and dQ included) are compared
with the exact float64 gradients of the oracle ``selective_scan_pq_ref`` on the same inputs
(``oracle.ssm_ref.selective_scan_pq_bwd_ref``, pinned in tests/test_oracle_pq_bwd.py): what the
reference returns in its default gradient mode (ssi.py:152-205).

Tolerances: the forward's (north_star) pair (rtol, atol) = (1e-4, 1e-5) for fp32 and (3e-2, 5e-2)
for 16-bit inputs, element-wise as |err| <= rtol |exact| + atol max(1, max |exact|), the absolute
part relative to the tensor's scale as for the diagonal backward (the parameter gradients are sums
over rows and steps).
"""
import ctypes
import os
import sys

import pytest
import torch

from oracle.ssm_ref import selective_scan_pq_bwd_ref, selective_scan_pq_ref
from tests import capi
from tests.test_gpu_pq import _pq_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias", "P", "Q"]


def _say(msg):
    print(f"\n[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _tol(dtype):
    return (1e-4, 1e-5) if dtype == torch.float32 else (3e-2, 5e-2)


# Gradients with one value per element of an input (du, ddelta, dz) are held element by element
# to |err| <= rtol |exact| + atol. The reduced gradients (dA, dD, ddelta_bias: sums over batch
# rows and steps; dB, dC: sums over the channels of a group; dP, dQ: sums over rows and steps)
# add thousands of terms of both signs: their float32 rounding is relative to the sum of the
# terms' magnitudes, which the result's own magnitude can fall far below where terms cancel, so
# the absolute part of their bound is taken relative to the tensor's scale, max(1, max |exact|).
ELEMENTWISE = {"du", "ddelta", "dz"}


def _check(got, exact, dtype, what):
    rtol, atol = _tol(dtype)
    got = got.double().cpu()
    exact = exact.double()
    elementwise = any(tok in ELEMENTWISE for tok in what.split())
    scale = 1.0 if elementwise else (max(1.0, exact.abs().max().item()) if exact.numel() else 1.0)
    err = (got - exact).abs()
    bound = rtol * exact.abs() + atol * scale
    bad = err > bound
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())}/{err.numel()} beyond tolerance; max err "
                                 f"{err.max().item():.3g} (scale {scale:.3g}, elementwise {elementwise})")


def _dout(seed, shape, dtype):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


def _autograd(case, dout):
    from motif_mamba_amd import selective_scan_fn
    g = {k: (v.to(DEV).requires_grad_(True) if torch.is_tensor(v) else v) for k, v in case.items()}
    out = selective_scan_fn(**g)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    return out.detach().cpu(), {n: g[n].grad for n in NAMES if torch.is_tensor(g[n])}


def _vs_exact(case, dout, dtype, what):
    _, grads = _autograd(case, dout)
    exact = selective_scan_pq_bwd_ref(**case, dout=dout)
    for n, gr in grads.items():
        assert gr.dtype == case[n].dtype, (n, gr.dtype)
        assert gr.shape == case[n].shape, (n, gr.shape)
        _check(gr, exact["d" + n], dtype, f"{what} d{n}")


@pytest.mark.parametrize("mode", ["exact", "fused"])
def test_pq_bwd_grad_modes(mode, monkeypatch):
    """MOTIFMAMBA_PQ_GRAD_MODE (ssi.py:157-158): for z-less calls the reference's "exact" mode takes
    dP / dQ from autograd through its full-matrix path, any other value from its dense CUDA
    backward, the only backward its launcher runs with P/Q (selective_scan_bwd_kernel.cuh:928-932),
    which accumulates the exact chain rule (:307, :334). Both are the exact gradient: the kernel's
    match the float64 adjoint under either value."""
    _say(f"pq bwd MOTIFMAMBA_PQ_GRAD_MODE={mode}")
    monkeypatch.setenv("MOTIFMAMBA_PQ_GRAD_MODE", mode)
    case = _pq_case(830, batch=2, dim=32, L=64, N=16, R=2, dtype=torch.float32, with_z=False)
    _vs_exact(case, _dout(831, (2, 32, 64), torch.float32), torch.float32, mode)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("per_dim", [True, False])
def test_pq_bwd_dtypes(dtype, per_dim):
    _say(f"pq bwd {dtype} per_dim={per_dim}")
    case = _pq_case(700 + per_dim, batch=2, dim=32, L=136, N=16, R=2, dtype=dtype, per_dim=per_dim)
    _vs_exact(case, _dout(701, (2, 32, 136), dtype), dtype, f"{dtype}")


@pytest.mark.parametrize("R", [1, 3, 4, 5, 8])
def test_pq_bwd_ranks(R):
    _say(f"pq bwd rank {R}")
    case = _pq_case(710 + R, batch=2, dim=32, L=64, N=16, R=R, dtype=torch.float32)
    _vs_exact(case, _dout(711, (2, 32, 64), torch.float32), torch.float32, f"R{R}")


@pytest.mark.parametrize("flags", [dict(with_z=False), dict(with_D=False), dict(with_bias=False),
                                   dict(softplus=False), dict(bkind="4d", G=2), dict(bkind="4d", G=4)])
def test_pq_bwd_options(flags):
    _say(f"pq bwd options {flags}")
    case = _pq_case(720 + len(str(flags)), batch=2, dim=64, L=72, N=16, R=2, dtype=torch.float32, **flags)
    _vs_exact(case, _dout(721, (2, 64, 72), torch.float32), torch.float32, str(flags))


@pytest.mark.parametrize("N", [1, 4, 12])
def test_pq_bwd_small_dstate(N):
    _say(f"pq bwd dstate {N}")
    case = _pq_case(730 + N, batch=3, dim=16, L=40, N=N, R=min(N, 2), dtype=torch.float32)
    _vs_exact(case, _dout(731, (3, 16, 40), torch.float32), torch.float32, f"N{N}")


@pytest.mark.parametrize("L", [8, 16, 1032])
def test_pq_bwd_lengths(L):
    _say(f"pq bwd L={L}")
    case = _pq_case(740 + L, batch=1, dim=16, L=L, N=16, R=2, dtype=torch.float32)
    _vs_exact(case, _dout(741, (1, 16, L), torch.float32), torch.float32, f"L{L}")


def test_pq_bwd_partial_grads_and_dtypes():
    """Only some inputs require grad; dP / dQ come back in P's / Q's dtype and shape."""
    _say("pq bwd partial requires_grad")
    from motif_mamba_amd import selective_scan_fn
    case = _pq_case(750, batch=2, dim=16, L=48, N=16, R=2, dtype=torch.bfloat16)
    dout = _dout(751, (2, 16, 48), torch.bfloat16)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    g["P"] = g["P"].to(torch.bfloat16).requires_grad_(True)
    g["Q"].requires_grad_(True)
    out = selective_scan_fn(**g)
    out.backward(dout.to(DEV))
    assert g["P"].grad.dtype == torch.bfloat16 and g["P"].grad.shape == (16, 16, 2)
    assert g["Q"].grad.dtype == torch.float32 and g["Q"].grad.shape == (16, 2, 16)
    assert g["u"].grad is None and g["A"].grad is None
    exact = selective_scan_pq_bwd_ref(**dict(case, P=case["P"].to(torch.bfloat16)), dout=dout)
    _check(g["P"].grad, exact["dP"], torch.bfloat16, "dP")
    _check(g["Q"].grad, exact["dQ"], torch.bfloat16, "dQ")


def test_pq_bwd_training_forward_matches_inference_forward():
    _say("pq training forward = inference forward")
    from motif_mamba_amd import selective_scan_fn
    case = _pq_case(760, batch=2, dim=32, L=256, N=16, R=2, dtype=torch.bfloat16)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    inf, inf_last = selective_scan_fn(**g, return_last_state=True)
    g["P"] = g["P"].clone().requires_grad_(True)
    tr, tr_last = selective_scan_fn(**g, return_last_state=True)
    torch.testing.assert_close(tr.detach(), inf, rtol=0, atol=0)
    torch.testing.assert_close(tr_last.detach(), inf_last, rtol=1e-6, atol=1e-6)


def test_pq_bwd_native_api_accumulates_into_dP_out():
    """selective_scan_cuda.bwd with P/Q: the reference's output list; dP / dQ are added into
    dP_out / dQ_out (selective_scan.cpp:580-590 accumulates into them)."""
    _say("pq bwd native API")
    from motif_mamba_amd import _native
    case = _pq_case(770, batch=2, dim=32, L=64, N=16, R=2, dtype=torch.float32)
    dout = _dout(771, (2, 32, 64), torch.float32)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    B4, C4 = g["B"].unsqueeze(1), g["C"].unsqueeze(1)
    out, x, out_z = _native.ext().fwd(g["u"], g["delta"], g["A"], B4, C4, g["D"], g["z"], g["delta_bias"],
                                      g["P"], g["Q"], None, True)
    dP = torch.ones(32, 16, 2, device=DEV)
    dQ = torch.full((32, 2, 16), 2.0, device=DEV)
    res = _native.ext().bwd(g["u"], g["delta"], g["A"], B4, C4, g["D"], g["z"], g["delta_bias"], g["P"], g["Q"],
                            None, dout.to(DEV), x, out, None, dP, dQ, True, True)
    assert len(res) == 9      # du, ddelta, dA, dB, dC, dD, ddelta_bias, dz, out_z
    torch.cuda.synchronize()
    exact = selective_scan_pq_bwd_ref(**case, dout=dout)
    _check(dP - 1.0, exact["dP"], torch.float32, "dP_out")
    _check(dQ - 2.0, exact["dQ"], torch.float32, "dQ_out")
    _check(res[0], exact["du"], torch.float32, "du")
    _check(res[7], exact["dz"], torch.float32, "dz")
    torch.testing.assert_close(res[8], out_z, rtol=1e-6, atol=1e-6)   # recomputed: same math, own rounding


def test_pq_bwd_c_abi_direct():
    _say("pq bwd C ABI direct")
    lib = capi.load()
    case = _pq_case(780, batch=2, dim=32, L=96, N=16, R=3, dtype=torch.float32, per_dim=False)
    dout = _dout(781, (2, 32, 96), torch.float32)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    B4, C4 = g["B"].unsqueeze(1), g["C"].unsqueeze(1)
    pre = selective_scan_pq_ref(**{**case, "z": None}).to(DEV)   # the forward's pre-gate output
    do = dout.to(DEV)
    du, ddelta, dz = torch.empty_like(g["u"]), torch.empty_like(g["delta"]), torch.empty_like(g["z"])
    dA = torch.full_like(g["A"], 7.0)            # overwritten, not accumulated into
    dB, dC = torch.full_like(B4, 7.0), torch.full_like(C4, 7.0)
    dD, dbias = torch.full_like(g["D"], 7.0), torch.full_like(g["delta_bias"], 7.0)
    dP, dQ = torch.full_like(g["P"], 7.0), torch.full_like(g["Q"], 7.0)
    p = capi.ScanBwdParams()
    p.batch, p.dim, p.seqlen, p.dstate, p.n_groups = 2, 32, 96, 16, 1
    p.itype, p.is_variable_B, p.is_variable_C, p.delta_softplus = 0, 1, 1, 1
    ptr = lambda t: t.data_ptr()
    p.u, p.delta, p.A, p.B, p.C, p.D, p.z, p.delta_bias = map(ptr, (g["u"], g["delta"], g["A"], B4, C4, g["D"],
                                                                  g["z"], g["delta_bias"]))
    p.dout, p.out = ptr(do), ptr(pre)
    p.du, p.ddelta, p.dz, p.dA, p.dB, p.dC, p.dD, p.ddelta_bias = map(ptr, (du, ddelta, dz, dA, dB, dC, dD, dbias))
    for nm, t in (("u", g["u"]), ("delta", g["delta"]), ("z", g["z"]), ("out", pre), ("dout", do), ("du", du),
                  ("ddelta", ddelta), ("dz", dz)):
        setattr(p, f"{nm}_batch_stride", t.stride(0))
        setattr(p, f"{nm}_d_stride", t.stride(1))
    p.A_d_stride, p.A_dstate_stride = g["A"].stride()
    p.dA_d_stride, p.dA_dstate_stride = dA.stride()
    p.B_batch_stride, p.B_group_stride, p.B_dstate_stride = B4.stride()[:3]
    p.C_batch_stride, p.C_group_stride, p.C_dstate_stride = C4.stride()[:3]
    p.dB_batch_stride, p.dB_group_stride, p.dB_dstate_stride = dB.stride()[:3]
    p.dC_batch_stride, p.dC_group_stride, p.dC_dstate_stride = dC.stride()[:3]
    p.P, p.Q, p.pq_rank = ptr(g["P"]), ptr(g["Q"]), 3
    p.P_dstate_stride, p.P_r_stride = g["P"].stride()
    p.Q_r_stride, p.Q_dstate_stride = g["Q"].stride()
    p.dP, p.dQ = ptr(dP), ptr(dQ)
    p.dP_dstate_stride, p.dP_r_stride = dP.stride()
    p.dQ_r_stride, p.dQ_dstate_stride = dQ.stride()
    nbytes = lib.mm_scan_bwd_workspace_size(ctypes.byref(p))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    rc = lib.mm_scan_bwd(ctypes.byref(p), capi.stream_handle())
    assert rc == 0, lib.mm_last_error().decode()
    torch.cuda.synchronize()
    exact = selective_scan_pq_bwd_ref(**case, dout=dout)
    for name, t in (("du", du), ("ddelta", ddelta), ("dz", dz), ("dA", dA), ("dB", dB.squeeze(1)),
                    ("dC", dC.squeeze(1)), ("dD", dD), ("ddelta_bias", dbias), ("dP", dP), ("dQ", dQ)):
        _check(t, exact[name], torch.float32, f"capi {name}")
    # Refusals, nothing launched: a rank past the reference's limit of 8, missing dP (invalid).
    p.pq_rank = 9
    assert lib.mm_scan_bwd(ctypes.byref(p), capi.stream_handle()) == capi.MM_ERR_INVALID_ARGUMENT
    assert b"pq_rank" in lib.mm_last_error()
    p.pq_rank, p.dP = 3, None
    assert lib.mm_scan_bwd(ctypes.byref(p), capi.stream_handle()) == capi.MM_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("L", [12, 1001])
def test_pq_bwd_padded_lengths(L):
    """Lengths that are not multiples of 8: the training forward and the backward run on copies
    padded in front with zero-u steps, which add nothing to any gradient; against the exact ones."""
    _say(f"pq bwd padded length L={L}")
    case = _pq_case(795 + L, batch=2, dim=32, L=L, N=16, R=2, dtype=torch.float32, bkind="4d", G=2)
    _vs_exact(case, _dout(796, (2, 32, L), torch.float32), torch.float32, f"padded L{L}")


GENERAL_SHAPES = {
    "dstate20": dict(N=20), "dstate32": dict(N=32), "dstate64": dict(N=64), "dstate32_rank5": dict(N=32, R=5),
    "dstate130": dict(N=130, R=3, dim=8, G=1), "constB": dict(G=1), "constBC": dict(bkind="const"),
    "dim24": dict(dim=24, G=1), "L100": dict(L=100), "shared_pq_dstate32": dict(N=32, per_dim=False),
    # workgroups whose rows span two groups (12 channels per group, 16 rows per workgroup) and two
    # batch rows (12 channels, 8 rows per workgroup): the dB/dC runs split there
    "dim24_G2": dict(dim=24, G=2), "dstate32_dim12": dict(N=32, dim=12, G=1),
    # lengths of one step and of one tile plus one; no z; no D, delta_bias or softplus
    "dstate32_L1": dict(N=32, L=1), "dstate32_L17": dict(N=32, L=17), "dstate32_noz": dict(N=32, with_z=False),
    "dstate32_bare": dict(N=32, with_D=False, with_bias=False, softplus=False),
}


@pytest.mark.parametrize("what", list(GENERAL_SHAPES))
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_pq_bwd_general_shapes(what, dtype, monkeypatch):
    """Shapes outside the 16-state kernel run the general P/Q backward (one lane per state, the sums
    over states as wave butterflies, LDS across waves past 64 states): dstate 20, 32, 64 and 130
    (the Motif module's "small" and "base" presets use 32 and 64, mamba_simplemotif.py:33-35; the
    reference's dense kernel takes up to 256), rank 5, a P/Q pair shared by every channel, constant
    B, constant B and C, 24 and 12 channels (workgroups spanning two groups or two batch rows), L 100
    with the training padding off; against the exact gradients (dP and dQ included), with z."""
    _say(f"pq bwd general {what} {dtype}")
    kw = dict(batch=2, dim=32, L=64, N=16, R=2, dtype=dtype, bkind="4d", G=2)
    kw.update(GENERAL_SHAPES[what])
    if what == "L100":
        monkeypatch.setenv("MM_SCAN_PAD", "0")
    case = _pq_case(790 + len(what), **kw)
    if what == "constB":
        case["B"] = torch.randn(kw["dim"], kw["N"], generator=torch.Generator().manual_seed(791))
    _vs_exact(case, _dout(792, (kw["batch"], kw["dim"], kw["L"]), dtype), dtype, what)


def test_pq_fwd_tile_states_are_the_prefix_states():
    """fwd(..., tile_states=True) appends the state before every 16-step tile: ck[j] is the last
    state of the scan over the first 16 j steps (tiled kernel, and the one-lane-per-row kernel that
    a strided u selects)."""
    _say("pq fwd tile_states")
    from motif_mamba_amd import _native
    for strided in (False, True):
        case = _pq_case(800 + strided, batch=2, dim=16, L=72, N=12, R=2, dtype=torch.float32)
        g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
        if strided:
            wide = torch.zeros(2, 16, 75, device=DEV)
            wide[:, :, 1:73] = g["u"]
            g["u"] = wide[:, :, 1:73]
        res = _native.ext().fwd(g["u"], g["delta"], g["A"], g["B"].unsqueeze(1), g["C"].unsqueeze(1), g["D"], g["z"],
                                g["delta_bias"], g["P"], g["Q"], None, True, tile_states=True)
        assert len(res) == 4
        ck = res[3].cpu()
        assert ck.shape == (5, 2, 16, 16)
        assert float(ck[0].abs().max()) == 0.0
        assert float(ck[:, :, :, 12:].abs().max()) == 0.0       # states past dstate
        for j in (1, 2, 4):
            pre = {k: (v[..., : 16 * j] if k in ("u", "delta", "z", "B", "C") else v) for k, v in case.items()}
            _, last = selective_scan_pq_ref(**pre, return_last_state=True)
            torch.testing.assert_close(ck[j, :, :, :12], last, rtol=1e-4, atol=1e-5)


def test_pq_bwd_with_and_without_tile_states():
    """The backward reading the forward's tile states equals the one recomputing them (the same
    recurrence in the same order with 8 lanes per channel in both)."""
    _say("pq bwd tile_states vs recompute")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _pq_case(810, batch=2, dim=64, L=200, N=16, R=2, dtype=torch.bfloat16)
    dout = _dout(811, (2, 64, 200), torch.bfloat16).to(DEV)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    B4, C4 = g["B"].unsqueeze(1), g["C"].unsqueeze(1)
    args = (g["u"], g["delta"], g["A"], B4, C4, g["D"], g["z"], g["delta_bias"], g["P"], g["Q"], None)
    old = os.environ.get("MM_PQ_LPR")
    os.environ["MM_PQ_LPR"] = "8"
    try:
        out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    finally:
        if old is None:
            os.environ.pop("MM_PQ_LPR")
        else:
            os.environ["MM_PQ_LPR"] = old
    grads = []
    for tiles in (ck, None):
        dP, dQ = torch.zeros_like(g["P"]), torch.zeros_like(g["Q"])
        r = ext.bwd(*args, dout, x, out, None, dP, dQ, True, False, tiles)
        grads.append(list(r) + [dP, dQ])
    torch.cuda.synchronize()
    # du, ddelta, dB, dC, dz bit for bit; dA, dD, ddelta_bias, dP, dQ are float32 atomic sums, whose
    # order (and so last bits) varies from run to run.
    atomic = {2, 5, 6, 8, 9}
    for i, (a, b) in enumerate(zip(*grads)):
        tol = 1e-6 if i in atomic else 0.0
        torch.testing.assert_close(a, b, rtol=tol, atol=tol)
    with pytest.raises(RuntimeError, match="tile_states"):
        ext.bwd(*args, dout, x, out, None, None, None, True, False, ck[:, :1])
    # Without P/Q the dstate-16 kernels write tile states too (the diagonal scan's own).
    res = ext.fwd(*args[:8], None, None, None, True, tile_states=True)
    assert res[-1] is not None and res[-1].shape == ck.shape


def test_pq_bwd_bench_shape_sampled_channels():
    """The P/Q training step at the benchmark shape (pq_1p4b: 4 x 4096 x 2048, rank 2, per-channel
    P/Q, fp16) against the exact float64 gradients of the oracle on sampled channels (independent
    given B and C): du, ddelta, dz, dA, dD, ddelta_bias, dP and dQ of those channels."""
    from motif_mamba_amd import selective_scan_fn
    from motif_mamba_amd.workloads import PQ_CONFIGS, pq_inputs
    c = PQ_CONFIGS["pq_1p4b"]
    _say(f"pq bwd bench shape {c}")
    case = pq_inputs(c)
    case.pop("return_last_state")
    dout = _dout(820, case["u"].shape, case["u"].dtype)
    names = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias", "P", "Q"]
    g = {k: (v.to(DEV).requires_grad_(True) if k in names else v) for k, v in case.items()}
    out = selective_scan_fn(**g)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    chans = torch.tensor([0, 1, 2049, c.dim - 1])
    per_ch = ("A", "D", "delta_bias", "P", "Q")
    sub = {k: (v[:, chans] if k in ("u", "delta", "z") else v[chans] if k in per_ch else v)
           for k, v in case.items()}
    exact = selective_scan_pq_bwd_ref(**sub, dout=dout[:, chans])
    for n in ("u", "delta", "z"):
        _check(g[n].grad[:, chans.to(DEV)], exact["d" + n], torch.float16, f"bench d{n}")
    for n in per_ch:
        _check(g[n].grad[chans.to(DEV)], exact["d" + n], torch.float16, f"bench d{n}")


def test_pq_bwd_rank_zero_is_the_diagonal_backward():
    """P/Q of rank 0 couple nothing: every gradient is the diagonal scan's, dP and dQ are empty."""
    _say("pq bwd rank 0")
    case = _pq_case(830, batch=2, dim=32, L=64, N=16, R=1, dtype=torch.float32)
    case["P"] = case["P"][..., :0].contiguous()
    case["Q"] = case["Q"][:, :0, :].contiguous()
    dout = _dout(831, (2, 32, 64), torch.float32)
    from motif_mamba_amd import selective_scan_fn
    g = {k: (v.to(DEV).requires_grad_(True) if torch.is_tensor(v) else v) for k, v in case.items()}
    out = selective_scan_fn(**g)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    from oracle.ssm_ref import selective_scan_bwd_ref
    kw = {k: v for k, v in case.items() if k not in ("P", "Q")}
    exact = selective_scan_bwd_ref(**kw, dout=dout, dtype=torch.float64)
    for n in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"):
        _check(g[n].grad, exact["d" + n], torch.float32, f"rank0 d{n}")
    assert g["P"].grad.shape == (32, 16, 0) and g["Q"].grad.shape == (32, 0, 16)


def test_pq_bwd_xz_chunk_views():
    """The Motif module's call form (mamba_simplemotif.py:314-332): u and z are the two halves of
    one (batch, 2 dim, L) activation, strided views, and delta is a (b, d, l) view of a
    channel-major matrix; gradients flow back into the shared parent tensors."""
    _say("pq bwd xz chunk views")
    from motif_mamba_amd import selective_scan_fn
    case = _pq_case(840, batch=2, dim=32, L=96, N=16, R=2, dtype=torch.bfloat16)
    dout = _dout(841, (2, 32, 96), torch.bfloat16)
    xz = torch.cat([case["u"], case["z"]], dim=1).to(DEV).requires_grad_(True)
    dl = case["delta"].permute(1, 0, 2).contiguous().to(DEV).requires_grad_(True)   # (dim, batch, L)
    u, z = xz.chunk(2, dim=1)
    delta = dl.permute(1, 0, 2)                                                     # (batch, dim, L) view
    assert u.stride() == (64 * 96, 96, 1) and delta.stride() == (96, 2 * 96, 1)
    g = {k: (v.to(DEV).requires_grad_(True) if torch.is_tensor(v) else v) for k, v in case.items()
         if k not in ("u", "z", "delta")}
    out = selective_scan_fn(u, delta, g["A"], g["B"], g["C"], D=g["D"], z=z, delta_bias=g["delta_bias"],
                            delta_softplus=True, P=g["P"], Q=g["Q"])
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    exact = selective_scan_pq_bwd_ref(**case, dout=dout)
    _check(xz.grad[:, :32], exact["du"], torch.bfloat16, "du via xz")
    _check(xz.grad[:, 32:], exact["dz"], torch.bfloat16, "dz via xz")
    _check(dl.grad.permute(1, 0, 2), exact["ddelta"], torch.bfloat16, "ddelta via the channel-major view")
    for n in ("A", "B", "C", "D", "delta_bias", "P", "Q"):
        _check(g[n].grad, exact["d" + n], torch.bfloat16, f"d{n}")


def test_pq_training_step_graph_replay_matches_eager():
    """The P/Q training forward (with tile states) and backward (dP/dQ added into dP_out/dQ_out)
    captured in one HIP graph; replays with fresh inputs equal the eager step."""
    _say("pq training step graph replay")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _pq_case(850, batch=2, dim=32, L=128, N=16, R=2, dtype=torch.bfloat16)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    dout = _dout(851, (2, 32, 128), torch.bfloat16).to(DEV)
    B4, C4 = g["B"].unsqueeze(1), g["C"].unsqueeze(1)
    args = (g["u"], g["delta"], g["A"], B4, C4, g["D"], g["z"], g["delta_bias"], g["P"], g["Q"], None)
    dP, dQ = torch.zeros_like(g["P"]), torch.zeros_like(g["Q"])

    def step():
        dP.zero_()
        dQ.zero_()
        out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
        res = ext.bwd(*args, dout, x, out, None, dP, dQ, True, False, ck)
        return [out_z] + list(res) + [dP.clone(), dQ.clone()]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    gen = torch.Generator().manual_seed(852)
    atomic = {3, 6, 7, 9, 10}          # dA, dD, ddelta_bias, dP, dQ (after out_z at index 0)
    for rep in range(3):
        for k in ("u", "delta", "z"):
            g[k].copy_(torch.randn(g[k].shape, generator=gen).to(g[k].dtype).to(DEV))
        dout.copy_(torch.randn(dout.shape, generator=gen).to(dout.dtype).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        exp = step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, exp)):
            tol = 1e-5 if i in atomic else 0.0
            torch.testing.assert_close(a, b, rtol=tol, atol=tol, msg=lambda m: f"replay {rep}, output {i}: {m}")
