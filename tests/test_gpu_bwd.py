"""GPU parity of the selective-scan backward (MI355X only).

``SelectiveScanFn.backward`` / the binding's ``bwd`` (selective_scan_cuda.bwd equivalent,
selective_scan.cpp:415-612) run the kernels of mm_scan_bwd.hip through the C ABI; the gradients
are compared with the exact (float64) gradients of the oracle ``selective_scan_ref`` on the same
inputs (``oracle.ssm_ref.selective_scan_bwd_ref``, pinned in tests/test_oracle_bwd.py).

Tolerances: the forward's (north_star) pair (rtol, atol) = (1e-4, 1e-5) for fp32 and (3e-2, 5e-2)
for 16-bit inputs, element by element: |err| <= rtol |exact| + atol for du, ddelta and dz, and
|err| <= rtol |exact| + atol max(1, max |exact|) for the reduced gradients dA, dB, dC, dD and
ddelta_bias (sums over rows and steps, whose rounding grows with the tensor's scale; see _check).
At the full benchmark shapes every element is compared with the float64 adjoint of
oracle/scan_f64.c.
"""
import ctypes
import sys

import pytest
import torch

from oracle.ssm_ref import selective_scan_bwd_ref, selective_scan_ref
from tests import capi
from tests.test_gpu_scan import _case

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ["u", "delta", "A", "B", "C", "D", "z", "delta_bias"]
GRAD = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz", "delta_bias": "ddelta_bias"}


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


def _autograd(case, dout, return_last_state=False):
    from motif_mamba_amd import selective_scan_fn
    g = {k: (v.to(DEV).requires_grad_(True) if torch.is_tensor(v) else v) for k, v in case.items()}
    res = selective_scan_fn(**g, return_last_state=return_last_state)
    out = res[0] if return_last_state else res
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    return out.detach().cpu(), {n: g[n].grad for n in NAMES if torch.is_tensor(g[n])}


def _vs_exact(case, dout, dtype, what):
    _, grads = _autograd(case, dout)
    exact = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    for n, gr in grads.items():
        assert gr.dtype == case[n].dtype, (n, gr.dtype)
        assert gr.shape == case[n].shape, (n, gr.shape)
        _check(gr, exact[GRAD[n]], dtype, f"{what} {GRAD[n]}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [16, 4, 64])
def test_bwd_shapes(dtype, N):
    _say(f"bwd N={N} {dtype}")
    case = _case(600 + N, 2, 32, 136, N, dtype)
    _vs_exact(case, _dout(601, (2, 32, 136), dtype), dtype, f"N{N}")


@pytest.mark.parametrize("N", [1, 4, 8, 12])
@pytest.mark.parametrize("via_pq", ["1", "0"], ids=["zero-pair", "general"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
def test_bwd_small_dstate(N, via_pq, dtype, monkeypatch):
    """Diagonal training at dstate < 16 (variable B/C): the forward and the backward on the P/Q
    kernels with a zero rank-1 pair (the forward's tile states handed over), or (MM_DIAG_VIA_PQ=0)
    on the general kernels; against the exact gradients, 3 dtypes."""
    monkeypatch.setenv("MM_DIAG_VIA_PQ", via_pq)
    _say(f"bwd dstate {N} via_pq={via_pq} {dtype}")
    case = _case(770 + N, 2, 64, 264, N, dtype, bkind="4d", G=2)
    _vs_exact(case, _dout(771, (2, 64, 264), dtype), dtype, f"N{N} via_pq={via_pq}")


@pytest.mark.parametrize("N,L,G", [(32, 264, 2), (48, 136, 1), (64, 200, 2)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("slots", ["", "6"], ids=["whole", "segmented"])
def test_bwd_state_split(N, L, G, dtype, slots, monkeypatch):
    """Diagonal backward at dstate 32, 48 and 64: the dstate-16 kernel once per group of 16 states,
    the sums over states (du, ddelta) carried between the parts in float32; whole rows and
    (MM_BWD_SLOTS) a segmented last round; against the exact gradients, and against the general
    kernel (MM_BWD_SPLIT=0) to float32 rounding."""
    if slots:
        monkeypatch.setenv("MM_BWD_SLOTS", slots)
    _say(f"bwd state split N={N} L={L} G={G} {dtype} slots={slots or 'auto'}")
    case = _case(850 + N, 2, 64, L, N, dtype, bkind="4d", G=G)
    dout = _dout(851, (2, 64, L), dtype)
    _vs_exact(case, dout, dtype, f"split N{N}")
    _, split = _autograd(case, dout)
    monkeypatch.setenv("MM_BWD_SPLIT", "0")
    _, general = _autograd(case, dout)
    for n in NAMES:
        a, b = split[n].float().cpu(), general[n].float().cpu()
        scale = max(1.0, b.abs().max().item())
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        torch.testing.assert_close(a, b, rtol=tol, atol=tol * 0.1 * scale, msg=lambda m: f"{n}: {m}")


@pytest.mark.parametrize("flags", [dict(with_z=False), dict(with_D=False), dict(with_bias=False),
                                   dict(softplus=False), dict(bkind="4d", G=2), dict(bkind="4d", G=4),
                                   dict(bkind="const")])
def test_bwd_options(flags):
    _say(f"bwd options {flags}")
    case = _case(610 + len(str(flags)), 2, 32, 100, 16, torch.float32, **flags)
    _vs_exact(case, _dout(611, (2, 32, 100), torch.float32), torch.float32, str(flags))


@pytest.mark.parametrize("pad", ["1", "0"], ids=["padded", "general"])
@pytest.mark.parametrize("L", [1, 7, 2049, 4100, 2056, 4096])
def test_bwd_lengths(L, pad, monkeypatch):
    """Odd lengths run padded (the fast kernels) or, with MM_SCAN_PAD=0, on the general kernels."""
    monkeypatch.setenv("MM_SCAN_PAD", pad)
    _say(f"bwd L={L} padding {pad}")
    case = _case(620 + L, 1, 16, L, 16, torch.float32)
    _vs_exact(case, _dout(621, (1, 16, L), torch.float32), torch.float32, f"L{L}")


def test_bwd_large_dstate_mixed_bc():
    _say("bwd dstate 130, constant B, variable C")
    case = _case(630, 2, 8, 64, 130, torch.float32)
    case["B"] = torch.randn(8, 130, generator=torch.Generator().manual_seed(631))
    _vs_exact(case, _dout(632, (2, 8, 64), torch.float32), torch.float32, "N130")


def test_bwd_partial_grads_and_three_dim_bc():
    """Only some inputs require grad; 3-D B/C come back with their own shape (ssi.py:84-85)."""
    _say("bwd partial requires_grad")
    from motif_mamba_amd import selective_scan_fn
    case = _case(640, 2, 16, 64, 16, torch.float32)
    dout = _dout(641, (2, 16, 64), torch.float32)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    g["u"].requires_grad_(True)
    g["B"].requires_grad_(True)
    out = selective_scan_fn(**g)
    out.backward(dout.to(DEV))
    exact = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    assert g["B"].grad.shape == case["B"].shape == (2, 16, 64)
    _check(g["u"].grad, exact["du"], torch.float32, "du")
    _check(g["B"].grad, exact["dB"], torch.float32, "dB")
    assert g["delta"].grad is None and g["A"].grad is None


def test_bwd_training_forward_matches_inference_forward():
    _say("bwd training forward = inference forward")
    from motif_mamba_amd import selective_scan_fn
    case = _case(650, 2, 32, 256, 16, torch.bfloat16)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    inf, inf_last = selective_scan_fn(**g, return_last_state=True)
    g["u"] = g["u"].clone().requires_grad_(True)
    tr, tr_last = selective_scan_fn(**g, return_last_state=True)
    torch.testing.assert_close(tr.detach(), inf, rtol=0, atol=0)
    torch.testing.assert_close(tr_last, inf_last, rtol=1e-6, atol=1e-6)


def test_bwd_native_api_outputs():
    """selective_scan_cuda.bwd's output list, with recompute_out_z (selective_scan.cpp:609-611)."""
    _say("bwd native API")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(660, 2, 16, 2100, 16, torch.bfloat16, bkind="4d", G=2)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    out, x, out_z = ext.fwd(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"],
                            None, None, None, True)
    dout = _dout(661, (2, 16, 2100), torch.bfloat16).to(DEV)
    res = ext.bwd(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None,
                  dout, x, out, None, None, None, True, True)
    assert len(res) == 9
    du, ddelta, dA, dB, dC, dD, dbias, dz, out_z2 = res
    assert dB.dtype == dC.dtype == torch.bfloat16 and dA.dtype == torch.float32
    torch.testing.assert_close(out_z2, out_z, rtol=1e-2, atol=1e-2)
    exact = selective_scan_bwd_ref(**case, dout=dout.cpu(), dtype=torch.float64)
    for name, t in (("du", du), ("ddelta", ddelta), ("dA", dA), ("dB", dB), ("dC", dC), ("dD", dD),
                    ("ddelta_bias", dbias), ("dz", dz)):
        _check(t, exact[name], torch.bfloat16, f"native {name}")
    with pytest.raises(RuntimeError):   # x is required past one chunk, as in the reference
        ext.bwd(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None,
                dout, None, out, None, None, None, True, False)
    # P/Q with 8 channels per group, outside the 16-state P/Q kernel: the general P/Q backward takes
    # it (its gradients are checked in test_gpu_pq_bwd.py); a zero pair leaves the diagonal ones.
    res = ext.bwd(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"],
                  torch.zeros(16, 2, device=DEV), torch.zeros(2, 16, device=DEV), None,
                  dout, x, out, None, None, None, True, False)
    torch.cuda.synchronize()
    for name, t in (("du", res[0]), ("ddelta", res[1]), ("dA", res[2])):
        _check(t, exact[name], torch.bfloat16, f"native zero P/Q {name}")


def test_bwd_c_abi_direct():
    _say("bwd C ABI direct")
    lib = capi.load()
    case = _case(670, 2, 32, 96, 16, torch.float32, bkind="4d", G=1)
    dout = _dout(671, (2, 32, 96), torch.float32)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    pre = selective_scan_ref(**{**case, "z": None}).to(DEV)   # the forward's pre-gate output
    do = dout.to(DEV)
    du, ddelta, dz = torch.empty_like(g["u"]), torch.empty_like(g["delta"]), torch.empty_like(g["z"])
    dA = torch.full_like(g["A"], 7.0)            # overwritten, not accumulated into
    dB, dC = torch.full_like(g["B"], 7.0), torch.full_like(g["C"], 7.0)
    dD, dbias = torch.full_like(g["D"], 7.0), torch.full_like(g["delta_bias"], 7.0)
    p = capi.ScanBwdParams()
    p.batch, p.dim, p.seqlen, p.dstate, p.n_groups = 2, 32, 96, 16, 1
    p.itype, p.is_variable_B, p.is_variable_C, p.delta_softplus = 0, 1, 1, 1
    ptr = lambda t: t.data_ptr()
    p.u, p.delta, p.A, p.B, p.C, p.D, p.z, p.delta_bias = map(ptr, (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"],
                                                                  g["z"], g["delta_bias"]))
    p.dout, p.out = ptr(do), ptr(pre)
    p.du, p.ddelta, p.dz, p.dA, p.dB, p.dC, p.dD, p.ddelta_bias = map(ptr, (du, ddelta, dz, dA, dB, dC, dD, dbias))
    for nm, t in (("u", g["u"]), ("delta", g["delta"]), ("z", g["z"]), ("out", pre), ("dout", do), ("du", du),
                  ("ddelta", ddelta), ("dz", dz)):
        setattr(p, f"{nm}_batch_stride", t.stride(0))
        setattr(p, f"{nm}_d_stride", t.stride(1))
    p.A_d_stride, p.A_dstate_stride = g["A"].stride()
    p.dA_d_stride, p.dA_dstate_stride = dA.stride()
    p.B_batch_stride, p.B_group_stride, p.B_dstate_stride = g["B"].stride()[:3]
    p.C_batch_stride, p.C_group_stride, p.C_dstate_stride = g["C"].stride()[:3]
    p.dB_batch_stride, p.dB_group_stride, p.dB_dstate_stride = dB.stride()[:3]
    p.dC_batch_stride, p.dC_group_stride, p.dC_dstate_stride = dC.stride()[:3]
    nbytes = lib.mm_scan_bwd_workspace_size(ctypes.byref(p))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
    rc = lib.mm_scan_bwd(ctypes.byref(p), capi.stream_handle())
    assert rc == 0, lib.mm_last_error().decode()
    torch.cuda.synchronize()
    exact = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    for name, t in (("du", du), ("ddelta", ddelta), ("dz", dz), ("dA", dA), ("dB", dB), ("dC", dC), ("dD", dD),
                    ("ddelta_bias", dbias)):
        _check(t, exact[name], torch.float32, f"capi {name}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("G", [1, 4])
def test_bwd_dstate16_kernel_medium_shape(dtype, G):
    """The dstate-16 kernel (16-channel blocks, per-block dB/dC partials) on 2 x 256 channels x L 1024."""
    _say(f"bwd dstate-16 kernel 2x256x1024 G={G} {dtype}")
    case = _case(680 + G, 2, 256, 1024, 16, dtype, bkind="4d", G=G)
    _vs_exact(case, _dout(681, (2, 256, 1024), dtype), dtype, f"G{G}")


def test_bwd_dstate16_kernel_matches_general_kernel():
    """Unaligned u rows send the same request to the general kernel: both agree."""
    _say("bwd dstate-16 vs general kernel")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(690, 2, 64, 512, 16, torch.float32, bkind="4d", G=2)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    out, x, out_z = ext.fwd(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"],
                            None, None, None, True)
    dout = _dout(691, (2, 64, 512), torch.float32).to(DEV)
    fast = ext.bwd(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None,
                   dout, x, out, None, None, None, True, False)
    wide = torch.zeros(2, 64, 513, device=DEV)
    wide[:, :, 1:] = g["u"]
    u_odd = wide[:, :, 1:]                     # rows start at odd elements: not 8-byte aligned
    slow = ext.bwd(u_odd, g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None,
                   dout, x, out, None, None, None, True, False)
    for name, a, b in zip(["du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"], fast, slow):
        scale = max(1.0, b.abs().max().item())
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-5 * scale, msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2"])
def test_bwd_full_size(cfg):
    """The backward at a benchmark configuration's full shape (config 1: 8 x 1536 x 2048, config 2:
    4 x 5120 x 4096, bf16), every gradient of every element -- du, ddelta, dz and the sums dA, dB,
    dC, dD, ddelta_bias -- against the float64 adjoint of oracle/scan_f64.c (pinned against the
    explicit adjoint brute.scan_bwd_brute in tests/test_oracle_bwd.py), run on the host's threads."""
    from motif_mamba_amd import selective_scan_fn
    from motif_mamba_amd.workloads import SCAN_CONFIGS, scan_inputs
    from oracle import cscan
    c = SCAN_CONFIGS[cfg]
    _say(f"bwd full size {cfg} {c}")
    case = scan_inputs(c)
    case.pop("return_last_state")
    dout = _dout(680, case["u"].shape, case["u"].dtype)
    g = {k: (v.to(DEV).requires_grad_(True) if torch.is_tensor(v) else v) for k, v in case.items()}
    out = selective_scan_fn(**g)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    exact = cscan.scan_bwd_all_rows(case["u"], case["delta"], case["A"], case["B"], case["C"], dout, D=case["D"],
                                    z=case["z"], delta_bias=case["delta_bias"], delta_softplus=True)
    for n in NAMES:
        _check(g[n].grad, torch.from_numpy(exact[GRAD[n]]), torch.bfloat16, f"{cfg} {GRAD[n]}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bwd_tile_states(dtype, monkeypatch):
    """fwd(..., tile_states=True) on the dstate-16 kernels appends the state before every 16-step
    tile (ck[j] = the last state of the scan over the first 16 j steps); the backward reading them
    equals the one recomputing them, bit for bit when both walk whole rows (MM_BWD_SEGMENTS=0:
    sequence segments reassociate the adjoint, test_bwd_segmented_tail covers them)."""
    _say(f"bwd tile states {dtype}")
    monkeypatch.setenv("MM_BWD_SEGMENTS", "0")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(690, 2, 32, 200, 16, dtype, bkind="4d", G=1)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)
    out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    assert ck is not None and ck.shape == (13, 2, 32, 16)
    ckc = ck.cpu()
    assert float(ckc[0].abs().max()) == 0.0
    for j in (1, 5, 12):
        pre = {k: (v[..., : 16 * j] if k in ("u", "delta", "z", "B", "C") else v) for k, v in case.items()}
        _, last = selective_scan_ref(**pre, return_last_state=True)
        torch.testing.assert_close(ckc[j], last, rtol=1e-4 if dtype == torch.float32 else 1e-3,
                                   atol=1e-5 if dtype == torch.float32 else 1e-4)
    dout = _dout(691, (2, 32, 200), dtype).to(DEV)
    a = ext.bwd(*args, dout, x, out, None, None, None, True, False, ck)
    b = ext.bwd(*args, dout, x, out, None, None, None, True, False)
    torch.cuda.synchronize()
    # dA, dD, ddelta_bias: float32 atomic sums of 8 lane partials per channel and batch row, added in
    # whatever order the lanes arrive: a few roundings of the partials' size apart between runs.
    atomic = {2, 5, 6}
    for i, (ta, tb) in enumerate(zip(a, b)):
        tol = 1e-5 if i in atomic else 0.0
        scale = max(1.0, tb.abs().max().item()) if i in atomic else 0.0
        torch.testing.assert_close(ta, tb, rtol=tol, atol=tol * scale)
    # A request no fast kernel takes (dstate 8 with the zero-coupling route off): no tile states.
    monkeypatch.setenv("MM_DIAG_VIA_PQ", "0")
    c8 = _case(692, 1, 16, 64, 8, dtype)
    g8 = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in c8.items()}
    B8, C8 = g8["B"].unsqueeze(1), g8["C"].unsqueeze(1)
    res = ext.fwd(g8["u"], g8["delta"], g8["A"], B8, C8, g8["D"], g8["z"], g8["delta_bias"], None, None, None, True,
                  tile_states=True)
    assert res[-1] is None


@pytest.mark.parametrize("N", [4, 8, 12])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_bwd_tile_states_small_dstate(N, dtype):
    """Below dstate 16 the training forward runs on the P/Q kernels with a zero coupling and writes
    the tile states too (ck[j] = the state after the first 16 j steps, states past dstate 0); the
    zero-coupling backward reading them matches the one recomputing them to float32 rounding, and
    both match the exact gradients."""
    _say(f"bwd tile states dstate {N} {dtype}")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(693 + N, 2, 64, 200, N, dtype, bkind="4d", G=2)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)
    out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    assert ck is not None and ck.shape == (13, 2, 64, 16)
    ckc = ck.cpu()
    assert float(ckc[0].abs().max()) == 0.0 and float(ckc[..., N:].abs().max()) == 0.0
    for j in (1, 6, 12):
        pre = {k: (v[..., : 16 * j] if k in ("u", "delta", "z", "B", "C") else v) for k, v in case.items()}
        _, last = selective_scan_ref(**pre, return_last_state=True)
        torch.testing.assert_close(ckc[j, ..., :N], last, rtol=1e-4 if dtype == torch.float32 else 1e-3,
                                   atol=1e-5 if dtype == torch.float32 else 1e-4)
    dout = _dout(694, (2, 64, 200), dtype)
    a = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False, ck)
    b = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False)
    torch.cuda.synchronize()
    names = ["du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"]
    for name, ta, tb in zip(names, a, b):
        scale = max(1.0, tb.abs().max().item())
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        torch.testing.assert_close(ta.float(), tb.float(), rtol=tol, atol=tol * 0.1 * scale,
                                   msg=lambda m: f"{name}: {m}")
    exact = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    got = dict(zip(names, a))
    for n in NAMES:
        _check(got[GRAD[n]], exact[GRAD[n]], dtype, f"N{N} tile states {GRAD[n]}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("slots,L", [(6, 1000), (7, 256), (64, 200)])
def test_bwd_segmented_tail(dtype, slots, L, monkeypatch):
    """With the forward's tile states, the dstate-16 backward cuts the units (batch row, 16-channel
    block) of a last, partial round of workgroups along the sequence and joins the segments with
    adjoint carries. MM_BWD_SLOTS sets the round size so that small shapes take that path
    (8 units: 6 whole + 2 in 3 segments; 7 whole + 1 in 4 segments; all 8 in 3 segments, the last
    with a padded tile). The gradients match the exact ones and the unsegmented backward."""
    _say(f"bwd segmented tail slots={slots} L={L} {dtype}")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(700 + slots, 2, 64, L, 16, dtype, bkind="4d", G=2)
    dout = _dout(701, (2, 64, L), dtype)
    monkeypatch.setenv("MM_BWD_SLOTS", str(slots))
    _vs_exact(case, dout, dtype, f"segmented slots={slots}")
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)
    out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    seg = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False, ck)
    monkeypatch.setenv("MM_BWD_SEGMENTS", "0")
    whole = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False, ck)
    torch.cuda.synchronize()
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    for name, a, b in zip(["du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"], seg, whole):
        scale = max(1.0, b.abs().max().item())
        torch.testing.assert_close(a.float(), b.float(), rtol=rtol, atol=rtol * 0.1 * scale,
                                   msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("slots,L", [(6, 1000), (64, 200), (6, 1024)])   # 1024: k2s states pass (16-bit)
def test_bwd_states_pass(dtype, slots, L, monkeypatch):
    """Without the forward's tile states (the callers that recompute, e.g. MambaInnerFn at
    checkpoint_lvl 1), the backward first runs a states-only forward into its workspace and then
    takes the segmented path a training forward's tile states would give it (MM_BWD_SLOTS sets the
    round size so that these small shapes have a partial last round). The gradients match the exact
    ones, and the backward with the forward's tile states, to float32 rounding."""
    _say(f"bwd states pass slots={slots} L={L} {dtype}")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(705 + slots, 2, 64, L, 16, dtype, bkind="4d", G=2)
    dout = _dout(706, (2, 64, L), dtype)
    monkeypatch.setenv("MM_BWD_SLOTS", str(slots))
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)
    out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    assert ck is not None
    recomputed = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False)       # no tile states
    saved = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False, ck)
    torch.cuda.synchronize()
    exact = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    names = ["du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"]
    for name, a, b in zip(names, recomputed, saved):
        _check(a, exact[name], dtype, f"states pass {name}")
        scale = max(1.0, b.abs().max().item())
        rtol = 1e-5 if dtype == torch.float32 else 1e-2
        torch.testing.assert_close(a.float(), b.float(), rtol=rtol, atol=rtol * 0.1 * scale,
                                   msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("q,dtype", [(3, torch.bfloat16), (5, torch.bfloat16), (5, torch.float16)])
def test_bwd_states_pass_balanced_grid(q, dtype):
    """Shapes with 3 or 5 sixteen-channel groups per compute unit run the backward's states pass on
    the balanced mixed grid (two-state and one-state groups, states only). Its checkpoints are the
    training forward's (same grid, same state arithmetic), so the backward recomputing them equals
    the one handed the forward's tile states bit for bit, up to the float32 atomic sums (dA, dD,
    ddelta_bias); du, ddelta and dz of rows of both group kinds match the exact gradients."""
    from motif_mamba_amd import _native
    ext = _native.ext()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    batch, dim, L = 2, q * cus * 16 // 2, 256
    _say(f"bwd states pass on the mixed grid q={q} {dtype} batch {batch} dim {dim} L {L}")
    case = _case(740 + q, batch, dim, L, 16, dtype, bkind="4d", G=1)
    dout = _dout(741, (batch, dim, L), dtype)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)
    out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    d = dout.to(DEV)
    recomputed = ext.bwd(*args, d, x, out, None, None, None, True, False)
    saved = ext.bwd(*args, d, x, out, None, None, None, True, False, ck)
    torch.cuda.synchronize()
    names = ["du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"]
    for i, (a, b) in enumerate(zip(recomputed, saved)):
        if names[i] in ("dA", "dD", "ddelta_bias"):
            scale = max(1.0, b.abs().max().item())
            torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5 * scale, msg=lambda m: f"{names[i]}: {m}")
        else:
            assert torch.equal(a, b), names[i]
    # Exact du / ddelta / dz of channels in the two-state groups, at the hand-over and in the
    # one-state groups (each channel's row needs only its own inputs and the shared B, C).
    first_k1 = 2 * (q // 2) * cus * 16            # first batch-major channel of the one-state groups
    flat = [0, 17, first_k1 - 1, first_k1, first_k1 + 31, batch * dim - 1]
    for bb in range(batch):
        chans = sorted({i % dim for i in flat if i // dim == bb})
        if not chans:
            continue
        sub = {k: v for k, v in case.items()}
        for k in ("u", "delta", "z"):
            sub[k] = case[k][bb:bb + 1, chans]
        for k in ("B", "C"):
            sub[k] = case[k][bb:bb + 1]
        for k in ("A", "D", "delta_bias"):
            sub[k] = case[k][chans]
        exact = selective_scan_bwd_ref(**sub, dout=dout[bb:bb + 1, chans], dtype=torch.float64)
        for name, idx in (("du", 0), ("ddelta", 1), ("dz", 7)):
            _check(recomputed[idx][bb:bb + 1, chans], exact[name], dtype, f"states pass q={q} b{bb} {name}")


@pytest.mark.parametrize("L,dtype,N", [(13, torch.float32, 16), (1001, torch.bfloat16, 16), (2047, torch.float32, 16),
                                       (13, torch.float32, 8), (1001, torch.bfloat16, 4)])
def test_bwd_padded_lengths(L, dtype, N):
    """Training at lengths that are not multiples of 8: selective_scan_fn pads the request in front
    with zero-u steps (forward and backward on the padded copies, gradients of the real steps
    returned); the output, last state and every gradient against the exact ones. dstate 16 runs
    the diagonal kernels, dstate 8 and 4 the P/Q ones with a zero pair."""
    _say(f"bwd padded length L={L} {dtype} dstate {N}")
    from motif_mamba_amd import selective_scan_fn
    case = _case(760 + L + N, 2, 64, L, N, dtype, bkind="4d", G=2)
    dout = _dout(761, (2, 64, L), dtype)
    g = {k: (v.to(DEV).requires_grad_(True) if torch.is_tensor(v) else v) for k, v in case.items()}
    out, last = selective_scan_fn(**g, return_last_state=True)
    assert out.shape == (2, 64, L) and out.is_contiguous()
    ref, ref_last = selective_scan_ref(**case, return_last_state=True)
    rtol, atol = _tol(dtype)
    torch.testing.assert_close(out.detach().cpu().float(), ref.float(), rtol=rtol, atol=atol)
    torch.testing.assert_close(last.cpu(), ref_last.float(), rtol=rtol, atol=atol)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    exact = selective_scan_bwd_ref(**case, dout=dout, dtype=torch.float64)
    for n in NAMES:
        gr = g[n].grad
        assert gr.shape == case[n].shape, (n, gr.shape)
        _check(gr, exact[GRAD[n]], dtype, f"padded L{L} {GRAD[n]}")


@pytest.mark.parametrize("L", [2, 6, 18, 1002, 2054])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bwd_even_lengths(L, dtype, monkeypatch):
    """Even lengths that are not multiples of 8 or 4 run the dstate-16 kernel (the last tile holds
    2 to 14 valid steps; the dB/dC slab rows are padded to whole float4s and the reduction stores
    only steps below L): against the exact gradients, whole rows and (MM_BWD_SLOTS) with a segmented
    last round, 16- and 32-channel workgroups."""
    _say(f"bwd even length L={L} {dtype}")
    case = _case(750 + L, 2, 64, L, 16, dtype, bkind="4d", G=1)
    dout = _dout(751, (2, 64, L), dtype)
    _vs_exact(case, dout, dtype, f"L{L}")
    monkeypatch.setenv("MM_BWD_SLOTS", "6")
    _vs_exact(case, dout, dtype, f"L{L} segmented")
    monkeypatch.setenv("MM_BWD_CH", "32")
    monkeypatch.setenv("MM_BWD_SLOTS", "3")
    _vs_exact(case, dout, dtype, f"L{L} 32 channels")


@pytest.mark.parametrize("split,slots,L", [(3, 7, 256), (3, 6, 1000), (1, 6, 1000)])
def test_bwd_carry_pieces(split, slots, L, monkeypatch):
    """The carry launch walks each segment as MM_BWD_CARRY_SPLIT pieces, which compose like
    segments: 4-tile segments in 3 pieces of 2 tiles (the last one empty), 21-tile segments in
    pieces of 7, and one piece per segment. The gradients match the exact ones and the unsegmented
    backward."""
    _say(f"bwd carry pieces split={split} slots={slots} L={L}")
    from motif_mamba_amd import _native
    ext = _native.ext()
    dtype = torch.float32
    case = _case(730 + slots, 2, 64, L, 16, dtype, bkind="4d", G=2)
    dout = _dout(731, (2, 64, L), dtype)
    monkeypatch.setenv("MM_BWD_SLOTS", str(slots))
    monkeypatch.setenv("MM_BWD_CARRY_SPLIT", str(split))
    _vs_exact(case, dout, dtype, f"carry pieces {split}")
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)
    out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    seg = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False, ck)
    monkeypatch.setenv("MM_BWD_SEGMENTS", "0")
    whole = ext.bwd(*args, dout.to(DEV), x, out, None, None, None, True, False, ck)
    torch.cuda.synchronize()
    for name, a, b in zip(["du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"], seg, whole):
        scale = max(1.0, b.abs().max().item())
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6 * scale, msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("dtype,G", [(torch.float32, 1), (torch.bfloat16, 1), (torch.float16, 2),
                                     (torch.bfloat16, 2)])
@pytest.mark.parametrize("ch,slots", [(32, 6)])
def test_bwd_channel_widths(dtype, G, ch, slots, monkeypatch):
    """The dstate-16 backward with 32-channel workgroups (MM_BWD_CH; one dB/dC partial slab per
    block of ch channels) on 2 x 128 channels, L 1000 (a padded last tile), one group or two (two
    blocks per group): against the exact gradients through autograd, and against the 16-channel
    kernel on the same inputs -- whole rows, a segmented last round (MM_BWD_SLOTS: 8 units as 6
    whole + 2 cut, whose carry launch also reduces the slab rows of the 3 complete (batch, group)
    pairs) and without tile states."""
    _say(f"bwd channel width {ch} slots={slots} {dtype} G={G}")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(720 + ch + G, 2, 128, 1000, 16, dtype, bkind="4d", G=G)
    dout = _dout(721, (2, 128, 1000), dtype)
    monkeypatch.setenv("MM_BWD_CH", str(ch))
    _vs_exact(case, dout, dtype, f"ch={ch}")
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)
    out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
    d = dout.to(DEV)
    runs = {}
    for width in (ch, 16):
        monkeypatch.setenv("MM_BWD_CH", str(width))
        monkeypatch.setenv("MM_BWD_SLOTS", str(slots))
        monkeypatch.delenv("MM_BWD_SEGMENTS", raising=False)
        runs[width, "seg"] = ext.bwd(*args, d, x, out, None, None, None, True, False, ck)
        runs[width, "none"] = ext.bwd(*args, d, x, out, None, None, None, True, False)
        monkeypatch.setenv("MM_BWD_SEGMENTS", "0")
        runs[width, "whole"] = ext.bwd(*args, d, x, out, None, None, None, True, False, ck)
    torch.cuda.synchronize()
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    names = ["du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"]
    for kind in ("seg", "none", "whole"):
        for name, a, b in zip(names, runs[ch, kind], runs[16, kind]):
            scale = max(1.0, b.abs().max().item())
            torch.testing.assert_close(a.float(), b.float(), rtol=rtol, atol=rtol * 0.1 * scale,
                                       msg=lambda m: f"{kind} {name}: {m}")
    # Whole rows at both widths walk the same steps in the same order: dz agrees bit for bit. du and
    # ddelta differ only in the order of their sums over states (a wave pre-adds the two slots it
    # holds per channel: slots rs and rs ^ 1 at 32 channels, rs and rs ^ 2 at 16), within the
    # bound above; the dB/dC block sums and the atomics are grouped differently too.
    assert torch.equal(runs[ch, "whole"][7], runs[16, "whole"][7]), names[7]


def test_training_step_graph_replay_matches_eager():
    """The training forward (with tile states) and the backward captured in one HIP graph: the
    workspace and outputs come from the graph's memory pool and the clears are fill kernels, so
    replays with fresh inputs equal the eager step (du, ddelta, dz, dB, dC bit for bit; dA, dD and
    ddelta_bias to float32 atomic-order rounding)."""
    _say("training step graph replay")
    from motif_mamba_amd import _native
    ext = _native.ext()
    case = _case(695, 2, 64, 256, 16, torch.bfloat16, bkind="4d", G=1)
    g = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in case.items()}
    dout = _dout(696, (2, 64, 256), torch.bfloat16).to(DEV)
    args = (g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], None, None, None)

    def step():
        out, x, out_z, ck = ext.fwd(*args, True, tile_states=True)
        return [out_z] + list(ext.bwd(*args, dout, x, out, None, None, None, True, False, ck))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    gen = torch.Generator().manual_seed(697)
    atomic = {3, 6, 7}                 # dA, dD, ddelta_bias (after out_z at index 0)
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
            # Atomic sums: one float32 partial per (batch row, sequence segment) workgroup, added
            # in whatever order they finish.
            tol = 1e-5 if i in atomic else 0.0
            torch.testing.assert_close(a, b, rtol=tol, atol=tol, msg=lambda m: f"replay {rep}, output {i}: {m}")
