"""GPU parity of the low-rank coupled (MotifMamba P/Q) forward scan (MI355X only).

``selective_scan_fn(..., P=P, Q=Q)`` runs the kernels of mm_scan_pq.hip through the C ABI and is
compared with ``oracle.ssm_ref.selective_scan_pq_ref`` (restating selective_scan_full_matrix_cuda,
ssi.py:262-350) on the same seeded inputs and, for long sequences and the benchmark shape, with the
float64 C restatement ``mm_oracle_scan_pq_rows_f64`` on sampled rows.
Tolerances (north_star): fp32 rtol 1e-4 / atol 1e-5; bf16/fp16 inputs rtol 3e-2 / atol 5e-2.
"""
import ctypes
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import cscan
from oracle.ssm_ref import selective_scan_pq_ref, selective_scan_ref
from tests import capi, fixtures

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _say(msg):
    print(f"\n[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _to(d, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}


def _close(a, b, dtype, what):
    rtol, atol = fixtures.tolerances(dtype)
    torch.testing.assert_close(a.float(), b.float(), rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


def _pq_case(seed, batch, dim, L, N, R, dtype, per_dim=True, bkind="3d", G=1, with_D=True, with_z=True,
             with_bias=True, softplus=True, pq_std=0.25):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, L, generator=g).to(dtype)
    delta = torch.randn(batch, dim, L, generator=g)
    z = torch.randn(batch, dim, L, generator=g).to(dtype) if with_z else None
    lo, hi = math.log(1e-3), math.log(1e-1)
    bias = (torch.rand(dim, generator=g) * (hi - lo) + lo).float() if with_bias else None
    if not softplus:
        delta = delta.abs() * 0.1
        if bias is not None:
            bias = bias.exp()
    delta = delta.to(dtype)
    if bkind == "4d":
        B = torch.randn(batch, G, N, L, generator=g).to(dtype)
        C = torch.randn(batch, G, N, L, generator=g).to(dtype)
    elif bkind == "3d":
        B = torch.randn(batch, N, L, generator=g).to(dtype)
        C = torch.randn(batch, N, L, generator=g).to(dtype)
    else:
        B = torch.randn(dim, N, generator=g)
        C = torch.randn(dim, N, generator=g)
    A = -(torch.rand(dim, N, generator=g) * 8 + 0.05)
    D = torch.randn(dim, generator=g) if with_D else None
    if per_dim:
        P = torch.randn(dim, N, R, generator=g) * pq_std
        Q = torch.randn(dim, R, N, generator=g) * pq_std
    else:
        P = torch.randn(N, R, generator=g) * pq_std
        Q = torch.randn(R, N, generator=g) * pq_std
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=bias, delta_softplus=softplus,
                P=P, Q=Q)


def _gpu(case, **kw):
    from motif_mamba_amd import selective_scan_fn
    out, last = selective_scan_fn(**_to(case, DEV), return_last_state=True, **kw)
    torch.cuda.synchronize()
    return out.cpu(), last.cpu()


def _vs_oracle(case, dtype, what):
    out, last = _gpu(case)
    ref, ref_last = selective_scan_pq_ref(**case, return_last_state=True)
    _close(out, ref, dtype, f"{what} out")
    _close(last, ref_last, dtype, f"{what} last_state")


class _lpr:
    """Forces the tiled kernel's lanes per row (MM_PQ_LPR) for the duration of a block."""

    def __init__(self, lpr):
        self.lpr = lpr

    def __enter__(self):
        self.old = os.environ.get("MM_PQ_LPR")
        if self.lpr:
            os.environ["MM_PQ_LPR"] = str(self.lpr)
        return self

    def __exit__(self, *a):
        if self.old is None:
            os.environ.pop("MM_PQ_LPR", None)
        else:
            os.environ["MM_PQ_LPR"] = self.old


# ---------------------------------------------------------------------------------------------
# Tiled kernel: every (states per lane, lanes per row) shape, rank padding, dtypes, P/Q layouts.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("N,lpr", [(16, 4), (16, 8), (16, 16), (32, 8), (32, 16), (64, 16), (12, 4), (24, 8)])
def test_pq_tiled_shapes(dtype, N, lpr):
    _say(f"pq tiled N={N} lpr={lpr} {dtype}")
    case = _pq_case(300 + N + lpr, batch=2, dim=48, L=136, N=N, R=2, dtype=dtype)
    with _lpr(lpr):
        _vs_oracle(case, dtype, f"N{N} lpr{lpr}")


@pytest.mark.parametrize("R", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("per_dim", [True, False])
def test_pq_tiled_ranks(R, per_dim):
    _say(f"pq tiled rank={R} per_dim={per_dim}")
    case = _pq_case(320 + R, batch=2, dim=32, L=96, N=16, R=R, dtype=torch.float32, per_dim=per_dim)
    _vs_oracle(case, torch.float32, f"R{R}")


@pytest.mark.parametrize("flags", [dict(with_z=False), dict(with_D=False), dict(with_bias=False),
                                   dict(softplus=False), dict(bkind="4d", G=4), dict(bkind="4d", G=2)])
def test_pq_tiled_options(flags):
    _say(f"pq tiled options {flags}")
    case = _pq_case(340 + len(str(flags)), batch=2, dim=64, L=72, N=16, R=2, dtype=torch.bfloat16, **flags)
    _vs_oracle(case, torch.bfloat16, str(flags))


def test_pq_partial_groups_and_tail_tile():
    """Channels per group not a multiple of the wave's channels, and L % 32 != 0."""
    _say("pq partial channel blocks, tail tile")
    for lpr in (4, 8, 16):
        case = _pq_case(350 + lpr, batch=3, dim=40, L=88, N=16, R=2, dtype=torch.float32, bkind="4d", G=2)
        with _lpr(lpr):
            _vs_oracle(case, torch.float32, f"lpr{lpr}")


# ---------------------------------------------------------------------------------------------
# Lane-per-row kernel: constant / mixed B and C, dstate > 64, odd lengths, strided rows, rank 0.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("bkind_b,bkind_c", [("const", "const"), ("3d", "const"), ("const", "3d")])
def test_pq_general_constant_bc(bkind_b, bkind_c):
    _say(f"pq general B={bkind_b} C={bkind_c}")
    case = _pq_case(360, batch=2, dim=20, L=45, N=16, R=2, dtype=torch.float32, bkind="3d")
    g = torch.Generator().manual_seed(361)
    if bkind_b == "const":
        case["B"] = torch.randn(20, 16, generator=g)
    if bkind_c == "const":
        case["C"] = torch.randn(20, 16, generator=g)
    _vs_oracle(case, torch.float32, f"{bkind_b}/{bkind_c}")


@pytest.mark.parametrize("N", [128, 200])
def test_pq_general_large_dstate(N):
    _say(f"pq general N={N}")
    case = _pq_case(370 + N, batch=1, dim=8, L=40, N=N, R=4, dtype=torch.float32, pq_std=0.1)
    _vs_oracle(case, torch.float32, f"N{N}")


@pytest.mark.parametrize("pad", ["0", "1"], ids=["general", "padded"])
def test_pq_general_odd_length_and_strided_rows(pad, monkeypatch):
    """Odd L with misaligned u rows: the lane-per-row P/Q kernel (MM_SCAN_PAD=0), or the fast
    kernel on the binding's front-padded copies."""
    _say(f"pq odd L and strided u, padding {pad}")
    monkeypatch.setenv("MM_SCAN_PAD", pad)
    from motif_mamba_amd import selective_scan_fn
    case = _pq_case(380, batch=2, dim=16, L=37, N=16, R=2, dtype=torch.bfloat16)
    g = _to(case, DEV)
    wide = torch.zeros(2, 16, 41, dtype=torch.bfloat16, device=DEV)
    wide[:, :, 2:39] = g["u"]
    g["u"] = wide[:, :, 2:39]              # stride(-1) == 1, row starts not 16-byte aligned
    assert g["u"].stride() == (16 * 41, 41, 1)
    out, last = selective_scan_fn(**g, return_last_state=True)
    ref, ref_last = selective_scan_pq_ref(**case, return_last_state=True)
    _close(out.cpu(), ref, torch.bfloat16, "odd L out")
    _close(last.cpu(), ref_last, torch.bfloat16, "odd L last")


@pytest.mark.parametrize("L,R", [(1, 2), (4, 2), (5, 2), (1001, 2), (2047, 4)])
def test_pq_padded_length(L, R):
    """P/Q inference at lengths that are not multiples of 8: from 5 steps on the fast kernel on
    front-padded copies (zero u keeps the coupled state at zero through the padding), below the
    lane-per-row kernel (L 1 is the Motif decode step's call); against selective_scan_pq_ref."""
    _say(f"pq padded length L={L} R={R}")
    case = _pq_case(390 + R, batch=2, dim=64, L=L, N=16, R=R, dtype=torch.bfloat16, bkind="4d", G=2)
    _vs_oracle(case, torch.bfloat16, f"padded L={L}")


def test_pq_rank_zero_is_the_diagonal_scan():
    _say("pq rank 0")
    case = _pq_case(390, batch=2, dim=32, L=64, N=16, R=1, dtype=torch.float32)
    case["P"] = case["P"][..., :0]
    case["Q"] = case["Q"][:, :0, :]
    out, last = _gpu(case)
    kw = {k: v for k, v in case.items() if k not in ("P", "Q")}
    ref, ref_last = selective_scan_ref(**kw, return_last_state=True)
    _close(out, ref, torch.float32, "rank0 out")
    _close(last, ref_last, torch.float32, "rank0 last")


def test_pq_zero_coupling_matches_diagonal_kernel():
    _say("pq P=0 vs the diagonal kernels")
    from motif_mamba_amd import selective_scan_fn
    case = _pq_case(395, batch=2, dim=128, L=512, N=16, R=2, dtype=torch.bfloat16)
    case["P"] = torch.zeros_like(case["P"])
    out, last = _gpu(case)
    kw = _to({k: v for k, v in case.items() if k not in ("P", "Q")}, DEV)
    ref, ref_last = selective_scan_fn(**kw, return_last_state=True)
    _close(out, ref.cpu(), torch.bfloat16, "P=0 out")
    torch.testing.assert_close(last, ref_last.cpu(), rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------------------------
# Chunk states, long sequences and the benchmark shape against the float64 restatement.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_pq_native_fwd_chunk_states(dtype):
    """ext.fwd returns [out, x, out_z] with x = (1, h) at every 2048-step chunk end, as the
    reference's dense forward writes it (selective_scan_fwd_kernel.cuh:244-249)."""
    _say(f"pq native fwd chunk states {dtype}")
    from motif_mamba_amd import _native
    L = 4200
    case = _pq_case(400, batch=1, dim=32, L=L, N=16, R=2, dtype=dtype)
    g = _to(case, DEV)
    B4 = g["B"].unsqueeze(1)
    C4 = g["C"].unsqueeze(1)
    out, x, out_z = _native.ext().fwd(g["u"], g["delta"], g["A"], B4, C4, g["D"], g["z"], g["delta_bias"],
                                      g["P"], g["Q"], None, True)
    torch.cuda.synchronize()
    assert x.shape == (1, 32, 3, 32) and x.dtype == torch.float32
    r = cscan.scan_rows(case["u"], case["delta"], case["A"], case["B"], case["C"], case["D"], case["z"],
                        case["delta_bias"], True, chunk=2048, P=case["P"], Q=case["Q"])
    xc = x.cpu().double()
    assert torch.all(xc[..., 0::2] == 1.0)
    h = torch.from_numpy(r["h_chunks"]).reshape(1, 32, 3, 16)
    torch.testing.assert_close(xc[..., 1::2], h, rtol=1e-3 if dtype == torch.float32 else 3e-2,
                               atol=1e-4 if dtype == torch.float32 else 5e-2)
    _close(out.cpu(), torch.from_numpy(r["out"]).reshape(1, 32, L), dtype, "pre-gate out")
    _close(out_z.cpu(), torch.from_numpy(r["out_z"]).reshape(1, 32, L), dtype, "out_z")


def test_pq_long_sequence_fp32_vs_f64():
    """8192 fp32 steps against float64, row by row in the max norm: max_t |gpu - f64| <= atol +
    rtol max_t |f64|, and the kernel's largest row error at most twice that of the reference's own
    float32 path (the restatement of ssi.py:262-350, evaluated by torch on this host) on the same
    inputs. Rounding accumulates over the coupled recurrence, and at the steps where a row's output
    cancels towards zero no float32 evaluation meets rtol 1e-4 / atol 1e-5 element by element (the
    torch float32 path misses float64 by 3e-5 to 1.4e-4 there, depending on the host CPU), so rows
    are compared in the max norm. The kernel's decays use the bias-compensated exp2 (decay_exp2):
    with the plain v_exp_f32 its error here was 3.2e-4, with the compensation a float32 emulation of
    its operation order gives 2.0e-5."""
    _say("pq fp32 L=8192 vs float64 and vs the torch float32 path, row max norm")
    case = _pq_case(410, batch=1, dim=64, L=8192, N=16, R=2, dtype=torch.float32)
    out, last = _gpu(case)
    r = cscan.scan_rows(case["u"], case["delta"], case["A"], case["B"], case["C"], case["D"], case["z"],
                        case["delta_bias"], True, P=case["P"], Q=case["Q"])
    ref_out, ref_last = selective_scan_pq_ref(**case, return_last_state=True)
    rtol, atol = fixtures.tolerances(torch.float32)
    for got, ref32, exact, what in ((out, ref_out, r["out_z"], "out"), (last, ref_last, r["last_state"], "last")):
        exact = torch.from_numpy(exact).reshape(got.shape)
        err = (got.double() - exact).abs().amax(dim=-1)
        err32 = (ref32.double() - exact).abs().amax(dim=-1)
        bound = atol + rtol * exact.abs().amax(dim=-1)
        assert bool((err <= bound).all()), f"{what}: row max error {err.max().item():.3g} beyond {bound.min().item():.3g}"
        assert err.max().item() <= 2 * err32.max().item(), \
            f"{what}: kernel row max error {err.max().item():.3g} > 2 x torch float32 {err32.max().item():.3g}"
        print(f"[gpu-case] {what}: kernel row max error {err.max().item():.3g}, torch float32 {err32.max().item():.3g}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pq_long_sequence_16bit_one_wave_layout(dtype):
    """8192 steps with 16-bit inputs on 64 channels: the layout of 16 lanes of one state, whose
    coupling carries Q h from step to step (Q hb + (Q P) q) instead of forming it from h. The
    16-bit output element by element at the 16-bit tolerance; the float32 last state row by row in
    the max norm at the float32 tolerance, the bound the direct form meets in the float32 case
    above, so a drift of the carried form over the sequence would show there."""
    _say(f"pq {dtype} L=8192 one-wave layout vs float64")
    case = _pq_case(420, batch=1, dim=64, L=8192, N=16, R=2, dtype=dtype)
    out, last = _gpu(case)
    r = cscan.scan_rows(case["u"], case["delta"], case["A"], case["B"], case["C"], case["D"], case["z"],
                        case["delta_bias"], True, P=case["P"], Q=case["Q"])
    _close(out.cpu(), torch.from_numpy(r["out_z"]).reshape(out.shape), dtype, "out")
    rtol, atol = fixtures.tolerances(torch.float32)
    exact = torch.from_numpy(r["last_state"]).reshape(last.shape)
    err = (last.double().cpu() - exact).abs().amax(dim=-1)
    bound = atol + rtol * exact.abs().amax(dim=-1)
    assert bool((err <= bound).all()), f"last: row max error {err.max().item():.3g} beyond {bound.min().item():.3g}"


def test_pq_bench_shape_every_row():
    """The PQ benchmark shape (Mamba-1.4B layer, rank 2, per-channel P/Q, fp16): every (batch,
    channel) row -- the gated output at every step and the last state -- against the float64
    restatement (run on the host's threads, one call per batch row sharing its B/C)."""
    from motif_mamba_amd.workloads import PQ_CONFIGS, pq_inputs
    c = PQ_CONFIGS["pq_1p4b"]
    _say(f"pq bench shape {c}: every row")
    inputs = pq_inputs(c, device="cuda")
    from motif_mamba_amd import selective_scan_fn
    out, last = selective_scan_fn(**inputs)
    torch.cuda.synchronize()
    cpu = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in inputs.items()}
    rtol, atol = fixtures.tolerances(torch.float16)
    out, last = out.cpu(), last.cpu()
    for b in range(c.batch):
        y64, last64 = cscan.scan_all_rows(cpu["u"], cpu["delta"], cpu["A"], cpu["B"], cpu["C"], cpu["D"],
                                          cpu["z"], cpu["delta_bias"], True, batches=[b], P=cpu["P"], Q=cpu["Q"])
        np.testing.assert_allclose(out[b].double().numpy(), y64[0], rtol=rtol, atol=atol,
                                   err_msg=f"pq bench batch {b} out_z")
        np.testing.assert_allclose(last[b].double().numpy(), last64[0], rtol=rtol, atol=atol,
                                   err_msg=f"pq bench batch {b} last_state")


@pytest.mark.parametrize("batch,dim,N", [(6, 4096, 16), (1, 2048, 16), (3, 4096, 32)])
def test_pq_automatic_layout_every_row(batch, dim, N):
    """The host's own choice of lanes per channel (no MM_PQ_LPR) at sizes where, on a device of
    1,024 SIMDs, it picks 4 lanes (6 x 4096, dstate 16: more than 2.5 waves of 8 lanes per SIMD),
    16 lanes (1 x 2048: one wave of 16 lanes per SIMD) and 8 lanes of 4 states (3 x 4096, dstate
    32): every row's gated output and last state against the float64 restatement."""
    import dataclasses
    from motif_mamba_amd import selective_scan_fn
    from motif_mamba_amd.workloads import PQ_CONFIGS, pq_inputs
    c = dataclasses.replace(PQ_CONFIGS["pq_1p4b"], batch=batch, dim=dim, seqlen=64, dstate=N, seed=400 + batch)
    _say(f"pq automatic layout {batch} x {dim} dstate {N}")
    with _lpr(None):
        os.environ.pop("MM_PQ_LPR", None)
        inputs = pq_inputs(c, device="cuda")
        out, last = selective_scan_fn(**inputs)
        torch.cuda.synchronize()
    cpu = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in inputs.items()}
    r = cscan.scan_rows(cpu["u"], cpu["delta"], cpu["A"], cpu["B"], cpu["C"], cpu["D"], cpu["z"],
                        cpu["delta_bias"], True, P=cpu["P"], Q=cpu["Q"])
    _close(out.cpu().reshape(batch * dim, -1), torch.from_numpy(r["out_z"]), torch.float16, "out")
    _close(last.cpu().reshape(batch * dim, -1), torch.from_numpy(r["last_state"]), torch.float16, "last")


# ---------------------------------------------------------------------------------------------
# Boundary: the C ABI with P/Q, argument errors.
# ---------------------------------------------------------------------------------------------
def test_pq_c_abi_direct():
    _say("pq C ABI direct")
    lib = capi.load()
    case = _pq_case(420, batch=2, dim=32, L=128, N=16, R=3, dtype=torch.bfloat16, per_dim=False)
    g = _to(case, DEV)
    B4, C4 = g["B"].unsqueeze(1), g["C"].unsqueeze(1)
    out_z = torch.empty_like(g["z"])
    last = torch.empty(2, 32, 16, device=DEV)
    p = capi.scan_fwd_params(g["u"], g["delta"], g["A"], B4, C4, g["D"], g["z"], g["delta_bias"], True,
                             out_z=out_z, last_state=last, P=g["P"], Q=g["Q"])
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(p)) == 0
    rc = lib.mm_scan_fwd(ctypes.byref(p), capi.stream_handle())
    assert rc == 0, lib.mm_last_error().decode()
    torch.cuda.synchronize()
    ref, ref_last = selective_scan_pq_ref(**case, return_last_state=True)
    _close(out_z.cpu(), ref, torch.bfloat16, "capi out_z")
    _close(last.cpu(), ref_last, torch.bfloat16, "capi last")


def test_pq_argument_errors():
    _say("pq argument errors")
    from motif_mamba_amd import _native, selective_scan_fn
    case = _to(_pq_case(430, batch=1, dim=8, L=16, N=16, R=2, dtype=torch.float32), DEV)
    with pytest.raises(ValueError, match="both be provided"):
        selective_scan_fn(**{**case, "Q": None})
    with pytest.raises(ValueError, match="both be 2D or both be 3D"):
        selective_scan_fn(**{**case, "P": case["P"][0]})
    with pytest.raises(ValueError, match=r"Expected P\(dim, n, r\)"):
        selective_scan_fn(**{**case, "P": case["P"][:4], "Q": case["Q"][:4]})
    with pytest.raises(NotImplementedError, match="pq_rank"):
        selective_scan_fn(**{**case, "P": torch.zeros(8, 16, 9, device=DEV), "Q": torch.zeros(8, 9, 16, device=DEV)})
    with pytest.raises(ValueError, match="CUDA"):
        selective_scan_fn(**{**case, "P": case["P"].cpu()})
    B4, C4 = case["B"].unsqueeze(1), case["C"].unsqueeze(1)
    with pytest.raises(RuntimeError, match="gamma"):
        _native.ext().fwd(case["u"], case["delta"], case["A"], B4, C4, None, None, None, case["P"], case["Q"],
                          torch.zeros(5, device=DEV), True)
    with pytest.raises(RuntimeError, match="Q must be provided"):
        _native.ext().fwd(case["u"], case["delta"], case["A"], B4, C4, None, None, None, case["P"], None, None, True)
    # gamma is carried, not read: any valid gamma leaves the result unchanged
    a = selective_scan_fn(**case)
    b = selective_scan_fn(**case, gamma=torch.randn(8, 16, device=DEV))
    torch.testing.assert_close(a, b, rtol=0, atol=0)
