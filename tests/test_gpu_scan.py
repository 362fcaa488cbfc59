"""GPU parity of the forward selective scan against the CPU oracle (MI355X only).

Every call goes through the C ABI of libmm_scan.so -- via the PyTorch-ROCm binding behind
``selective_scan_fn`` or directly through ctypes -- and is compared with
``oracle.ssm_ref.selective_scan_ref`` (restating ssi.py:353-451) on the same seeded inputs, or,
at the full benchmark shapes, with the float64 C restatement on every row.
Tolerances (north_star): fp32 rtol 1e-4 / atol 1e-5; bf16/fp16 inputs rtol 3e-2 / atol 5e-2.
"""
import ctypes
import math
import sys

import numpy as np
import pytest
import torch
from einops import rearrange

from oracle import cscan
from oracle.ssm_ref import chunk_states_ref, selective_scan_ref
from tests import capi, fixtures

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(f"\n[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _to(d, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}


def _run(inputs, **kw):
    from motif_mamba_amd import selective_scan_fn
    g = _to(inputs, DEV)
    out, last = selective_scan_fn(**g, return_last_state=True, **kw)
    torch.cuda.synchronize()
    return out.cpu(), last.cpu()


def _close(a, b, dtype, what):
    rtol, atol = fixtures.tolerances(dtype)
    torch.testing.assert_close(a.float(), b.float(), rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


def _case(seed, batch, dim, L, N, dtype, bkind="3d", G=1, with_D=True, with_z=True, with_bias=True,
          softplus=True):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, L, generator=g).to(dtype)
    delta = torch.randn(batch, dim, L, generator=g)
    z = torch.randn(batch, dim, L, generator=g).to(dtype) if with_z else None
    lo, hi = math.log(1e-3), math.log(1e-1)
    bias = (torch.rand(dim, generator=g) * (hi - lo) + lo).float() if with_bias else None
    if not softplus:
        # without softplus the step size is used raw: keep delta + bias >= 0 as real callers do
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
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=bias, delta_softplus=softplus)


# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("name", fixtures.names())
def test_golden_fixture(name):
    _say(f"golden fixture {name}")
    inputs, exp = fixtures.load(name)
    out, last = _run(inputs)
    assert out.dtype == exp["out"].dtype
    _close(out, exp["out"], inputs["u"].dtype, f"{name} out")
    _close(last, exp["last_state"], inputs["u"].dtype, f"{name} last_state")


SHAPES = [
    # (batch, dim, L, N, bkind, G)
    (2, 64, 1, 16, "3d", 1),
    (2, 64, 5, 16, "3d", 1),
    (2, 64, 64, 16, "3d", 1),
    (3, 96, 130, 16, "4d", 2),
    (1, 128, 257, 16, "4d", 4),
    (2, 40, 33, 16, "3d", 1),        # dim not a multiple of 64
    (2, 64, 96, 8, "3d", 1),         # N < 16
    (1, 64, 48, 1, "3d", 1),
    (2, 64, 72, 32, "4d", 2),
    (1, 64, 40, 64, "3d", 1),
    (1, 8, 24, 100, "3d", 1),        # N > 64 (generic path)
    (2, 64, 50, 16, "const", 1),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"b{s[0]}d{s[1]}L{s[2]}N{s[3]}{s[4]}G{s[5]}" for s in SHAPES])
def test_random_shapes(shape, dtype):
    batch, dim, L, N, bkind, G = shape
    _say(f"random shape {shape} {dtype}")
    case = _case(7, batch, dim, L, N, dtype, bkind, G)
    exp, exp_last = selective_scan_ref(**case, return_last_state=True)
    out, last = _run(case)
    _close(out, exp, dtype, "out_z")
    _close(last, exp_last, dtype, "last_state")


@pytest.mark.parametrize("shape", [s for s in SHAPES if s[2] % 8 != 0],
                         ids=[f"b{s[0]}d{s[1]}L{s[2]}N{s[3]}{s[4]}G{s[5]}" for s in SHAPES if s[2] % 8 != 0])
def test_random_shapes_general_kernels(shape, monkeypatch):
    """The shapes with L % 8 != 0 again with the front padding off (MM_SCAN_PAD=0), so that the
    general kernels that serve them then stay covered."""
    monkeypatch.setenv("MM_SCAN_PAD", "0")
    batch, dim, L, N, bkind, G = shape
    _say(f"random shape {shape} bf16, padding off")
    case = _case(7, batch, dim, L, N, torch.bfloat16, bkind, G)
    exp, exp_last = selective_scan_ref(**case, return_last_state=True)
    out, last = _run(case)
    _close(out, exp, torch.bfloat16, "out_z")
    _close(last, exp_last, torch.bfloat16, "last_state")


@pytest.mark.parametrize("N", [4, 8, 12, 24, 32, 64])
@pytest.mark.parametrize("via_pq", ["1", "0"], ids=["zero-pair", "general"])
def test_other_dstate_every_row(N, via_pq, monkeypatch):
    """Diagonal inference at dstate != 16 (variable B/C): the P/Q kernels with a zero rank-1 pair,
    which leaves the recurrence exactly diagonal, or (MM_DIAG_VIA_PQ=0) the general kernel; every
    row's output and last state against the float64 restatement, G = 2, L = 256."""
    monkeypatch.setenv("MM_DIAG_VIA_PQ", via_pq)
    batch, dim, L = 2, 128, 256
    _say(f"dstate {N} via_pq={via_pq}")
    case = _case(130 + N, batch, dim, L, N, torch.bfloat16, bkind="4d", G=2)
    out, last = _run(case)
    _rows_vs_f64(case, out, last, f"dstate {N}")


@pytest.mark.parametrize("N,L", [(8, 4104), (32, 4096), (4, 2056)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("via_pq", ["1", "0"], ids=["zero-pair", "general"])
def test_other_dstate_reference_fwd_chunk_states(N, L, dtype, via_pq, monkeypatch):
    """The training forward (ext.fwd with chunk states) at dstate != 16: on the P/Q kernels with a
    zero pair, which then write x in the diagonal form, (prod a, h) per 2048-step chunk, or
    (MM_DIAG_VIA_PQ=0) on the general kernel. Whole and partial last chunks; the prod-a half
    against the closed form exp(A * sum delta'), the h half and the outputs of sampled rows against
    the float64 restatement (16-bit outputs element by element; float32 ones row by row in the max
    norm, as the long float32 P/Q check does: over thousands of steps, where a row's output cancels
    towards zero, no float32 evaluation meets the element-wise bound)."""
    monkeypatch.setenv("MM_DIAG_VIA_PQ", via_pq)
    _say(f"reference-format fwd dstate {N} L={L} {dtype} via_pq={via_pq}")
    from motif_mamba_amd import _native
    case = _case(140 + N, 2, 64, L, N, dtype, bkind="4d", G=2)
    g = _to(case, DEV)
    out, x, out_z = _native.ext().fwd(g["u"], g["delta"], g["A"], g["B"], g["C"], D=g["D"], z=g["z"],
                                      delta_bias=g["delta_bias"], delta_softplus=True)
    torch.cuda.synchronize()
    assert x.shape == (2, 64, (L + 2047) // 2048, 2 * N) and x.dtype == torch.float32
    rows = [(b, d) for b in (0, 1) for d in range(b, 64, 11)]
    r = cscan.scan_rows(**case, rows=rows, chunk=2048)    # out: pre-gate, out_z: gated
    rtol, atol = fixtures.tolerances(dtype)
    for got, exact, what in ((out, r["out"], "out"), (out_z, r["out_z"], "out_z")):
        got = torch.stack([got[b, d] for b, d in rows]).cpu().double()
        exact = torch.from_numpy(exact)
        if dtype == torch.float32:
            err = (got - exact).abs().amax(dim=-1)
            bound = atol + rtol * exact.abs().amax(dim=-1)
            assert bool((err <= bound).all()), f"{what}: row max error {err.max().item():.3g}"
        else:
            torch.testing.assert_close(got, exact, rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")
    for i, (b, d) in enumerate(rows):
        np.testing.assert_allclose(x[b, d, :, 1::2].cpu().double().numpy(), r["h_chunks"][i], rtol=1e-3, atol=1e-3)
    pa = chunk_states_ref(case["delta"], case["A"], case["delta_bias"], True)
    np.testing.assert_allclose(x[..., 0::2].cpu().double().numpy(), pa.numpy(), rtol=1e-3, atol=1e-30)


@pytest.mark.parametrize("L", [7, 13, 14, 1001, 2047])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("with_z", [True, False], ids=["z", "noz"])
def test_padded_lengths_every_row(L, dtype, with_z):
    """Inference requests whose length is not a multiple of 8 run the fast kernels on copies padded
    in front to a multiple of 32 steps with zero u (the binding's fwd_infer) from 14 steps on, the
    general kernel below (L 7, 13): every row's output and last state against the float64
    restatement, G = 2."""
    batch, dim = 2, 256
    _say(f"padded length L={L} {dtype} z={with_z}")
    case = _case(110 + L, batch, dim, L, 16, dtype, bkind="4d", G=2, with_z=with_z)
    out, last = _run(case)
    assert out.shape == (batch, dim, L) and out.is_contiguous() and last.shape == (batch, dim, 16)
    _rows_vs_f64(case, out, last, f"padded L={L}")


@pytest.mark.parametrize("flags", [dict(with_D=False), dict(with_z=False), dict(with_bias=False),
                                   dict(softplus=False), dict(with_D=False, with_z=False, with_bias=False,
                                                              softplus=False)],
                         ids=["noD", "noz", "nobias", "nosoftplus", "bare"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("L", [80, 96], ids=["L80", "L96"])  # 96: whole 32-step pairs (k2s)
def test_optional_inputs(flags, dtype, L):
    _say(f"optional inputs {flags} {dtype} L={L}")
    case = _case(8, 2, 64, L, 16, dtype, **flags)
    exp, exp_last = selective_scan_ref(**case, return_last_state=True)
    out, last = _run(case)
    _close(out, exp, dtype, "out")
    _close(last, exp_last, dtype, "last_state")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_strided_inputs_like_mamba_block(dtype):
    """x, z = xz.chunk(2, dim=1) and delta with strides (L, B*L, 1), as Mambamotif passes them
    (mamba_simplemotif.py:288, 308-313)."""
    _say(f"strided inputs {dtype}")
    batch, dim, L, N = 2, 64, 96, 16
    g = torch.Generator().manual_seed(9)
    xz = torch.randn(batch, 2 * dim, L, generator=g).to(dtype)
    dt_base = torch.randn(dim, batch * L, generator=g).to(dtype)
    B = torch.randn(batch, N, L, generator=g).to(dtype)
    C = torch.randn(batch, N, L, generator=g).to(dtype)
    A = -torch.rand(dim, N, generator=g) * 4
    D = torch.randn(dim, generator=g)
    bias = torch.rand(dim, generator=g) - 4

    def views(xz_, dt_base_):
        x, z = xz_.chunk(2, dim=1)
        return x, z, rearrange(dt_base_, "d (b l) -> b d l", l=L)

    x, z, dt = views(xz, dt_base)
    exp, exp_last = selective_scan_ref(x, dt, A, B, C, D, z, bias, True, return_last_state=True)
    gx, gz, gdt = views(xz.to(DEV), dt_base.to(DEV))
    assert not gx.is_contiguous() and gdt.stride() == (L, batch * L, 1)
    from motif_mamba_amd import selective_scan_fn
    out, last = selective_scan_fn(gx, gdt, A.to(DEV), B.to(DEV), C.to(DEV), D.to(DEV), gz, bias.to(DEV),
                                  True, return_last_state=True)
    torch.cuda.synchronize()
    _close(out.cpu(), exp, dtype, "out_z")
    _close(last.cpu(), exp_last, dtype, "last_state")


@pytest.mark.parametrize("L", [4100, 4096])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_reference_fwd_outputs(dtype, L):
    """ext.fwd returns [out, x, out_z] in the layout of selective_scan_cuda.fwd
    (selective_scan.cpp:383-412): out pre-gate, x = (B, D, ceil(L/2048), 2N) (prod a, h) pairs.
    L = 4100 runs the general kernel, L = 4096 the dstate-16 kernels (bf16: the buffer-addressed
    path for L a multiple of 32), both with a partial or whole last 2048-step chunk."""
    _say(f"reference-format fwd {dtype} L={L}")
    from motif_mamba_amd import _native
    case = _case(10, 1, 64, L, 16, dtype, bkind="4d", G=1)
    exp_z, exp_last = selective_scan_ref(**case, return_last_state=True)
    exp_out = selective_scan_ref(**{**case, "z": None})
    g = _to(case, DEV)
    out, x, out_z = _native.ext().fwd(g["u"], g["delta"], g["A"], g["B"], g["C"], D=g["D"], z=g["z"],
                                      delta_bias=g["delta_bias"], delta_softplus=True)
    torch.cuda.synchronize()
    assert x.shape == (1, 64, (L + 2047) // 2048, 32) and x.dtype == torch.float32
    _close(out.cpu(), exp_out, dtype, "out")
    _close(out_z.cpu(), exp_z, dtype, "out_z")
    _close(x[:, :, -1, 1::2].cpu(), exp_last, dtype, "x[..., -1, 1::2]")
    rows = [(0, d) for d in range(0, 64, 9)]
    r = cscan.scan_rows(**case, rows=rows, chunk=2048)
    for i, (b, d) in enumerate(rows):
        np.testing.assert_allclose(x[b, d, :, 1::2].cpu().double().numpy(), r["h_chunks"][i], rtol=1e-3, atol=1e-3)
    pa = chunk_states_ref(case["delta"], case["A"], case["delta_bias"], True)
    np.testing.assert_allclose(x[..., 0::2].cpu().double().numpy(), pa.numpy(), rtol=1e-3, atol=1e-30)


def test_c_abi_direct_call():
    """libmm_scan.so called through ctypes (no torch binding) on the config-0 fixture."""
    _say("C ABI via ctypes, cfg0")
    lib = capi.load()
    inputs, exp = fixtures.load("cfg0")
    g = _to(inputs, DEV)
    Bv = g["B"].unsqueeze(1)
    Cv = g["C"].unsqueeze(1)
    out_z = torch.empty_like(g["z"])
    last = torch.empty(g["u"].shape[0], g["u"].shape[1], g["A"].shape[1], device=DEV)
    p = capi.scan_fwd_params(g["u"], g["delta"], g["A"], Bv, Cv, g["D"], g["z"], g["delta_bias"], True,
                             out_z=out_z, last_state=last)
    rc = lib.mm_scan_fwd(ctypes.byref(p), capi.stream_handle())
    assert rc == 0, lib.mm_last_error()
    torch.cuda.synchronize()
    _close(out_z.cpu(), exp["out"], torch.float32, "out_z")
    _close(last.cpu(), exp["last_state"], torch.float32, "last_state")


def test_deterministic():
    _say("determinism cfg-like bf16")
    case = _to(_case(11, 2, 128, 600, 16, torch.bfloat16), DEV)
    from motif_mamba_amd import selective_scan_fn
    a, la = selective_scan_fn(**case, return_last_state=True)
    b, lb = selective_scan_fn(**case, return_last_state=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(la, lb)


def test_no_grad_with_inputs_requiring_grad_takes_inference_path():
    """Under torch.no_grad() with inputs that require grad (a module's A, D and delta_bias
    parameters), selective_scan_fn runs the inference forward: the output has the bits of the
    training forward's, carries no graph, and nothing for a backward is allocated (the training
    forward would add the pre-gate out, the chunk states and the tile states: about 3x the output)."""
    _say("selective_scan_fn no_grad with inputs requiring grad")
    from motif_mamba_amd import selective_scan_fn
    case = _case(40, 2, 64, 1024, 16, torch.bfloat16)
    g = _to(case, DEV)
    for k in ("A", "D", "delta_bias"):
        g[k].requires_grad_(True)
    out_train = selective_scan_fn(**g)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    with torch.no_grad():
        out = selective_scan_fn(**g)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    assert not out.requires_grad and out_train.requires_grad
    assert torch.equal(out, out_train.detach())
    out_bytes = out.numel() * out.element_size()
    assert peak < 2 * out_bytes, f"peak {peak} bytes for a {out_bytes}-byte output"


# ---------------------------------------------------------------------------------------------
# Full benchmark shapes: every row against the float64 C restatement.
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("cfg", ["cfg1", "cfg2", "cfg3_g1", "cfg3_g4"])
def test_full_size_config(cfg):
    """Every (batch, channel) row of the configuration -- out_z at every step and last_state --
    against the float64 C restatement of ssi.py:353-451 (run on the host's threads, one call per
    (batch, group) sharing that group's B/C), element by element at the north_star tolerances.
    An indexing mistake confined to one batch row, one 16-channel workgroup or one sequence
    segment cannot pass."""
    from motif_mamba_amd.workloads import SCAN_CONFIGS, scan_inputs
    c = SCAN_CONFIGS[cfg]
    _say(f"full-size {cfg}: {c}")
    inputs = scan_inputs(c)
    inputs.pop("return_last_state")
    dtype = inputs["u"].dtype
    out, last = _run(inputs)
    assert out.shape == inputs["u"].shape and out.dtype == dtype
    rtol, atol = fixtures.tolerances(dtype)
    for b in range(c.batch):   # one batch row at a time keeps the float64 copies small
        y64, last64 = cscan.scan_all_rows(**inputs, batches=[b])
        np.testing.assert_allclose(out[b].double().numpy(), y64[0], rtol=rtol, atol=atol,
                                   err_msg=f"{cfg} batch {b} out_z")
        np.testing.assert_allclose(last[b].double().numpy(), last64[0], rtol=rtol, atol=atol,
                                   err_msg=f"{cfg} batch {b} last_state")


@pytest.mark.parametrize("mix", ["varB_constC", "constB_varC"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_mixed_constant_variable_bc(mix, dtype):
    """B and C are independently input-dependent or constant (is_variable_B / is_variable_C,
    selective_scan.cpp:284-285, 316-327): one of each, 3-D and 4-D variable layouts. The group
    count comes from B alone (selective_scan.cpp:307: n_groups = is_variable_B ? B.size(1) : 1),
    so with a constant B a variable C must have one group; a grouped C is refused, as there."""
    _say(f"mixed B/C {mix} {dtype}")
    if mix == "constB_varC":
        bad = _case(23, 2, 64, 77, 16, dtype, "4d", 2)
        bad["B"] = _case(23, 2, 64, 77, 16, dtype, "const", 1)["B"]
        with pytest.raises(RuntimeError, match="C must have shape"):
            _run(bad)
    for bkind, G in (("3d", 1), ("4d", 2 if mix == "varB_constC" else 1)):
        var = _case(23, 2, 64, 77, 16, dtype, bkind, G)
        const = _case(23, 2, 64, 77, 16, dtype, "const", 1)
        case = dict(var)
        if mix == "varB_constC":
            case["C"] = const["C"]
        else:
            case["B"] = const["B"]
        exp, exp_last = selective_scan_ref(**case, return_last_state=True)
        out, last = _run(case)
        _close(out, exp, dtype, f"{mix} {bkind} out_z")
        _close(last, exp_last, dtype, f"{mix} {bkind} last_state")


# ---------------------------------------------------------------------------------------------
# Sequence-parallel segments: few (batch, 16-channel) groups and a long sequence.
# ---------------------------------------------------------------------------------------------

def _seg_rows(out, last, case, what):
    rows = [(0, d) for d in range(case["u"].shape[1])]
    r = cscan.scan_rows(**case, rows=rows)
    rtol, atol = fixtures.tolerances(case["u"].dtype)
    exp = r["out_z"] if case["z"] is not None else r["out"]   # without z the pre-gate out is returned
    for i, (b, d) in enumerate(rows):
        np.testing.assert_allclose(out[b, d].double().numpy(), exp[i], rtol=rtol, atol=atol,
                                   err_msg=f"{what} row {(b, d)} out_z")
        np.testing.assert_allclose(last[b, d].double().numpy(), r["last_state"][i], rtol=rtol, atol=atol,
                                   err_msg=f"{what} row {(b, d)} last_state")


# L 8192: 256 tile pairs in 16 segments of 16 pairs (k2s segments). L 8864: 277 pairs in 17
# segments of 17, the last of 5 (odd pair counts, a short last segment). L 8200: not whole 32-step
# pairs (the pipelined kernel's segments, a partial last tile).
@pytest.mark.parametrize("L", [8192, 8864, 8200])
@pytest.mark.parametrize("G", [1, 2])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_segmented_scan(dtype, G, L):
    """batch 1 x 64 channels is 4 channel groups, so a long scan runs in sequence segments
    (state-only pass, carry chain, full pass); every row against the float64 restatement."""
    _say(f"segmented scan {dtype} G={G} L={L}")
    case = _case(20 + G, 1, 64, L, 16, dtype, bkind="4d", G=G)
    out, last = _run(case)
    _seg_rows(out, last, case, f"segmented G={G} L={L}")


@pytest.mark.parametrize("flags", [dict(with_z=False), dict(softplus=False), dict(with_D=False, with_bias=False)],
                         ids=["noz", "nosoftplus", "noD_nobias"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_segmented_optional_inputs(dtype, flags):
    """The segmented kernels without z (the pre-gate out is the output), without softplus, and
    without D and delta_bias; every row against the float64 restatement."""
    _say(f"segmented optional inputs {flags} {dtype}")
    case = _case(26, 1, 64, 4096, 16, dtype, bkind="4d", G=1, **flags)
    out, last = _run(case)
    _seg_rows(out, last, case, f"segmented {flags}")


def test_segmented_reference_fwd_chunk_states():
    """The reference-format fwd on a segmented shape: x's (prod a, h) per 2048-step chunk carry
    the delta' prefix and the state across segment boundaries."""
    _say("segmented reference-format fwd")
    from motif_mamba_amd import _native
    case = _case(30, 1, 64, 8192 + 96, 16, torch.float32, bkind="4d", G=1)
    g = _to(case, DEV)
    out, x, out_z = _native.ext().fwd(g["u"], g["delta"], g["A"], g["B"], g["C"], D=g["D"], z=g["z"],
                                      delta_bias=g["delta_bias"], delta_softplus=True)
    torch.cuda.synchronize()
    assert x.shape == (1, 64, 5, 32)
    rows = [(0, d) for d in range(64)]
    r = cscan.scan_rows(**case, rows=rows, chunk=2048)
    for i, (b, d) in enumerate(rows):
        np.testing.assert_allclose(x[b, d, :, 1::2].cpu().double().numpy(), r["h_chunks"][i], rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(out_z[b, d].cpu().double().numpy(), r["out_z"][i], rtol=1e-4, atol=1e-5)
    pa = chunk_states_ref(case["delta"], case["A"], case["delta_bias"], True)
    np.testing.assert_allclose(x[..., 0::2].cpu().double().numpy(), pa.numpy(), rtol=1e-3, atol=1e-30)
    exp_out = selective_scan_ref(**{**case, "z": None})
    _close(out.cpu(), exp_out, torch.float32, "out (pre-gate)")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_segmented_reference_fwd_chunk_states_16bit(dtype):
    """The reference-format fwd without z on a segmented 16-bit shape (k2s segments with chunk
    states): x's (prod a, h) per 2048-step chunk carry the delta' prefix and the state across
    segment boundaries; out against the float64 restatement."""
    _say(f"segmented reference-format fwd, {dtype}, no z")
    from motif_mamba_amd import _native
    case = _case(32, 1, 64, 8192 + 96, 16, dtype, bkind="4d", G=1, with_z=False)
    g = _to(case, DEV)
    res = _native.ext().fwd(g["u"], g["delta"], g["A"], g["B"], g["C"], D=g["D"], z=None,
                            delta_bias=g["delta_bias"], delta_softplus=True)
    torch.cuda.synchronize()
    assert len(res) == 2
    out, x = res
    assert x.shape == (1, 64, 5, 32)
    rows = [(0, d) for d in range(64)]
    r = cscan.scan_rows(**case, rows=rows, chunk=2048)
    rtol, atol = fixtures.tolerances(dtype)
    for i, (b, d) in enumerate(rows):
        np.testing.assert_allclose(x[b, d, :, 1::2].cpu().double().numpy(), r["h_chunks"][i], rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(out[b, d].cpu().double().numpy(), r["out"][i], rtol=rtol, atol=atol)
    pa = chunk_states_ref(case["delta"], case["A"], case["delta_bias"], True)
    np.testing.assert_allclose(x[..., 0::2].cpu().double().numpy(), pa.numpy(), rtol=1e-3, atol=1e-30)


def test_segmented_c_abi_with_and_without_workspace():
    """Through ctypes: with the queried workspace the segmented kernels run, without it the single
    pass; both match the float64 restatement."""
    _say("segmented C ABI, workspace / none")
    lib = capi.load()
    case = _case(31, 1, 32, 4096, 16, torch.bfloat16, bkind="4d", G=1)
    g = _to(case, DEV)
    res = []
    for use_ws in (True, False):
        out_z = torch.empty_like(g["z"])
        last = torch.empty(1, 32, 16, device=DEV)
        p = capi.scan_fwd_params(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"], True,
                                 out_z=out_z, last_state=last)
        need = lib.mm_scan_fwd_workspace_size(ctypes.byref(p))
        assert need > 0
        ws = torch.empty(need, dtype=torch.uint8, device=DEV) if use_ws else None
        if ws is not None:
            p.workspace, p.workspace_bytes = ws.data_ptr(), need
        rc = lib.mm_scan_fwd(ctypes.byref(p), capi.stream_handle())
        assert rc == 0, lib.mm_last_error()
        torch.cuda.synchronize()
        res.append((out_z.cpu(), last.cpu()))
    for (o, l), what in zip(res, ("with workspace", "without workspace")):
        _seg_rows(o, l, case, what)


# ---------------------------------------------------------------------------------------------
# The balanced mixed grid (scan_fwd_mix): 3 or 5 sixteen-channel groups per compute unit.
# ---------------------------------------------------------------------------------------------
def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _rows_vs_f64(inputs, out, last, what):
    rtol, atol = fixtures.tolerances(inputs["u"].dtype)
    y64, last64 = cscan.scan_all_rows(**inputs)
    np.testing.assert_allclose(out.double().numpy(), y64, rtol=rtol, atol=atol, err_msg=f"{what} out")
    if last is not None:
        np.testing.assert_allclose(last.double().numpy(), last64, rtol=rtol, atol=atol,
                                   err_msg=f"{what} last_state")


@pytest.mark.parametrize("q", [3, 5])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["fp32", "bf16", "fp16"])
def test_balanced_grid_every_row(q, dtype):
    """Shapes whose 16-channel groups number 3 or 5 per compute unit run the mixed grid: two-state
    (k2s) groups in the first blocks, one-state (k1s) groups in the last ones. Every row -- both
    paths and the group where one hands over to the other -- against the float64 restatement. With
    batch 2 the one-state groups sit in the second batch row; L = 96 is an odd number of 32-step
    pairs."""
    cus = _cus()
    batch, dim = 2, q * cus * 16 // 2
    _say(f"balanced grid q={q} {dtype} batch {batch} dim {dim} L 96 (CUs {cus})")
    case = _case(70 + q, batch, dim, 96, 16, dtype)
    out, last = _run(case)
    _rows_vs_f64(case, out, last, f"q={q} {dtype}")


@pytest.mark.parametrize("q,dtype,with_z", [(3, torch.bfloat16, True), (5, torch.bfloat16, True),
                                             (3, torch.float16, True), (5, torch.float16, True),
                                             (5, torch.bfloat16, False)],
                         ids=["q3-bf16", "q5-bf16", "q3-fp16", "q5-fp16", "q5-bf16-no-z"])
def test_balanced_grid_training_outputs(q, dtype, with_z):
    """The training forward (pre-gate out, out_z, chunk states x and tile states) on the mixed grid,
    16-bit inputs: out and out_z of every row against the float64 restatement; x's (prod a, h)
    pairs and the tile states (the state before every 16-step tile) on rows of both group kinds and
    of the groups where one hands over to the other. L = 2144: a whole 2048-step chunk and a
    partial one."""
    from motif_mamba_amd import _native
    cus = _cus()
    batch, dim, L = 2, q * cus * 16 // 2, 2144
    _say(f"balanced grid training outputs q={q} {dtype} batch {batch} dim {dim} L {L}")
    case = _case(90 + q, batch, dim, L, 16, dtype, bkind="4d", G=1, with_z=with_z)
    g = _to(case, DEV)
    res = _native.ext().fwd(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["z"], g["delta_bias"],
                            None, None, None, True, tile_states=True)
    torch.cuda.synchronize()
    if with_z:
        out, x, out_z, ck = res
        _rows_vs_f64(case, out_z.cpu(), None, f"q={q} {dtype} out_z")
    else:
        out, x, ck = res
    n_tiles = L // 16
    assert x.shape == (batch, dim, 2, 32) and ck.shape == (n_tiles, batch, dim, 16)
    _rows_vs_f64(dict(case, z=None), out.cpu(), None, f"q={q} {dtype} pre-gate out")
    pa = chunk_states_ref(case["delta"], case["A"], case["delta_bias"], True)
    np.testing.assert_allclose(x[..., 0::2].cpu().double().numpy(), pa.numpy(), rtol=1e-3, atol=1e-30)
    first_k1 = 2 * (q // 2) * cus * 16     # first (batch-major) channel of the one-state groups
    sel = [0, 1, 15, first_k1 - 16, first_k1 - 1, first_k1, first_k1 + 15, batch * dim - 1]
    rows = [(i // dim, i % dim) for i in sel]
    r2 = cscan.scan_rows(**case, rows=rows, chunk=2048)
    r16 = cscan.scan_rows(**case, rows=rows, chunk=16)
    xc, ckc = x.cpu(), ck.cpu()
    for i, (b, d) in enumerate(rows):
        np.testing.assert_allclose(xc[b, d, :, 1::2].double().numpy(), r2["h_chunks"][i], rtol=1e-3, atol=1e-3,
                                   err_msg=f"x row {(b, d)}")
        assert float(ckc[0, b, d].abs().max()) == 0.0
        np.testing.assert_allclose(ckc[1:, b, d].double().numpy(), r16["h_chunks"][i][:n_tiles - 1], rtol=1e-3,
                                   atol=1e-3, err_msg=f"tile states row {(b, d)}")


@pytest.mark.parametrize("flags", [dict(with_z=False), dict(with_D=False, with_bias=False), dict(softplus=False),
                                   dict(bkind="4d", G=4)], ids=["no_z", "no_D_bias", "no_softplus", "G4"])
def test_balanced_grid_optional_inputs(flags):
    cus = _cus()
    dim = 3 * cus * 16
    _say(f"balanced grid optional inputs {flags} batch 1 dim {dim} L 64")
    case = _case(75, 1, dim, 64, 16, torch.bfloat16, **flags)
    out, last = _run(case)
    _rows_vs_f64(case, out, last, f"balanced grid {flags}")


def test_balanced_grid_out_and_out_z_c_abi():
    """The pre-gate out and out_z written together (no chunk states) through the C ABI on the mixed
    grid, plus two identical calls giving the same bits."""
    lib = capi.load()
    cus = _cus()
    dim = 5 * cus * 16
    _say(f"balanced grid out + out_z via C ABI, batch 1 dim {dim} L 64")
    case = _case(76, 1, dim, 64, 16, torch.bfloat16)
    g = _to(case, DEV)
    res = []
    for _ in range(2):
        out = torch.empty_like(g["u"])
        out_z = torch.empty_like(g["u"])
        last = torch.empty(1, dim, 16, device=DEV)
        p = capi.scan_fwd_params(g["u"], g["delta"], g["A"], g["B"].unsqueeze(1), g["C"].unsqueeze(1), g["D"],
                                 g["z"], g["delta_bias"], True, out=out, out_z=out_z, last_state=last)
        rc = lib.mm_scan_fwd(ctypes.byref(p), capi.stream_handle())
        assert rc == 0, lib.mm_last_error()
        torch.cuda.synchronize()
        res.append((out.cpu(), out_z.cpu(), last.cpu()))
    assert all(torch.equal(a, b) for a, b in zip(res[0], res[1]))
    _rows_vs_f64(case, res[0][1], res[0][2], "out_z")
    no_z = dict(case, z=None)
    _rows_vs_f64(no_z, res[0][0], None, "pre-gate out")


@pytest.mark.parametrize("L", [64, 2048])
def test_fp32_group_span_above_4_gib(L):
    """An fp32 u whose channel stride puts the 16-channel group's span above 2^32 bytes (but below
    2^31 elements): the kernels that address a group with 32-bit byte offsets (k2s, k1s) would wrap
    and read other rows, so the request must go to the element-offset kernels (L 64: one pass;
    L 2048: sequence segments). Checked against the oracle."""
    from motif_mamba_amd import selective_scan_fn
    S = (1 << 26) + (1 << 24)                # 15 * S * 4 bytes > 2^32, 15 * S + L < 2^31
    _say(f"fp32 u channel stride {S} (5.4 GB view), L {L}")
    case = _case(80, 1, 16, L, 16, torch.float32)
    base = torch.zeros(16 * S, device=DEV)
    u = base.as_strided((1, 16, L), (16 * S, S, 1))
    u.copy_(case["u"].to(DEV))
    g = _to(case, DEV)
    g["u"] = u
    out, last = selective_scan_fn(**g, return_last_state=True)
    torch.cuda.synchronize()
    del base, u
    exp, exp_last = selective_scan_ref(**case, return_last_state=True)
    _close(out.cpu(), exp, torch.float32, "out_z")
    _close(last.cpu(), exp_last, torch.float32, "last_state")
