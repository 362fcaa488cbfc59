"""GPU parity of the causal depthwise conv1d (forward, backward and decode update, mm_conv1d.hip) against the
CPU oracle oracle/conv_ref.py (the Mamba module's torch fallback, mamba_simplemotif.py:298-299 and
:353-358, and the published semantics of the causal-conv1d API the reference calls).
Tolerances (north_star): fp32 rtol 1e-4 / atol 1e-5; bf16/fp16 rtol 3e-2 / atol 5e-2.
"""
import ctypes
import sys

import pytest
import torch

from oracle.conv_ref import causal_conv1d_ref, causal_conv1d_update_ref
from tests import capi, fixtures

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(f"\n[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _close(a, b, dtype, what):
    rtol, atol = fixtures.tolerances(dtype)
    torch.testing.assert_close(a.float().cpu(), b.float().cpu(), rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


def _case(seed, batch, dim, L, W, dtype, wdtype=None, with_bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, dim, L, generator=g).to(dtype)
    w = (torch.randn(dim, W, generator=g) * 0.5).to(wdtype or dtype)
    b = (torch.randn(dim, generator=g) * 0.1).to(wdtype or dtype) if with_bias else None
    return x, w, b


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("L", [1, 7, 64, 1000])
def test_conv_fwd(dtype, W, L):
    _say(f"conv fwd {dtype} W={W} L={L}")
    from causal_conv1d import causal_conv1d_fn
    x, w, b = _case(700 + W + L, 2, 24, L, W, dtype)
    for act in (None, "silu"):
        got = causal_conv1d_fn(x.to(DEV), w.to(DEV), b.to(DEV), activation=act)
        _close(got, causal_conv1d_ref(x, w, b, activation=act), dtype, f"act={act}")


@pytest.mark.parametrize("W", [2, 4])
def test_conv_fwd_initial_and_final_states(W):
    _say(f"conv fwd initial/final states W={W}")
    from causal_conv1d import causal_conv1d_fn
    x, w, b = _case(710 + W, 2, 16, 40, W, torch.float32)
    ini = torch.randn(2, 16, W - 1, generator=torch.Generator().manual_seed(711))
    got, fin = causal_conv1d_fn(x.to(DEV), w.to(DEV), b.to(DEV), initial_states=ini.to(DEV),
                                return_final_states=True, activation="silu")
    ref, ref_fin = causal_conv1d_ref(x, w, b, initial_states=ini, return_final_states=True, activation="silu")
    _close(got, ref, torch.float32, "out")
    torch.testing.assert_close(fin.cpu(), ref_fin)
    # shorter than width - 1: final states come partly from the initial states
    got2, fin2 = causal_conv1d_fn(x[..., :1].to(DEV), w.to(DEV), None, initial_states=ini.to(DEV),
                                  return_final_states=True)
    ref2, rfin2 = causal_conv1d_ref(x[..., :1], w, None, initial_states=ini, return_final_states=True)
    _close(got2, ref2, torch.float32, "short out")
    torch.testing.assert_close(fin2.cpu(), rfin2)


def test_conv_fwd_strided_and_mixed_dtypes():
    """x as the first half of an xz projection (batch stride 2*dim*L), unaligned rows, fp32 weights on
    bf16 activations (the module's float32 parameters under bf16 activations)."""
    _say("conv fwd strided / mixed dtypes")
    from causal_conv1d import causal_conv1d_fn
    g = torch.Generator().manual_seed(720)
    xz = torch.randn(2, 64, 256, generator=g).to(torch.bfloat16)
    w = torch.randn(32, 4, generator=g) * 0.5
    b = torch.randn(32, generator=g) * 0.1
    x, _ = xz.to(DEV).chunk(2, dim=1)
    got = causal_conv1d_fn(x, w.to(DEV), b.to(DEV), activation="silu")
    _close(got, causal_conv1d_ref(xz[:, :32], w, b, activation="silu"), torch.bfloat16, "xz half")
    odd = torch.zeros(2, 32, 257, dtype=torch.bfloat16, device=DEV)
    odd[..., 1:] = xz[:, :32].to(DEV)
    got2 = causal_conv1d_fn(odd[..., 1:], w.to(DEV), b.to(DEV), activation="silu")
    _close(got2, causal_conv1d_ref(xz[:, :32], w, b, activation="silu"), torch.bfloat16, "unaligned")


@pytest.mark.parametrize("dtype,sdtype", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                          (torch.float32, torch.float32), (torch.float16, torch.float16)])
@pytest.mark.parametrize("state_len", [3, 4, 6])
@pytest.mark.parametrize("seqlen", [1, 3])
def test_conv_update(dtype, sdtype, state_len, seqlen):
    _say(f"conv update {dtype} state {sdtype} S={state_len} seqlen={seqlen}")
    from causal_conv1d import causal_conv1d_update
    g = torch.Generator().manual_seed(730 + state_len + seqlen)
    x = torch.randn(3, 40, seqlen, generator=g).to(dtype)
    w = (torch.randn(40, 4, generator=g) * 0.5).to(dtype)
    b = (torch.randn(40, generator=g) * 0.1).to(dtype)
    st = torch.randn(3, 40, state_len, generator=g).to(sdtype)
    st_ref = st.clone()
    st_gpu = st.to(DEV)
    xin = x[..., 0] if seqlen == 1 else x
    got = causal_conv1d_update(xin.to(DEV), st_gpu, w.to(DEV), b.to(DEV), activation="silu")
    ref = causal_conv1d_update_ref(xin, st_ref, w, b, activation="silu")
    assert got.shape == xin.shape
    _close(got, ref, dtype, "out")
    _close(st_gpu, st_ref, sdtype, "state")



@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32], ids=["w_bf16", "w_fp32"])
def test_conv_update_decode_many_rows(wdtype):
    """The decode form with four batch rows per workgroup (222 x 4700: a partial last block of
    channels, 4700 = 18 x 256 + 92, and of batch rows, 222 = 55 x 4 + 2), bf16 tokens and state with
    bf16 or float32 weights."""
    _say(f"conv update 222 x 4700 weight {wdtype}")
    from causal_conv1d import causal_conv1d_update
    g = torch.Generator().manual_seed(760)
    batch, dim = 222, 4700
    x = torch.randn(batch, dim, generator=g).to(torch.bfloat16)
    w = (torch.randn(dim, 4, generator=g) * 0.5).to(wdtype)
    b = (torch.randn(dim, generator=g) * 0.1).to(wdtype)
    st = torch.randn(batch, dim, 4, generator=g).to(torch.bfloat16)
    st_ref = st.clone()
    st_gpu = st.to(DEV)
    got = causal_conv1d_update(x.to(DEV), st_gpu, w.to(DEV), b.to(DEV), activation="silu")
    ref = causal_conv1d_update_ref(x, st_ref, w, b, activation="silu")
    _close(got, ref, torch.bfloat16, "out")
    assert torch.equal(st_gpu.cpu(), st_ref), "state: the shifted entries must be moved exactly"

def test_conv_prefill_then_decode_matches_forward():
    """The module's hand-off (mamba_simplemotif.py:292-293): the state after a prefill is the last
    d_conv inputs; decoding the following tokens one by one reproduces the forward of the sequence."""
    _say("conv prefill + decode")
    from causal_conv1d import causal_conv1d_fn, causal_conv1d_update
    x, w, b = _case(740, 2, 48, 40, 4, torch.float32)
    full = causal_conv1d_fn(x.to(DEV), w.to(DEV), b.to(DEV), activation="silu")
    state = torch.nn.functional.pad(x[..., :32], (4 - 32, 0)).to(DEV).contiguous()   # last 4 inputs
    for t in range(32, 40):
        y = causal_conv1d_update(x[:, :, t].to(DEV), state, w.to(DEV), b.to(DEV), activation="silu")
        torch.testing.assert_close(y, full[:, :, t], rtol=1e-5, atol=1e-6)


def test_conv_fwd_benchmark_shape_rows():
    """The conv before the config-2 scan (batch 4, 5120 channels, L 4096, bf16, width 4): a slice of
    channels against the oracle."""
    _say("conv fwd config-2 shape")
    from causal_conv1d import causal_conv1d_fn
    g = torch.Generator().manual_seed(750)
    x = torch.randn(4, 5120, 4096, generator=g).to(torch.bfloat16)
    w = (torch.randn(5120, 4, generator=g) * 0.5).to(torch.bfloat16)
    b = (torch.randn(5120, generator=g) * 0.1).to(torch.bfloat16)
    got = causal_conv1d_fn(x.to(DEV), w.to(DEV), b.to(DEV), activation="silu").cpu()
    sl = slice(1000, 1064)
    _close(got[:, sl], causal_conv1d_ref(x[:, sl], w[sl], b[sl], activation="silu"), torch.bfloat16, "rows")
    _close(got[:, -8:], causal_conv1d_ref(x[:, -8:], w[-8:], b[-8:], activation="silu"), torch.bfloat16, "last rows")


def test_conv_c_abi_direct():
    _say("conv C ABI direct")
    lib = capi.load()
    x, w, b = _case(760, 2, 16, 128, 4, torch.float32)
    xg, wg, bg = x.to(DEV), w.to(DEV), b.to(DEV)
    out = torch.empty_like(xg)
    p = capi.Conv1dFwdParams()
    p.batch, p.dim, p.seqlen, p.width, p.itype, p.wtype, p.silu = 2, 16, 128, 4, 0, 0, 1
    p.x, p.weight, p.bias, p.out = xg.data_ptr(), wg.data_ptr(), bg.data_ptr(), out.data_ptr()
    p.x_batch_stride, p.x_d_stride = xg.stride(0), xg.stride(1)
    p.out_batch_stride, p.out_d_stride = out.stride(0), out.stride(1)
    p.weight_d_stride, p.weight_w_stride, p.bias_stride = wg.stride(0), wg.stride(1), 1
    rc = lib.mm_causal_conv1d_fwd(ctypes.byref(p), capi.stream_handle())
    assert rc == 0, lib.mm_last_error().decode()
    torch.cuda.synchronize()
    _close(out, causal_conv1d_ref(x, w, b, activation="silu"), torch.float32, "capi fwd")


# Backward (mm_causal_conv1d_bwd): gradients of the oracle's float32 forward by autograd, on the same
# inputs, element-wise |err| <= rtol |exact| + atol max(1, max |exact|) with the forward's (rtol,
# atol) pair: dweight and dbias are sums over batch and steps whose rounding grows with their scale.

def _gcheck(got, exact, dtype, what):
    rtol, atol = fixtures.tolerances(dtype)
    got, exact = got.double().cpu(), exact.double()
    scale = max(1.0, exact.abs().max().item()) if exact.numel() else 1.0
    err = (got - exact).abs()
    bad = err > rtol * exact.abs() + atol * scale
    assert not bool(bad.any()), f"{what}: {int(bad.sum())}/{err.numel()} beyond tolerance, max err {err.max().item():.3g}"


def _ref_grads(x, w, b, dout, act):
    xr = x.detach().float().clone().requires_grad_(True)
    wr = w.detach().float().clone().requires_grad_(True)
    br = b.detach().float().clone().requires_grad_(True) if b is not None else None
    causal_conv1d_ref(xr, wr, br, activation=act, compute_dtype=torch.float64).float().backward(dout.float())
    return xr.grad, wr.grad, (br.grad if br is not None else None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("W", [2, 3, 4])
# The kernel takes 2,048-step tiles (8 positions per lane) where they leave fewer idle lanes than
# 4,096-step tiles (16 per lane): L 1 .. 1000 and 9000 (five tiles, the last partial) take the
# former, 4000 (one partial tile either way) the latter.
@pytest.mark.parametrize("L", [1, 7, 64, 1000, 4000, 9000])
def test_conv_bwd(dtype, W, L):
    _say(f"conv bwd {dtype} W={W} L={L}")
    from causal_conv1d import causal_conv1d_fn
    x, w, b = _case(800 + W + L, 2, 24, L, W, dtype)
    dout = torch.randn(2, 24, L, generator=torch.Generator().manual_seed(801)).to(dtype)
    for act in (None, "silu"):
        xg, wg, bg = (t.to(DEV).requires_grad_(True) for t in (x, w, b))
        causal_conv1d_fn(xg, wg, bg, activation=act).backward(dout.to(DEV))
        torch.cuda.synchronize()
        ex, ew, eb = _ref_grads(x, w, b, dout, act)
        assert xg.grad.dtype == dtype and wg.grad.dtype == w.dtype
        _gcheck(xg.grad, ex, dtype, f"dx act={act}")
        _gcheck(wg.grad, ew, dtype, f"dweight act={act}")
        _gcheck(bg.grad, eb, dtype, f"dbias act={act}")


def test_conv_bwd_function_into_dxz_slice_no_bias():
    """causal_conv1d_bwd_function as MambaInnerFn calls it (ssi.py:635-637): x a half of xz, dout in a
    channel-major layout, dx written into the matching half of a preallocated dxz, no bias."""
    _say("conv bwd function into dxz slice")
    from causal_conv1d.cpp_functions import causal_conv1d_bwd_function
    g = torch.Generator().manual_seed(810)
    xz = torch.randn(3, 64, 96, generator=g).to(torch.bfloat16)
    w = torch.randn(32, 4, generator=g) * 0.5
    dcm = torch.randn(32, 3, 96, generator=g).to(torch.bfloat16)          # (d, b, l) storage
    x = xz.to(DEV).chunk(2, dim=1)[0]
    dout = dcm.to(DEV).transpose(0, 1)                                       # (b, d, l) view
    dxz = torch.full((3, 64, 96), 7.0, dtype=torch.bfloat16, device=DEV)
    dx_slot = dxz.chunk(2, dim=1)[0]
    dx, dw, db, dini = causal_conv1d_bwd_function(x, w.to(DEV), None, dout, None, None, None, dx_slot, False, True)
    torch.cuda.synchronize()
    assert db is None and dini is None and dx.data_ptr() == dx_slot.data_ptr()
    ex, ew, _ = _ref_grads(xz[:, :32], w, None, dcm.transpose(0, 1), "silu")
    _gcheck(dxz[:, :32], ex, torch.bfloat16, "dx")
    assert bool((dxz[:, 32:] == 7.0).all()), "the z half of dxz was written"
    _gcheck(dw, ew, torch.bfloat16, "dweight")


def test_conv_bwd_benchmark_shape_rows():
    """Config-2 conv shape (batch 4, 5120 channels, L 4096, bf16): a slice of channels against the oracle."""
    _say("conv bwd config-2 shape")
    from motif_mamba_amd.causal_conv1d import causal_conv1d_bwd
    g = torch.Generator().manual_seed(820)
    x = torch.randn(4, 5120, 4096, generator=g).to(torch.bfloat16)
    w = (torch.randn(5120, 4, generator=g) * 0.5).to(torch.bfloat16)
    b = (torch.randn(5120, generator=g) * 0.1).to(torch.bfloat16)
    dout = torch.randn(4, 5120, 4096, generator=g).to(torch.bfloat16)
    gx, gw, gb, gd = x.to(DEV), w.to(DEV), b.to(DEV), dout.to(DEV)
    dx, dw, db = causal_conv1d_bwd(gx, gw, gb, gd, None, True)
    dx2, dw2, db2 = causal_conv1d_bwd(gx, gw, gb, gd, None, True)
    # one workgroup per channel sums dweight / dbias in a fixed order: the same bits on every call
    assert torch.equal(dw, dw2) and torch.equal(db, db2) and torch.equal(dx, dx2)
    dx, dw, db = dx.cpu(), dw.cpu(), db.cpu()
    for sl in (slice(1000, 1032), slice(5112, 5120)):
        ex, ew, eb = _ref_grads(x[:, sl], w[sl], b[sl], dout[:, sl], "silu")
        _gcheck(dx[:, sl], ex, torch.bfloat16, "dx rows")
        _gcheck(dw[sl], ew, torch.bfloat16, "dweight rows")
        _gcheck(db[sl], eb, torch.bfloat16, "dbias rows")


def test_conv_bwd_config1_shape_rows():
    """Config-1 conv shape (batch 8, 1536 channels, L 2048, bf16: one 2,048-step tile per row): a
    slice of channels against the oracle, and the same bits on a second call."""
    _say("conv bwd config-1 shape")
    from motif_mamba_amd.causal_conv1d import causal_conv1d_bwd
    g = torch.Generator().manual_seed(830)
    x = torch.randn(8, 1536, 2048, generator=g).to(torch.bfloat16)
    w = (torch.randn(1536, 4, generator=g) * 0.5).to(torch.bfloat16)
    b = (torch.randn(1536, generator=g) * 0.1).to(torch.bfloat16)
    dout = torch.randn(8, 1536, 2048, generator=g).to(torch.bfloat16)
    gx, gw, gb, gd = x.to(DEV), w.to(DEV), b.to(DEV), dout.to(DEV)
    dx, dw, db = causal_conv1d_bwd(gx, gw, gb, gd, None, True)
    dx2, dw2, db2 = causal_conv1d_bwd(gx, gw, gb, gd, None, True)
    assert torch.equal(dw, dw2) and torch.equal(db, db2) and torch.equal(dx, dx2)
    dx, dw, db = dx.cpu(), dw.cpu(), db.cpu()
    for sl in (slice(0, 16), slice(1520, 1536)):
        ex, ew, eb = _ref_grads(x[:, sl], w[sl], b[sl], dout[:, sl], "silu")
        _gcheck(dx[:, sl], ex, torch.bfloat16, "dx rows")
        _gcheck(dw[sl], ew, torch.bfloat16, "dweight rows")
        _gcheck(db[sl], eb, torch.bfloat16, "dbias rows")


def test_conv_bwd_c_abi_direct():
    _say("conv bwd C ABI direct")
    lib = capi.load()
    x, w, b = _case(830, 2, 16, 128, 4, torch.float32)
    dout = torch.randn(2, 16, 128, generator=torch.Generator().manual_seed(831))
    xg, wg, bg, dg = x.to(DEV), w.to(DEV), b.to(DEV), dout.to(DEV)
    dx = torch.empty_like(xg)
    dw = torch.full((16, 4), 5.0, device=DEV)                                # cleared by the call
    db = torch.full((16,), 5.0, device=DEV)
    p = capi.Conv1dBwdParams()
    p.batch, p.dim, p.seqlen, p.width, p.itype, p.wtype, p.silu = 2, 16, 128, 4, 0, 0, 1
    p.x, p.weight, p.bias, p.dout = xg.data_ptr(), wg.data_ptr(), bg.data_ptr(), dg.data_ptr()
    p.dx, p.dweight, p.dbias = dx.data_ptr(), dw.data_ptr(), db.data_ptr()
    p.x_batch_stride, p.x_d_stride = xg.stride(0), xg.stride(1)
    p.dout_batch_stride, p.dout_d_stride = dg.stride(0), dg.stride(1)
    p.dx_batch_stride, p.dx_d_stride = dx.stride(0), dx.stride(1)
    p.weight_d_stride, p.weight_w_stride, p.bias_stride = wg.stride(0), wg.stride(1), 1
    rc = lib.mm_causal_conv1d_bwd(ctypes.byref(p), capi.stream_handle())
    assert rc == 0, lib.mm_last_error().decode()
    torch.cuda.synchronize()
    ex, ew, eb = _ref_grads(x, w, b, dout, "silu")
    _gcheck(dx, ex, torch.float32, "dx")
    _gcheck(dw, ew, torch.float32, "dweight")
    _gcheck(db, eb, torch.float32, "dbias")
