"""GPU parity of the fused Mamba inner function (``mamba_inner_fn`` / ``MambaInnerFn``, reference
selective_scan_interface.py:454-656) against the CPU oracle ``oracle.inner_ref.mamba_inner_ref``
(pinned in tests/test_oracle_inner.py).

Forward: the oracle evaluates the block in float32 and, for 16-bit inputs, rounds its
intermediates where the reference writes them in the activation dtype. Backward: the oracle's
autograd gradients (float32 arithmetic on the same input values, no intermediate rounding).
Tolerances: the north_star pair (rtol, atol) = (1e-4, 1e-5) for fp32 and (3e-2, 5e-2) for 16-bit
inputs, element-wise as |err| <= rtol |exact| + atol max(1, max |exact|) (the projections and the
weight gradients are sums over thousands of terms whose rounding grows with their scale).
"""
import sys

import pytest
import torch

from oracle.inner_ref import mamba_inner_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
ARGS = ["xz", "conv1d_weight", "conv1d_bias", "x_proj_weight", "delta_proj_weight", "out_proj_weight",
        "out_proj_bias", "A", "B", "C", "D", "delta_bias", "B_proj_bias", "C_proj_bias"]


def _say(msg):
    print(f"\n[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _check(got, exact, dtype, what, loose=1.0):
    rtol, atol = (1e-4, 1e-5) if dtype == torch.float32 else (3e-2, 5e-2)
    got, exact = got.double().cpu(), exact.double().cpu()
    assert got.shape == exact.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(exact.shape)}"
    scale = max(1.0, exact.abs().max().item()) if exact.numel() else 1.0
    err = (got - exact).abs()
    bad = err > loose * (rtol * exact.abs() + atol * scale)
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())}/{err.numel()} beyond tolerance; max err "
                                 f"{err.max().item():.3g} (scale {scale:.3g})")


def _case(seed, batch=2, d_inner=64, L=96, d_state=16, rank=4, d_model=32, W=4, dtype=torch.float32,
          wdtype=None, biases=True, bc_bias=False):
    """Weights scaled like a trained Mamba layer (dt_proj init ~ rank^-0.5, A = -exp(A_log))."""
    g = torch.Generator().manual_seed(seed)
    wd = wdtype or dtype
    r = lambda *s, sc=1.0, dt=wd: (torch.randn(*s, generator=g) * sc).to(dt)     # noqa: E731
    c = dict(
        xz=r(batch, 2 * d_inner, L, dt=dtype),
        conv1d_weight=r(d_inner, 1, W, sc=0.5),
        conv1d_bias=r(d_inner, sc=0.1) if biases else None,
        x_proj_weight=r(rank + 2 * d_state, d_inner, sc=d_inner ** -0.5),
        delta_proj_weight=r(d_inner, rank, sc=rank ** -0.5),
        out_proj_weight=r(d_model, d_inner, sc=d_inner ** -0.5),
        out_proj_bias=r(d_model, sc=0.1) if biases else None,
        A=-torch.exp(torch.rand(d_inner, d_state, generator=g) * 2.0),
        B=None, C=None,
        D=torch.randn(d_inner, generator=g),
        delta_bias=torch.rand(d_inner, generator=g) * 2.0 - 4.0,
        B_proj_bias=r(d_state, sc=0.1) if bc_bias else None,
        C_proj_bias=r(d_state, sc=0.1) if bc_bias else None,
    )
    return c


def _dev(c, grad):
    out = {}
    for k, v in c.items():
        if torch.is_tensor(v):
            v = v.to(DEV)
            if grad and v.is_floating_point():
                v.requires_grad_(True)
        out[k] = v
    return out


def _run(c, dout=None, **kw):
    from mamba_ssm.ops.selective_scan_interface import mamba_inner_fn
    g = _dev(c, dout is not None)
    y = mamba_inner_fn(*[g[k] for k in ARGS], **kw)
    grads = None
    if dout is not None:
        y.backward(dout.to(DEV))
        grads = {k: g[k].grad for k in ARGS if torch.is_tensor(g[k])}
    torch.cuda.synchronize()
    return y.detach().cpu(), grads


def _oracle(c, dout=None, **kw):
    rnd = "input" if dout is None else None
    cc = {k: (v.clone().float().requires_grad_(True) if torch.is_tensor(v) and dout is not None else v)
          for k, v in c.items()}
    y = mamba_inner_ref(*[cc[k] for k in ARGS], round_to=rnd, **kw)
    if dout is None:
        return y, None
    y.backward(dout.float())
    return y.detach(), {k: cc[k].grad for k in ARGS if torch.is_tensor(cc[k])}


def _dout(seed, c):
    b, _, L = c["xz"].shape
    e = c["out_proj_weight"].shape[0]
    return torch.randn(b, L, e, generator=torch.Generator().manual_seed(seed)).to(c["xz"].dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("L", [96, 100])
def test_forward(dtype, L):
    _say(f"mamba_inner fwd {dtype} L={L}")
    c = _case(900 + L, L=L, dtype=dtype)
    got, _ = _run(c)
    want, _ = _oracle(c)
    assert got.dtype == dtype and got.shape == (2, L, 32)
    _check(got, want, dtype, "out")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ckpt", [0, 1])
@pytest.mark.parametrize("bc_bias", [False, True])
def test_backward(dtype, ckpt, bc_bias):
    _say(f"mamba_inner bwd {dtype} checkpoint_lvl={ckpt} bc_bias={bc_bias}")
    c = _case(910 + ckpt + 2 * bc_bias, L=128, dtype=dtype, bc_bias=bc_bias)
    dout = _dout(911, c)
    got, gg = _run(c, dout, checkpoint_lvl=ckpt)
    want, eg = _oracle(c, dout)
    _check(got, want, dtype, "out")
    for k, v in eg.items():
        assert gg[k] is not None, k
        assert gg[k].dtype == c[k].dtype, f"{k}: grad dtype {gg[k].dtype}"
        _check(gg[k], v, dtype, f"d{k}")


@pytest.mark.parametrize("pad", ["1", "0"], ids=["padded", "general"])
@pytest.mark.parametrize("ckpt", [0, 1])
def test_backward_without_biases_ragged_length(pad, ckpt, monkeypatch):
    """L = 37: the scan runs on copies padded in front with zero-u steps (forward and backward), or,
    with MM_SCAN_PAD=0, on the general kernels."""
    monkeypatch.setenv("MM_SCAN_PAD", pad)
    _say(f"mamba_inner bwd no biases L=37 padding {pad} checkpoint_lvl={ckpt}")
    c = _case(920, L=37, biases=False)
    dout = _dout(921, c)
    got, gg = _run(c, dout, checkpoint_lvl=ckpt)
    want, eg = _oracle(c, dout)
    _check(got, want, torch.float32, "out")
    for k, v in eg.items():
        _check(gg[k], v, torch.float32, f"d{k}")


def test_checkpoint_levels_agree_and_inference_path():
    _say("mamba_inner checkpoint 0 vs 1, inference")
    c = _case(930, L=256, dtype=torch.bfloat16)
    dout = _dout(931, c)
    y1, g1 = _run(c, dout, checkpoint_lvl=1)
    y0, g0 = _run(c, dout, checkpoint_lvl=0)
    yi, _ = _run(c)                                   # no gradients: the scan's inference outputs
    torch.testing.assert_close(y0, y1, rtol=0, atol=0)
    torch.testing.assert_close(yi, y1, rtol=1e-2, atol=1e-2)
    for k in g1:
        torch.testing.assert_close(g0[k], g1[k], rtol=1e-2, atol=1e-2, msg=lambda m: f"d{k}: {m}")


def test_no_grad_with_weights_requiring_grad_takes_inference_path():
    """A module evaluated under torch.no_grad() passes weights that require grad: mamba_inner_fn
    takes the inference path then too (the caller's grad mode is passed in), so its output has the
    same bits as with weights that do not require grad, and carries no graph."""
    _say("mamba_inner no_grad with weights requiring grad")
    from mamba_ssm.ops.selective_scan_interface import mamba_inner_fn
    c = _case(940, L=256, dtype=torch.bfloat16)
    yi, _ = _run(c)
    g = _dev(c, True)
    with torch.no_grad():
        y = mamba_inner_fn(*[g[k] for k in ARGS])
    torch.cuda.synchronize()
    assert not y.requires_grad
    assert torch.equal(y.cpu(), yi)


def test_given_B_C():
    """B and C passed in (not projected): variable (batch, 1, N, L) and constant (d, N) forms; the
    x_proj rows that would have produced them get a zero gradient."""
    _say("mamba_inner given B/C")
    c = _case(940, L=64)
    g = torch.Generator().manual_seed(941)
    c["B"] = torch.randn(2, 1, 16, 64, generator=g)
    c["C"] = torch.randn(64, 16, generator=g)
    dout = _dout(942, c)
    got, gg = _run(c, dout)
    want, eg = _oracle(c, dout)
    _check(got, want, torch.float32, "out")
    for k, v in eg.items():
        if v is not None:
            _check(gg[k], v, torch.float32, f"d{k}")


def _rms_weights(seed, d_state=16, d_inner=64):
    g = torch.Generator().manual_seed(seed)
    return dict(b_rms_weight=torch.rand(d_state, generator=g) + 0.5, c_rms_weight=torch.rand(d_state, generator=g) + 0.5,
                dt_rms_weight=torch.rand(d_inner, generator=g) + 0.5)


def test_rms_norm_forward():
    _say("mamba_inner rms weights forward")
    c = _case(950, L=64, dtype=torch.bfloat16)
    rw = _rms_weights(951)
    got, _ = _run(c, **{k: v.to(DEV) for k, v in rw.items()})
    want, _ = _oracle(c, **rw)
    _check(got, want, torch.bfloat16, "out")
    for only in ("b_rms_weight", "dt_rms_weight"):
        got1, _ = _run(c, **{only: rw[only].to(DEV)})
        want1, _ = _oracle(c, **{only: rw[only]})
        _check(got1, want1, torch.bfloat16, f"out {only}")
    # A given (batch, 1, dstate, seqlen) B and C are normalised too (ssi.py:515-524).
    g = torch.Generator().manual_seed(953)
    cg = dict(c, B=torch.randn(2, 1, 16, 64, generator=g).to(torch.bfloat16),
              C=torch.randn(2, 1, 16, 64, generator=g).to(torch.bfloat16))
    kw = {k: rw[k] for k in ("b_rms_weight", "c_rms_weight")}
    got2, _ = _run(cg, **{k: v.to(DEV) for k, v in kw.items()})
    want2, _ = _oracle(cg, **kw)
    _check(got2, want2, torch.bfloat16, "out given B/C")
    cc = dict(c, C=torch.randn(64, 16, generator=g))                  # a constant C cannot be normalised
    with pytest.raises(ValueError, match="RMS"):
        _run(cc, c_rms_weight=rw["c_rms_weight"].to(DEV))


@pytest.mark.parametrize("lvl", [0, 1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rms_norm_backward(lvl, dtype):
    """The reference's backward with RMSNorm weights (ssi.py:571-645): the norms passed unchanged and,
    at checkpoint_lvl 1, B and C normalised a second time -- against its step-by-step restatement
    (oracle.inner_ref.mamba_inner_bwd_ref, pinned in tests/test_oracle_inner.py)."""
    from oracle.inner_ref import mamba_inner_bwd_ref
    _say(f"mamba_inner rms weights backward lvl {lvl} {dtype}")
    c = _case(960 + lvl, L=64, dtype=dtype, bc_bias=True)
    rw = _rms_weights(962)
    dout = _dout(963, c)
    _, gg = _run(c, dout, checkpoint_lvl=lvl, **{k: v.to(DEV) for k, v in rw.items()})
    eg = mamba_inner_bwd_ref(*[c[k] for k in ARGS[:8]], dout, B=c["B"], C=c["C"], D=c["D"],
                             delta_bias=c["delta_bias"], B_proj_bias=c["B_proj_bias"], C_proj_bias=c["C_proj_bias"],
                             checkpoint_lvl=lvl, **rw)
    for k in ARGS:
        if eg[k] is None:
            assert gg.get(k) is None, k
            continue
        assert gg[k].dtype == c[k].dtype, f"{k}: grad dtype {gg[k].dtype}"
        _check(gg[k], eg[k], dtype, f"d{k}")


def test_rms_norm_kernel_layouts():
    """rms_norm_fwd over dim 1 in the scan layout and on a plain row-major matrix, fp32 and bf16."""
    _say("rms_norm kernel")
    from motif_mamba_amd._native import ext
    from oracle.inner_ref import rms_norm_ref
    g = torch.Generator().manual_seed(960)
    for dtype in (torch.float32, torch.bfloat16):
        x = torch.randn(3, 5120, 77, generator=g).to(dtype)
        w = torch.rand(5120, generator=g) + 0.5
        got = ext().rms_norm_fwd(x.to(DEV), w.to(DEV), 1e-6, None).cpu()
        _check(got, rms_norm_ref(x, w, 1e-6, dim=1), dtype, f"scan layout {dtype}")
        m = torch.randn(1000, 16, generator=g).to(dtype)          # (rows, cols) as (rows, cols, 1)
        got = ext().rms_norm_fwd(m.to(DEV).unsqueeze(-1), w[:16].to(DEV), 1e-5, None).cpu()[..., 0]
        _check(got, rms_norm_ref(m, w[:16], 1e-5, dim=1), dtype, f"rows {dtype}")
    x = torch.randn(2, 16, 64, generator=g).to(DEV)
    y = ext().rms_norm_fwd(x, torch.ones(16, device=DEV), 0.0, x)           # in place
    torch.cuda.synchronize()
    assert y.data_ptr() == x.data_ptr()
    torch.testing.assert_close(x.pow(2).mean(dim=1), torch.ones(2, 64, device=DEV), rtol=1e-5, atol=1e-5)


def test_autocast_fp32_weights():
    """The module's case: float32 parameters, bf16 activations under torch.autocast (ssi.py:469-474)."""
    _say("mamba_inner autocast")
    c = _case(970, L=64, dtype=torch.bfloat16, wdtype=torch.float32)
    from mamba_ssm.ops.selective_scan_interface import mamba_inner_fn
    g = _dev(c, True)
    dout = _dout(971, c)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = mamba_inner_fn(*[g[k] for k in ARGS])
    y.backward(dout.to(DEV))
    torch.cuda.synchronize()
    cw = dict(c)
    for k in ("x_proj_weight", "delta_proj_weight", "out_proj_weight", "out_proj_bias"):
        cw[k] = c[k].to(torch.bfloat16)
    want, _ = _oracle(cw)
    _check(y.detach().cpu(), want, torch.bfloat16, "out")
    assert g["x_proj_weight"].grad.dtype == torch.float32
    _, eg = _oracle(cw, dout)
    for k in ("xz", "x_proj_weight", "out_proj_weight", "conv1d_weight", "A", "D"):
        _check(g[k].grad, eg[k], torch.bfloat16, f"d{k}")


def test_mamba_2p8b_layer_shape():
    """The Mamba-2.8B layer (d_model 2560, d_inner 5120, dt_rank 160, d_state 16) at a short length,
    bf16, forward and backward."""
    _say("mamba_inner 2.8B layer shape")
    c = _case(980, batch=1, d_inner=5120, L=256, rank=160, d_model=2560, dtype=torch.bfloat16)
    dout = _dout(981, c)
    got, gg = _run(c, dout)
    want, _ = _oracle(c)
    _check(got, want, torch.bfloat16, "out")
    _, eg = _oracle(c, dout)
    for k, v in eg.items():
        _check(gg[k], v, torch.bfloat16, f"d{k}")
