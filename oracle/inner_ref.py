"""CPU restatement of the fused Mamba inner function -- TEST INFRASTRUCTURE ONLY.

Follows ``MambaInnerFn.forward`` (reference mamba_ssm/ops/selective_scan_interface.py:458-553) and
``mamba_inner_ref`` (:659-694), the block between the input projection and the output of a Mamba
layer, for real A:

    x, z        = xz split in half along channels                                  (ssi.py:482)
    conv1d_out  = silu(causal_conv1d(x, conv1d_weight, conv1d_bias))             (ssi.py:484-486)
    x_dbl       = conv1d_out as (b l, d) @ x_proj_weight^T                          (ssi.py:490)
    delta       = delta_proj_weight @ x_dbl[:, :delta_rank]^T, as (b, d, l)         (ssi.py:491)
    B, C        = x_dbl[:, delta_rank:delta_rank + d_state], x_dbl[:, -d_state:]
                  (+ B_proj_bias / C_proj_bias), as (b, 1, d_state, l)             (ssi.py:496-514)
    optional RMSNorm over d_state of B and C, over d of delta                      (ssi.py:515-529)
    out_z       = selective_scan(conv1d_out, delta, A, B, C, D, z, delta_bias, softplus)
    result      = out_z as (b, l, d) @ out_proj_weight^T + out_proj_bias           (ssi.py:553)

B or C given explicitly (not None) are used as they are (the "constant" forms).

The arithmetic is float32 (float64 with ``compute_dtype``); ``round_to`` (default: xz's dtype)
rounds the intermediates where the reference's kernels and torch ops write them in the activation
dtype (conv1d_out, x_dbl, delta, the normalised B/C/delta, out_z, the result), so a bf16 run of
the reference and this restatement see the same roundings. Gradients: the function is built from
differentiable torch ops, so ``torch.autograd`` gives the exact gradients of this forward (with
``round_to=None`` no rounding enters the graph).

RMSNorm (rms_norm_forward, ssi.py:217-234, computed by the un-vendored Triton ``_layer_norm_fwd``
of mamba_ssm): y = x * weight / sqrt(mean(x^2) + eps), float32, written in x's dtype.
"""
from __future__ import annotations

import math

import torch

from .conv_ref import causal_conv1d_ref
from .ssm_ref import selective_scan_bwd_ref, selective_scan_ref


def rms_norm_ref(x, weight, eps=1e-6, dim=-1, compute_dtype=torch.float32):
    """RMSNorm of x over ``dim``; result in x's dtype."""
    xf = x.to(compute_dtype)
    shape = [1] * x.dim()
    shape[dim] = -1
    rstd = torch.rsqrt(xf.pow(2).mean(dim=dim, keepdim=True) + eps)
    return (xf * rstd * weight.to(compute_dtype).reshape(shape)).to(x.dtype)


def mamba_inner_ref(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                    out_proj_bias, A, B=None, C=None, D=None, delta_bias=None, B_proj_bias=None, C_proj_bias=None,
                    delta_softplus=True, b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None,
                    b_c_dt_rms_eps=1e-6, round_to="input", compute_dtype=torch.float32):
    """xz: (batch, 2 d_inner, seqlen); conv1d_weight: (d_inner, 1, width); x_proj_weight:
    (delta_rank + 2 d_state, d_inner); delta_proj_weight: (d_inner, delta_rank); out_proj_weight:
    (d_model, d_inner); A: (d_inner, d_state) real. Returns (batch, seqlen, d_model)."""
    if A.is_complex():
        raise NotImplementedError("complex A is not restated")
    rt = xz.dtype if round_to == "input" else round_to

    def rnd(t):
        return t if rt is None or rt == compute_dtype else t.to(rt).to(compute_dtype)

    cd = compute_dtype
    batch, two_d, L = xz.shape
    d_inner = two_d // 2
    delta_rank = delta_proj_weight.shape[1]
    d_state = A.shape[-1]
    x, z = xz.to(cd).chunk(2, dim=1)
    w = conv1d_weight.reshape(d_inner, -1).to(cd)
    cb = None if conv1d_bias is None else conv1d_bias.to(cd)
    conv1d_out = rnd(causal_conv1d_ref(x, w, cb, activation="silu", compute_dtype=cd))
    x_dbl = rnd(conv1d_out.transpose(1, 2).reshape(batch * L, d_inner) @ x_proj_weight.to(cd).t())
    delta = rnd(delta_proj_weight.to(cd) @ x_dbl[:, :delta_rank].t())              # (d, b l)
    delta = delta.reshape(d_inner, batch, L).permute(1, 0, 2)

    def proj(cols, bias):
        v = x_dbl[:, cols]
        if bias is not None:
            v = rnd(v + rnd(bias.to(cd)))       # the reference adds bias.to(B.dtype) (ssi.py:498, :508)
        return v.reshape(batch, L, d_state).permute(0, 2, 1).unsqueeze(1)           # (b, 1, n, l)

    Bv = proj(slice(delta_rank, delta_rank + d_state), B_proj_bias) if B is None else B.to(cd)
    Cv = proj(slice(x_dbl.shape[1] - d_state, None), C_proj_bias) if C is None else C.to(cd)
    if b_rms_weight is not None:
        Bv = rnd(rms_norm_ref(Bv, b_rms_weight, b_c_dt_rms_eps, dim=2, compute_dtype=cd))
    if c_rms_weight is not None:
        Cv = rnd(rms_norm_ref(Cv, c_rms_weight, b_c_dt_rms_eps, dim=2, compute_dtype=cd))
    if dt_rms_weight is not None:
        delta = rnd(rms_norm_ref(delta, dt_rms_weight, b_c_dt_rms_eps, dim=1, compute_dtype=cd))
    if B is None:
        Bv = Bv[:, 0]                                                                 # (b, n, l)
    if C is None:
        Cv = Cv[:, 0]
    out_z = rnd(selective_scan_ref(conv1d_out, delta, A.to(cd), Bv, Cv, None if D is None else D.to(cd), z=z,
                                   delta_bias=None if delta_bias is None else delta_bias.to(cd),
                                   delta_softplus=delta_softplus, compute_dtype=cd))
    y = out_z.transpose(1, 2) @ out_proj_weight.to(cd).t()
    if out_proj_bias is not None:
        y = y + out_proj_bias.to(cd)
    return y if rt is None else y.to(rt)


def mamba_inner_brute(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                      out_proj_bias, A, D, delta_bias, B_proj_bias=None, C_proj_bias=None, b_rms_weight=None,
                      c_rms_weight=None, dt_rms_weight=None, eps=1e-6):
    """Float64 nested-loop evaluation of the same function (variable B and C, softplus) on tiny
    shapes, with the scan as the closed sum of oracle/brute.py; every index written out."""
    from .brute import scan_brute
    from .conv_ref import causal_conv1d_brute
    t = lambda v: v.double().tolist() if v is not None else None     # noqa: E731
    XZ, XW, DW, OW = t(xz), t(x_proj_weight), t(delta_proj_weight), t(out_proj_weight)
    batch, two_d, L = len(XZ), len(XZ[0]), len(XZ[0][0])
    d = two_d // 2
    R, N = len(DW[0]), len(t(A)[0])
    x = [[XZ[b][c] for c in range(d)] for b in range(batch)]
    z = [[XZ[b][d + c] for c in range(d)] for b in range(batch)]
    cw = [row[0] for row in t(conv1d_weight)]
    u = causal_conv1d_brute(x, cw, t(conv1d_bias), None, "silu")
    n_out = len(XW)
    dbl = [[[sum(XW[j][c] * u[b][c][l] for c in range(d)) for j in range(n_out)] for l in range(L)]
           for b in range(batch)]
    bpb, cpb = t(B_proj_bias), t(C_proj_bias)
    delta = [[[sum(DW[c][r] * dbl[b][l][r] for r in range(R)) for l in range(L)] for c in range(d)]
             for b in range(batch)]
    Bm = [[[dbl[b][l][R + n] + (bpb[n] if bpb else 0.0) for l in range(L)] for n in range(N)] for b in range(batch)]
    Cm = [[[dbl[b][l][n_out - N + n] + (cpb[n] if cpb else 0.0) for l in range(L)] for n in range(N)]
          for b in range(batch)]

    def rms_cols(M, wgt, n_rows, n_cols, get, put):      # normalise over the column index
        for b in range(batch):
            for l in range(L):
                ms = sum(get(M, b, i, l) ** 2 for i in range(n_cols)) / n_cols
                r = 1.0 / math.sqrt(ms + eps)
                for i in range(n_cols):
                    put(M, b, i, l, get(M, b, i, l) * r * wgt[i])

    get = lambda M, b, i, l: M[b][i][l]                  # noqa: E731

    def put(M, b, i, l, v):
        M[b][i][l] = v
    if b_rms_weight is not None:
        rms_cols(Bm, t(b_rms_weight), L, N, get, put)
    if c_rms_weight is not None:
        rms_cols(Cm, t(c_rms_weight), L, N, get, put)
    if dt_rms_weight is not None:
        rms_cols(delta, t(dt_rms_weight), L, d, get, put)
    _, out_z, _ = scan_brute(u, delta, t(A), Bm, Cm, t(D), z, t(delta_bias), True, "3d", "3d")
    opb = t(out_proj_bias)
    return [[[sum(OW[e][c] * out_z[b][c][l] for c in range(d)) + (opb[e] if opb else 0.0)
              for e in range(len(OW))] for l in range(L)] for b in range(batch)]


def mamba_inner_bwd_ref(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                        out_proj_bias, A, dout, B=None, C=None, D=None, delta_bias=None, B_proj_bias=None,
                        C_proj_bias=None, delta_softplus=True, checkpoint_lvl=1, b_rms_weight=None,
                        c_rms_weight=None, dt_rms_weight=None, b_c_dt_rms_eps=1e-6, compute_dtype=torch.float32):
    """The gradients ``MambaInnerFn.backward`` returns (ssi.py:555-645), step by step, in
    ``compute_dtype`` without intermediate rounding. Returns a dict keyed by the input names (xz,
    conv1d_weight, ..., C_proj_bias; None where the reference returns None).

    The steps: the forward's quantities (ssi.py:482-553); dout_y = out_proj_weight^T dout; the scan
    backward (selective_scan_bwd_ref) at the point the reference evaluates it -- the forward's
    delta, B and C, except that at checkpoint_lvl 1 the saved B and C, already RMS-normalised, are
    normalised again (ssi.py:582-593); dz from the forward's pre-gate output (the kernel reads the
    saved ``out``); dB, dC into the x_dbl rows and ddelta into the delta projection unchanged, i.e.
    without a backward through the RMSNorms, whose weights get no gradient (ssi.py:598-645); then the
    x_proj products and the conv1d backward. Without RMSNorm weights this is the gradient of
    ``mamba_inner_ref`` at either checkpoint level (tests/test_oracle_inner.py checks that against
    autograd)."""
    cd = compute_dtype
    f = lambda t: None if t is None else t.detach().to(cd)          # noqa: E731
    xz, A, D, delta_bias, dout = f(xz), f(A), f(D), f(delta_bias), f(dout)
    Wc, bc, Wx, Wd, Wo = f(conv1d_weight), f(conv1d_bias), f(x_proj_weight), f(delta_proj_weight), f(out_proj_weight)
    batch, two_d, L = xz.shape
    d_inner = two_d // 2
    R, N = Wd.shape[1], A.shape[-1]
    eps = b_c_dt_rms_eps
    x, z = xz.chunk(2, dim=1)
    x = x.clone().requires_grad_(True)
    Wc = Wc.clone().requires_grad_(True)
    if bc is not None:
        bc = bc.clone().requires_grad_(True)
    conv_out = causal_conv1d_ref(x, Wc.reshape(d_inner, -1), bc, activation="silu", compute_dtype=cd)
    u = conv_out.detach()
    x_dbl = u.transpose(1, 2).reshape(batch * L, d_inner) @ Wx.t()                   # (b l, R + 2N)
    delta = (Wd @ x_dbl[:, :R].t()).reshape(d_inner, batch, L).permute(1, 0, 2)      # (b, d, l)

    def bc_in(given, cols, bias):
        if given is not None:
            return f(given)
        v = x_dbl[:, cols]
        if bias is not None:
            v = v + f(bias)
        return v.reshape(batch, L, N).permute(0, 2, 1).unsqueeze(1)                   # (b, 1, N, l)

    norm = lambda t, w, dim: rms_norm_ref(t, w, eps, dim=dim, compute_dtype=cd)     # noqa: E731
    Bs = bc_in(B, slice(R, R + N), B_proj_bias)
    Cs = bc_in(C, slice(x_dbl.shape[1] - N, None), C_proj_bias)
    if b_rms_weight is not None:
        Bs = norm(Bs, b_rms_weight, 2)
    if c_rms_weight is not None:
        Cs = norm(Cs, c_rms_weight, 2)
    if dt_rms_weight is not None:
        delta = norm(delta, dt_rms_weight, 1)
    sq = lambda t: t[:, 0] if t.dim() == 4 else t                                    # noqa: E731
    out = selective_scan_ref(u, delta, A, sq(Bs), sq(Cs), D, None, delta_bias, delta_softplus, compute_dtype=cd)
    out_z = out * torch.nn.functional.silu(z)
    # The point of the scan backward.
    Bb, Cb = Bs, Cs
    if checkpoint_lvl == 1:
        if b_rms_weight is not None:
            Bb = norm(Bb, b_rms_weight, 2)
        if c_rms_weight is not None:
            Cb = norm(Cb, c_rms_weight, 2)
    dout2 = dout.reshape(batch * L, -1)                                               # (b l, e)
    dout_y = (dout2 @ Wo).reshape(batch, L, d_inner).permute(0, 2, 1)                  # (b, d, l)
    sg = torch.sigmoid(z)
    g = dout_y * sg * z                                                               # the pre-gate cotangent
    sb = selective_scan_bwd_ref(u, delta, A, sq(Bb), sq(Cb), g, D, None, delta_bias, delta_softplus, dtype=cd)
    dz = dout_y * out * sg * (1 + z * (1 - sg))
    res = {"out_proj_weight": dout2.t() @ out_z.permute(0, 2, 1).reshape(batch * L, d_inner),
           "out_proj_bias": dout2.sum(dim=0) if out_proj_bias is not None else None,
           "A": sb["dA"], "D": sb["dD"] if D is not None else None,
           "delta_bias": sb["ddelta_bias"] if delta_bias is not None else None,
           "B": None, "C": None, "B_proj_bias": None, "C_proj_bias": None}
    dx_dbl = torch.zeros_like(x_dbl)
    for name, given, cols, grad, bias in (("B", B, slice(R, R + N), sb["dB"], B_proj_bias),
                                           ("C", C, slice(x_dbl.shape[1] - N, None), sb["dC"], C_proj_bias)):
        if given is None:
            gr = grad.permute(0, 2, 1).reshape(batch * L, N)                          # (b, N, l) -> (b l, N)
            dx_dbl[:, cols] = gr
            res[name + "_proj_bias"] = gr.sum(dim=0) if bias is not None else None
        else:
            res[name] = grad.reshape(given.shape)
    dd = sb["ddelta"].permute(1, 0, 2).reshape(d_inner, batch * L)                    # (d, b l)
    res["delta_proj_weight"] = dd @ x_dbl[:, :R]
    dx_dbl[:, :R] = dd.t() @ Wd
    res["x_proj_weight"] = dx_dbl.t() @ u.transpose(1, 2).reshape(batch * L, d_inner)
    dconv = sb["du"] + (Wx.t() @ dx_dbl.t()).reshape(d_inner, batch, L).permute(1, 0, 2)
    conv_out.backward(dconv)
    res["xz"] = torch.cat([x.grad, dz], dim=1)
    res["conv1d_weight"] = Wc.grad
    res["conv1d_bias"] = bc.grad if bc is not None else None
    return res
