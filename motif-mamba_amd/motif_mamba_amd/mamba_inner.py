"""Drop-in ``mamba_inner_fn`` / ``MambaInnerFn``: the fused Mamba block between the input
projection and the output (reference mamba_ssm/ops/selective_scan_interface.py:454-656), forward
and backward, on the gfx950 kernels of this package plus library GEMMs.

Signature, argument meanings, defaults and return value are the reference's:
``mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None, B_proj_bias=None,
C_proj_bias=None, delta_softplus=True, checkpoint_lvl=1, b_rms_weight=None, c_rms_weight=None,
dt_rms_weight=None, b_c_dt_rms_eps=1e-6)`` -> (batch, seqlen, d_model). The function computed is

    x, z = xz halves; u = silu(causal_conv1d(x)); x_dbl = x_proj(u); delta = delta_proj(x_dbl[:R]);
    B, C = x_dbl[R:R+N] (+ B_proj_bias), x_dbl[-N:] (+ C_proj_bias)   [or the given B / C];
    optional RMSNorm of B, C (over N) and delta (over d);
    out = out_proj(selective_scan(u, delta, A, B, C, D, z, delta_bias, delta_softplus)).

Kernels: the causal conv1d forward/backward (mm_conv1d.hip), the selective scan forward/backward
(mm_scan_*.hip), the RMSNorm (mm_norm.hip); the five projections are plain GEMMs (hipBLASLt via
torch.mm), the MFMA-bound part of the block.

Layout (the MI355X design choice; the values are the reference's): every activation of the block
is kept channel-major, as a (channels, batch * seqlen) matrix, and exposed to the kernels as a
(batch, channels, seqlen) view with strides (seqlen, batch * seqlen, 1). The conv writes its output
straight into that layout, x_dbl is produced as (R + 2N, batch * seqlen), and delta, B and C are
views or GEMM outputs in it, so every projection is a single 2-D GEMM and no activation is ever
transposed in memory (the reference transposes conv1d_out, B, C and out_z through (b l, d) copies).

Checkpointing as the reference: ``checkpoint_lvl=1`` keeps neither conv1d_out nor delta and
recomputes both in the backward; ``0`` keeps them, and with dstate 16 also the scan's 16-step tile
states, so that the scan backward need not recompute them (``MM_TILE_STATES=0`` turns that off). Autocast: the projection weights are cast to
the autocast dtype as the reference does (ssi.py:469-474).

RMSNorm weights (b_rms_weight, c_rms_weight, dt_rms_weight) as the reference: the forward
normalises B and C over dstate (projected or given; a given B/C must then be (batch, 1, dstate,
seqlen)) and delta over channels (ssi.py:515-529). The backward is the reference's, which is not the
gradient of its forward (ssi.py:571-645): dB, dC and ddelta pass the norms unchanged (no norm
backward; the norm weights get no gradient), and at checkpoint_lvl=1 the saved B and C, already
normalised, are normalised a second time before the scan backward (ssi.py:582-593) while delta is
recomputed and normalised once. No reference caller passes these weights
(mamba_simplemotif.py:272-285).

Not provided (raises, as in the other parts of this build): complex A.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from ._native import ext
from .selective_scan import _pad_front, _save_tile_states, _train_pad, _unpad


def _cm_empty(batch, ch, L, like, dtype=None):
    """A (batch, ch, L) tensor stored channel-major, i.e. as a contiguous (ch, batch * L) matrix."""
    return torch.empty(ch, batch, L, device=like.device, dtype=dtype or like.dtype).transpose(0, 1)


def _cm_flat(t):
    """(batch, ch, L) -> (ch, batch * L): a view for channel-major tensors, a copy otherwise."""
    b, c, l = t.shape
    return t.transpose(0, 1).reshape(c, b * l)


def _cm_view(m, batch):
    """(ch, batch * L) matrix -> (batch, ch, L) view."""
    c, bl = m.shape
    return m.view(c, batch, bl // batch).transpose(0, 1)


def _conv(x, weight, bias):
    out = _cm_empty(x.shape[0], x.shape[1], x.shape[2], x)
    return ext().conv1d_fwd(x, weight, bias, None, None, True, out)


def _rms(t, weight, eps):
    """RMSNorm over dim 1 of a (n0, cols, n2) tensor (rms_norm_forward, ssi.py:217-234)."""
    return ext().rms_norm_fwd(t, weight.contiguous(), eps)


def _delta(delta_proj_weight, x_dbl, delta_rank, batch, dt_rms_weight, eps):
    delta = _cm_view(delta_proj_weight @ x_dbl[:delta_rank], batch)
    if dt_rms_weight is not None:
        delta = _rms(delta, dt_rms_weight, eps)
    return delta


def _rms_bc(t, weight, eps, name):
    """RMSNorm over dstate of a (batch, 1, dstate, seqlen) B or C (ssi.py:515-524 reshapes it to
    ((b l), dstate), which needs that form)."""
    if t.dim() != 4 or t.shape[1] != 1:
        raise ValueError(f"{name} must have shape (batch, 1, dstate, seqlen) to be RMS-normalised")
    return _rms(t[:, 0], weight, eps).unsqueeze(1)


def _state_input(x_dbl, rows, bias, batch, rms_weight, eps):
    """B or C of the scan from rows of x_dbl: (batch, 1, N, L), channel-major unless a bias or RMSNorm
    makes a new tensor."""
    v = _cm_view(x_dbl[rows], batch)                          # (batch, N, L)
    if bias is not None:
        v = v + bias.to(dtype=v.dtype)[None, :, None]
    if rms_weight is not None:
        v = _rms(v, rms_weight, eps)
    return v.unsqueeze(1)


class MambaInnerFn(torch.autograd.Function):

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                out_proj_bias, A, B=None, C=None, D=None, delta_bias=None, B_proj_bias=None, C_proj_bias=None,
                delta_softplus=True, checkpoint_lvl=1, b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None,
                b_c_dt_rms_eps=1e-6, grad_enabled=True):
        """xz: (batch, 2 d_inner, seqlen) -> (batch, seqlen, d_model). grad_enabled: the caller's grad
        mode (mamba_inner_fn passes it): under torch.no_grad() the inference path runs even when the
        weights require grad."""
        assert checkpoint_lvl in (0, 1), "checkpoint_lvl must be 0 or 1"
        if A.is_complex():
            raise NotImplementedError("complex A is not supported by the MI355X build")
        batch, L = xz.shape[0], xz.shape[-1]
        delta_rank = delta_proj_weight.shape[1]
        d_state = A.shape[-1]
        if torch.is_autocast_enabled("cuda"):
            dt = torch.get_autocast_dtype("cuda")
            x_proj_weight = x_proj_weight.to(dtype=dt)
            delta_proj_weight = delta_proj_weight.to(dtype=dt)
            out_proj_weight = out_proj_weight.to(dtype=dt)
            out_proj_bias = out_proj_bias.to(dtype=dt) if out_proj_bias is not None else None
        if xz.stride(-1) != 1:
            xz = xz.contiguous()
        ctx.conv1d_weight_shape = conv1d_weight.shape
        conv1d_weight = conv1d_weight.reshape(conv1d_weight.shape[0], conv1d_weight.shape[-1])   # d 1 w -> d w
        conv1d_bias = conv1d_bias.contiguous() if conv1d_bias is not None else None
        x, z = xz.chunk(2, dim=1)
        conv1d_out = _conv(x, conv1d_weight, conv1d_bias)
        x_dbl = x_proj_weight @ _cm_flat(conv1d_out)                     # (R + 2N, batch * L)
        delta = _delta(delta_proj_weight, x_dbl, delta_rank, batch, dt_rms_weight, b_c_dt_rms_eps)
        ctx.is_variable_B = B is None
        ctx.is_variable_C = C is None
        ctx.B_proj_bias_is_None = B_proj_bias is None
        ctx.C_proj_bias_is_None = C_proj_bias is None
        if B is None:
            B = _state_input(x_dbl, slice(delta_rank, delta_rank + d_state), B_proj_bias, batch, b_rms_weight,
                             b_c_dt_rms_eps)
        else:
            if B.stride(-1) != 1:
                B = B.contiguous()
            if b_rms_weight is not None:
                B = _rms_bc(B, b_rms_weight, b_c_dt_rms_eps, "B")
        if C is None:
            C = _state_input(x_dbl, slice(x_dbl.shape[0] - d_state, None), C_proj_bias, batch, c_rms_weight,
                             b_c_dt_rms_eps)
        else:
            if C.stride(-1) != 1:
                C = C.contiguous()
            if c_rms_weight is not None:
                C = _rms_bc(C, c_rms_weight, b_c_dt_rms_eps, "C")
        if D is not None:
            D = D.contiguous()
        if not grad_enabled or not any(ctx.needs_input_grad):
            # Inference: the scan writes only the gated output; nothing is kept for a backward.
            out_z = ext().fwd_infer(conv1d_out, delta, A, B, C, D=D, z=z, delta_bias=delta_bias,
                                    delta_softplus=delta_softplus, return_last_state=False)[0]
            y = F.linear(_cm_flat(out_z).t(), out_proj_weight, out_proj_bias)
            return y.view(batch, L, -1)
        # checkpoint_lvl 0 keeps activations rather than recomputing them: the scan's 16-step tile
        # states too (None where the kernels do not write them), which spare the backward a recompute.
        want_ck = checkpoint_lvl == 0 and A.shape[-1] <= 16 and _save_tile_states()
        # A length that is not a multiple of 8: the scan runs on copies padded in front with zero-u
        # steps, forward and backward (as selective_scan_fn pads), and its outputs are cut back.
        pad = ctx.scan_pad = _train_pad(conv1d_out, A, B, C)
        out, scan_states, out_z, *ck = ext().fwd(*(_pad_front(t, pad) for t in (conv1d_out, delta)), A,
                                                 *(_pad_front(t, pad) for t in (B, C)), D, _pad_front(z, pad),
                                                 delta_bias, None, None, None, delta_softplus, tile_states=want_ck)
        ck = ck[0] if want_ck else None
        out_z = _unpad(out_z, pad)
        ctx.delta_softplus = delta_softplus
        ctx.out_proj_bias_is_None = out_proj_bias is None
        ctx.checkpoint_lvl = checkpoint_lvl
        ctx.b_rms_weight = b_rms_weight
        ctx.c_rms_weight = c_rms_weight
        ctx.dt_rms_weight = dt_rms_weight
        ctx.b_c_dt_rms_eps = b_c_dt_rms_eps
        if checkpoint_lvl >= 1:
            conv1d_out, delta = None, None
        ctx.save_for_backward(xz, conv1d_weight, conv1d_bias, x_dbl, x_proj_weight, delta_proj_weight,
                              out_proj_weight, conv1d_out, delta, A, B, C, D, delta_bias, scan_states, out, ck)
        y = F.linear(_cm_flat(out_z).t(), out_proj_weight, out_proj_bias)  # (batch * L, d_model)
        return y.view(batch, L, -1)

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        """Gradients of every tensor input as the reference returns them (ssi.py:555-645); dout:
        (batch, seqlen, d_model). With RMSNorm weights these are the reference's, not the gradient of
        the forward: the norms are passed unchanged and, at checkpoint_lvl=1, B and C normalised twice."""
        (xz, conv1d_weight, conv1d_bias, x_dbl, x_proj_weight, delta_proj_weight, out_proj_weight, conv1d_out,
         delta, A, B, C, D, delta_bias, scan_states, out, ck) = ctx.saved_tensors
        batch, L = xz.shape[0], xz.shape[-1]
        delta_rank = delta_proj_weight.shape[1]
        d_state = A.shape[-1]
        x, z = xz.chunk(2, dim=1)
        eps = ctx.b_c_dt_rms_eps
        if ctx.checkpoint_lvl == 1:
            conv1d_out = _conv(x, conv1d_weight, conv1d_bias)
            delta = _delta(delta_proj_weight, x_dbl, delta_rank, batch, ctx.dt_rms_weight, eps)
            # The saved B and C are the normalised ones; the reference normalises them again here
            # (ssi.py:582-593), so its scan backward runs at RMSNorm(RMSNorm(.)).
            if ctx.b_rms_weight is not None:
                B = _rms_bc(B, ctx.b_rms_weight, eps, "B")
            if ctx.c_rms_weight is not None:
                C = _rms_bc(C, ctx.c_rms_weight, eps, "C")
        dout2 = dout.reshape(batch * L, dout.shape[-1])                   # (batch * L, d_model)
        dxz = torch.empty_like(xz)
        dx, dz = dxz.chunk(2, dim=1)
        dout_y = _cm_view(out_proj_weight.t() @ dout2.t(), batch)          # (batch, d_inner, L), channel-major
        pad = ctx.scan_pad
        if pad:
            # The forward's padded scan (dout zero over the padding): dz comes back padded and is
            # copied into dxz; du, ddelta, dB, dC and out_z are cut back to the real steps.
            du, ddelta, dA, dB, dC, dD, ddelta_bias, dz_p, out_z = ext().bwd(
                *(_pad_front(t, pad) for t in (conv1d_out, delta)), A, *(_pad_front(t, pad) for t in (B, C)),
                D=D, z=_pad_front(z, pad), delta_bias=delta_bias, dout=_pad_front(dout_y, pad), x=scan_states,
                out=out, dz=None, delta_softplus=ctx.delta_softplus, recompute_out_z=True, tile_states=ck)
            dz.copy_(_unpad(dz_p, pad))
            du, ddelta, dB, dC, out_z = (_unpad(t, pad) for t in (du, ddelta, dB, dC, out_z))
        else:
            du, ddelta, dA, dB, dC, dD, ddelta_bias, dz, out_z = ext().bwd(
                conv1d_out, delta, A, B, C, D=D, z=z, delta_bias=delta_bias, dout=dout_y, x=scan_states, out=out,
                dz=dz, delta_softplus=ctx.delta_softplus, recompute_out_z=True, tile_states=ck)
        dout_proj_weight = dout2.t() @ _cm_flat(out_z).t()                 # (d_model, d_inner)
        dout_proj_bias = dout2.sum(dim=0) if not ctx.out_proj_bias_is_None else None
        # Rows of x_dbl that feed nothing (B or C given by the caller) get a zero gradient; the
        # reference leaves them uninitialised (torch.empty_like, ssi.py:609).
        dx_dbl = torch.empty_like(x_dbl)                                   # (R + 2N, batch * L)
        dB_proj_bias = dC_proj_bias = None
        rows_B = slice(delta_rank, delta_rank + d_state)
        rows_C = slice(x_dbl.shape[0] - d_state, None)
        if ctx.is_variable_B:
            dB2 = _cm_flat(dB[:, 0])
            dB_proj_bias = dB2.sum(dim=1) if not ctx.B_proj_bias_is_None else None
            dx_dbl[rows_B] = dB2
            dB = None
        else:
            dx_dbl[rows_B] = 0
        if ctx.is_variable_C:
            dC2 = _cm_flat(dC[:, 0])
            dC_proj_bias = dC2.sum(dim=1) if not ctx.C_proj_bias_is_None else None
            dx_dbl[rows_C] = dC2
            dC = None
        else:
            dx_dbl[rows_C] = 0
        ddelta2 = _cm_flat(ddelta)                                         # (d_inner, batch * L)
        ddelta_proj_weight = ddelta2 @ x_dbl[:delta_rank].t()
        torch.mm(delta_proj_weight.t(), ddelta2, out=dx_dbl[:delta_rank])
        u2 = _cm_flat(conv1d_out)
        dx_proj_weight = dx_dbl @ u2.t()
        du2 = _cm_flat(du)
        if du2.data_ptr() == du.data_ptr() and du2.is_contiguous():
            torch.addmm(du2, x_proj_weight.t(), dx_dbl, out=du2)
            dconv1d_out = du
        else:
            dconv1d_out = _cm_view(torch.addmm(du2, x_proj_weight.t(), dx_dbl), batch)
        res = ext().conv1d_bwd(x, conv1d_weight, conv1d_bias, dconv1d_out, dx, True)   # dx written into dxz
        dconv1d_weight = res[1].reshape(ctx.conv1d_weight_shape)          # (d_inner, 1, width)
        dconv1d_bias = res[2] if conv1d_bias is not None else None
        return (dxz, dconv1d_weight, dconv1d_bias, dx_proj_weight, ddelta_proj_weight,
                dout_proj_weight, dout_proj_bias,
                dA, dB, dC, dD if D is not None else None,
                ddelta_bias if delta_bias is not None else None,
                dB_proj_bias, dC_proj_bias, None, None, None, None, None, None, None)


def mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                   out_proj_bias, A, B=None, C=None, D=None, delta_bias=None, B_proj_bias=None, C_proj_bias=None,
                   delta_softplus=True, checkpoint_lvl=1, b_rms_weight=None, c_rms_weight=None, dt_rms_weight=None,
                   b_c_dt_rms_eps=1e-6):
    """ssi.py:648-656."""
    return MambaInnerFn.apply(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                              out_proj_bias, A, B, C, D, delta_bias, B_proj_bias, C_proj_bias, delta_softplus,
                              checkpoint_lvl, b_rms_weight, c_rms_weight, dt_rms_weight, b_c_dt_rms_eps,
                              torch.is_grad_enabled())
