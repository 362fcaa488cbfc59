"""Drop-in ``selective_scan_fn`` / ``SelectiveScanFn`` backed by the gfx950 kernels.

Mirrors the reference interface ``mamba_ssm/ops/selective_scan_interface.py``:
``selective_scan_fn`` (ssi.py:237-259) and ``SelectiveScanFn.forward`` (ssi.py:24-61), with the
same argument names, defaults, input normalisation and return values:

* inputs whose last dimension is not contiguous are made contiguous (ssi.py:29-40);
* 3-D B/C ``(batch, dstate, L)`` are viewed as ``(batch, 1, dstate, L)`` (ssi.py:41-46);
* returns ``out_z`` when z is given, else ``out``; with ``return_last_state`` also the float32
  ``(batch, dim, dstate)`` state after the last step (ssi.py:54-61).

With P/Q (the MotifMamba low-rank coupling, ssi.py:243-258) ``selective_scan_fn`` computes
``h_t = exp(dt A) h_{t-1} + dt P (Q h_{t-1}) + dt u B_t`` on the GPU whether or not z is given: the
reference sends z-less calls to its dense CUDA kernel (``SelectiveScanPQFn``, ssi.py:93-150) and
calls with z to a torch loop (``selective_scan_full_matrix_cuda``, ssi.py:262-350); both compute
the same function, and so does this build's single kernel. Argument errors are the reference's
(ValueError for P without Q, mismatched P/Q shapes or non-CUDA tensors). gamma is validated
and, as in both reference paths, not used.

``SelectiveScanFn.backward`` (ssi.py:63-91) runs the gfx950 backward (``selective_scan_cuda.bwd``
equivalent); with gradients required, the forward saves the reference's tensors (u, delta, A, B,
C, D, [z], delta_bias, x, [out]); without, it writes only what it returns.

``SelectiveScanPQFn.backward`` returns the exact gradients of the coupled recurrence (dP and dQ
included), which is what the reference returns in both of its gradient modes
(``MOTIFMAMBA_PQ_GRAD_MODE``, ssi.py:157-158): its dense CUDA backward (z-less calls) and autograd
through its torch loop (calls with z) differentiate the same function; "exact" takes dP/dQ of
z-less calls from that autograd, any other value ("fused") from the dense kernel, the only backward
its launcher runs with P/Q (selective_scan_bwd_kernel.cuh:928-932), which accumulates the same
chain rule (:307, :334). The variable is therefore not read here. The fast gfx950 backward covers
pq_rank 1..8, dstate <= 16, dim and dim / n_groups multiples of 16 and seqlen a multiple of 8, with
variable B and C; training requests of other lengths are padded in front with zero-u steps
(_train_pad); the other shapes the reference takes (dstate <= 256, rank <= 8, constant B or C) run
a general P/Q backward with one lane per state.

Differences (all raise instead of computing something else): complex A is not part of this build.
"""
from __future__ import annotations

import os

import torch
from einops import rearrange

from ._native import ext


def _save_tile_states():
    """Whether training forwards keep the 16-step tile states for the backward (default on;
    MM_TILE_STATES=0 trades the B * dim * L float32 of saved activations for the backward's recompute
    of the scan)."""
    return os.environ.get("MM_TILE_STATES", "1") != "0"


def _train_pad(u, A, B, C):
    """Steps to put in front of a training request whose length is not a multiple of 8, so that
    the forward and backward run the fast kernels (the diagonal ones at dstate 16, the P/Q ones at
    dstate <= 16, which also run the diagonal scan at other dstate values with a zero coupling;
    with other lengths the diagonal scan would run the general kernels, ~14x and ~100x slower, and
    the P/Q backward would refuse the call). The padded steps carry zero u, delta, z, B and C, and
    dout is zero over them: from the zero initial state a zero-u step leaves every state exactly
    zero, so the real steps run the unpadded recurrence, and the padded steps add nothing to dA,
    dD, ddelta_bias, dP or dQ (each of their terms holds u, h or Q h of a padded step). 0 when no
    padding applies, or with MM_SCAN_PAD=0 (which also turns off the binding's padding of
    inference requests)."""
    L = u.shape[-1]
    if L % 8 == 0 or B.dim() != 4 or C.dim() != 4 or os.environ.get("MM_SCAN_PAD", "1") == "0":
        return 0
    if A.shape[1] > 16:
        return 0
    dim, groups = u.shape[1], B.shape[1]
    if dim % 16 or (dim // groups) % 16:
        return 0
    return (-L) % 32


def _pad_front(t, pad):
    return t if t is None or pad == 0 else torch.nn.functional.pad(t, (pad, 0))


def _unpad(t, pad):
    return t if t is None or pad == 0 else t[..., pad:]


def _infer(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state, P=None, Q=None, gamma=None):
    """The inference forward (no gradient needed): the stride fix-ups of the autograd forwards
    (ssi.py:24-36) and the binding's fwd_infer, which writes only what is returned."""
    if u.stride(-1) != 1:
        u = u.contiguous()
    if delta.stride(-1) != 1:
        delta = delta.contiguous()
    if D is not None:
        D = D.contiguous()
    if B.stride(-1) != 1:
        B = B.contiguous()
    if C.stride(-1) != 1:
        C = C.contiguous()
    if z is not None and z.stride(-1) != 1:
        z = z.contiguous()
    if delta_bias is not None and delta_bias.stride(-1) != 1:
        delta_bias = delta_bias.contiguous()
    if B.dim() == 3:
        B = B.unsqueeze(1)
    if C.dim() == 3:
        C = C.unsqueeze(1)
    res = ext().fwd_infer(u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias, delta_softplus=delta_softplus,
                          return_last_state=return_last_state, P=P, Q=Q, gamma=gamma)
    return (res[0], res[1]) if return_last_state else res[0]


class SelectiveScanFn(torch.autograd.Function):

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                return_last_state=False, grad_enabled=True):
        # grad_enabled: the grad mode of the caller (selective_scan_fn passes it; forward itself runs
        # with grad disabled, and needs_input_grad reflects requires_grad alone, so a module called
        # under torch.no_grad() with parameters that require grad would otherwise take the training path).
        if u.stride(-1) != 1:
            u = u.contiguous()
        if delta.stride(-1) != 1:
            delta = delta.contiguous()
        if D is not None:
            D = D.contiguous()
        if B.stride(-1) != 1:
            B = B.contiguous()
        if C.stride(-1) != 1:
            C = C.contiguous()
        if z is not None and z.stride(-1) != 1:
            z = z.contiguous()
        if B.dim() == 3:
            B = rearrange(B, "b dstate l -> b 1 dstate l")
            ctx.squeeze_B = True
        if C.dim() == 3:
            C = rearrange(C, "b dstate l -> b 1 dstate l")
            ctx.squeeze_C = True
        if not grad_enabled or not any(ctx.needs_input_grad[:8]):
            # Inference: only what is returned is written (no pre-gate out, no chunk states).
            return _infer(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state)
        # Training: the reference's outputs and saved tensors (ssi.py:47-61), plus, for dstate <= 16,
        # the states before every 16-step tile (None where the kernels do not write them), which
        # spare the backward its recompute of the scan.
        want_ck = A.shape[1] <= 16 and _save_tile_states()
        pad = ctx.pad = _train_pad(u, A, B, C)
        u, delta, z, B, C = (_pad_front(t, pad) for t in (u, delta, z, B, C))
        out, x, *rest = ext().fwd(u, delta, A, B, C, D, z, delta_bias, None, None, None, delta_softplus,
                                  tile_states=want_ck)
        ck = rest.pop() if want_ck else None
        ctx.delta_softplus = delta_softplus
        ctx.has_z = z is not None
        last_state = x[:, :, -1, 1::2]
        if not ctx.has_z:
            ctx.save_for_backward(u, delta, A, B, C, D, delta_bias, x, ck)
            out = _unpad(out, pad).contiguous() if pad else out
            return out if not return_last_state else (out, last_state)
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, x, out, ck)
        out_z = _unpad(rest[0], pad).contiguous() if pad else rest[0]
        return out_z if not return_last_state else (out_z, last_state)

    @staticmethod
    def backward(ctx, dout, *args):
        """ssi.py:63-91: the gradient of last_state is not propagated, as in the reference."""
        if not ctx.has_z:
            u, delta, A, B, C, D, delta_bias, x, ck = ctx.saved_tensors
            z = None
            out = None
        else:
            u, delta, A, B, C, D, z, delta_bias, x, out, ck = ctx.saved_tensors
        if dout.stride(-1) != 1:
            dout = dout.contiguous()
        pad = ctx.pad
        dout = _pad_front(dout, pad)
        du, ddelta, dA, dB, dC, dD, ddelta_bias, *rest = ext().bwd(
            u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias, dout=dout, x=x, out=out, dz=None,
            delta_softplus=ctx.delta_softplus, recompute_out_z=False, tile_states=ck)
        dz = rest[0] if ctx.has_z else None
        du, ddelta, dz, dB, dC = (_unpad(t, pad) for t in (du, ddelta, dz, dB, dC))
        dB = dB.squeeze(1) if getattr(ctx, "squeeze_B", False) else dB
        dC = dC.squeeze(1) if getattr(ctx, "squeeze_C", False) else dC
        return (du, ddelta, dA, dB, dC,
                dD if D is not None else None,
                dz,
                ddelta_bias if delta_bias is not None else None,
                None,
                None,
                None)


class SelectiveScanPQFn(torch.autograd.Function):
    """Forward of the low-rank coupled scan (ssi.py:93-150 and ssi.py:262-350), z optional."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                return_last_state=False, P=None, Q=None, gamma=None, grad_enabled=True):
        if u.stride(-1) != 1:
            u = u.contiguous()
        if delta.stride(-1) != 1:
            delta = delta.contiguous()
        if D is not None:
            D = D.contiguous()
        if B.stride(-1) != 1:
            B = B.contiguous()
        if C.stride(-1) != 1:
            C = C.contiguous()
        if z is not None and z.stride(-1) != 1:
            z = z.contiguous()
        if delta_bias is not None and delta_bias.stride(-1) != 1:
            delta_bias = delta_bias.contiguous()
        if B.dim() == 3:
            B = rearrange(B, "b dstate l -> b 1 dstate l")
            ctx.squeeze_B = True
        if C.dim() == 3:
            C = rearrange(C, "b dstate l -> b 1 dstate l")
            ctx.squeeze_C = True
        if not grad_enabled or not (any(ctx.needs_input_grad[:8]) or any(ctx.needs_input_grad[10:12])):
            return _infer(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state, P, Q, gamma)
        # Training: the forward's outputs plus what the backward reads (ssi.py:123-137 saves
        # u, delta, A, B, C, D, delta_bias, P, Q, gamma, x; out joins them when z is given). With
        # dstate <= 16 the forward also writes the states before every 16-step tile (B * dim * L
        # float32, about one float32 copy of u), which spare the backward a recompute of the scan.
        want_ck = A.shape[1] <= 16 and P.shape[-1] > 0 and _save_tile_states()
        pad = ctx.pad = _train_pad(u, A, B, C)
        u, delta, z, B, C = (_pad_front(t, pad) for t in (u, delta, z, B, C))
        out, x, *rest = ext().fwd(u, delta, A, B, C, D, z, delta_bias, P, Q, gamma, delta_softplus,
                                  tile_states=want_ck)
        ck = rest.pop() if want_ck else None
        ctx.delta_softplus = delta_softplus
        ctx.has_z = z is not None
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias, P, Q, gamma, x,
                              out if ctx.has_z else None, ck)
        last_state = x[:, :, -1, 1::2]
        result = rest[0] if ctx.has_z else out
        result = _unpad(result, pad).contiguous() if pad else result
        return result if not return_last_state else (result, last_state)

    @staticmethod
    def backward(ctx, dout, *args):
        """Exact gradients of the coupled recurrence, dP and dQ included: what the reference's
        default ("exact") mode returns (ssi.py:152-205: its CUDA backward for u, delta, A, B, C,
        D, delta_bias and autograd through selective_scan_full_matrix_cuda for dP, dQ; with z,
        autograd through that torch loop for everything). gamma gets no gradient, as there."""
        u, delta, A, B, C, D, z, delta_bias, P, Q, gamma, x, out, ck = ctx.saved_tensors
        if dout.stride(-1) != 1:
            dout = dout.contiguous()
        pad = ctx.pad
        dout = _pad_front(dout, pad)
        dP = torch.zeros(P.shape, dtype=torch.float32, device=P.device)
        dQ = torch.zeros(Q.shape, dtype=torch.float32, device=Q.device)
        du, ddelta, dA, dB, dC, dD, ddelta_bias, *rest = ext().bwd(
            u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias, P=P, Q=Q, gamma=gamma, dout=dout,
            x=x, out=out, dz=None, dP_out=dP, dQ_out=dQ, delta_softplus=ctx.delta_softplus,
            recompute_out_z=False, tile_states=ck)
        dz = rest[0] if ctx.has_z else None
        du, ddelta, dz, dB, dC = (_unpad(t, pad) for t in (du, ddelta, dz, dB, dC))
        dB = dB.squeeze(1) if getattr(ctx, "squeeze_B", False) else dB
        dC = dC.squeeze(1) if getattr(ctx, "squeeze_C", False) else dC
        return (du, ddelta, dA, dB, dC,
                dD if D is not None else None,
                dz,
                ddelta_bias if delta_bias is not None else None,
                None,
                None,
                dP.to(P.dtype), dQ.to(Q.dtype),
                None,
                None)


def _check_pq(u, delta, A, B, C, P, Q):
    """The argument errors of selective_scan_full_matrix_cuda (ssi.py:266-271, 303-318)."""
    if P is None or Q is None:
        raise ValueError("P and Q must both be provided for full-matrix path")
    if A.is_complex():
        raise NotImplementedError("Full-matrix P/Q path currently supports real A only")
    if not (u.is_cuda and delta.is_cuda and A.is_cuda and B.is_cuda and C.is_cuda and P.is_cuda and Q.is_cuda):
        raise ValueError("Full-matrix path requires CUDA tensors")
    dim, dstate = u.shape[1], A.shape[1]
    if P.dim() == 2 and Q.dim() == 2:
        if P.shape[0] != dstate or Q.shape[1] != dstate or P.shape[1] != Q.shape[0]:
            raise ValueError("Expected P(n, r), Q(r, n) with n=dstate")
    elif P.dim() == 3 and Q.dim() == 3:
        if P.shape[0] != dim or Q.shape[0] != dim:
            raise ValueError("Expected P(dim, n, r), Q(dim, r, n)")
        if P.shape[1] != dstate or Q.shape[2] != dstate or P.shape[2] != Q.shape[1]:
            raise ValueError("Expected P(dim, n, r), Q(dim, r, n)")
    else:
        raise ValueError("P and Q must both be 2D or both be 3D")
    if P.shape[-1] > 8:
        raise NotImplementedError("pq_rank > 8 is not supported (the reference's dense forward limit)")


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                      return_last_state=False, P=None, Q=None, gamma=None):
    """if return_last_state is True, returns (out, last_state)
    last_state has shape (batch, dim, dstate). Note that the gradient of the last state is
    not considered in the backward pass.
    """
    pq = P is not None or Q is not None or gamma is not None
    if pq:
        _check_pq(u, delta, A, B, C, P, Q)
    # Without a gradient to take (grad mode off, or no input that requires one) the inference
    # forward runs directly, without the autograd Function's own host cost (~5 us per call; the
    # Motif decode step calls the P/Q scan once per layer and token, mamba_simplemotif.py:378-396).
    grads = (u, delta, A, B, C, D, z, delta_bias) + ((P, Q) if pq else ())
    if not torch.is_grad_enabled() or not any(t is not None and t.requires_grad for t in grads):
        return _infer(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state,
                      *((P, Q, gamma) if pq else ()))
    if pq:
        return SelectiveScanPQFn.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus,
                                       return_last_state, P, Q, gamma, True)
    return SelectiveScanFn.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state, True)
