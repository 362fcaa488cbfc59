"""Drop-in ``selective_scan_fn`` / ``SelectiveScanFn`` backed by the gfx950 kernels.

Mirrors the reference interface ``mamba_ssm/ops/selective_scan_interface.py``:
``selective_scan_fn`` (ssi.py:237-259) and ``SelectiveScanFn.forward`` (ssi.py:24-61), with the
same argument names, defaults, input normalisation and return values:

* inputs whose last dimension is not contiguous are made contiguous (ssi.py:29-40);
* 3-D B/C ``(batch, dstate, L)`` are viewed as ``(batch, 1, dstate, L)`` (ssi.py:41-46);
* returns ``out_z`` when z is given, else ``out``; with ``return_last_state`` also the float32
  ``(batch, dim, dstate)`` state after the last step (ssi.py:54-61).

Differences (all raise instead of computing something else): the backward pass, the MotifMamba
P/Q/gamma paths (ssi.py:243-258) and complex A are not part of this build.
"""
from __future__ import annotations

import torch
from einops import rearrange

from ._native import ext


class SelectiveScanFn(torch.autograd.Function):

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                return_last_state=False):
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
        if C.dim() == 3:
            C = rearrange(C, "b dstate l -> b 1 dstate l")
        res = ext().fwd_infer(u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias,
                              delta_softplus=delta_softplus, return_last_state=return_last_state)
        if return_last_state:
            return res[0], res[1]
        return res[0]

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(
            "selective_scan backward is not implemented by the MI355X build (forward and decode only)")


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                      return_last_state=False, P=None, Q=None, gamma=None):
    """if return_last_state is True, returns (out, last_state)
    last_state has shape (batch, dim, dstate). Note that the gradient of the last state is
    not considered in the backward pass.
    """
    if P is not None or Q is not None or gamma is not None:
        raise NotImplementedError(
            "the MotifMamba P/Q/gamma low-rank coupling path is not part of the MI355X selective scan")
    return SelectiveScanFn.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state)
