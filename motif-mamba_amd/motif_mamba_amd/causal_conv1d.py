"""Drop-in ``causal_conv1d_fn`` / ``causal_conv1d_update`` backed by the gfx950 kernels of
mm_conv1d.hip.

The reference imports both from the third-party package causal-conv1d (mamba_simplemotif.py:16-19,
selective_scan_interface.py:10-17; pinned ``causal-conv1d>=1.2.0``, pyproject.toml:33-34, not
vendored) and otherwise runs its own torch fallback (mamba_simplemotif.py:298-299 forward,
:353-358 decode update). Signatures, argument meanings and errors are the package's:

* ``causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None,
  return_final_states=False, final_states_out=None, activation=None)`` -> out, or
  (out, final_states) with ``return_final_states``;
* ``causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, cache_seqlens=None,
  conv_state_indices=None)`` -> out, conv_state updated in place.

``causal_conv1d_fn`` is differentiable in x, weight and bias (the package's CausalConv1dFn), and
``causal_conv1d_bwd`` is the functional backward MambaInnerFn calls
(selective_scan_interface.py:635-637).

``activation`` is None, "silu" or "swish" (else NotImplementedError). Not provided (raise
NotImplementedError): ``seq_idx`` (packed variable-length batches), ``cache_seqlens`` (circular
state buffers), ``conv_state_indices``, and gradients through ``initial_states`` / the returned
final states -- none is used on the reference's path. x that is not contiguous along seqlen is
copied first (the package also reads channel-last x directly).
"""
from __future__ import annotations

import torch

from ._native import ext


def _silu(activation):
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    return activation in ("silu", "swish")


def _fwd(x, weight, bias, initial_states, return_final_states, final_states_out, silu):
    if x.stride(-1) != 1 and x.shape[-1] != 1:
        x = x.contiguous()
    if bias is not None:
        bias = bias.contiguous()
    if return_final_states and final_states_out is None:
        final_states_out = torch.empty(x.shape[0], x.shape[1], weight.shape[1] - 1, device=x.device, dtype=x.dtype)
    out = ext().conv1d_fwd(x, weight, bias, initial_states,
                           final_states_out if return_final_states else None, silu)
    return x, bias, out, final_states_out


def causal_conv1d_bwd(x, weight, bias, dout, dx=None, silu=False):
    """Gradients of ``causal_conv1d_fn(x, weight, bias, activation="silu" if silu else None)`` for
    the output gradient dout: (dx, dweight, dbias); dx is written into the given tensor when one is
    passed. dweight / dbias are summed in float32 and returned in the dtypes of weight / bias."""
    if x.stride(-1) != 1 and x.shape[-1] != 1:
        x = x.contiguous()
    if dout.stride(-1) != 1 and dout.shape[-1] != 1:
        dout = dout.contiguous()
    res = ext().conv1d_bwd(x, weight, None if bias is None else bias.contiguous(), dout, dx, silu)
    return res[0], res[1], (res[2] if bias is not None else None)


class CausalConv1dFn(torch.autograd.Function):
    """The package's autograd form of causal_conv1d_fn: gradients for x, weight and bias."""

    @staticmethod
    def forward(ctx, x, weight, bias=None, initial_states=None, return_final_states=False,
                final_states_out=None, silu=False):
        x, bias_c, out, fin = _fwd(x, weight, bias, initial_states, return_final_states, final_states_out, silu)
        ctx.silu = silu
        ctx.has_initial = initial_states is not None
        ctx.has_bias = bias is not None
        ctx.set_materialize_grads(False)
        if final_states_out is not None:
            ctx.mark_dirty(final_states_out)
        ctx.save_for_backward(x, weight, bias_c)
        return (out, fin) if return_final_states else out

    @staticmethod
    def backward(ctx, dout, *rest):
        if ctx.has_initial or (rest and rest[0] is not None):
            raise NotImplementedError("gradients through initial_states / final states are not part of this build")
        x, weight, bias = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros_like(x)
        dx, dweight, dbias = causal_conv1d_bwd(x, weight, bias, dout, None, ctx.silu)
        return dx, dweight, dbias if ctx.has_bias else None, None, None, None, None


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None, return_final_states=False,
                     final_states_out=None, activation=None):
    """x: (batch, dim, seqlen); weight: (dim, width); bias: (dim,); initial_states:
    (batch, dim, width - 1). Returns out (batch, dim, seqlen) [, final_states (batch, dim, width - 1)]."""
    silu = _silu(activation)
    if seq_idx is not None:
        raise NotImplementedError("seq_idx (variable-length packing) is not part of this build")
    return CausalConv1dFn.apply(x, weight, bias, initial_states, return_final_states, final_states_out, silu)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, cache_seqlens=None,
                         conv_state_indices=None):
    """x: (batch, dim) or (batch, dim, seqlen); conv_state: (batch, dim, state_len), state_len >=
    width - 1, updated in place; weight: (dim, width); bias: (dim,). Returns out shaped like x."""
    silu = _silu(activation)
    if cache_seqlens is not None or conv_state_indices is not None:
        raise NotImplementedError("cache_seqlens / conv_state_indices are not part of this build")
    return ext().conv1d_update(x, conv_state, weight, bias, silu)
