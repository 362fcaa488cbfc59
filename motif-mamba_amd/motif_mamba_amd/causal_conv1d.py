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

``activation`` is None, "silu" or "swish" (else NotImplementedError). Not provided (raise
NotImplementedError): ``seq_idx`` (packed variable-length batches), ``cache_seqlens`` (circular
state buffers), ``conv_state_indices`` and the backward -- none is used on the reference's path.
x that is not contiguous along seqlen is copied first (the package also reads channel-last x
directly).
"""
from __future__ import annotations

import torch

from ._native import ext


def _silu(activation):
    if activation not in (None, "silu", "swish"):
        raise NotImplementedError("activation must be None, silu, or swish")
    return activation in ("silu", "swish")


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None, return_final_states=False,
                     final_states_out=None, activation=None):
    """x: (batch, dim, seqlen); weight: (dim, width); bias: (dim,); initial_states:
    (batch, dim, width - 1). Returns out (batch, dim, seqlen) [, final_states (batch, dim, width - 1)]."""
    silu = _silu(activation)
    if seq_idx is not None:
        raise NotImplementedError("seq_idx (variable-length packing) is not part of this build")
    if x.stride(-1) != 1 and x.shape[-1] != 1:
        x = x.contiguous()
    if bias is not None:
        bias = bias.contiguous()
    if return_final_states and final_states_out is None:
        final_states_out = torch.empty(x.shape[0], x.shape[1], weight.shape[1] - 1, device=x.device, dtype=x.dtype)
    out = ext().conv1d_fwd(x, weight, bias, initial_states,
                           final_states_out if return_final_states else None, silu)
    return (out, final_states_out) if return_final_states else out


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, cache_seqlens=None,
                         conv_state_indices=None):
    """x: (batch, dim) or (batch, dim, seqlen); conv_state: (batch, dim, state_len), state_len >=
    width - 1, updated in place; weight: (dim, width); bias: (dim,). Returns out shaped like x."""
    silu = _silu(activation)
    if cache_seqlens is not None or conv_state_indices is not None:
        raise NotImplementedError("cache_seqlens / conv_state_indices are not part of this build")
    return ext().conv1d_update(x, conv_state, weight, bias, silu)
