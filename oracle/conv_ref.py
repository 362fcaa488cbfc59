"""CPU restatement of the causal depthwise conv1d that precedes the scan -- TEST INFRASTRUCTURE ONLY.

The reference imports ``causal_conv1d_fn`` / ``causal_conv1d_update`` from the third-party package
``causal-conv1d`` (pinned ``causal-conv1d>=1.2.0`` in the reference's pyproject.toml:33-34; not
vendored, not installed here), and otherwise runs the module's own torch fallback, which is the
algorithm restated here:

* forward (mamba_simplemotif.py:298-299): ``act(conv1d(x)[..., :seqlen])`` with the depthwise
  ``nn.Conv1d(d_inner, d_inner, kernel_size=d_conv, groups=d_inner, padding=d_conv - 1)`` of
  mamba_simplemotif.py:75-82, i.e.
      out[b, d, t] = bias[d] + sum_{k < W} weight[d, k] * x[b, d, t - (W - 1) + k]
  with x = 0 before t = 0 (or, as the package's API allows, the given ``initial_states``, the W - 1
  inputs before t = 0), then SiLU when activation is "silu"/"swish";
* decode update (mamba_simplemotif.py:353-358): the state (batch, dim, state_len) shifts left by
  one and takes the new input; out = sum(state * weight) + bias over the last W entries; SiLU.
  Generalised as the package's API allows to several new tokens per call (each one appended in
  turn) and state_len >= W - 1.

Arithmetic in float32 (inputs, weight and bias upcast), the result cast to x's dtype.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _act(y, activation):
    if activation in ("silu", "swish"):
        return F.silu(y)
    if activation is None:
        return y
    raise NotImplementedError("activation must be None, silu, or swish")


def causal_conv1d_ref(x, weight, bias=None, initial_states=None, return_final_states=False, activation=None,
                      compute_dtype=torch.float32):
    """x: (batch, dim, seqlen); weight: (dim, width); bias: (dim,) or None;
    initial_states: (batch, dim, width - 1) or None. Returns out (batch, dim, seqlen) in x's dtype,
    and with ``return_final_states`` also the last width - 1 inputs (batch, dim, width - 1).
    ``compute_dtype=torch.float64`` evaluates the same formula in double precision."""
    dtype_in = x.dtype
    dim, width = weight.shape
    seqlen = x.shape[-1]
    cd = compute_dtype
    xf = x.to(cd)
    wf = weight.to(cd).unsqueeze(1)
    bf = None if bias is None else bias.to(cd)
    if initial_states is not None:
        xf = torch.cat([initial_states.to(cd), xf], dim=-1)
        y = F.conv1d(xf, wf, bf, padding=0, groups=dim)
    else:
        y = F.conv1d(xf, wf, bf, padding=width - 1, groups=dim)
    y = _act(y[..., :seqlen], activation).to(dtype_in)
    if not return_final_states:
        return y
    final = F.pad(xf, (width - 1 - xf.shape[-1], 0)).to(dtype_in)
    return y, final


def causal_conv1d_update_ref(x, conv_state, weight, bias=None, activation=None):
    """x: (batch, dim) or (batch, dim, seqlen); conv_state: (batch, dim, state_len), state_len >=
    width - 1, updated in place; weight: (dim, width); bias: (dim,) or None. Returns out with x's
    shape and dtype."""
    dtype_in = x.dtype
    squeeze = x.dim() == 2
    xs = x.unsqueeze(-1) if squeeze else x
    dim, width = weight.shape
    state_len = conv_state.shape[-1]
    if state_len < width - 1:
        raise ValueError("conv_state must hold at least width - 1 steps")
    seqlen = xs.shape[-1]
    seq = torch.cat([conv_state.float(), xs.float()], dim=-1)
    conv_state.copy_(seq[..., -state_len:].to(conv_state.dtype))
    y = F.conv1d(seq[..., -(seqlen + width - 1):], weight.float().unsqueeze(1),
                 None if bias is None else bias.float(), padding=0, groups=dim)
    y = _act(y, activation).to(dtype_in)
    return y.squeeze(-1) if squeeze else y


def causal_conv1d_brute(x, weight, bias=None, initial_states=None, activation=None):
    """Float64 explicit sum, nested lists in and out (tiny shapes only)."""
    import math
    batch, dim, L = len(x), len(x[0]), len(x[0][0])
    W = len(weight[0])
    out = [[[0.0] * L for _ in range(dim)] for _ in range(batch)]
    for b in range(batch):
        for d in range(dim):
            for t in range(L):
                acc = float(bias[d]) if bias is not None else 0.0
                for k in range(W):
                    s = t - (W - 1) + k
                    if s >= 0:
                        v = float(x[b][d][s])
                    elif initial_states is not None:
                        v = float(initial_states[b][d][W - 1 + s])
                    else:
                        v = 0.0
                    acc += float(weight[d][k]) * v
                if activation in ("silu", "swish"):
                    acc = acc / (1.0 + math.exp(-acc))
                out[b][d][t] = acc
    return out
