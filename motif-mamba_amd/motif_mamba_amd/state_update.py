"""Drop-in ``selective_state_update`` backed by the gfx950 decode kernel.

Signature of the upstream ``mamba_ssm.ops.triton.selective_state_update.selective_state_update``
(mamba_ssm 2.2.6.post3) as called by the reference at ``mamba_simplemotif.py:397-399``:
``selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
dt_softplus=False) -> out``; ``state`` is updated in place.

Accepted layouts: state (batch, dim, dstate) with x/dt/z (batch, dim), A (dim, dstate),
B/C (batch, dstate) or (batch, n_groups, dstate), D/dt_bias (dim,); and the multi-head form
state (batch, nheads, headdim, dstate) with x/dt/z (batch, nheads, headdim), A (nheads, headdim,
dstate), B/C (batch, n_groups, dstate), D/dt_bias (nheads, headdim), flattened to dim =
nheads * headdim (group of a channel = head // (nheads / n_groups) = channel // (dim / n_groups)).
The state may be float32, float16 or bfloat16 (a bf16/fp16 model's ``allocate_inference_cache``
creates it in ``dt_proj.weight.dtype``, ``mamba_simplemotif.py:410-414``), and so may D and
dt_bias (passed uncast at ``mamba_simplemotif.py:397-399``): everything is widened to float32,
the state is stored back in its own dtype with round-to-nearest-even, and the output is read
from the float32 state, as the upstream kernel does.
"""
from __future__ import annotations

from ._native import ext


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False):
    if state.dim() == 4:
        batch, nheads, headdim, dstate = state.shape
        flat = state.view(batch, nheads * headdim, dstate)  # raises if not viewable: state is in place
        dim = nheads * headdim
        out = ext().state_update(
            flat, x.reshape(batch, dim), dt.reshape(batch, dim), A.reshape(dim, dstate), B, C,
            D=None if D is None else D.reshape(dim), z=None if z is None else z.reshape(batch, dim),
            dt_bias=None if dt_bias is None else dt_bias.reshape(dim), dt_softplus=dt_softplus)
        return out.view(batch, nheads, headdim)
    return ext().state_update(state, x, dt, A, B, C, D=D, z=z, dt_bias=dt_bias, dt_softplus=dt_softplus)
