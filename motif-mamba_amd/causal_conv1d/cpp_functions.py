"""``causal_conv1d.cpp_functions`` names imported by selective_scan_interface.py:12 (the functional
forms MambaInnerFn calls, selective_scan_interface.py:482-484, :567-569, :635-637)."""
from motif_mamba_amd.causal_conv1d import causal_conv1d_bwd, causal_conv1d_fn, causal_conv1d_update


def causal_conv1d_fwd_function(x, weight, bias, seq_idx, initial_states, final_states_out, silu_activation):
    """(x, weight, bias, seq_idx, initial_states, final_states_out, silu_activation) -> out; the last
    width - 1 inputs are written into final_states_out when it is given."""
    res = causal_conv1d_fn(x, weight, bias, seq_idx=seq_idx, initial_states=initial_states,
                           return_final_states=final_states_out is not None, final_states_out=final_states_out,
                           activation="silu" if silu_activation else None)
    return res[0] if final_states_out is not None else res


def causal_conv1d_update_function(x, conv_state, weight, bias, silu_activation, cache_seqlens=None,
                                  conv_state_indices=None):
    return causal_conv1d_update(x, conv_state, weight, bias, activation="silu" if silu_activation else None,
                                cache_seqlens=cache_seqlens, conv_state_indices=conv_state_indices)


def causal_conv1d_bwd_function(x, weight, bias, dout, seq_idx, initial_states, dfinal_states, dx,
                               return_dinitial_states, silu_activation):
    """-> (dx, dweight, dbias, dinitial_states): dx written into the given dx when not None, dweight /
    dbias in the dtypes of weight / bias, dinitial_states None. seq_idx, initial_states,
    dfinal_states and return_dinitial_states are not provided (NotImplementedError when set)."""
    if seq_idx is not None or initial_states is not None or dfinal_states is not None or return_dinitial_states:
        raise NotImplementedError("seq_idx / initial_states / dfinal_states gradients are not part of this build")
    dx, dweight, dbias = causal_conv1d_bwd(x, weight, bias, dout, dx, silu_activation)
    return dx, dweight, dbias, None
