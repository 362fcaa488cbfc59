"""``causal_conv1d.cpp_functions`` names imported by selective_scan_interface.py:12 (the functional
forms MambaInnerFn calls, selective_scan_interface.py:482-484, :567-569, :635-637)."""
from motif_mamba_amd.causal_conv1d import causal_conv1d_fn, causal_conv1d_update


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


def causal_conv1d_bwd_function(*args, **kwargs):
    raise NotImplementedError("the causal_conv1d backward is not part of the MI355X build")
