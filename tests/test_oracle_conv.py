"""Pins for the causal-conv1d oracle (oracle/conv_ref.py), the restatement of the Mamba module's torch
fallback (mamba_simplemotif.py:298-299 forward, :353-358 decode update) and of the third-party
``causal-conv1d`` API the reference calls (not vendored; its published semantics):

* a hand-worked known answer and a float64 explicit-sum brute force (no F.conv1d) on tiny shapes;
* the decode update written literally as the module writes it (roll, write the last slot, dot with
  the weights) against ``causal_conv1d_update_ref``;
* L decode updates from a zero state reproduce the forward over the same L tokens;
* ``initial_states`` continue a split sequence exactly; ``final_states`` are the last width-1 inputs.

CPU only.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.conv_ref import causal_conv1d_brute, causal_conv1d_ref, causal_conv1d_update_ref


def _case(seed, batch=2, dim=3, L=9, W=4, with_bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, dim, L, generator=g)
    w = torch.randn(dim, W, generator=g)
    b = torch.randn(dim, generator=g) if with_bias else None
    return x, w, b


def test_known_answer():
    x = torch.tensor([[[1.0, 2.0, 3.0]]])
    w = torch.tensor([[1.0, 2.0]])
    np.testing.assert_allclose(causal_conv1d_ref(x, w)[0, 0].numpy(), [2.0, 5.0, 8.0])
    np.testing.assert_allclose(causal_conv1d_ref(x, w, torch.tensor([0.5]))[0, 0].numpy(), [2.5, 5.5, 8.5])


@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("act", [None, "silu"])
@pytest.mark.parametrize("init", [False, True])
def test_forward_vs_brute(W, act, init):
    x, w, b = _case(10 + W, W=W)
    ini = torch.randn(2, 3, W - 1, generator=torch.Generator().manual_seed(3)) if init else None
    got = causal_conv1d_ref(x, w, b, initial_states=ini, activation=act)
    ref = causal_conv1d_brute(x.tolist(), w.tolist(), b.tolist(), None if ini is None else ini.tolist(), act)
    np.testing.assert_allclose(got.double().numpy(), np.array(ref), rtol=1e-5, atol=1e-6)


def _module_step(conv_state, x, weight, bias):
    """mamba_simplemotif.py:353-358, literally (SiLU activation)."""
    conv_state.copy_(torch.roll(conv_state, shifts=-1, dims=-1))
    conv_state[:, :, -1] = x
    y = torch.sum(conv_state * weight, dim=-1)
    if bias is not None:
        y = y + bias
    return F.silu(y)


def test_update_matches_module_fallback_and_forward():
    x, w, b = _case(20, batch=2, dim=5, L=12, W=4)
    st_ref = torch.zeros(2, 5, 4)
    st_mod = torch.zeros(2, 5, 4)
    full = causal_conv1d_ref(x, w, b, activation="silu")
    for t in range(12):
        y_ref = causal_conv1d_update_ref(x[:, :, t], st_ref, w, b, activation="silu")
        y_mod = _module_step(st_mod, x[:, :, t], w, b)
        torch.testing.assert_close(y_ref, y_mod, rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(st_ref, st_mod)
        torch.testing.assert_close(y_ref, full[:, :, t], rtol=1e-5, atol=1e-6)


def test_update_several_tokens_and_short_state():
    """seqlen > 1 per call equals one call per token; state_len = width - 1 keeps what is needed."""
    x, w, b = _case(30, batch=2, dim=4, L=6, W=4)
    s1 = torch.randn(2, 4, 3, generator=torch.Generator().manual_seed(31))
    s2 = s1.clone()
    many = causal_conv1d_update_ref(x, s1, w, b, activation=None)
    one = torch.stack([causal_conv1d_update_ref(x[:, :, t], s2, w, b) for t in range(6)], dim=-1)
    torch.testing.assert_close(many, one, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(s1, s2)
    torch.testing.assert_close(s1, x[:, :, -3:])


def test_initial_and_final_states_split_a_sequence():
    x, w, b = _case(40, batch=2, dim=3, L=20, W=4)
    full = causal_conv1d_ref(x, w, b, activation="silu")
    a, fin = causal_conv1d_ref(x[..., :7], w, b, return_final_states=True, activation="silu")
    torch.testing.assert_close(fin, x[..., 4:7])
    rest = causal_conv1d_ref(x[..., 7:], w, b, initial_states=fin, activation="silu")
    torch.testing.assert_close(torch.cat([a, rest], -1), full, rtol=1e-6, atol=1e-6)
    # shorter than width - 1: the final states are left-padded with zeros
    _, fin2 = causal_conv1d_ref(x[..., :2], w, b, return_final_states=True)
    torch.testing.assert_close(fin2, F.pad(x[..., :2], (1, 0)))


def test_activation_errors():
    x, w, b = _case(50)
    with pytest.raises(NotImplementedError):
        causal_conv1d_ref(x, w, b, activation="relu")
