"""ctypes mirror of include/mm_scan.h, used by the tests to call libmm_scan.so directly (the
binding a Python maintainer would add on the reference side uses the same structures)."""
from __future__ import annotations

import ctypes
import os
import re

import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "mm_scan.h")
HEADERS = [os.path.join(REPO, "include", h) for h in ("mm_scan.h", "mm_conv1d.h", "mm_norm.h")]

i64, i32, vp = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p

MM_OK, MM_ERR_INVALID_ARGUMENT, MM_ERR_UNSUPPORTED = 0, -1, -2
DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


class ScanFwdParams(ctypes.Structure):
    _fields_ = [("batch", i64), ("dim", i64), ("seqlen", i64), ("dstate", i64), ("n_groups", i64),
                ("itype", i32), ("is_variable_B", i32), ("is_variable_C", i32), ("delta_softplus", i32),
                ("u", vp), ("delta", vp), ("A", vp), ("B", vp), ("C", vp), ("D", vp), ("z", vp),
                ("delta_bias", vp), ("out", vp), ("out_z", vp), ("last_state", vp), ("chunk_states", vp),
                ("u_batch_stride", i64), ("u_d_stride", i64),
                ("delta_batch_stride", i64), ("delta_d_stride", i64),
                ("z_batch_stride", i64), ("z_d_stride", i64),
                ("out_batch_stride", i64), ("out_d_stride", i64),
                ("out_z_batch_stride", i64), ("out_z_d_stride", i64),
                ("A_d_stride", i64), ("A_dstate_stride", i64),
                ("B_batch_stride", i64), ("B_group_stride", i64), ("B_dstate_stride", i64), ("B_d_stride", i64),
                ("C_batch_stride", i64), ("C_group_stride", i64), ("C_dstate_stride", i64), ("C_d_stride", i64),
                ("workspace", vp), ("workspace_bytes", i64),
                ("P", vp), ("Q", vp), ("gamma", vp), ("pq_rank", i64),
                ("P_d_stride", i64), ("P_dstate_stride", i64), ("P_r_stride", i64),
                ("Q_d_stride", i64), ("Q_r_stride", i64), ("Q_dstate_stride", i64),
                ("gamma_d_stride", i64), ("gamma_dstate_stride", i64),
                ("tile_states", vp)]


class ScanBwdParams(ctypes.Structure):
    _fields_ = [("batch", i64), ("dim", i64), ("seqlen", i64), ("dstate", i64), ("n_groups", i64),
                ("itype", i32), ("is_variable_B", i32), ("is_variable_C", i32), ("delta_softplus", i32),
                ("u", vp), ("delta", vp), ("A", vp), ("B", vp), ("C", vp), ("D", vp), ("z", vp),
                ("delta_bias", vp), ("dout", vp), ("out", vp),
                ("du", vp), ("ddelta", vp), ("dz", vp), ("out_z", vp), ("dA", vp), ("dB", vp), ("dC", vp),
                ("dD", vp), ("ddelta_bias", vp),
                ("u_batch_stride", i64), ("u_d_stride", i64),
                ("delta_batch_stride", i64), ("delta_d_stride", i64),
                ("z_batch_stride", i64), ("z_d_stride", i64),
                ("out_batch_stride", i64), ("out_d_stride", i64),
                ("dout_batch_stride", i64), ("dout_d_stride", i64),
                ("du_batch_stride", i64), ("du_d_stride", i64),
                ("ddelta_batch_stride", i64), ("ddelta_d_stride", i64),
                ("dz_batch_stride", i64), ("dz_d_stride", i64),
                ("out_z_batch_stride", i64), ("out_z_d_stride", i64),
                ("A_d_stride", i64), ("A_dstate_stride", i64),
                ("B_batch_stride", i64), ("B_group_stride", i64), ("B_dstate_stride", i64), ("B_d_stride", i64),
                ("C_batch_stride", i64), ("C_group_stride", i64), ("C_dstate_stride", i64), ("C_d_stride", i64),
                ("dA_d_stride", i64), ("dA_dstate_stride", i64),
                ("dB_batch_stride", i64), ("dB_group_stride", i64), ("dB_dstate_stride", i64), ("dB_d_stride", i64),
                ("dC_batch_stride", i64), ("dC_group_stride", i64), ("dC_dstate_stride", i64), ("dC_d_stride", i64),
                ("workspace", vp), ("workspace_bytes", i64),
                ("P", vp), ("Q", vp), ("pq_rank", i64),
                ("P_d_stride", i64), ("P_dstate_stride", i64), ("P_r_stride", i64),
                ("Q_d_stride", i64), ("Q_r_stride", i64), ("Q_dstate_stride", i64),
                ("dP", vp), ("dQ", vp),
                ("dP_d_stride", i64), ("dP_dstate_stride", i64), ("dP_r_stride", i64),
                ("dQ_d_stride", i64), ("dQ_r_stride", i64), ("dQ_dstate_stride", i64),
                ("tile_states", vp)]


class Conv1dFwdParams(ctypes.Structure):
    _fields_ = [("batch", i64), ("dim", i64), ("seqlen", i64), ("width", i64),
                ("itype", i32), ("wtype", i32), ("silu", i32),
                ("x", vp), ("weight", vp), ("bias", vp), ("initial_states", vp), ("out", vp), ("final_states", vp),
                ("x_batch_stride", i64), ("x_d_stride", i64), ("out_batch_stride", i64), ("out_d_stride", i64),
                ("weight_d_stride", i64), ("weight_w_stride", i64), ("bias_stride", i64),
                ("init_batch_stride", i64), ("init_d_stride", i64), ("init_w_stride", i64),
                ("final_batch_stride", i64), ("final_d_stride", i64), ("final_w_stride", i64)]


class Conv1dUpdateParams(ctypes.Structure):
    _fields_ = [("batch", i64), ("dim", i64), ("seqlen", i64), ("width", i64), ("state_len", i64),
                ("itype", i32), ("wtype", i32), ("stype", i32), ("silu", i32),
                ("x", vp), ("conv_state", vp), ("weight", vp), ("bias", vp), ("out", vp),
                ("x_batch_stride", i64), ("x_d_stride", i64), ("x_l_stride", i64),
                ("state_batch_stride", i64), ("state_d_stride", i64), ("state_l_stride", i64),
                ("out_batch_stride", i64), ("out_d_stride", i64), ("out_l_stride", i64),
                ("weight_d_stride", i64), ("weight_w_stride", i64), ("bias_stride", i64)]


class Conv1dBwdParams(ctypes.Structure):
    _fields_ = [("batch", i64), ("dim", i64), ("seqlen", i64), ("width", i64),
                ("itype", i32), ("wtype", i32), ("silu", i32),
                ("x", vp), ("weight", vp), ("bias", vp), ("dout", vp), ("dx", vp), ("dweight", vp), ("dbias", vp),
                ("x_batch_stride", i64), ("x_d_stride", i64), ("dout_batch_stride", i64), ("dout_d_stride", i64),
                ("dx_batch_stride", i64), ("dx_d_stride", i64),
                ("weight_d_stride", i64), ("weight_w_stride", i64), ("bias_stride", i64)]


class RmsNormParams(ctypes.Structure):
    _fields_ = [("n0", i64), ("cols", i64), ("n2", i64), ("itype", i32), ("wtype", i32), ("eps", ctypes.c_float),
                ("x", vp), ("weight", vp), ("out", vp),
                ("x_stride0", i64), ("x_stride_c", i64), ("x_stride2", i64),
                ("out_stride0", i64), ("out_stride_c", i64), ("out_stride2", i64), ("weight_stride", i64)]


class StateUpdateParams(ctypes.Structure):
    _fields_ = [("batch", i64), ("dim", i64), ("dstate", i64), ("n_groups", i64),
                ("itype", i32), ("dt_softplus", i32),
                ("state", vp), ("x", vp), ("dt", vp), ("A", vp), ("B", vp), ("C", vp), ("D", vp), ("z", vp),
                ("dt_bias", vp), ("out", vp),
                ("state_batch_stride", i64), ("state_d_stride", i64), ("state_dstate_stride", i64),
                ("x_batch_stride", i64), ("x_d_stride", i64),
                ("dt_batch_stride", i64), ("dt_d_stride", i64),
                ("z_batch_stride", i64), ("z_d_stride", i64),
                ("out_batch_stride", i64), ("out_d_stride", i64),
                ("A_d_stride", i64), ("A_dstate_stride", i64),
                ("B_batch_stride", i64), ("B_group_stride", i64), ("B_dstate_stride", i64),
                ("C_batch_stride", i64), ("C_group_stride", i64), ("C_dstate_stride", i64),
                ("state_type", i32), ("D_type", i32), ("dt_bias_type", i32)]


def header_functions():
    """Names of the functions the headers in include/ declare."""
    text = "\n".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mm_\w+)\s*\(", text, re.M)))


def load():
    """libmm_scan.so with argtypes set (loaded through the package loader, which imports torch first)."""
    from motif_mamba_amd import _native
    lib = _native.lib()
    lib.mm_scan_fwd.argtypes = [ctypes.POINTER(ScanFwdParams), vp]
    lib.mm_scan_fwd.restype = ctypes.c_int
    lib.mm_state_update.argtypes = [ctypes.POINTER(StateUpdateParams), vp]
    lib.mm_state_update.restype = ctypes.c_int
    lib.mm_scan_fwd_noalloc.argtypes = [ctypes.POINTER(ScanFwdParams), vp]
    lib.mm_scan_fwd_noalloc.restype = ctypes.c_int
    lib.mm_scan_fwd_workspace_size.argtypes = [ctypes.POINTER(ScanFwdParams)]
    lib.mm_scan_fwd_workspace_size.restype = ctypes.c_int64
    lib.mm_scan_fwd_tile_states_size.argtypes = [ctypes.POINTER(ScanFwdParams)]
    lib.mm_scan_fwd_tile_states_size.restype = ctypes.c_int64
    lib.mm_scan_bwd.argtypes = [ctypes.POINTER(ScanBwdParams), vp]
    lib.mm_scan_bwd.restype = ctypes.c_int
    lib.mm_scan_bwd_workspace_size.argtypes = [ctypes.POINTER(ScanBwdParams)]
    lib.mm_scan_bwd_workspace_size.restype = ctypes.c_int64
    lib.mm_causal_conv1d_fwd.argtypes = [ctypes.POINTER(Conv1dFwdParams), vp]
    lib.mm_causal_conv1d_fwd.restype = ctypes.c_int
    lib.mm_causal_conv1d_update.argtypes = [ctypes.POINTER(Conv1dUpdateParams), vp]
    lib.mm_causal_conv1d_update.restype = ctypes.c_int
    lib.mm_causal_conv1d_bwd.argtypes = [ctypes.POINTER(Conv1dBwdParams), vp]
    lib.mm_causal_conv1d_bwd.restype = ctypes.c_int
    lib.mm_rms_norm_fwd.argtypes = [ctypes.POINTER(RmsNormParams), vp]
    lib.mm_rms_norm_fwd.restype = ctypes.c_int
    return lib


def _ptr(t):
    return None if t is None else t.data_ptr()


def scan_fwd_params(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False,
                    out=None, out_z=None, last_state=None, chunk_states=None, workspace=None,
                    P=None, Q=None, gamma=None):
    """Fill ScanFwdParams from torch tensors in the reference layouts (B/C 4-D or 2-D; P/Q 2-D
    shared or 3-D per channel, float32)."""
    p = ScanFwdParams()
    p.batch, p.dim, p.seqlen = u.shape
    p.dstate = A.shape[1]
    p.n_groups = B.shape[1] if B.dim() == 4 else 1
    p.itype = DTYPES[u.dtype]
    p.is_variable_B = int(B.dim() >= 3)
    p.is_variable_C = int(C.dim() >= 3)
    p.delta_softplus = int(bool(delta_softplus))
    p.u, p.delta, p.A, p.B, p.C = _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C)
    p.D, p.z, p.delta_bias = _ptr(D), _ptr(z), _ptr(delta_bias)
    p.out, p.out_z, p.last_state, p.chunk_states = _ptr(out), _ptr(out_z), _ptr(last_state), _ptr(chunk_states)
    p.u_batch_stride, p.u_d_stride = u.stride(0), u.stride(1)
    p.delta_batch_stride, p.delta_d_stride = delta.stride(0), delta.stride(1)
    if z is not None:
        p.z_batch_stride, p.z_d_stride = z.stride(0), z.stride(1)
    if out is not None:
        p.out_batch_stride, p.out_d_stride = out.stride(0), out.stride(1)
    if out_z is not None:
        p.out_z_batch_stride, p.out_z_d_stride = out_z.stride(0), out_z.stride(1)
    p.A_d_stride, p.A_dstate_stride = A.stride(0), A.stride(1)
    if B.dim() == 4:
        p.B_batch_stride, p.B_group_stride, p.B_dstate_stride = B.stride(0), B.stride(1), B.stride(2)
    else:
        p.B_d_stride, p.B_dstate_stride = B.stride(0), B.stride(1)
    if C.dim() == 4:
        p.C_batch_stride, p.C_group_stride, p.C_dstate_stride = C.stride(0), C.stride(1), C.stride(2)
    else:
        p.C_d_stride, p.C_dstate_stride = C.stride(0), C.stride(1)
    if workspace is not None:
        p.workspace, p.workspace_bytes = _ptr(workspace), workspace.numel() * workspace.element_size()
    if P is not None:
        p.P, p.Q, p.pq_rank = _ptr(P), _ptr(Q), P.shape[-1]
        if P.dim() == 3:
            p.P_d_stride, p.P_dstate_stride, p.P_r_stride = P.stride()
            p.Q_d_stride, p.Q_r_stride, p.Q_dstate_stride = Q.stride()
        else:
            p.P_dstate_stride, p.P_r_stride = P.stride()
            p.Q_r_stride, p.Q_dstate_stride = Q.stride()
    if gamma is not None:
        p.gamma = _ptr(gamma)
        if gamma.dim() == 2:
            p.gamma_d_stride, p.gamma_dstate_stride = gamma.stride()
        else:
            p.gamma_dstate_stride = gamma.stride(0)
    return p


def state_update_params(state, x, dt, A, B, C, out, D=None, z=None, dt_bias=None, dt_softplus=False):
    p = StateUpdateParams()
    p.batch, p.dim, p.dstate = state.shape
    p.n_groups = B.shape[1] if B.dim() == 3 else 1
    p.itype = DTYPES[x.dtype]
    p.dt_softplus = int(bool(dt_softplus))
    p.state, p.x, p.dt, p.A, p.B, p.C = map(_ptr, (state, x, dt, A, B, C))
    p.D, p.z, p.dt_bias, p.out = _ptr(D), _ptr(z), _ptr(dt_bias), _ptr(out)
    p.state_type = DTYPES[state.dtype]
    p.D_type = DTYPES[D.dtype] if D is not None else 0
    p.dt_bias_type = DTYPES[dt_bias.dtype] if dt_bias is not None else 0
    p.state_batch_stride, p.state_d_stride, p.state_dstate_stride = state.stride()
    p.x_batch_stride, p.x_d_stride = x.stride()
    p.dt_batch_stride, p.dt_d_stride = dt.stride()
    if z is not None:
        p.z_batch_stride, p.z_d_stride = z.stride()
    p.out_batch_stride, p.out_d_stride = out.stride()
    p.A_d_stride, p.A_dstate_stride = A.stride()
    if B.dim() == 3:
        p.B_batch_stride, p.B_group_stride, p.B_dstate_stride = B.stride()
        p.C_batch_stride, p.C_group_stride, p.C_dstate_stride = C.stride()
    else:
        p.B_batch_stride, p.B_dstate_stride = B.stride()
        p.C_batch_stride, p.C_dstate_stride = C.stride()
    return p


def stream_handle(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
