"""CPU checks of the drop-in boundary: the C-ABI library loads, exports every function the header
declares, its parameter structs have the layout of include/mm_scan.h, and invalid requests are
rejected before anything is launched. No GPU needed (no call here reaches a kernel launch)."""
import ctypes
import os
import subprocess

import pytest
import torch

from tests import capi


def test_library_exports_every_header_function():
    lib = capi.load()
    names = capi.header_functions()
    assert set(names) == {"mm_scan_fwd", "mm_scan_fwd_noalloc", "mm_scan_fwd_workspace_size",
                          "mm_scan_fwd_tile_states_size",
                          "mm_scan_bwd", "mm_scan_bwd_workspace_size",
                          "mm_state_update", "mm_last_error", "mm_abi_version", "mm_causal_conv1d_fwd",
                          "mm_causal_conv1d_update", "mm_causal_conv1d_bwd", "mm_rms_norm_fwd"}
    for n in names:
        assert hasattr(lib, n), n
    assert lib.mm_abi_version() == 10


def _c_layout(struct, fields, tmp_path):
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "mm_scan.h"', '#include "mm_conv1d.h"', '#include "mm_norm.h"',
             'int main(void) {',
             f'  printf("%zu\\n", sizeof({struct}));']
    lines += [f'  printf("%zu\\n", offsetof({struct}, {f}));' for f in fields]
    lines += ['  return 0;', '}']
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.check_call(["gcc", "-std=c11", f"-I{os.path.join(capi.REPO, 'include')}", str(src), "-o", str(exe)])
    return [int(x) for x in subprocess.check_output([str(exe)]).split()]


@pytest.mark.parametrize("cname,pystruct", [("mm_scan_fwd_params", capi.ScanFwdParams),
                                            ("mm_scan_bwd_params", capi.ScanBwdParams),
                                            ("mm_conv1d_fwd_params", capi.Conv1dFwdParams),
                                            ("mm_conv1d_update_params", capi.Conv1dUpdateParams),
                                            ("mm_conv1d_bwd_params", capi.Conv1dBwdParams),
                                            ("mm_rms_norm_params", capi.RmsNormParams),
                                            ("mm_state_update_params", capi.StateUpdateParams)])
def test_struct_layout_matches_header(tmp_path, cname, pystruct):
    fields = [f for f, _ in pystruct._fields_]
    got = _c_layout(cname, fields, tmp_path)
    assert got[0] == ctypes.sizeof(pystruct)
    assert got[1:] == [getattr(pystruct, f).offset for f in fields]


def _valid_looking_params():
    p = capi.ScanFwdParams()
    p.batch, p.dim, p.seqlen, p.dstate, p.n_groups = 2, 8, 16, 16, 1
    p.itype = 2
    p.is_variable_B = p.is_variable_C = 1
    fake = 0x1000
    p.u = p.delta = p.A = p.B = p.C = p.out = fake
    return p


@pytest.mark.parametrize("mutate,needle", [
    (lambda p: setattr(p, "dstate", 257), "state dimension"),
    (lambda p: setattr(p, "dstate", 0), "state dimension"),
    (lambda p: setattr(p, "n_groups", 3), "multiple of n_groups"),
    (lambda p: setattr(p, "itype", 7), "itype"),
    (lambda p: setattr(p, "seqlen", -1), "negative"),
    (lambda p: setattr(p, "u", None), "required"),
    (lambda p: setattr(p, "z", 0x2000), "out_z is required"),
    (lambda p: (setattr(p, "out", None)), "no output"),
])
def test_scan_fwd_rejects_invalid_params(mutate, needle):
    lib = capi.load()
    p = _valid_looking_params()
    mutate(p)
    for entry in (lib.mm_scan_fwd, lib.mm_scan_fwd_noalloc):   # same validation, nothing launched
        rc = entry(ctypes.byref(p), None)
        assert rc == capi.MM_ERR_INVALID_ARGUMENT
        assert needle in lib.mm_last_error().decode()


def test_scan_fwd_null_params_and_empty_batch():
    lib = capi.load()
    assert lib.mm_scan_fwd(None, None) == capi.MM_ERR_INVALID_ARGUMENT
    p = _valid_looking_params()
    p.batch = 0          # nothing to do: returns before touching any pointer or the GPU
    assert lib.mm_scan_fwd(ctypes.byref(p), None) == capi.MM_OK


def test_state_update_rejects_invalid_params():
    lib = capi.load()
    assert lib.mm_state_update(None, None) == capi.MM_ERR_INVALID_ARGUMENT
    p = capi.StateUpdateParams()
    p.batch, p.dim, p.dstate, p.n_groups, p.itype = 1, 4, 16, 1, 2
    assert lib.mm_state_update(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "required" in lib.mm_last_error().decode()
    for field in ("state_type", "D_type", "dt_bias_type"):
        setattr(p, field, 5)
        assert lib.mm_state_update(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
        assert "state_type, D_type or dt_bias_type" in lib.mm_last_error().decode()
        setattr(p, field, 0)
    p.dstate = 300
    assert lib.mm_state_update(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT


def test_binding_checks_mirror_reference():
    """TORCH_CHECK failures raise RuntimeError like selective_scan.cpp:280-381 (CPU tensors fail
    the is_cuda check before anything is launched)."""
    from motif_mamba_amd import _native
    ext = _native.ext()
    u = torch.zeros(1, 4, 8)
    A = -torch.ones(4, 16)
    B = torch.zeros(1, 1, 16, 8)
    with pytest.raises(RuntimeError):
        ext.fwd(u, u, A, B, B)
    with pytest.raises(RuntimeError):
        ext.fwd(u.to(torch.int32), u, A, B, B)
    with pytest.raises(RuntimeError):
        ext.fwd(u, u, A, B, B, P=torch.zeros(16, 2), Q=torch.zeros(2, 16))
    with pytest.raises(RuntimeError):
        ext.state_update(torch.zeros(1, 4, 16), u[:, :, 0], u[:, :, 0], A, B[:, 0, :, 0], B[:, 0, :, 0])


def test_python_api_pq_argument_errors():
    """The argument errors of selective_scan_full_matrix_cuda (ssi.py:266-271, 303-318), raised
    before anything reaches the GPU."""
    from motif_mamba_amd import selective_scan_fn
    u = torch.zeros(1, 4, 8)
    A = -torch.ones(4, 16)
    B = torch.zeros(1, 16, 8)
    with pytest.raises(ValueError, match="both be provided"):
        selective_scan_fn(u, u, A, B, B, P=torch.zeros(16, 2))
    with pytest.raises(ValueError, match="both be provided"):
        selective_scan_fn(u, u, A, B, B, gamma=torch.zeros(16))
    with pytest.raises(NotImplementedError):
        selective_scan_fn(u, u, A.to(torch.complex64), B, B, P=torch.zeros(16, 2), Q=torch.zeros(2, 16))
    with pytest.raises(ValueError, match="CUDA"):
        selective_scan_fn(u, u, A, B, B, P=torch.zeros(16, 2), Q=torch.zeros(2, 16))


def test_scan_fwd_rejects_invalid_pq_params():
    lib = capi.load()
    p = _valid_looking_params()
    p.P = 0x3000
    assert lib.mm_scan_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "P and Q" in lib.mm_last_error().decode()
    p.Q, p.pq_rank = 0x4000, 9
    assert lib.mm_scan_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "pq_rank" in lib.mm_last_error().decode()
    p.pq_rank = 2
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(p)) == 0   # the P/Q kernels use no scratch


def test_mamba_ssm_import_paths_resolve_to_hip_kernels():
    import mamba_ssm.ops.selective_scan_interface as ssi
    import mamba_ssm.ops.triton.selective_state_update as ssu
    import motif_mamba_amd
    assert ssi.selective_scan_fn is motif_mamba_amd.selective_scan_fn
    assert ssi.SelectiveScanFn is motif_mamba_amd.SelectiveScanFn
    assert ssu.selective_state_update is motif_mamba_amd.selective_state_update


def test_workspace_size_query():
    """mm_scan_fwd_workspace_size reads sizes, flags and strides only (fake pointers are never
    dereferenced): segments for few channel groups and long sequences, none otherwise."""
    lib = capi.load()

    def params(batch, dim, L, N=16, itype=2):
        p = capi.ScanFwdParams()
        p.batch, p.dim, p.seqlen, p.dstate, p.n_groups = batch, dim, L, N, 1
        p.itype, p.is_variable_B, p.is_variable_C, p.delta_softplus = itype, 1, 1, 1
        p.u = p.delta = p.A = p.B = p.C = p.z = p.out_z = 4096
        p.u_batch_stride = p.delta_batch_stride = p.z_batch_stride = p.out_z_batch_stride = dim * L
        p.u_d_stride = p.delta_d_stride = p.z_d_stride = p.out_z_d_stride = L
        p.A_d_stride, p.A_dstate_stride = N, 1
        p.B_batch_stride = p.C_batch_stride = p.B_group_stride = p.C_group_stride = N * L
        p.B_dstate_stride = p.C_dstate_stride = L
        return p

    seg = lib.mm_scan_fwd_workspace_size(ctypes.byref(params(1, 2560, 65536, itype=0)))
    assert seg > 0 and seg % (1 * 2560 * 18 * 4) == 0           # config 3: segmented
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(params(4, 5120, 4096))) == 0   # config 2: one pass
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(params(1, 64, 256))) == 0      # too short to split
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(params(1, 64, 8192, N=32))) == 0  # not dstate 16
    bad = params(1, 64, 8192)
    bad.dstate = 0
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(bad)) == 0                      # invalid request
    assert lib.mm_scan_fwd_workspace_size(None) == 0
    odd = params(1, 2560, 65536, itype=0)
    odd.u = 4098                         # rows not 16-byte aligned: the row-per-lane kernel, no segments
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(odd)) == 0


def test_tile_states_size_query(monkeypatch):
    """mm_scan_fwd_tile_states_size (sizes, flags, strides and pointer alignment only; fake pointers
    are never dereferenced): the training forward of the dstate-16 kernels, the diagonal training
    forward below dstate 16 (the P/Q kernels with a zero coupling) and every P/Q request with
    dstate <= 16 write them; other requests do not."""
    lib = capi.load()

    def params(batch, dim, L, N=16, chunks=True, pq=False):
        p = capi.ScanFwdParams()
        p.batch, p.dim, p.seqlen, p.dstate, p.n_groups = batch, dim, L, N, 1
        p.itype, p.is_variable_B, p.is_variable_C, p.delta_softplus = 2, 1, 1, 1
        p.u = p.delta = p.A = p.B = p.C = p.z = p.out_z = p.out = 4096
        p.u_batch_stride = p.delta_batch_stride = p.z_batch_stride = p.out_z_batch_stride = dim * L
        p.out_batch_stride = dim * L
        p.u_d_stride = p.delta_d_stride = p.z_d_stride = p.out_z_d_stride = p.out_d_stride = L
        p.A_d_stride, p.A_dstate_stride = N, 1
        p.B_batch_stride = p.C_batch_stride = p.B_group_stride = p.C_group_stride = N * L
        p.B_dstate_stride = p.C_dstate_stride = L
        if chunks:
            p.chunk_states = 8192
        if pq:
            p.P, p.Q, p.pq_rank = 8192, 16384, 2
            p.P_dstate_stride, p.P_r_stride, p.Q_r_stride, p.Q_dstate_stride = 2, 1, N, 1
        return p

    size = lambda p: lib.mm_scan_fwd_tile_states_size(ctypes.byref(p))   # noqa: E731
    assert size(params(4, 5120, 4096)) == 256 * 4 * 5120 * 16 * 4           # config 2 training forward
    assert size(params(2, 64, 200)) == 13 * 2 * 64 * 16 * 4                 # ragged last tile
    assert size(params(4, 5120, 4096, chunks=False)) == 0                  # the inference forward
    assert size(params(2, 64, 256, N=8)) == 16 * 2 * 64 * 16 * 4           # zero-coupling P/Q kernels
    monkeypatch.setenv("MM_DIAG_VIA_PQ", "0")
    assert size(params(2, 64, 256, N=8)) == 0                              # that route off: none
    monkeypatch.delenv("MM_DIAG_VIA_PQ")
    assert size(params(2, 64, 100)) == 0                                   # L % 8 != 0
    assert size(params(2, 64, 256, N=8, chunks=False, pq=True)) == 16 * 2 * 64 * 16 * 4   # P/Q
    assert size(params(2, 64, 256, N=32, pq=True)) == 0                    # P/Q, dstate > 16
    assert lib.mm_scan_fwd_tile_states_size(None) == 0
    # A diagonal request the kernels cannot serve is refused when tile states are asked for.
    monkeypatch.setenv("MM_DIAG_VIA_PQ", "0")
    p = params(2, 64, 256, N=8)
    p.tile_states = 32768
    assert lib.mm_scan_fwd(ctypes.byref(p), None) == capi.MM_ERR_UNSUPPORTED
    monkeypatch.delenv("MM_DIAG_VIA_PQ")
    p = params(2, 64, 256, chunks=False)
    p.tile_states = 32768
    assert lib.mm_scan_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT


def test_scan_bwd_rejects_invalid_params():
    """Validation of mm_scan_bwd happens before anything is launched (fake pointers)."""
    lib = capi.load()
    assert lib.mm_scan_bwd(None, None) == capi.MM_ERR_INVALID_ARGUMENT
    p = capi.ScanBwdParams()
    p.batch, p.dim, p.seqlen, p.dstate, p.n_groups, p.itype = 2, 8, 64, 16, 1, 2
    p.is_variable_B = p.is_variable_C = 1
    fake = 0x1000
    p.u = p.delta = p.A = p.B = p.C = p.dout = fake
    assert lib.mm_scan_bwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "du, ddelta" in lib.mm_last_error().decode()
    p.du = p.ddelta = p.dA = p.dB = p.dC = fake
    p.z = fake
    assert lib.mm_scan_bwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "out and dz" in lib.mm_last_error().decode()
    p.z = None
    p.D = fake
    assert lib.mm_scan_bwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "dD" in lib.mm_last_error().decode()
    p.D = None
    need = lib.mm_scan_bwd_workspace_size(ctypes.byref(p))
    assert need == 2 * 8 * (64 // 16) * 16 * 4                     # one float per state per 16-step tile
    assert lib.mm_scan_bwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "workspace" in lib.mm_last_error().decode()
    p.dstate = 300
    assert lib.mm_scan_bwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert lib.mm_scan_bwd_workspace_size(ctypes.byref(p)) == 0
    p.dstate = 16
    for groups in (0, -1, 3):   # no groups, or dim (8) not a multiple of them: size 0, call refused
        p.n_groups = groups
        assert lib.mm_scan_bwd_workspace_size(ctypes.byref(p)) == 0
        assert lib.mm_scan_bwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
        assert "n_groups" in lib.mm_last_error().decode()
    p.n_groups = 1
    p.batch = 0   # nothing to do: returns before touching any pointer or the GPU
    assert lib.mm_scan_bwd(ctypes.byref(p), None) == capi.MM_OK


def test_conv1d_rejects_invalid_params():
    lib = capi.load()
    assert lib.mm_causal_conv1d_fwd(None, None) == capi.MM_ERR_INVALID_ARGUMENT
    p = capi.Conv1dFwdParams()
    p.batch, p.dim, p.seqlen, p.width, p.itype, p.wtype = 2, 8, 16, 4, 2, 2
    assert lib.mm_causal_conv1d_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "required" in lib.mm_last_error().decode()
    p.width = 9
    assert lib.mm_causal_conv1d_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "width" in lib.mm_last_error().decode()
    p.width, p.wtype = 4, 7
    assert lib.mm_causal_conv1d_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    q = capi.Conv1dUpdateParams()
    q.batch, q.dim, q.seqlen, q.width, q.state_len = 2, 8, 1, 4, 2
    q.x = q.conv_state = q.weight = q.out = 0x1000
    assert lib.mm_causal_conv1d_update(ctypes.byref(q), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "state_len" in lib.mm_last_error().decode()
    q.batch = 0
    q.state_len = 4
    assert lib.mm_causal_conv1d_update(ctypes.byref(q), None) == capi.MM_OK
    assert lib.mm_causal_conv1d_bwd(None, None) == capi.MM_ERR_INVALID_ARGUMENT
    r = capi.Conv1dBwdParams()
    r.batch, r.dim, r.seqlen, r.width, r.itype, r.wtype = 2, 8, 16, 4, 2, 2
    r.x = r.dout = r.dx = r.weight = r.dweight = 0x1000
    r.bias = 0x1000                      # bias without dbias
    assert lib.mm_causal_conv1d_bwd(ctypes.byref(r), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "dbias" in lib.mm_last_error().decode()
    r.bias, r.x = None, None
    assert lib.mm_causal_conv1d_bwd(ctypes.byref(r), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "required" in lib.mm_last_error().decode()
    r.x, r.width = 0x1000, 0
    assert lib.mm_causal_conv1d_bwd(ctypes.byref(r), None) == capi.MM_ERR_INVALID_ARGUMENT
    r.width, r.dim = 4, 1 << 24          # one 256-lane workgroup per channel: the grid's lanes reach 2^32
    assert lib.mm_causal_conv1d_bwd(ctypes.byref(r), None) == capi.MM_ERR_UNSUPPORTED
    assert "2^24" in lib.mm_last_error().decode()
    r.dim = 0                            # nothing to write: returns before any launch
    assert lib.mm_causal_conv1d_bwd(ctypes.byref(r), None) == capi.MM_OK


def test_rms_norm_rejects_invalid_params():
    lib = capi.load()
    assert lib.mm_rms_norm_fwd(None, None) == capi.MM_ERR_INVALID_ARGUMENT
    p = capi.RmsNormParams()
    p.n0, p.cols, p.n2, p.itype, p.wtype, p.eps = 2, 16, 64, 2, 0, 1e-6
    assert lib.mm_rms_norm_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    assert "required" in lib.mm_last_error().decode()
    p.x = p.weight = p.out = 0x1000
    p.eps = -1.0
    assert lib.mm_rms_norm_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    p.eps, p.itype = 1e-6, 9
    assert lib.mm_rms_norm_fwd(ctypes.byref(p), None) == capi.MM_ERR_INVALID_ARGUMENT
    p.itype, p.n2 = 2, 0
    assert lib.mm_rms_norm_fwd(ctypes.byref(p), None) == capi.MM_OK


def test_causal_conv1d_import_paths_and_argument_errors():
    import causal_conv1d
    import causal_conv1d.cpp_functions as cf
    import motif_mamba_amd
    assert causal_conv1d.causal_conv1d_fn is motif_mamba_amd.causal_conv1d_fn
    assert causal_conv1d.causal_conv1d_update is motif_mamba_amd.causal_conv1d_update
    x = torch.zeros(1, 4, 8)
    w = torch.zeros(4, 4)
    with pytest.raises(NotImplementedError):
        causal_conv1d.causal_conv1d_fn(x, w, activation="relu")
    with pytest.raises(NotImplementedError):
        causal_conv1d.causal_conv1d_fn(x, w, seq_idx=torch.zeros(1, 8, dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        cf.causal_conv1d_bwd_function(x, w, None, x, torch.zeros(1, 8, dtype=torch.int32), None, None, None,
                                      False, True)
    with pytest.raises(RuntimeError):       # CPU tensors are refused by the binding
        causal_conv1d.causal_conv1d_fn(x, w)
