"""Writes the golden fixtures of tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no golden vectors or tests, so the fixtures are produced by this repo's CPU
oracle -- the torch restatement of ``selective_scan_ref`` (reference
mamba_ssm/ops/selective_scan_interface.py:353-451) -- and cross-checked, before writing, against
the float64 C restatement (oracle/scan_f64.c); both are pinned by tests/test_oracle.py.

Each fixture is an .npz (no pickles) holding the inputs exactly as fed to the kernels, the
flags, and the expected outputs: ``out`` (out_z when z is present), ``last_state`` and the float64
``out64`` / ``last64`` from the C restatement.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.join(REPO, "motif-mamba_amd")]

from motif_mamba_amd.workloads import SCAN_CONFIGS, scan_inputs  # noqa: E402
from oracle import cscan  # noqa: E402
from oracle.ssm_ref import selective_scan_ref  # noqa: E402


def _edge_case(seed, batch, dim, L, N, G, dtype, bkind, with_D=True, with_z=True, with_bias=True,
               softplus=True):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, L, generator=g).to(dtype)
    delta = torch.randn(batch, dim, L, generator=g)
    z = torch.randn(batch, dim, L, generator=g).to(dtype) if with_z else None
    lo, hi = np.log(1e-3), np.log(1e-1)
    bias = (torch.rand(dim, generator=g) * (hi - lo) + lo).float() if with_bias else None
    if not softplus:
        # the raw step size is used: keep it non-negative, as callers without softplus do
        delta = delta.abs() * 0.1
        if bias is not None:
            bias = bias.exp()
    delta = delta.to(dtype)
    if bkind == "4d":
        B = torch.randn(batch, G, N, L, generator=g).to(dtype)
        C = torch.randn(batch, G, N, L, generator=g).to(dtype)
    elif bkind == "3d":
        B = torch.randn(batch, N, L, generator=g).to(dtype)
        C = torch.randn(batch, N, L, generator=g).to(dtype)
    else:  # constant (dim, N) float32
        B = torch.randn(dim, N, generator=g)
        C = torch.randn(dim, N, generator=g)
    A = -torch.rand(dim, N, generator=g) * 4 - 0.05
    D = torch.randn(dim, generator=g) if with_D else None
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=bias, delta_softplus=softplus)


CASES = {
    "edge_L1_fp32": lambda: _edge_case(101, 2, 8, 1, 16, 1, torch.float32, "3d"),
    "edge_L7_ragged_bf16": lambda: _edge_case(102, 2, 8, 7, 16, 1, torch.bfloat16, "3d"),
    "edge_L2049_chunk_fp32": lambda: _edge_case(103, 1, 4, 2049, 16, 1, torch.float32, "3d"),
    "edge_G2_4d_fp16": lambda: _edge_case(104, 2, 8, 40, 16, 2, torch.float16, "4d"),
    "edge_constBC_noz_fp32": lambda: _edge_case(105, 2, 8, 33, 8, 1, torch.float32, "const", with_z=False),
    "edge_noD_nobias_nosoftplus_bf16": lambda: _edge_case(106, 2, 8, 24, 16, 1, torch.bfloat16, "3d",
                                                          with_D=False, with_bias=False, softplus=False),
    "edge_N64_fp32": lambda: _edge_case(107, 1, 4, 20, 64, 1, torch.float32, "3d"),
}


def _save(name, case):
    out, last = selective_scan_ref(**case, return_last_state=True)
    r = cscan.scan_rows(**case)
    key = "out_z" if case["z"] is not None else "out"
    ref64 = r[key].reshape(out.shape)
    # the float32 oracle must agree with the float64 restatement before anything is written
    tol = 1e-4 if case["u"].dtype == torch.float32 else 3e-2
    np.testing.assert_allclose(out.double().numpy(), ref64, rtol=tol, atol=tol * 0.1 if tol < 1e-3 else 5e-2)
    arrays = {}
    for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"):
        v = case[k]
        if v is None:
            continue
        arrays[k] = v.float().numpy()
        arrays[k + "__dtype"] = np.array(str(v.dtype).replace("torch.", ""))
    arrays["delta_softplus"] = np.array(bool(case["delta_softplus"]))
    arrays["out"] = out.float().numpy()
    arrays["out__dtype"] = np.array(str(out.dtype).replace("torch.", ""))
    arrays["last_state"] = last.numpy()
    arrays["out64"] = ref64
    arrays["last64"] = r["last_state"].reshape(last.shape)
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def main():
    cscan.build(force=False)
    cfg0 = scan_inputs(SCAN_CONFIGS["cfg0"])
    cfg0.pop("return_last_state")
    _save("cfg0", cfg0)
    for name, mk in CASES.items():
        _save(name, mk())


if __name__ == "__main__":
    main()
