"""Build recipe for the native parts of motif_mamba_amd (gfx950 only).

* ``libmm_scan.so``      -- the HIP kernels and the C ABI (include/mm_scan.h), built with hipcc.
* ``mm_scan_torch*.so``  -- the PyTorch-ROCm binding (pybind), built with g++ against torch's
                            headers and linked to ``libmm_scan.so`` through an $ORIGIN rpath.
* ``libmm_probe.so``     -- instruction-issue probes (csrc/mm_probe.hip) that bench.py runs to
                            measure the transcendental and VALU issue rates behind its rooflines;
                            not part of the scan library.

Both land next to this file so they travel with the source tree. ``build()`` always recompiles.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
import time

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SRC_ROOT = os.path.dirname(PKG_DIR)                      # .../motif-mamba_amd
CSRC = os.path.join(SRC_ROOT, "csrc")
REPO = os.path.dirname(SRC_ROOT)
INCLUDE = os.path.join(REPO, "include")
LIB_NAME = "libmm_scan.so"
PROBE_NAME = "libmm_probe.so"
EXT_NAME = "mm_scan_torch"
ARCH = "gfx950"

# mm_scan_tiled_{f16,bf16}.hip include mm_scan_tiled.hip for their input type (parallel builds).
HIP_SOURCES = ["mm_scan.hip", "mm_scan_tiled.hip", "mm_scan_tiled_f16.hip", "mm_scan_tiled_bf16.hip",
               "mm_scan_pq.hip", "mm_scan_bwd.hip", "mm_scan_pq_bwd.hip", "mm_conv1d.hip", "mm_norm.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed fp32 VALU ops are disabled: the compiler would otherwise form v_pk_{add,mul,fma}_f32
# from scalar float code, and those have given silent wrong results on these GPUs.
HIP_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-cuda-compat", f"-I{INCLUDE}", f"-I{CSRC}"]


def ext_filename() -> str:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return EXT_NAME + suffix


def _run_parallel(cmds, verbose):
    procs = []
    for cmd in cmds:
        if verbose:
            print("[build]", " ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for cmd, pr in procs:
        out, _ = pr.communicate()
        text = out.decode(errors="replace")
        # hipcc's host pass does not know the packed-fp32 target feature; that warning is noise.
        lines = [l for l in text.splitlines() if "packed-fp32-ops" not in l]
        if pr.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        elif verbose and any(l.strip() for l in lines):
            print("\n".join(lines))
    if failed:
        msg = "\n\n".join(f"$ {' '.join(c)}\n{t}" for c, t in failed)
        raise RuntimeError(f"native build failed:\n{msg}")


def build_library(verbose: bool = True) -> str:
    """Compile every .hip source for gfx950 and link libmm_scan.so."""
    objdir = os.path.join(PKG_DIR, "_obj")
    os.makedirs(objdir, exist_ok=True)
    objs, cmds = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    probe = os.path.join(PKG_DIR, PROBE_NAME)
    cmds.append([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, "mm_probe.hip"), "-o", probe + ".tmp"])
    _run_parallel(cmds, verbose)
    os.replace(probe + ".tmp", probe)
    out = os.path.join(PKG_DIR, LIB_NAME)
    tmp = out + ".tmp"
    _run_parallel([[HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]], verbose)
    os.replace(tmp, out)
    return out


def build_torch_binding(verbose: bool = True) -> str:
    """Compile the pybind binding against torch's headers, linked to libmm_scan.so."""
    import torch
    from torch.utils import cpp_extension as ce

    torch_dir = os.path.dirname(torch.__file__)
    incs = ce.include_paths(device_type="cuda") if "device_type" in ce.include_paths.__code__.co_varnames \
        else ce.include_paths(True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = os.path.join(PKG_DIR, ext_filename())
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in incs], f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
           os.path.join(CSRC, "mm_scan_torch.cpp"),
           f"-L{PKG_DIR}", "-lmm_scan",
           f"-L{os.path.join(torch_dir, 'lib')}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           "-lc10_hip", "-ltorch_hip",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(torch_dir, 'lib')}",
           "-o", tmp]
    _run_parallel([cmd], verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = True) -> None:
    t0 = time.time()
    build_library(verbose)
    build_torch_binding(verbose)
    if verbose:
        print(f"[build] native parts built in {time.time() - t0:.1f}s", flush=True)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
