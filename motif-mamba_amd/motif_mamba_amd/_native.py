"""Loader of the native parts: ``libmm_scan.so`` (C ABI) and the ``mm_scan_torch`` binding.

Both must have been built (``python -m motif_mamba_amd._build`` or ``__graft_entry__.build()``).
There is no fallback: a missing or stale library raises, so no call can silently run anything
but the gfx950 kernels. torch is imported first so that the HIP runtime already loaded by
torch (same SONAME ``libamdhip64.so.7``) is the one the library binds to.
"""
from __future__ import annotations

import ctypes
import importlib.machinery
import importlib.util
import os

import torch  # noqa: F401  (must precede loading libmm_scan.so, see module docstring)

from ._build import EXT_NAME, LIB_NAME, PKG_DIR, ext_filename

ABI_VERSION = 10

_lib = None
_ext = None


class NativeLibraryMissing(ImportError):
    pass


def lib_path() -> str:
    return os.path.join(PKG_DIR, LIB_NAME)


def ext_path() -> str:
    return os.path.join(PKG_DIR, ext_filename())


def lib() -> ctypes.CDLL:
    """The C ABI library (ctypes handle)."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise NativeLibraryMissing(
                f"{path} is missing: build it with `python -m motif_mamba_amd._build` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        handle = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        handle.mm_abi_version.restype = ctypes.c_int
        got = handle.mm_abi_version()
        if got != ABI_VERSION:
            raise NativeLibraryMissing(f"{path} has ABI version {got}, expected {ABI_VERSION}; rebuild it")
        handle.mm_last_error.restype = ctypes.c_char_p
        _lib = handle
    return _lib


def ext():
    """The PyTorch-ROCm binding module (fwd, fwd_infer, state_update)."""
    global _ext
    if _ext is None:
        lib()  # loads libmm_scan.so first (RTLD_GLOBAL) and checks its ABI version
        path = ext_path()
        if not os.path.exists(path):
            raise NativeLibraryMissing(
                f"{path} is missing: build it with `python -m motif_mamba_amd._build`; "
                "there is no non-HIP fallback")
        loader = importlib.machinery.ExtensionFileLoader(EXT_NAME, path)
        spec = importlib.util.spec_from_file_location(EXT_NAME, path, loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        if mod.abi_version() != ABI_VERSION:
            raise NativeLibraryMissing(f"{path} was built against another ABI version; rebuild it")
        _ext = mod
    return _ext
