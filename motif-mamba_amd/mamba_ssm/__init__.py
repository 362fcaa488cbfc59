"""Import-path shim: ``mamba_ssm`` names resolved to the MI355X selective-scan kernels.

Only the hot-path modules are provided: ``mamba_ssm.ops.selective_scan_interface`` and
``mamba_ssm.ops.triton.selective_state_update`` (the path the reference's Mambamotif imports at
mamba_ssm/modules/mamba_simplemotif.py:13, :20-23), and the two top-level names of the reference's
mamba_ssm/__init__.py:3. Nothing here is Triton.
"""
__version__ = "2.2.6.post3+mi355x"

from mamba_ssm.ops.selective_scan_interface import mamba_inner_fn, selective_scan_fn  # noqa: E402,F401
