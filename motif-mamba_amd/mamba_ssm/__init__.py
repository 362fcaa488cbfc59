"""Import-path shim: ``mamba_ssm`` names resolved to the MI355X selective-scan kernels.

Only the hot-path modules are provided: ``mamba_ssm.ops.selective_scan_interface`` and
``mamba_ssm.ops.triton.selective_state_update`` (the path the reference's Mambamotif imports at
mamba_ssm/modules/mamba_simplemotif.py:20-23). Nothing here is Triton.
"""
__version__ = "2.2.6.post3+mi355x"
