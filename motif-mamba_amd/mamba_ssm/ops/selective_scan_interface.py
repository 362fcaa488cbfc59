"""``mamba_ssm.ops.selective_scan_interface`` hot-path names, served by the gfx950 kernels
(reference mamba_ssm/ops/selective_scan_interface.py:24-61, 93-150, 237-259, 262-350, 454-656)."""
from motif_mamba_amd.mamba_inner import MambaInnerFn, mamba_inner_fn
from motif_mamba_amd.selective_scan import SelectiveScanFn, SelectiveScanPQFn, selective_scan_fn

__all__ = ["SelectiveScanFn", "SelectiveScanPQFn", "selective_scan_fn", "MambaInnerFn", "mamba_inner_fn"]
