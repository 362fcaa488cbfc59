"""motif_mamba_amd -- MI355X (gfx950) selective-scan hot path of Motif-Mamba.

Public API (drop-in for the reference's):
  selective_scan_fn, SelectiveScanFn   (mamba_ssm/ops/selective_scan_interface.py:24-61, 237-259)
  SelectiveScanPQFn                    (selective_scan_interface.py:93-150, forward; with z too)
  selective_state_update               (upstream mamba_ssm.ops.triton.selective_state_update)
  causal_conv1d_fn, causal_conv1d_update (package causal-conv1d, mamba_simplemotif.py:16-19)
  mamba_inner_fn, MambaInnerFn         (selective_scan_interface.py:454-656)
"""
from .selective_scan import SelectiveScanFn, SelectiveScanPQFn, selective_scan_fn
from .causal_conv1d import causal_conv1d_fn, causal_conv1d_update
from .state_update import selective_state_update
from .mamba_inner import MambaInnerFn, mamba_inner_fn

__all__ = ["SelectiveScanFn", "SelectiveScanPQFn", "selective_scan_fn", "selective_state_update",
           "causal_conv1d_fn", "causal_conv1d_update", "MambaInnerFn", "mamba_inner_fn"]
