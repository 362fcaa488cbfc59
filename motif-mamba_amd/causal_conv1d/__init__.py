"""``causal_conv1d`` names the reference imports (mamba_simplemotif.py:16-19), served by the gfx950
kernels of motif_mamba_amd (the third-party package itself is not part of this build)."""
from motif_mamba_amd.causal_conv1d import causal_conv1d_fn, causal_conv1d_update

__all__ = ["causal_conv1d_fn", "causal_conv1d_update"]
