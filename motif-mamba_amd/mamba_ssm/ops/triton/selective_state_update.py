"""``mamba_ssm.ops.triton.selective_state_update`` import path (the name Mambamotif imports at
mamba_ssm/modules/mamba_simplemotif.py:21), served by the gfx950 HIP decode kernel. Despite the
module path, nothing here is Triton."""
from motif_mamba_amd.state_update import selective_state_update

__all__ = ["selective_state_update"]
