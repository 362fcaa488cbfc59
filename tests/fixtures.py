"""Loader of the golden fixtures in tests/golden/ (written by tests/golden/make_golden.py)."""
import glob
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def names():
    return sorted(os.path.splitext(os.path.basename(p))[0] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))


def load(name):
    """Returns (inputs, expected): inputs are the selective_scan_fn kwargs as torch CPU tensors
    in their original dtypes; expected has out (input dtype), last_state, out64, last64."""
    f = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    inputs = {}
    for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"):
        if k in f:
            inputs[k] = torch.from_numpy(f[k]).to(_DT[str(f[k + "__dtype"])])
        else:
            inputs[k] = None
    inputs["delta_softplus"] = bool(f["delta_softplus"])
    expected = {
        "out": torch.from_numpy(f["out"]).to(_DT[str(f["out__dtype"])]),
        "last_state": torch.from_numpy(f["last_state"]),
        "out64": torch.from_numpy(f["out64"]),
        "last64": torch.from_numpy(f["last64"]),
    }
    return inputs, expected


def tolerances(dtype):
    """north_star tolerances: fp32 rtol 1e-4 / atol 1e-5; 16-bit inputs rtol 3e-2 / atol 5e-2."""
    return (1e-4, 1e-5) if dtype == torch.float32 else (3e-2, 5e-2)
