"""GPU checks of mm_scan_fwd_noalloc, the forward entry point that allocates nothing (its
sequence-segment scratch is a static device array): through the C ABI, its outputs equal those of
mm_scan_fwd given a caller-allocated workspace, bit for bit (the same kernels on the same inputs),
on two calls in a row, the second with a smaller input, on shapes that take the segmented path;
and on a shape that needs no scratch. The forward's own parity against the oracle is covered by
test_gpu_scan.py."""
import ctypes
import sys

import pytest
import torch

from tests import capi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(f"\n[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _inputs(seed, batch, dim, L, dtype, G=1):
    g = torch.Generator().manual_seed(seed)
    u, delta, z = (torch.randn(batch, dim, L, generator=g).to(dtype).to(DEV) for _ in range(3))
    B, C = (torch.randn(batch, G, 16, L, generator=g).to(dtype).to(DEV) for _ in range(2))
    A = (-torch.arange(1, 17, dtype=torch.float32).repeat(dim, 1) * (0.5 + torch.rand(dim, 1, generator=g))).to(DEV)
    D = torch.randn(dim, generator=g).to(DEV)
    bias = (torch.rand(dim, generator=g) - 4.0).to(DEV)
    return u, delta, A, B, C, D, z, bias


def _run(entry, lib, inp, workspace=None):
    u, delta, A, B, C, D, z, bias = inp
    out_z = torch.full_like(z, float("nan"))
    last = torch.full((u.shape[0], u.shape[1], 16), float("nan"), device=DEV)
    p = capi.scan_fwd_params(u, delta, A, B, C, D, z, bias, True, out_z=out_z, last_state=last, workspace=workspace)
    rc = entry(ctypes.byref(p), capi.stream_handle())
    assert rc == 0, lib.mm_last_error().decode()
    return out_z, last, p


# (batch, dim, L, dtype, groups): few (batch, 16-channel) groups and long sequences, so that the
# dstate-16 forward cuts the sequence into segments; the second of each pair is smaller. The third
# pair is BASELINE config 3 (G = 4), whose 16-segment plan needs 2,949,120 bytes of scratch.
PAIRS = [((1, 256, 8192, torch.bfloat16, 1), (1, 128, 4096, torch.bfloat16, 1)),
         ((1, 160, 16384, torch.float32, 2), (2, 32, 2048, torch.float32, 1)),
         ((1, 2560, 65536, torch.float32, 4), (1, 1280, 65536, torch.float32, 1))]


@pytest.mark.parametrize("pair", PAIRS, ids=["bf16", "fp32", "cfg3"])
def test_noalloc_matches_workspace_entry(pair):
    lib = capi.load()
    for i, (batch, dim, L, dtype, G) in enumerate(pair):
        _say(f"mm_scan_fwd_noalloc call {i}: batch {batch} dim {dim} L {L} {dtype} G {G}")
        inp = _inputs(30 + i, batch, dim, L, dtype, G)
        got_z, got_last, p = _run(lib.mm_scan_fwd_noalloc, lib, inp)
        need = lib.mm_scan_fwd_workspace_size(ctypes.byref(p))
        assert 0 < need <= 4 << 20, need          # the shape takes the segmented path
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        exp_z, exp_last, _ = _run(lib.mm_scan_fwd, lib, inp, workspace=ws)
        torch.cuda.synchronize()
        assert torch.isfinite(got_z.float()).all() and torch.isfinite(got_last).all()
        assert torch.equal(got_z, exp_z), f"call {i}: out_z differs from mm_scan_fwd's"
        assert torch.equal(got_last, exp_last), f"call {i}: last_state differs from mm_scan_fwd's"


def test_noalloc_without_scratch():
    """A shape the single-pass kernel serves (no scratch needed), after the segmented calls."""
    lib = capi.load()
    _say("mm_scan_fwd_noalloc without scratch: batch 2 dim 64 L 128")
    inp = _inputs(40, 2, 64, 128, torch.float32)
    got_z, got_last, p = _run(lib.mm_scan_fwd_noalloc, lib, inp)
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(p)) == 0
    exp_z, exp_last, _ = _run(lib.mm_scan_fwd, lib, inp)
    torch.cuda.synchronize()
    assert torch.equal(got_z, exp_z) and torch.equal(got_last, exp_last)


def test_noalloc_plan_larger_than_scratch(monkeypatch):
    """A segment plan that needs more than the static scratch (forced here with MM_SCAN_SEGMENTS,
    which the library reads on every call) runs the single-pass kernels: the outputs equal those of
    mm_scan_fwd given no workspace."""
    lib = capi.load()
    monkeypatch.setenv("MM_SCAN_SEGMENTS", "64")
    _say("mm_scan_fwd_noalloc with a forced 64-segment plan: batch 1 dim 1024 L 65536 fp32")
    inp = _inputs(50, 1, 1024, 65536, torch.float32)
    got_z, got_last, p = _run(lib.mm_scan_fwd_noalloc, lib, inp)
    assert lib.mm_scan_fwd_workspace_size(ctypes.byref(p)) > 4 << 20
    exp_z, exp_last, _ = _run(lib.mm_scan_fwd, lib, inp)
    torch.cuda.synchronize()
    assert torch.isfinite(got_z.float()).all() and torch.isfinite(got_last).all()
    assert torch.equal(got_z, exp_z) and torch.equal(got_last, exp_last)
