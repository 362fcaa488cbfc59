"""Seeded synthetic inputs for the benchmark configurations of the selective-scan hot path.

Every tensor is drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in a fixed order,
cast to its dtype, and only then moved to ``device``, so the GPU and any host-side checker see
bit-identical inputs. Distributions (shared by all configs):

* u, z ~ N(0, 1); raw delta ~ N(0, 1)
* delta_bias ~ U(log 1e-3, log 1e-1) per channel, float32
* A = -[1 .. N] for every channel (S4D-real init), float32; D = ones, float32
* input-dependent B, C ~ N(0, 1)

Draw order: u, delta, z, delta_bias, B, C.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

_DT = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


@dataclass(frozen=True)
class ScanConfig:
    name: str
    batch: int
    dim: int
    seqlen: int
    dstate: int = 16
    dtype: str = "bf16"
    n_groups: int = 1
    bc_4d: bool = False      # B/C passed as (batch, G, N, L) instead of (batch, N, L)
    seed: int = 0


# BASELINE.json "configs"; index = config id. Config 3 is listed with both group counts.
SCAN_CONFIGS = {
    "cfg0": ScanConfig("cfg0", 2, 64, 128, 16, "fp32", 1, False, 0),
    "cfg1": ScanConfig("cfg1", 8, 1536, 2048, 16, "bf16", 1, False, 1),
    "cfg2": ScanConfig("cfg2", 4, 5120, 4096, 16, "bf16", 1, False, 2),
    "cfg3_g1": ScanConfig("cfg3_g1", 1, 2560, 65536, 16, "fp32", 1, True, 3),
    "cfg3_g4": ScanConfig("cfg3_g4", 1, 2560, 65536, 16, "fp32", 4, True, 3),
}


def scan_inputs(cfg: ScanConfig, device="cpu", batch=None, dim=None, seqlen=None):
    """Inputs of one selective_scan_fn call for ``cfg`` (optionally with overridden sizes).

    Returns a dict with u, delta, A, B, C, D, z, delta_bias (+ the flags delta_softplus=True,
    return_last_state=True of every config)."""
    batch = cfg.batch if batch is None else batch
    dim = cfg.dim if dim is None else dim
    L = cfg.seqlen if seqlen is None else seqlen
    N, G = cfg.dstate, cfg.n_groups
    dt = _DT[cfg.dtype]
    g = torch.Generator().manual_seed(cfg.seed)
    u = torch.randn(batch, dim, L, generator=g).to(dt)
    delta = torch.randn(batch, dim, L, generator=g).to(dt)
    z = torch.randn(batch, dim, L, generator=g).to(dt)
    lo, hi = math.log(1e-3), math.log(1e-1)
    delta_bias = (torch.rand(dim, generator=g) * (hi - lo) + lo).float()
    if cfg.bc_4d:
        B = torch.randn(batch, G, N, L, generator=g).to(dt)
        C = torch.randn(batch, G, N, L, generator=g).to(dt)
    else:
        B = torch.randn(batch, N, L, generator=g).to(dt)
        C = torch.randn(batch, N, L, generator=g).to(dt)
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(dim, 1).contiguous()
    D = torch.ones(dim, dtype=torch.float32)
    t = dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=delta_bias)
    if device != "cpu":
        t = {k: v.to(device) for k, v in t.items()}
    t.update(delta_softplus=True, return_last_state=True)
    return t


def scan_bytes(batch, dim, seqlen, dstate, n_groups, in_bytes, write_out=False, has_z=True):
    """Algorithmic HBM bytes of one forward scan (each tensor touched once): u, delta, z read and
    out_z written, B and C read, A, D, delta_bias read, last_state written (+ pre-gate out)."""
    per_elem = 3 if has_z else 2
    per_elem += 1  # the output actually written (out_z, or out when there is no z)
    if write_out and has_z:
        per_elem += 1
    return (batch * dim * seqlen * per_elem * in_bytes
            + 2 * batch * n_groups * dstate * seqlen * in_bytes
            + dim * dstate * 4 + 2 * dim * 4 + batch * dim * dstate * 4)


def scan_transcendentals(batch, dim, seqlen, dstate, softplus=True, has_z=True):
    """N exp2 per element for the decay, plus exp+log for softplus and exp+rcp for silu(z)."""
    return batch * dim * seqlen * (dstate + (2 if softplus else 0) + (2 if has_z else 0))


@dataclass(frozen=True)
class DecodeConfig:
    name: str
    batch: int
    dim: int = 5120
    dstate: int = 16
    dtype: str = "bf16"
    steps: int = 1024
    seed: int = 4


DECODE_CONFIGS = {f"cfg4_b{b}": DecodeConfig(f"cfg4_b{b}", b) for b in (1, 64, 256)}


def decode_inputs(cfg: DecodeConfig, device="cpu", steps=None):
    """Initial state ~ N(0, 0.1) (std 0.1) and ``steps`` fresh (x, dt, z, B, C) draws.

    Draw order: state, dt_bias, then per step x, dt, z, B, C."""
    steps = cfg.steps if steps is None else steps
    dt_ = _DT[cfg.dtype]
    g = torch.Generator().manual_seed(cfg.seed)
    Bt, D, N = cfg.batch, cfg.dim, cfg.dstate
    state = (torch.randn(Bt, D, N, generator=g) * 0.1).float()
    lo, hi = math.log(1e-3), math.log(1e-1)
    dt_bias = (torch.rand(D, generator=g) * (hi - lo) + lo).float()
    xs = torch.empty(steps, Bt, D, dtype=dt_)
    dts = torch.empty(steps, Bt, D, dtype=dt_)
    zs = torch.empty(steps, Bt, D, dtype=dt_)
    Bs = torch.empty(steps, Bt, N, dtype=dt_)
    Cs = torch.empty(steps, Bt, N, dtype=dt_)
    for s in range(steps):
        xs[s] = torch.randn(Bt, D, generator=g).to(dt_)
        dts[s] = torch.randn(Bt, D, generator=g).to(dt_)
        zs[s] = torch.randn(Bt, D, generator=g).to(dt_)
        Bs[s] = torch.randn(Bt, N, generator=g).to(dt_)
        Cs[s] = torch.randn(Bt, N, generator=g).to(dt_)
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(D, 1).contiguous()
    Dv = torch.ones(D, dtype=torch.float32)
    t = dict(state=state, x=xs, dt=dts, z=zs, B=Bs, C=Cs, A=A, D=Dv, dt_bias=dt_bias)
    if device != "cpu":
        t = {k: v.to(device) for k, v in t.items()}
    return t


def decode_bytes(batch, dim, dstate, n_groups=1, in_bytes=2):
    """Algorithmic HBM bytes of one decode step: state read+written (f32), x, dt, z read and out
    written, B and C read, A, D, dt_bias read."""
    return (batch * (2 * dim * dstate * 4 + 4 * dim * in_bytes + 2 * n_groups * dstate * in_bytes)
            + dim * dstate * 4 + 2 * dim * 4)


@dataclass(frozen=True)
class PQConfig:
    """A MotifMamba layer with the low-rank P/Q coupling (mamba_simplemotif.py:139-151, 314-332)."""
    name: str
    batch: int
    dim: int
    seqlen: int
    dstate: int = 16
    rank: int = 2
    per_dim: bool = True
    dtype: str = "fp16"
    pq_std: float = 0.1
    seed: int = 5


# Mamba-1.4B (d_model 2048, d_inner 4096, d_state 16), the model train_kpq_motif_pile_lm.py adapts,
# with its defaults: pq_rank 2, per-channel P/Q, float16 activations.
PQ_CONFIGS = {
    "pq_1p4b": PQConfig("pq_1p4b", 4, 4096, 2048),
}


def pq_inputs(cfg: PQConfig, device="cpu"):
    """Inputs of one selective_scan_fn(..., P=P, Q=Q) call as the Motif module makes it (z gate,
    delta_bias + softplus, last state). Draw order: u, delta, z, delta_bias, B, C, P, Q.
    P, Q ~ N(0, pq_std) (the module draws N(0, 1e-2) and scales P by pq_k; a larger spread keeps
    the coupling visible in parity checks and does not change the work)."""
    N, L, R = cfg.dstate, cfg.seqlen, cfg.rank
    dt = _DT[cfg.dtype]
    g = torch.Generator().manual_seed(cfg.seed)
    u = torch.randn(cfg.batch, cfg.dim, L, generator=g).to(dt)
    delta = torch.randn(cfg.batch, cfg.dim, L, generator=g).to(dt)
    z = torch.randn(cfg.batch, cfg.dim, L, generator=g).to(dt)
    lo, hi = math.log(1e-3), math.log(1e-1)
    delta_bias = (torch.rand(cfg.dim, generator=g) * (hi - lo) + lo).float()
    B = torch.randn(cfg.batch, N, L, generator=g).to(dt)
    C = torch.randn(cfg.batch, N, L, generator=g).to(dt)
    shp_p, shp_q = ((cfg.dim, N, R), (cfg.dim, R, N)) if cfg.per_dim else ((N, R), (R, N))
    P = (torch.randn(*shp_p, generator=g) * cfg.pq_std).float()
    Q = (torch.randn(*shp_q, generator=g) * cfg.pq_std).float()
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(cfg.dim, 1).contiguous()
    D = torch.ones(cfg.dim, dtype=torch.float32)
    t = dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z, delta_bias=delta_bias, P=P, Q=Q)
    if device != "cpu":
        t = {k: v.to(device) for k, v in t.items()}
    t.update(delta_softplus=True, return_last_state=True)
    return t


def pq_flops(batch, dim, seqlen, dstate, rank):
    """Multiply-adds of the coupling per step (Q h then P q: 2 N R) as flops, per call."""
    return batch * dim * seqlen * 4 * dstate * rank
