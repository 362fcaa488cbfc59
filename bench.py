#!/usr/bin/env python3
"""Benchmark of the MI355X selective-scan hot path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]``

One "step" is one forward selective scan over BASELINE config 2 (the headline: Mamba-2.8B layer
shape, batch 4, d_inner 5120, L 4096, dstate 16, bf16 in / fp32 accumulate, z gate, delta_bias +
softplus, last state returned), with all inputs resident in HBM before timing starts. ``value``
is the algorithmic HBM throughput of that step (bytes of u, delta, z, B, C, A, D, delta_bias read
and out_z, last_state written, each once) divided by the measured time per step, in GB/s.

The run starts with the issue-rate probes of libmm_probe.so (csrc/mm_probe.hip), which measure the
v_exp_f32 and v_fma_f32 rates of this GPU (and bring it to its loaded clock before anything is
timed). The JSON line carries the forward kernel's rooflines: ``roofline_hbm`` (8 TB/s published
peak), ``roofline_trans`` (the measured v_exp_f32 rate), ``roofline`` = the binding one of those two
(north_star: the larger floor), and ``roofline_issue`` (transcendentals plus the 4 VALU operations
of a state update, at the measured rates); ``cpu_baseline`` (the CPU oracle timed on the host on a
bounded sample of the same workload, and one per other configuration), per-config results for
configs 1 and 3, decode tokens/s for config 4, the MotifMamba P/Q forward on a Mamba-1.4B layer and
the training forward + backward of configs 1 and 2, the causal conv1d that precedes the scan
(forward on the config 1 and 2 shapes, decode update) and the fused Mamba block mamba_inner_fn on
the config-2 tokens of a Mamba-2.8B layer (inference and training; unless --quick).
Only one GPU is used; --gpus N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [REPO, os.path.join(REPO, "motif-mamba_amd")]

HBM_PEAK_GBS = 8000.0
METRIC = "selective-scan fwd GB/s & % of binding roofline; decode tokens/s, 1 GPU"
# Issue rates of this GPU, measured at the start of every run by issue_rates() (libmm_probe.so):
# "trans_per_s" (v_exp_f32 lane operations per second, chip-wide) and "valu_per_s" (v_fma_f32).
RATES = {}


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


RAMP_S = 0.25


def _time_loop(fn, steps, warmup, torch):
    """ms per step of fn over `steps` timed calls after `warmup` untimed ones. Before those, fn runs
    untimed for RAMP_S seconds: an idle MI355X takes ~50 ms of sustained load to reach its loaded
    clocks (config 2 measured 0.88, 0.45, 0.43 then a steady 0.42 ms per step over its first
    batches of 20 calls, and back to 0.50 after a 1 s pause), and a throughput figure is meant to be
    the steady-state one."""
    t0 = time.time()
    i = 0
    while time.time() - t0 < RAMP_S:
        fn(i)
        i += 1
        if i % 4 == 0:
            torch.cuda.synchronize()
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step (events on the launch stream)


def _graph_ms_per_step(step, n_calls, steps, torch):
    """step(0 .. n_calls-1) captured once in a HIP graph and replayed steps / n_calls times: the
    per-call GPU time of a serving loop that does not pay one Python call per token."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n_calls):  # warm the allocator and the binding on the capture stream
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        for i in range(n_calls):
            step(i)
    reps = max(1, steps // n_calls)
    return _time_loop(lambda i: graph.replay(), reps, 2, torch) / n_calls


def bench_scan(cfg_name, steps, warmup, torch, rotate=1):
    from motif_mamba_amd import selective_scan_fn
    from motif_mamba_amd.workloads import SCAN_CONFIGS, scan_bytes, scan_inputs, scan_transcendentals
    c = SCAN_CONFIGS[cfg_name]
    sets = []
    for r in range(rotate):
        cc = c if r == 0 else type(c)(**{**c.__dict__, "seed": c.seed + 100 * r})
        sets.append(scan_inputs(cc, device="cuda"))
    in_bytes = 2 if c.dtype in ("bf16", "fp16") else 4

    def step(i):
        selective_scan_fn(**sets[i % rotate])

    ms = _time_loop(step, steps, warmup, torch)
    nbytes = scan_bytes(c.batch, c.dim, c.seqlen, c.dstate, c.n_groups, in_bytes)
    trans = scan_transcendentals(c.batch, c.dim, c.seqlen, c.dstate)
    elems = c.batch * c.dim * c.seqlen
    del sets
    torch.cuda.empty_cache()
    return {
        "shape": [c.batch, c.dim, c.seqlen, c.dstate], "n_groups": c.n_groups, "dtype": c.dtype,
        "ms": ms, "GB_s": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes,
        "elements_per_s": elems / (ms * 1e-3), "state_updates_per_s": elems * c.dstate / (ms * 1e-3),
        "trans_per_s": trans / (ms * 1e-3), "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        **scan_floors(nbytes, trans, elems * c.dstate, ms), "input_rotation": rotate,
    }


def scan_floors(nbytes, trans, updates, ms):
    """The scan's rooflines at one shape, from the algorithmic work of one call:

    * HBM: nbytes at the published 8 TB/s;
    * transcendental issue: trans (N exp2 per element for the decay, exp + log for softplus,
      exp + rcp for silu) at the v_exp_f32 rate measured on this GPU;
    * VALU + transcendental issue: the same transcendentals plus 4 VALU operations per state update
      (the exp argument, B * delta' u, the state FMA, y += C h) at the v_fma_f32 rate measured on
      this GPU, added because the probes show no co-issue of the two on a SIMD.

    The binding roofline is the larger of the first two (north_star: "HBM bandwidth or exp issue
    rate"); ``binding_frac`` is its floor over the measured time. The issue floor is reported
    beside it as the tighter bound this kernel design can reach."""
    t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
    t_trans = trans / RATES["trans_per_s"]
    t_issue = t_trans + 4 * updates / RATES["valu_per_s"]
    binding = "hbm" if t_hbm >= t_trans else "trans"
    t_bind = max(t_hbm, t_trans)
    t = ms * 1e-3
    return {"t_hbm_us": t_hbm * 1e6, "t_trans_us": t_trans * 1e6, "t_issue_us": t_issue * 1e6,
            "binding": binding, "t_floor_us": t_bind * 1e6, "binding_frac": t_bind / t,
            "issue_frac": t_issue / t}


def bench_decode(batch, steps, warmup, torch, sets_max=64):
    from motif_mamba_amd import selective_state_update
    from motif_mamba_amd.workloads import DECODE_CONFIGS, decode_bytes
    c = DECODE_CONFIGS[f"cfg4_b{batch}"]
    dt = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(c.seed)
    S = min(steps, sets_max)
    state = torch.randn(batch, c.dim, c.dstate, device="cuda", generator=g) * 0.1
    x = torch.randn(S, batch, c.dim, device="cuda", generator=g).to(dt)
    dts = torch.randn(S, batch, c.dim, device="cuda", generator=g).to(dt)
    z = torch.randn(S, batch, c.dim, device="cuda", generator=g).to(dt)
    B = torch.randn(S, batch, c.dstate, device="cuda", generator=g).to(dt)
    C = torch.randn(S, batch, c.dstate, device="cuda", generator=g).to(dt)
    A = -torch.arange(1, c.dstate + 1, dtype=torch.float32, device="cuda").repeat(c.dim, 1).contiguous()
    D = torch.ones(c.dim, device="cuda")
    bias = torch.empty(c.dim, device="cuda").uniform_(-6.907755, -2.302585, generator=g)

    # Per-step views made once, outside the timed region: the step is the decode call alone, as in
    # a decode loop that hands each layer the tensors the previous ops produced (slicing five
    # tensors per step would add ~4 us of Python/ATen indexing to every eager step).
    xs, dtl, zs, Bs, Cs = (list(t.unbind(0)) for t in (x, dts, z, B, C))

    def step(i):
        j = i % S
        selective_state_update(state, xs[j], dtl[j], A, Bs[j], Cs[j], D, zs[j], bias, True)

    ms = _time_loop(step, steps, warmup, torch)
    nbytes = decode_bytes(batch, c.dim, c.dstate)

    gms = _graph_ms_per_step(step, S, steps, torch)
    return {"batch": batch, "dim": c.dim, "dstate": c.dstate, "steps": steps, "us_per_step": ms * 1e3,
            "tokens_per_s": batch / (ms * 1e-3), "GB_s": nbytes / (ms * 1e-3) / 1e9,
            "graph_us_per_step": gms * 1e3, "graph_tokens_per_s": batch / (gms * 1e-3),
            "graph_GB_s": nbytes / (gms * 1e-3) / 1e9,
            "note": "state (batch*5120*16*4 B) fits the 256 MB Infinity Cache; GB/s may exceed HBM peak; "
                    "graph_*: the steps replayed from one captured HIP graph (no per-call host overhead)"}


def bench_pq(name, steps, warmup, torch):
    """Forward of the low-rank coupled scan (selective_scan_fn with P/Q) on a MotifMamba layer."""
    from motif_mamba_amd import selective_scan_fn
    from motif_mamba_amd.workloads import PQ_CONFIGS, pq_flops, pq_inputs, scan_bytes, scan_transcendentals
    c = PQ_CONFIGS[name]
    inputs = pq_inputs(c, device="cuda")

    def step(i):
        selective_scan_fn(**inputs)

    ms = _time_loop(step, steps, warmup, torch)
    in_bytes = 2 if c.dtype in ("bf16", "fp16") else 4
    nbytes = scan_bytes(c.batch, c.dim, c.seqlen, c.dstate, 1, in_bytes) + 2 * c.dim * c.dstate * c.rank * 4
    trans = scan_transcendentals(c.batch, c.dim, c.seqlen, c.dstate)
    flops = pq_flops(c.batch, c.dim, c.seqlen, c.dstate, c.rank)
    elems = c.batch * c.dim * c.seqlen
    floor = max(nbytes / (HBM_PEAK_GBS * 1e9), trans / RATES["trans_per_s"])
    del inputs
    torch.cuda.empty_cache()
    return {"shape": [c.batch, c.dim, c.seqlen, c.dstate], "rank": c.rank, "per_dim": c.per_dim, "dtype": c.dtype,
            "ms": ms, "GB_s": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "elements_per_s": elems / (ms * 1e-3),
            "trans_per_s": trans / (ms * 1e-3), "coupling_TFLOP_s": flops / (ms * 1e-3) / 1e12,
            "t_floor_us": floor * 1e6, "floor_frac": floor / (ms * 1e-3)}


def bench_presets(steps, warmup, torch):
    """Training steps (forward + backward through selective_scan_fn, bf16) at the Motif module's
    "small" and "base" state sizes (d_state 32 and 64, mamba_simplemotif.py:33-35), diagonal and
    with a rank-2 per-channel P/Q pair, batch 8, L 1024, 1,024 / 1,536 channels; synthetic inputs.
    The diagonal backward runs split into groups of 16 states, the P/Q one the general kernel."""
    from motif_mamba_amd import selective_scan_fn
    res = {}
    for kind in ("diag", "pq"):
        for N, dim in ((16, 1024), (32, 1024), (64, 1536)):
            g = torch.Generator(device="cuda").manual_seed(N + dim)
            batch, L = 8, 1024

            def rn(*shape, scale=1.0):
                return (torch.randn(*shape, device="cuda", generator=g) * scale)

            t = dict(u=rn(batch, dim, L).bfloat16(), delta=rn(batch, dim, L).bfloat16(),
                     A=-(torch.rand(dim, N, device="cuda", generator=g) * 8 + 0.05), B=rn(batch, N, L).bfloat16(),
                     C=rn(batch, N, L).bfloat16(), D=rn(dim), z=rn(batch, dim, L).bfloat16(),
                     delta_bias=rn(dim, scale=0.5) - 4.0)
            if kind == "pq":
                t["P"], t["Q"] = rn(dim, N, 2, scale=0.25), rn(dim, 2, N, scale=0.25)
            for v in t.values():
                v.requires_grad_(True)
            dout = rn(batch, dim, L).bfloat16()

            def step(i):
                out = selective_scan_fn(**t, delta_softplus=True)
                out.backward(dout)

            res[f"{kind}_dstate{N}_train_ms"] = _time_loop(step, steps, warmup, torch)
    return res


def bench_pq_train(name, steps, warmup, torch):
    """Training forward and backward of the low-rank coupled scan (P/Q) on a MotifMamba layer, as
    SelectiveScanPQFn runs them: the forward saving pre-gate out, chunk states and the 16-step tile
    states, and the backward (reading those tile states) with dP / dQ."""
    from motif_mamba_amd import _native
    from motif_mamba_amd.workloads import PQ_CONFIGS, pq_inputs
    ext = _native.ext()
    c = PQ_CONFIGS[name]
    t = pq_inputs(c, device="cuda")
    B, C = t["B"].unsqueeze(1), t["C"].unsqueeze(1)
    args = (t["u"], t["delta"], t["A"], B, C, t["D"], t["z"], t["delta_bias"], t["P"], t["Q"], None, True)
    out, x, out_z, ck = ext.fwd(*args, tile_states=True)
    dout = torch.randn(out_z.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(7)).to(out_z.dtype)
    dP, dQ = torch.zeros_like(t["P"]), torch.zeros_like(t["Q"])

    def fwd(i):
        ext.fwd(*args, tile_states=True)

    def bwd(i):
        ext.bwd(*args[:11], dout, x, out, None, dP, dQ, True, False, ck)

    def both(i):
        o, xx, oz, cc = ext.fwd(*args, tile_states=True)
        ext.bwd(*args[:11], dout, xx, o, None, dP, dQ, True, False, cc)

    def bwd_self(i):                   # without the forward's tile states: the backward recomputes them
        ext.bwd(*args[:11], dout, x, out, None, dP, dQ, True, False)

    f_ms = _time_loop(fwd, steps, warmup, torch)
    b_ms = _time_loop(bwd, steps, warmup, torch)
    s_ms = _time_loop(both, steps, warmup, torch)
    bs_ms = _time_loop(bwd_self, steps, warmup, torch)
    elems = c.batch * c.dim * c.seqlen
    del t, out, x, out_z, dout, ck
    torch.cuda.empty_cache()
    return {"shape": [c.batch, c.dim, c.seqlen, c.dstate], "rank": c.rank, "per_dim": c.per_dim, "dtype": c.dtype,
            "fwd_train_ms": f_ms, "bwd_ms": b_ms, "fwd_bwd_ms": s_ms, "bwd_recompute_ms": bs_ms,
            "elements_per_s": elems / (s_ms * 1e-3)}


def bench_pq_layouts(steps, warmup, torch):
    """The P/Q forward at the Motif layer's settings (rank 2, per-channel P/Q, fp16, L 2048) over
    channel counts and batch sizes, with each tiled layout forced through MM_PQ_LPR (lanes per
    channel: 4, 8, 16) and with the host's own choice ("auto"): the measurement behind that
    choice. Milliseconds per call."""
    import dataclasses
    import os
    from motif_mamba_amd import selective_scan_fn
    from motif_mamba_amd.workloads import PQ_CONFIGS, pq_inputs
    base = PQ_CONFIGS["pq_1p4b"]
    grid = [(16, dim, (4, 8, 16)) for dim in (2048, 3072, 4096, 5120)] + [(32, dim, (8, 16)) for dim in (2048, 4096)]
    rows = []
    old = os.environ.get("MM_PQ_LPR")
    try:
        for n, dim, lprs in grid:
            for batch in (1, 2, 3, 4, 6, 8):
                x = pq_inputs(dataclasses.replace(base, batch=batch, dim=dim, dstate=n), device="cuda")
                row = {"dstate": n, "dim": dim, "batch": batch}
                for lpr in (*lprs, None):
                    if lpr:
                        os.environ["MM_PQ_LPR"] = str(lpr)
                    else:
                        os.environ.pop("MM_PQ_LPR", None)
                    row[f"lpr{lpr}" if lpr else "auto"] = _time_loop(lambda i: selective_scan_fn(**x), steps, warmup, torch)
                del x
                torch.cuda.empty_cache()
                _log(f"pq layouts {row}")
                rows.append(row)
    finally:
        if old is None:
            os.environ.pop("MM_PQ_LPR", None)
        else:
            os.environ["MM_PQ_LPR"] = old
    return {"rank": base.rank, "per_dim": base.per_dim, "dtype": base.dtype, "seqlen": base.seqlen, "rows": rows}


def bench_train(cfg_name, steps, warmup, torch):
    """Forward in training mode (pre-gate out and chunk states saved, ssi.py:47-61, plus the 16-step
    tile states SelectiveScanFn keeps) and the backward (selective_scan_cuda.bwd equivalent, reading
    those tile states) on one configuration: times of each and of the pair, and of the backward that
    recomputes the tile states itself."""
    from motif_mamba_amd import _native
    from motif_mamba_amd.workloads import SCAN_CONFIGS, scan_inputs
    ext = _native.ext()
    c = SCAN_CONFIGS[cfg_name]
    t = scan_inputs(c, device="cuda")
    B = t["B"].unsqueeze(1) if t["B"].dim() == 3 else t["B"]
    C = t["C"].unsqueeze(1) if t["C"].dim() == 3 else t["C"]
    args = (t["u"], t["delta"], t["A"], B, C, t["D"], t["z"], t["delta_bias"], None, None, None, True)
    out, x, out_z, ck = ext.fwd(*args, tile_states=True)
    ck_ok = ck is not None
    dout = torch.randn(out_z.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(7)).to(out_z.dtype)

    def fwd(i):
        ext.fwd(*args, tile_states=True)

    def bwd(i):
        ext.bwd(*args[:11], dout, x, out, None, None, None, True, False, ck)

    def both(i):
        o, xx, oz, cc = ext.fwd(*args, tile_states=True)
        ext.bwd(*args[:11], dout, xx, o, None, None, None, True, False, cc)

    def bwd_self(i):                   # without the forward's tile states: the backward recomputes them
        ext.bwd(*args[:11], dout, x, out, None, None, None, True, False)

    f_ms = _time_loop(fwd, steps, warmup, torch)
    b_ms = _time_loop(bwd, steps, warmup, torch)
    s_ms = _time_loop(both, steps, warmup, torch)
    bs_ms = _time_loop(bwd_self, steps, warmup, torch)
    elems = c.batch * c.dim * c.seqlen
    del t, out, x, out_z, dout, ck
    torch.cuda.empty_cache()
    return {"shape": [c.batch, c.dim, c.seqlen, c.dstate], "dtype": c.dtype, "fwd_train_ms": f_ms, "bwd_ms": b_ms,
            "fwd_bwd_ms": s_ms, "bwd_recompute_ms": bs_ms, "tile_states": ck_ok,
            "elements_per_s": elems / (s_ms * 1e-3)}


def bench_conv(cfg_name, steps, warmup, torch):
    """causal_conv1d_fn (width 4, bias, SiLU) on the conv that feeds a scan configuration: HBM
    throughput of x read and out written once."""
    from motif_mamba_amd import causal_conv1d_fn
    from motif_mamba_amd.workloads import SCAN_CONFIGS
    c = SCAN_CONFIGS[cfg_name]
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[c.dtype]
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(c.batch, c.dim, c.seqlen, device="cuda", generator=g).to(dt)
    w = (torch.randn(c.dim, 4, device="cuda", generator=g) * 0.5).to(dt)
    b = (torch.randn(c.dim, device="cuda", generator=g) * 0.1).to(dt)
    ms = _time_loop(lambda i: causal_conv1d_fn(x, w, b, activation="silu"), steps, warmup, torch)
    nbytes = 2 * x.numel() * x.element_size() + w.numel() * w.element_size() + b.numel() * b.element_size()
    del x
    torch.cuda.empty_cache()
    return {"shape": [c.batch, c.dim, c.seqlen], "width": 4, "dtype": c.dtype, "us": ms * 1e3,
            "GB_s": nbytes / (ms * 1e-3) / 1e9, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def bench_conv_bwd(cfg_name, steps, warmup, torch):
    """causal_conv1d's backward (width 4, bias, SiLU: dx, dweight, dbias, as MambaInnerFn's
    backward calls it) on the conv that feeds a scan configuration: HBM throughput of x and dout
    read and dx written once."""
    from motif_mamba_amd.causal_conv1d import causal_conv1d_bwd
    from motif_mamba_amd.workloads import SCAN_CONFIGS
    c = SCAN_CONFIGS[cfg_name]
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[c.dtype]
    g = torch.Generator(device="cuda").manual_seed(13)
    x = torch.randn(c.batch, c.dim, c.seqlen, device="cuda", generator=g).to(dt)
    dout = torch.randn(c.batch, c.dim, c.seqlen, device="cuda", generator=g).to(dt)
    w = (torch.randn(c.dim, 4, device="cuda", generator=g) * 0.5).to(dt)
    b = (torch.randn(c.dim, device="cuda", generator=g) * 0.1).to(dt)
    dx = torch.empty_like(x)
    ms = _time_loop(lambda i: causal_conv1d_bwd(x, w, b, dout, dx, True), steps, warmup, torch)
    nbytes = 3 * x.numel() * x.element_size() + 2 * (w.numel() + b.numel()) * w.element_size()
    del x, dout, dx
    torch.cuda.empty_cache()
    return {"shape": [c.batch, c.dim, c.seqlen], "width": 4, "dtype": c.dtype, "us": ms * 1e3,
            "GB_s": nbytes / (ms * 1e-3) / 1e9, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


def bench_conv_update(batch, steps, warmup, torch, dim=5120):
    """causal_conv1d_update of one decode token (state (batch, dim, 4) bf16, width 4, SiLU)."""
    from motif_mamba_amd import causal_conv1d_update
    g = torch.Generator(device="cuda").manual_seed(12)
    x = torch.randn(batch, dim, device="cuda", generator=g).to(torch.bfloat16)
    st = torch.zeros(batch, dim, 4, device="cuda").to(torch.bfloat16)
    w = (torch.randn(dim, 4, device="cuda", generator=g) * 0.5).to(torch.bfloat16)
    b = (torch.randn(dim, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    step = lambda i: causal_conv1d_update(x, st, w, b, activation="silu")  # noqa: E731
    ms = _time_loop(step, steps, warmup, torch)
    gms = _graph_ms_per_step(step, 64, max(steps, 256), torch)
    nbytes = batch * dim * (2 * 4 * 2 + 2 * 2) + dim * 5 * 2
    return {"batch": batch, "dim": dim, "us_per_step": ms * 1e3, "tokens_per_s": batch / (ms * 1e-3),
            "GB_s": nbytes / (ms * 1e-3) / 1e9, "graph_us_per_step": gms * 1e3,
            "graph_GB_s": nbytes / (gms * 1e-3) / 1e9}


def bench_inner(steps, warmup, torch, batch=4, seqlen=4096, d_model=2560, d_inner=5120, rank=160, d_state=16):
    """mamba_inner_fn (selective_scan_interface.py:454-656) on a Mamba-2.8B layer (bf16 weights and
    activations, float32 A / D / dt bias, conv width 4, checkpoint_lvl 1): the inference forward
    (no gradients), and the training forward + backward with the gradients of every input. The
    projections' GEMM flops are reported with the achieved rate over the whole block."""
    from motif_mamba_amd import mamba_inner_fn
    bf = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(13)

    def r(*shape, sc=1.0, dt=bf, grad=True):
        return (torch.randn(*shape, device="cuda", generator=g) * sc).to(dt).requires_grad_(grad)
    xz = r(batch, 2 * d_inner, seqlen)
    p = [r(d_inner, 1, 4, sc=0.5), r(d_inner, sc=0.1), r(rank + 2 * d_state, d_inner, sc=d_inner ** -0.5),
         r(d_inner, rank, sc=rank ** -0.5), r(d_model, d_inner, sc=d_inner ** -0.5), None,
         (-torch.exp(torch.rand(d_inner, d_state, device="cuda", generator=g) * 2.0)).requires_grad_(True)]
    D = torch.ones(d_inner, device="cuda", requires_grad=True)
    dtb = (torch.rand(d_inner, device="cuda", generator=g) * 2.0 - 4.0).requires_grad_(True)
    dout = torch.randn(batch, seqlen, d_model, device="cuda", generator=g).to(bf)

    def infer(i):
        with torch.no_grad():
            mamba_inner_fn(xz, *p, None, None, D, dtb, delta_softplus=True)

    def train(i):
        for t in [xz, D, dtb] + [q for q in p if q is not None]:
            t.grad = None
        mamba_inner_fn(xz, *p, None, None, D, dtb, delta_softplus=True).backward(dout)

    f_ms = _time_loop(infer, steps, warmup, torch)
    t_ms = _time_loop(train, steps, warmup, torch)
    tokens = batch * seqlen
    fwd_flops = 2 * tokens * (d_inner * (rank + 2 * d_state) + rank * d_inner + d_inner * d_model)
    # backward: two GEMMs per forward projection, and delta recomputed (checkpoint_lvl 1)
    train_flops = 3 * fwd_flops + 2 * tokens * rank * d_inner
    del xz, p, dout
    torch.cuda.empty_cache()
    return {"shape": {"batch": batch, "seqlen": seqlen, "d_model": d_model, "d_inner": d_inner, "dt_rank": rank,
                      "d_state": d_state, "d_conv": 4}, "dtype": "bf16",
            "fwd_ms": f_ms, "fwd_bwd_ms": t_ms, "tokens_per_s_fwd": tokens / (f_ms * 1e-3),
            "tokens_per_s_fwd_bwd": tokens / (t_ms * 1e-3), "gemm_gflop_fwd": fwd_flops / 1e9,
            "gemm_gflop_fwd_bwd": train_flops / 1e9}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _time_cpu(fn, seconds_target):
    t0 = time.time()
    fn()
    t1 = time.time() - t0
    reps = max(1, int(seconds_target / max(t1, 1e-3)))
    t0 = time.time()
    for _ in range(reps):
        fn()
    return (time.time() - t0) / reps, reps


def cpu_scan_sample(torch, cfg_name, batch, dims, seconds_target):
    """The CPU oracle (oracle.ssm_ref.selective_scan_ref, the torch restatement of the reference's
    selective_scan_ref, selective_scan_interface.py:353-451) on a bounded sample of one scan
    configuration: `batch` rows x `dims` channels at the configuration's full L, scaled to the
    configuration's algorithmic bytes per element (GB/s) and elements per second."""
    from motif_mamba_amd.workloads import SCAN_CONFIGS, scan_bytes, scan_inputs
    from oracle.ssm_ref import selective_scan_ref
    c = SCAN_CONFIGS[cfg_name]
    inputs = scan_inputs(c, batch=batch, dim=dims)
    inputs.pop("return_last_state")
    per, reps = _time_cpu(lambda: selective_scan_ref(**inputs, return_last_state=True), seconds_target)
    frac = (batch * dims) / (c.batch * c.dim)
    in_bytes = 2 if c.dtype in ("bf16", "fp16") else 4
    nbytes = scan_bytes(c.batch, c.dim, c.seqlen, c.dstate, c.n_groups, in_bytes) * frac
    elems = batch * dims * c.seqlen
    threads = torch.get_num_threads()
    return {"value": nbytes / per / 1e9, "unit": "GB/s", "elements_per_s": elems / per, "cores": threads,
            "kind": "port",
            "sample": f"{cfg_name} restricted to batch {batch} x {dims} channels x L {c.seqlen} "
                      f"(1/{round(1 / frac)} of the work), {reps} timed run(s) of {per:.3f}s; "
                      f"oracle/ssm_ref.selective_scan_ref, torch {torch.__version__}, {threads} threads on "
                      f"{_cpu_model()} ({os.cpu_count()} logical CPUs visible)"}


def cpu_decode_sample(torch, batch, dims, steps, seconds_target):
    """The CPU restatement of the decode step (oracle.ssm_ref.selective_state_update_ref, the math of
    mamba_simplemotif.py:369-376 with the upstream kernel's float32 discretisation) over `steps`
    consecutive steps of config 4 at `batch`, on `dims` of its 5120 channels, scaled to tokens/s
    of the whole layer."""
    from oracle.ssm_ref import selective_state_update_ref
    g = torch.Generator().manual_seed(4)
    N = 16
    state0 = torch.randn(batch, dims, N, generator=g) * 0.1
    bias = torch.rand(dims, generator=g) * 4.6 - 6.9
    A = -torch.arange(1, N + 1, dtype=torch.float32).repeat(dims, 1)
    D = torch.ones(dims)
    S = min(steps, 16)
    xs = [torch.randn(batch, dims, generator=g).to(torch.bfloat16) for _ in range(3 * S)]
    BC = [torch.randn(batch, N, generator=g).to(torch.bfloat16) for _ in range(2 * S)]

    def run():
        st = state0.clone()
        for i in range(steps):
            j = i % S
            selective_state_update_ref(st, xs[3 * j], xs[3 * j + 1], A, BC[2 * j], BC[2 * j + 1], D, xs[3 * j + 2],
                                       bias, dt_softplus=True)
    per, reps = _time_cpu(run, seconds_target)
    frac = dims / 5120
    threads = torch.get_num_threads()
    return {"value": batch * steps * frac / per, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"config 4 batch {batch}: {steps} steps on {dims} of 5120 channels (1/{round(1 / frac)} "
                      f"of the layer), {reps} timed run(s) of {per:.3f}s; oracle/ssm_ref.selective_state_update_ref, "
                      f"{threads} threads on {_cpu_model()}"}


def cpu_baselines(torch):
    """The headline CPU baseline (config 2) and one per other configuration, each a few seconds."""
    head = cpu_scan_sample(torch, "cfg2", 1, 64, 10.0)
    per_cfg = {
        "cfg1": cpu_scan_sample(torch, "cfg1", 1, 64, 4.0),
        "cfg3_g1": cpu_scan_sample(torch, "cfg3_g1", 1, 16, 4.0),
        "cfg3_g4": cpu_scan_sample(torch, "cfg3_g4", 1, 16, 4.0),
        "cfg4_b1": cpu_decode_sample(torch, 1, 5120, 1024, 2.0),
        "cfg4_b64": cpu_decode_sample(torch, 64, 320, 1024, 3.0),
        "cfg4_b256": cpu_decode_sample(torch, 256, 80, 1024, 3.0),
    }
    return head, per_cfg


# Instructions per round and lane of each probe kind of libmm_probe.so (csrc/mm_probe.hip), as
# (transcendental, VALU) counts; kind 4 runs kind 1 on even waves and kind 0 on odd waves.
PROBE_KINDS = {0: ("v_fma_f32", 0, 32), 1: ("v_exp_f32", 32, 0), 2: ("v_mul_f32_dpp row_newbcast", 0, 32),
               3: ("v_exp_f32 + 4 v_fma_f32 (one wave)", 8, 32), 4: ("v_exp_f32 / v_fma_f32 (alternate waves)", 16, 16),
               5: ("v_fmac_f32_dpp row_newbcast", 0, 32), 6: ("v_exp_f32 + v_fma_f32 (one wave)", 16, 16),
               7: ("scan core (per state update: exp2, 2 DPP, 2 VALU)", 16, 64),
               8: ("scan core, plain VALU instead of DPP", 16, 64),
               9: ("scan core without exp2", 0, 64)}


def issue_rates(torch, waves=(2, 3, 4, 8), iters=2000):
    """Issue rates of the instructions a state update is made of, measured on this GPU with the
    probe kernels of libmm_probe.so: for each kind and W waves per SIMD, the SIMD cycles one wave64
    instruction takes (kernel time x shader clock / instructions per SIMD) and the chip-wide rate in
    lane operations per second. The shader clock comes from the probes' own s_memtime /
    s_memrealtime ticks."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(REPO, "motif-mamba_amd", "motif_mamba_amd", "libmm_probe.so"))
    lib.mm_probe_launch.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_void_p]
    lib.mm_probe_device.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    cus, wall_khz = ctypes.c_int(), ctypes.c_int()
    if lib.mm_probe_device(ctypes.byref(cus), ctypes.byref(wall_khz)) != 0:
        raise RuntimeError("mm_probe_device failed")
    n_simd = cus.value * 4
    stream = torch.cuda.current_stream()
    res = {"cus": cus.value, "wall_clock_khz": wall_khz.value, "iters": iters, "kinds": {}}
    clocks = []
    for kind, (name, n_trans, n_valu) in PROBE_KINDS.items():
        rows = []
        for W in waves:
            blocks = cus.value * W
            out = torch.empty(blocks * 256, device="cuda")
            ticks = torch.zeros(blocks * 8, dtype=torch.int64, device="cuda")

            def launch():
                rc = lib.mm_probe_launch(kind, blocks, iters, out.data_ptr(), ticks.data_ptr(),
                                         ctypes.c_void_p(stream.cuda_stream))
                if rc != 0:
                    raise RuntimeError(f"mm_probe_launch kind {kind}: hip error {rc}")
            launch()
            torch.cuda.synchronize()
            best = None
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                launch()
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1)
                best = ms if best is None else min(best, ms)
            tk = ticks.view(-1, 2).double()
            clk_hz = (tk[:, 0].sum() / tk[:, 1].sum()).item() * wall_khz.value * 1e3
            clocks.append(clk_hz)
            instr_simd = W * iters * (n_trans + n_valu)        # wave64 instructions per SIMD
            row = {"waves_per_simd": W, "ms": round(best, 4), "clock_mhz": round(clk_hz / 1e6, 1),
                   "simd_cycles_per_instr": round(best * 1e-3 * clk_hz / instr_simd, 3),
                   "lane_ops_per_s": n_simd * instr_simd * 64 / (best * 1e-3)}
            if kind >= 7:   # the scan-core kinds: 16 state updates per lane and round
                row["simd_cycles_per_wave_update"] = round(best * 1e-3 * clk_hz / (W * iters * 16), 3)
            rows.append(row)
            del out, ticks
        res["kinds"][name] = rows
    res["clock_mhz"] = round(sum(clocks) / len(clocks) / 1e6, 1)

    def best_rate(name):
        return max(r["lane_ops_per_s"] for r in res["kinds"][name])
    res["trans_per_s"] = best_rate("v_exp_f32")                 # exp2 lane operations per second, chip
    res["valu_per_s"] = best_rate("v_fma_f32")
    res["dpp_valu_per_s"] = best_rate("v_mul_f32_dpp row_newbcast")
    return res


def _traffic():
    """HBM bytes per launch of the headline kernel, from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs
    recorded in profiles/traffic_cfg2.json (static: counters cannot be read from inside this run)."""
    path = os.path.join(REPO, "profiles", "traffic_cfg2.json")
    if os.path.exists(path):
        with open(path) as f:
            d = json.load(f)
        return d.get("hbm_bytes_per_launch"), ("static: profiles/traffic_cfg2.json, rocprofv3 --pmc FETCH_SIZE and "
                                              "WRITE_SIZE of " + str(d.get("kernel", "the headline kernel")))
    return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--quick", action="store_true", help="headline config only (no secondary configs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-ref", action="store_true",
                    help="also run three 1 GiB device-to-device copies: the reference that scales the "
                         "FETCH_SIZE / WRITE_SIZE byte counters of a profiled run to HBM bytes")
    ap.add_argument("--only", default=None,
                    help="run one secondary configuration alone (cfg1, cfg3_g1, cfg3_g4, cfg4_b<batch>, pq_1p4b, pq_1p4b_train, pq_layouts, "
                         "cfg1_train, cfg2_train, conv_cfg1, conv_cfg2, conv_bwd_cfg1, conv_bwd_cfg2, conv_update_b<batch>, inner_2p8b, "
                         "presets) "
                         "and print its result as JSON: the profiled command of that configuration")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from motif_mamba_amd import _native
    _native.ext()  # the HIP library must be present: no fallback path exists
    torch.cuda.init()
    _log(f"device: {torch.cuda.get_device_name(0)}")

    if args.only:
        name = args.only
        RATES.update(issue_rates(torch))
        if name == "probe":
            res = RATES
        elif name == "cpu":
            head, per_cfg = cpu_baselines(torch)
            res = {"cfg2": head, **per_cfg}
        elif name.startswith("cfg4_b"):
            res = bench_decode(int(name[len("cfg4_b"):]), 1024, 16, torch)
        elif name == "pq_layouts":
            res = bench_pq_layouts(args.steps, 2, torch)
        elif name == "presets":
            res = bench_presets(min(args.steps, 10), 2, torch)
        elif name.startswith("pq_") and name.endswith("_train"):
            res = bench_pq_train(name[: -len("_train")], args.steps, args.warmup, torch)
        elif name.startswith("pq_"):
            res = bench_pq(name, args.steps, args.warmup, torch)
        elif name == "inner_2p8b":
            res = bench_inner(args.steps, args.warmup, torch)
        elif name.endswith("_train"):
            res = bench_train(name[: -len("_train")], args.steps, args.warmup, torch)
        elif name.startswith("conv_update_b"):
            res = bench_conv_update(int(name[len("conv_update_b"):]), max(args.steps, 100), args.warmup, torch)
        elif name.startswith("conv_bwd_"):
            res = bench_conv_bwd(name[len("conv_bwd_"):], args.steps, args.warmup, torch)
        elif name.startswith("conv_"):
            res = bench_conv(name[len("conv_"):], args.steps, args.warmup, torch)
        else:
            res = bench_scan(name, args.steps, args.warmup, torch, rotate=2 if name == "cfg1" else 1)
        print(json.dumps({"config": name, **res}), flush=True)
        return

    _log("issue-rate probes (also bring the GPU to its loaded clock before the timed runs)")
    RATES.update(issue_rates(torch))
    _log("config 2 (headline)")
    head = bench_scan("cfg2", args.steps, args.warmup, torch)
    if args.copy_ref:
        src = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()
    extra = {}
    if not args.quick:
        _log("config 1 (rotating 2 input sets: 2 x 203 MB > Infinity Cache)")
        extra["cfg1"] = bench_scan("cfg1", max(5, args.steps), 2, torch, rotate=2)
        for name in ("cfg3_g1", "cfg3_g4"):
            _log(f"config 3 ({name})")
            extra[name] = bench_scan(name, max(3, args.steps // 4), 1, torch)
        for b in (1, 64, 256):
            _log(f"config 4 decode batch {b}")
            extra[f"cfg4_b{b}"] = bench_decode(b, 1024, 16, torch)
        _log("MotifMamba P/Q forward (Mamba-1.4B layer, rank 2, per-channel P/Q)")
        extra["pq_1p4b"] = bench_pq("pq_1p4b", max(5, args.steps), 2, torch)
        _log("MotifMamba P/Q training forward + backward (same layer)")
        extra["pq_1p4b_train"] = bench_pq_train("pq_1p4b", max(5, args.steps // 2), 2, torch)
        for name in ("cfg1", "cfg2"):
            _log(f"training forward + backward ({name})")
            extra[f"{name}_train"] = bench_train(name, max(5, args.steps // 2), 2, torch)
        for name in ("cfg1", "cfg2"):
            _log(f"causal_conv1d forward ({name} shape)")
            extra[f"conv_{name}"] = bench_conv(name, max(10, args.steps), 3, torch)
        for name in ("cfg1", "cfg2"):
            _log(f"causal_conv1d backward ({name} shape)")
            extra[f"conv_bwd_{name}"] = bench_conv_bwd(name, max(10, args.steps), 3, torch)
        for b in (64, 256):
            _log(f"causal_conv1d decode update batch {b}")
            extra[f"conv_update_b{b}"] = bench_conv_update(b, 200, 10, torch)
        _log("mamba_inner_fn forward and forward + backward (Mamba-2.8B layer, config-2 tokens)")
        extra["inner_2p8b"] = bench_inner(max(5, args.steps // 2), 2, torch)
    cpu, cpu_cfgs = None, None
    if not args.no_cpu:
        _log("CPU baselines (oracle on bounded samples of configs 1-4)")
        cpu, cpu_cfgs = cpu_baselines(torch)
        for name, res in cpu_cfgs.items():
            if name in extra:
                extra[name]["cpu_baseline"] = res

    value = head["GB_s"]
    t = head["ms"] * 1e-3
    traffic, traffic_src = _traffic()
    hbm = {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src}
    trans = {"bound": "trans", "achieved": round(head["trans_per_s"] / 1e12, 3),
             "peak": round(RATES["trans_per_s"] / 1e12, 3), "unit": "T/s",
             "frac": round(head["trans_per_s"] / RATES["trans_per_s"], 4), "traffic": traffic,
             "traffic_source": traffic_src,
             "peak_source": "v_exp_f32 lane operations per second measured in this run by libmm_probe.so "
                            "(csrc/mm_probe.hip), the best of 2-8 waves per SIMD"}
    issue = {"bound": "valu+trans issue", "t_floor_us": round(head["t_issue_us"], 2),
             "frac": round(head["issue_frac"], 4),
             "model": "B*D*L*(N+4) transcendentals at the measured v_exp_f32 rate plus 4 VALU operations per "
                      "state update at the measured v_fma_f32 rate, issued serially (the probes show no co-issue)"}
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["ms"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "accumulate_dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "cfg2: selective_scan_fn fwd, Mamba-2.8B layer (batch 4, d_inner 5120, "
                               "L 4096, dstate 16, bf16, z gate, delta_bias+softplus, last_state)",
                   "batch": 4, "dim": 5120, "seqlen": 4096, "dstate": 16, "n_groups": 1, "io_dtype": "bf16"},
        # The binding roofline of north_star ("HBM bandwidth or exp issue rate", the larger floor).
        "roofline": trans if head["binding"] == "trans" else hbm,
        "roofline_hbm": hbm, "roofline_trans": trans, "roofline_issue": issue,
        "cpu_baseline": cpu,
        "issue_rates": {k: RATES[k] for k in ("clock_mhz", "trans_per_s", "valu_per_s", "dpp_valu_per_s")},
        "headline_detail": head,
        "configs": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
