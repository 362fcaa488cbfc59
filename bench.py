#!/usr/bin/env python3
"""Benchmark of the MI355X selective-scan hot path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]``

One "step" is one forward selective scan over BASELINE config 2 (the headline: Mamba-2.8B layer
shape, batch 4, d_inner 5120, L 4096, dstate 16, bf16 in / fp32 accumulate, z gate, delta_bias +
softplus, last state returned), with all inputs resident in HBM before timing starts. ``value``
is the algorithmic HBM throughput of that step (bytes of u, delta, z, B, C, A, D, delta_bias read
and out_z, last_state written, each once) divided by the measured time per step, in GB/s.

The JSON line also carries: ``roofline`` for the forward-scan kernel (HBM bound, 8 TB/s peak),
``roofline_trans`` (the same kernel against the v_exp_f32 issue rate, which binds it), ``cpu_baseline``
(the CPU oracle timed on the host on a bounded sample of the same workload), per-config results for
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
# v_exp_f32 throughput of the whole MI355X, measured with a kernel-time microbenchmark (8 waves per
# SIMD, independent chains): the transcendental issue roofline of the scan.
TRANS_PEAK_PER_S = 16.14e12
METRIC = "selective-scan fwd GB/s & % of binding roofline; decode tokens/s, 1 GPU"


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _time_loop(fn, steps, warmup, torch):
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
        "t_floor_us": max(nbytes / (HBM_PEAK_GBS * 1e9), trans / TRANS_PEAK_PER_S) * 1e6,
        "floor_frac": max(nbytes / (HBM_PEAK_GBS * 1e9), trans / TRANS_PEAK_PER_S) / (ms * 1e-3),
        "input_rotation": rotate,
    }


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

    def step(i):
        j = i % S
        selective_state_update(state, x[j], dts[j], A, B[j], C[j], D, z[j], bias, True)

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
    floor = max(nbytes / (HBM_PEAK_GBS * 1e9), trans / TRANS_PEAK_PER_S)
    del inputs
    torch.cuda.empty_cache()
    return {"shape": [c.batch, c.dim, c.seqlen, c.dstate], "rank": c.rank, "per_dim": c.per_dim, "dtype": c.dtype,
            "ms": ms, "GB_s": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "elements_per_s": elems / (ms * 1e-3),
            "trans_per_s": trans / (ms * 1e-3), "coupling_TFLOP_s": flops / (ms * 1e-3) / 1e12,
            "t_floor_us": floor * 1e6, "floor_frac": floor / (ms * 1e-3)}


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


def cpu_baseline(torch, seconds_target=15.0):
    """The CPU oracle (torch restatement of selective_scan_ref) on a bounded sample of config 2:
    one batch row and a slice of channels at the full L = 4096, scaled to GB/s of the config's
    algorithmic bytes per element."""
    from motif_mamba_amd.workloads import SCAN_CONFIGS, scan_bytes, scan_inputs
    from oracle.ssm_ref import selective_scan_ref
    c = SCAN_CONFIGS["cfg2"]
    threads = torch.get_num_threads()
    dims = 64
    inputs = scan_inputs(c, batch=1, dim=dims)
    inputs.pop("return_last_state")
    t0 = time.time()
    selective_scan_ref(**inputs, return_last_state=True)
    t1 = time.time() - t0
    reps = max(1, int(seconds_target / max(t1, 1e-3)))
    t0 = time.time()
    for _ in range(reps):
        selective_scan_ref(**inputs, return_last_state=True)
    per = (time.time() - t0) / reps
    frac = (1 * dims) / (c.batch * c.dim)
    nbytes = scan_bytes(c.batch, c.dim, c.seqlen, c.dstate, c.n_groups, 2) * frac
    return {"value": nbytes / per / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"config 2 shape restricted to batch 1 x {dims} channels x L {c.seqlen} "
                      f"(1/{int(1 / frac)} of the work), {reps} timed run(s) of {per:.3f}s; "
                      f"oracle/ssm_ref.selective_scan_ref, torch {torch.__version__} on "
                      f"{platform.processor() or platform.machine()} with {threads} threads"}


def _traffic():
    path = os.path.join(REPO, "profiles", "traffic_cfg2.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


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
                    help="run one secondary configuration alone (cfg1, cfg3_g1, cfg3_g4, cfg4_b<batch>, pq_1p4b, pq_1p4b_train, "
                         "cfg1_train, cfg2_train, conv_cfg1, conv_cfg2, conv_update_b<batch>, inner_2p8b) "
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
        if name.startswith("cfg4_b"):
            res = bench_decode(int(name[len("cfg4_b"):]), 1024, 16, torch)
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
        elif name.startswith("conv_"):
            res = bench_conv(name[len("conv_"):], args.steps, args.warmup, torch)
        else:
            res = bench_scan(name, args.steps, args.warmup, torch, rotate=2 if name == "cfg1" else 1)
        print(json.dumps({"config": name, **res}), flush=True)
        return

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
        for b in (64, 256):
            _log(f"causal_conv1d decode update batch {b}")
            extra[f"conv_update_b{b}"] = bench_conv_update(b, 200, 10, torch)
        _log("mamba_inner_fn forward and forward + backward (Mamba-2.8B layer, config-2 tokens)")
        extra["inner_2p8b"] = bench_inner(max(5, args.steps // 2), 2, torch)
    cpu = None
    if not args.no_cpu:
        _log("CPU baseline (oracle on a bounded sample)")
        cpu = cpu_baseline(torch)

    value = head["GB_s"]
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["ms"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "cfg2: selective_scan_fn fwd, Mamba-2.8B layer (batch 4, d_inner 5120, "
                               "L 4096, dstate 16, bf16, z gate, delta_bias+softplus, last_state)",
                   "batch": 4, "dim": 5120, "seqlen": 4096, "dstate": 16, "n_groups": 1, "io_dtype": "bf16"},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": _traffic()},
        "roofline_trans": {"bound": "v_exp_f32 issue", "achieved": round(head["trans_per_s"] / 1e12, 3),
                           "peak": TRANS_PEAK_PER_S / 1e12, "unit": "T/s",
                           "frac": round(head["trans_per_s"] / TRANS_PEAK_PER_S, 4),
                           "t_floor_us": round(head["t_floor_us"], 2), "floor_frac": round(head["floor_frac"], 4)},
        "cpu_baseline": cpu,
        "headline_detail": head,
        "configs": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
