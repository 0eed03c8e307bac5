"""Benchmark of the routed-expert MoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config decode_t1]

One step is one routed-expert MoE layer (route plan, fused gate/up FP8
projection + SwiGLU, down FP8 projection + route weighting, route combine)
over one batch of synthetic tokens, with every input already resident in HBM.
All 256 experts of the layer are resident (9.7 GB of e4m3 bytes + scales) and
every step uses a different routing drawn from 64 seeds, so consecutive steps
touch different experts and the 256 MB Infinity Cache cannot hold the decode
working set.

Prints ONE JSON line: the headline metric (us per MoE layer of the
``--config`` workload), the roofline of the dominant kernel (the fused gate/up
projection: algorithmic bytes or flops per launch / its mean launch time from
HIP events recorded on the launch stream), the CPU baseline (the numpy oracle
on the host cores, a bounded sample), and secondary figures for the other
configurations.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "glm-tpu_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
ROTATIONS = 64
# The GPU's kernels reach their steady speed only after some tens of ms of work
# (measured: the decode kernels run 7 % slower in the first 10 ms), so every
# timed loop is preceded by untimed replays for at least WARM_SECONDS.
WARM_SECONDS = 0.3
TIMED_REPLAYS = 5       # timed replays of the K captured steps (at least)
MIN_TIMED_CALLS = 50    # ... and at least this many timed calls in all; value = median per call
TABLE_KEYS = ("gate_bits", "gate_scale", "up_bits", "up_scale", "down_bits", "down_scale")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", default="decode_t1")
    p.add_argument("--secondary",
                   default="decode_t4,batch_t64,prefill_t128,prefill_t2048,prefill_t8192_zipf,prefill_t2048:fp8,"
                           "prefill_t8192_zipf:fp8,"
                           "prefill_t2048:share8",
                   help="comma-separated extra configs measured after the headline ('' for none); a ':fp8' "
                        "suffix runs the native FP8 MFMA mode and reports its error against the reference "
                        "numerics; ':share8' times the eight expert-parallel shares of the layer one by one")
    p.add_argument("--secondary-steps", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--headline-only", action="store_true",
                   help="time the headline config's routed layer alone (no full-layer, router or "
                        "MLP-from-logits figures): in a rocprofv3 run, the kernels replayed from HIP graphs "
                        "(listed under their symbol names) are then the routed layer's only")
    p.add_argument("--copy-calibration", action="store_true",
                   help="after the headline, copy a 1 GiB device buffer 3 times (the known-size kernel that "
                        "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    return p.parse_args()


def copy_calibration(device, nbytes=1 << 30, times=3):
    """Device-to-device copies of a known size, for calibrating HBM byte counters."""
    import torch

    src = torch.ones(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(times):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


class Workload:
    """Rotated synthetic routings of one config on the device, plus their costs."""

    def __init__(self, cfg, tables, device, rotations=ROTATIONS, seed0=1000, activations="bfloat16"):
        import torch

        from glm_moe import synthetic as S

        self.cfg = cfg
        self.activations = activations
        self.tables = tables
        self.inputs = []
        self.host = []
        self.bytes_total, self.bytes_gate_up = [], []
        for r in range(rotations):
            seed = seed0 + r
            ids, w = S.routes(cfg, seed)
            x = S.hidden_states(cfg, seed)
            xd = torch.from_numpy(x).to(torch.bfloat16).to(device)
            self.inputs.append((xd, torch.from_numpy(ids).to(device), torch.from_numpy(w).to(device)))
            self.host.append((x, ids, w))
            b = S.algorithmic_bytes(cfg, ids)
            self.bytes_total.append(b["total"])
            self.bytes_gate_up.append(b["gate_up"])
        self.flops = S.algorithmic_flops(cfg)


def _timed_replays(run_batch, steps):
    """Untimed batches for at least WARM_SECONDS, then at least TIMED_REPLAYS
    batches (and MIN_TIMED_CALLS calls) each bracketed by synchronisations and
    HIP events on the current stream.  Returns (median ms per call, every
    batch's ms per call)."""
    import torch

    t0 = time.perf_counter()
    warm = 0
    while warm < 3 or time.perf_counter() - t0 < WARM_SECONDS:
        run_batch()
        torch.cuda.synchronize()
        warm += 1
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    per_call = []
    for _ in range(max(TIMED_REPLAYS, math.ceil(MIN_TIMED_CALLS / steps))):
        torch.cuda.synchronize()
        start.record()
        run_batch()
        stop.record()
        torch.cuda.synchronize()
        per_call.append(start.elapsed_time(stop) / steps)
    return float(np.median(per_call)), per_call


def graph_time(body, steps, warmup):
    """``body(i)`` (one call of the timed operation on the i-th rotated input)
    replayed from one HIP graph of ``steps`` calls, captured after ``warmup``
    eager calls: (median ms per call, per-replay ms per call).  The time is the
    GPU's, without the host's per-call launch cost (a serving loop replays its
    decode steps the same way)."""
    import torch

    for i in range(max(warmup, 1)):
        body(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            body(warmup + i)
    try:
        return _timed_replays(graph.replay, steps)
    finally:
        del graph


def eager_time(body, steps, warmup):
    """The same ``steps`` calls launched one by one from Python (batches
    bracketed like the graph replays): (median ms per call, per-batch ms)."""
    for i in range(warmup):
        body(i)

    def batch():
        for i in range(steps):
            body(warmup + i)

    return _timed_replays(batch, steps)


def layer_body(work):
    """``body(i)``: one routed-expert layer call on rotated input i."""
    import torch

    from glm_moe.layers.moe.routed_experts import routed_experts

    tables = [work.tables[k] for k in TABLE_KEYS]
    out = torch.empty((work.cfg.tokens, work.cfg.hidden), dtype=torch.bfloat16, device=tables[0].device)
    n_rot = len(work.inputs)

    def body(i):
        x, ids, w = work.inputs[i % n_rot]
        routed_experts(x, ids, w, *tables, out=out, activations=work.activations)

    return body


def stage_times(work, steps, warmup):
    """Per-kernel times of ``steps`` layer calls after the warm-up: HIP events
    that each stage's kernel records at its own start and end on the launch
    stream.  Returns (ms per call of the loop, per-call stage timings, the
    rotated inputs used)."""
    import torch

    from glm_moe.layers.moe.routed_experts import StageEvents, routed_experts

    tables = [work.tables[k] for k in TABLE_KEYS]
    out = torch.empty((work.cfg.tokens, work.cfg.hidden), dtype=torch.bfloat16, device=tables[0].device)
    n_rot = len(work.inputs)
    body = layer_body(work)
    t0 = time.perf_counter()
    i = 0
    while i < warmup or time.perf_counter() - t0 < WARM_SECONDS:
        body(i)
        i += 1
        if i % 32 == 0:
            torch.cuda.synchronize()
    events = [StageEvents() for _ in range(steps)]
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for j in range(steps):
        x, ids, w = work.inputs[(warmup + j) % n_rot]
        routed_experts(x, ids, w, *tables, out=out, events=events[j], activations=work.activations)
    stop.record()
    torch.cuda.synchronize()
    stages = [ev.elapsed() for ev in events]
    for ev in events:
        ev.close()
    order = [(warmup + j) % n_rot for j in range(steps)]
    return start.elapsed_time(stop) / steps, stages, order


def router_time(cfg, device, steps=20):
    """The GPU noaux_tc router on the config's [T, E] FP32 logits (replayed from
    one HIP graph): us per call and its algorithmic bytes (logits in, ids and
    weights out)."""
    import torch

    from glm_moe import synthetic as S
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    logits = torch.from_numpy(S.router_logits(cfg, 0)).to(device)
    bias = torch.zeros(cfg.experts, dtype=torch.float32, device=device)
    ms, _ = graph_time(lambda i: route_glm_noaux_tc_logits(logits, bias, top_k=cfg.top_k), steps, 3)
    us = ms * 1e3
    nbytes = cfg.tokens * cfg.experts * 4 + cfg.experts * 4 + cfg.tokens * cfg.top_k * 8
    return {"us": us, "bytes": nbytes, "hbm_gbs": nbytes / (us * 1e-6) / 1e9}


def with_router(s, cfg, device):
    try:
        s["router"] = router_time(cfg, device)
    except Exception as exc:  # a secondary figure: report it, keep the headline
        print(f"[bench] router timing failed: {exc!r}", file=sys.stderr, flush=True)
        s["router"] = {"error": repr(exc)}
    return s


def full_layer(work, steps, warmup):
    """The whole MoE layer (K calls replayed from one HIP graph), as the reference's layer bodies compute it: the bf16
    shared expert (random-init N(0, 0.02) weights of the contract's shape,
    I_shared = I) and the routed experts with the epilogue
    bf16(bf16(routed * 2.5) + shared) fused into their route-sum kernel.  On
    decode shapes the shared expert runs inside the two decode kernels
    (glm_moe_moe_layer_resident); for 2-8 rows in the few-row shared-expert
    kernels (glm_moe_shared_expert_rows); else as torch GEMMs on hipBLASLt.
    Returns (us per layer, algorithmic bytes of the shared expert, how)."""
    import torch

    from glm_moe.layers.moe.routed_experts import (_shared_expert, routed_experts, shared_expert_rows_fit,
                                                   uses_decode_kernels)

    cfg = work.cfg
    device = work.inputs[0][0].device
    g = torch.Generator(device=device).manual_seed(11)
    inter_shared = cfg.intermediate  # one shared expert of the routed experts' width (contract local_shared_intermediate x stage_size)
    sg = (torch.randn((inter_shared, cfg.hidden), generator=g, device=device) * 0.02).to(torch.bfloat16)
    su = (torch.randn((inter_shared, cfg.hidden), generator=g, device=device) * 0.02).to(torch.bfloat16)
    sd = (torch.randn((cfg.hidden, inter_shared), generator=g, device=device) * 0.02).to(torch.bfloat16)
    t = work.tables
    tables = [t[k] for k in TABLE_KEYS]
    out = torch.empty((cfg.tokens, cfg.hidden), dtype=torch.bfloat16, device=device)
    n_rot = len(work.inputs)

    # up to 8 rows on the decode kernels: the shared expert inside them (one row: the
    # decode body); more: hipBLASLt (each reads the shared weights once)
    resident = work.activations == "bfloat16" and cfg.tokens <= 8 and uses_decode_kernels(
        cfg.tokens, cfg.top_k, cfg.hidden, cfg.intermediate)

    def layer(i):
        x, ids, w = work.inputs[i % n_rot]
        if resident:
            routed_experts(x, ids, w, *tables, out=out, shared_tables=(sg, su, sd), routed_scale=2.5)
        else:
            shared = _shared_expert(x, sg, su, sd)
            routed_experts(x, ids, w, *tables, out=out, shared=shared, routed_scale=2.5,
                           activations=work.activations)

    ms, _ = graph_time(layer, steps, warmup)
    shared_bytes = 3 * inter_shared * cfg.hidden * 2
    if resident:
        how = ("shared expert inside the two decode kernels (glm_moe_moe_layer_resident"
               + (")" if cfg.tokens == 1 else "; routes grouped by expert, shared rows streamed once per token group)"))
    elif shared_expert_rows_fit(cfg.tokens, cfg.hidden, inter_shared):
        how = "shared expert on the few-row kernels (glm_moe_shared_expert_rows), epilogue fused (glm_moe_moe_layer)"
    else:
        how = "shared expert on torch/hipBLASLt GEMMs and the library SwiGLU kernel, epilogue fused (glm_moe_moe_layer)"
    return ms * 1e3, shared_bytes, how


def mlp_from_logits(work, steps, warmup):
    """The decode MLP body from router logits (one row; K calls replayed from
    one HIP graph), both ways: the router kernel then moe_grouped_routes (three
    launches), and moe_mlp_from_router_logits with the routing inside the decode
    gate/up kernel (two launches).  Rotated logits, so each call touches its own
    experts.  Returns {"two_step_us", "fused_us"}."""
    import torch

    from glm_moe import synthetic as S
    from glm_moe.contracts import single_gpu_contract
    from glm_moe.layers.moe.routed_experts import moe_grouped_routes, moe_mlp_from_router_logits
    from glm_moe.layers.moe.router import route_glm_noaux_tc_logits

    cfg = work.cfg
    device = work.inputs[0][0].device
    contract = single_gpu_contract(hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
                                   num_experts=cfg.experts, top_k=cfg.top_k)
    g = torch.Generator(device=device).manual_seed(11)
    shared = tuple((torch.randn(shape, generator=g, device=device) * 0.02).to(torch.bfloat16)
                   for shape in ((cfg.intermediate, cfg.hidden), (cfg.intermediate, cfg.hidden),
                                 (cfg.hidden, cfg.intermediate)))
    t = work.tables
    tables = [t[k] for k in TABLE_KEYS]
    n_rot = len(work.inputs)
    logits = [torch.from_numpy(S.router_logits(cfg, 1000 + r)).to(device) for r in range(n_rot)]
    bias = torch.zeros(cfg.experts, dtype=torch.float32, device=device)

    def two_step(i):
        ids, w = route_glm_noaux_tc_logits(logits[i % n_rot], bias, top_k=cfg.top_k)
        moe_grouped_routes(work.inputs[i % n_rot][0], ids, w, *tables, contract=contract, shared_bf16=shared)

    def fused(i):
        moe_mlp_from_router_logits(work.inputs[i % n_rot][0], logits[i % n_rot], bias, *tables, contract=contract,
                                   shared_bf16=shared)

    result = {}
    for name, body in (("two_step_us", two_step), ("fused_us", fused)):
        ms, _ = graph_time(body, steps, warmup)
        result[name] = ms * 1e3
    result["note"] = ("decode MLP body from router logits incl. the resident shared expert: router kernel + "
                      "moe_grouped_routes, vs routing inside the decode gate/up kernel (glm_moe_moe_layer_from_logits)")
    return result


def with_mlp_from_logits(s, work, steps):
    cfg = work.cfg
    if work.activations != "bfloat16" or cfg.tokens != 1 or cfg.experts > 256:
        return s
    try:
        s["mlp_from_logits"] = mlp_from_logits(work, steps, 3)
    except Exception as exc:  # a secondary figure: report it, keep the headline
        print(f"[bench] MLP from logits failed: {exc!r}", file=sys.stderr, flush=True)
        s["mlp_from_logits"] = {"error": repr(exc)}
    return s


def with_full_layer(s, work, steps):
    try:
        us, shared_bytes, how = full_layer(work, steps, 3)
    except Exception as exc:  # a secondary figure: report it, keep the headline
        print(f"[bench] full layer failed: {exc!r}", file=sys.stderr, flush=True)
        s["full_layer_error"] = repr(exc)
        return s
    s["full_layer_us"] = us
    s["full_layer_hbm_gbs"] = (s["layer_bytes"] + shared_bytes) / (us * 1e-6) / 1e9
    s["full_layer_note"] = f"routed experts + bf16 shared expert + fused routed*2.5+shared epilogue; {how}"
    return s


def summarize(work, ms, stages, order):
    gate_up_ms = np.array([s.gate_up for s in stages])
    down_ms = np.array([s.down for s in stages])
    plan_ms = np.array([s.plan for s in stages])
    combine_ms = np.array([s.combine for s in stages])
    bytes_total = np.array([work.bytes_total[i] for i in order], np.float64)
    bytes_gu = np.array([work.bytes_gate_up[i] for i in order], np.float64)
    return {
        "us_per_layer": ms * 1e3,
        "stage_us": {
            "plan": float(plan_ms.mean() * 1e3),
            "gate_up": float(gate_up_ms.mean() * 1e3),
            "down": float(down_ms.mean() * 1e3),
            "combine": float(combine_ms.mean() * 1e3),
        },
        "layer_hbm_gbs": float(bytes_total.mean() / (ms * 1e-3) / 1e9),
        "gate_up_hbm_gbs": float(bytes_gu.mean() / (gate_up_ms.mean() * 1e-3) / 1e9),
        "layer_tflops": float(work.flops["total"] / (ms * 1e-3) / 1e12),
        "gate_up_tflops": float(work.flops["gate_up"] / (gate_up_ms.mean() * 1e-3) / 1e12),
        "gate_up_bytes": float(bytes_gu.mean()),
        "gate_up_flops": float(work.flops["gate_up"]),
        "layer_bytes": float(bytes_total.mean()),
        "distinct_experts": float(np.mean([len(np.unique(work.host[i][1])) for i in order])),
    }


DECODE_PATH_MAX_ROUTES = 64  # routes handled by the two decode GEMV kernels (libglm_moe)
PROFILES = ROOT / "profiles"


def measured_traffic():
    """HBM bytes per launch of each config's gate/up kernel, read from the
    profiles/*_hbm_traffic.md summaries: their lines
    ``bench-traffic: <config[:mode]> <kernel> <bytes>`` hold the rocprofv3 --pmc
    FETCH_SIZE + WRITE_SIZE per dispatch (scaled by the 1 GiB copy calibration
    of ``bench.py --copy-calibration``), the figure the summary's table derives."""
    found = {}
    for path in sorted(PROFILES.glob("*_hbm_traffic.md")) if PROFILES.is_dir() else []:
        for line in path.read_text().splitlines():
            if line.startswith("bench-traffic:"):
                _, name, kernel, nbytes = line.split()
                found[name] = {"bytes": float(nbytes), "kernel": kernel, "source": f"profiles/{path.name}"}
    return found


def dominant_roofline(cfg, s, mode=""):
    """Roofline of the stage that dominates the layer: the gate/up projection.

    The bound follows the kernel's arithmetic intensity (algorithmic flops per
    algorithmic byte) against the ridge point of the MFMA peak it computes on
    (bf16, or fp8 in the native FP8 mode) over the 8 TB/s HBM peak: below the
    ridge it is HBM-bound and achieved = its algorithmic bytes (the selected
    experts' gate and up e4m3 bytes and scales, the token rows read and the
    activations written) / its kernel time; above it, achieved = its
    algorithmic flops / its kernel time against the MFMA peak.  Kernel times
    come from HIP events the kernel records at its own start and end on the
    launch stream.  ``traffic`` is the measured HBM bytes per launch of that
    config's profile summary (null where there is none).
    """
    gate_up_us = s["stage_us"]["gate_up"]
    decode_path = cfg.tokens * cfg.top_k <= DECODE_PATH_MAX_ROUTES
    fp8 = mode == "fp8"
    peak_tflops = FP8_PEAK_TFLOPS if fp8 else BF16_PEAK_TFLOPS
    ridge = peak_tflops * 1e12 / (HBM_PEAK_GBS * 1e9)
    intensity = s["gate_up_flops"] / s["gate_up_bytes"]
    if decode_path:
        kernel = "decode_gate_up_kernel" if cfg.tokens == 1 else "decode_gate_up_multi_kernel"
    else:
        kernel = "prefill_gemm_fp8_kernel" if fp8 else "prefill_gemm_kernel"
    if decode_path or intensity < ridge:
        achieved = s["gate_up_bytes"] / (gate_up_us * 1e-6) / 1e9
        line = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS}
    else:
        achieved = s["gate_up_tflops"]
        line = {"bound": "mfma", "achieved": achieved, "peak": peak_tflops, "unit": "TFLOP/s",
                "frac": achieved / peak_tflops}
    measured = measured_traffic().get(cfg.name + (":" + mode if mode else ""))
    line["traffic"] = measured["bytes"] if measured else None
    line["kernel"] = kernel
    line["kernel_us"] = gate_up_us
    line["algorithmic_bytes"] = s["gate_up_bytes"]
    line["algorithmic_flops"] = s["gate_up_flops"]
    line["arithmetic_intensity"] = intensity
    line["ridge"] = ridge
    line["mfma_frac"] = s["gate_up_tflops"] / peak_tflops
    if measured:
        line["traffic_source"] = measured["source"]
        line["traffic_over_algorithmic"] = measured["bytes"] / s["gate_up_bytes"]
    return line


def fp8_error(work, device):
    """Error of the native FP8 mode against the reference numerics: the same
    layer on the library's bf16 path (decoded weights, bf16 activations; the
    GPU parity tests hold it to the oracle within max-abs 2e-2 / mean-rel 5e-3),
    over every token of the workload's first routing."""
    from glm_moe.layers.moe.routed_experts import routed_experts

    xd, idd, wd = work.inputs[0]
    tables = [work.tables[k] for k in TABLE_KEYS]
    got, _ = routed_experts(xd, idd, wd, *tables, activations="float8_e4m3fn")
    ref, _ = routed_experts(xd, idd, wd, *tables)
    got = got.double()
    ref = ref.double()
    err = (got - ref).abs()
    return {"max_abs": float(err.max()), "mean_rel": float(err.mean() / ref.abs().mean()),
            "sample": f"all {xd.shape[0]} tokens vs the bf16 path (reference numerics)"}


def cpu_baseline(work, device):
    """The numpy oracle on this host's cores, on one layer of the same workload."""
    import torch

    from oracle import moe_oracle as O

    try:
        from threadpoolctl import threadpool_info

        blas_threads = max((p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"),
                           default=1)
    except Exception:  # pragma: no cover - threadpoolctl missing
        blas_threads = 1
    x, ids, w = work.host[0]
    used = np.unique(ids.reshape(-1))
    index = torch.as_tensor(used, dtype=torch.long, device=device)
    host = {k: work.tables[k].index_select(0, index).cpu().numpy() for k in TABLE_KEYS}
    remap = np.searchsorted(used, ids).astype(np.int32)
    tokens = ids.shape[0]
    sample_tokens = tokens if tokens <= 4 else 4
    times = []
    budget_s = 20.0
    t_all = time.perf_counter()
    while len(times) < 3 and (time.perf_counter() - t_all) < budget_s:
        t0 = time.perf_counter()
        O.routed_experts(x[:sample_tokens], remap[:sample_tokens], w[:sample_tokens], **host)
        times.append(time.perf_counter() - t0)
    per_layer_us = float(np.median(times)) * 1e6 * (tokens / sample_tokens)
    return {
        "value": per_layer_us,
        "unit": "us/layer",
        "cores": len(os.sched_getaffinity(0)),
        "threads": int(blas_threads),
        "extrapolated": sample_tokens < tokens,
        "kind": "port",
        "sample": (f"numpy oracle (oracle/moe_oracle.py) on {sample_tokens} of {tokens} tokens of routing seed "
                   f"{1000}, {len(used)} experts decoded per run, median of {len(times)} runs; elementwise "
                   f"e4m3 decode single-threaded, FP32 BLAS on {blas_threads} threads"),
    }


def cpu_baseline_sampled(work, device):
    """The numpy oracle on a stratified sample of the experts of one prefill
    layer, scaled to the whole layer.

    The oracle's cost is a fixed part (route grouping over every route, the
    restore and the FP32 slot sum) plus one job per selected expert (its table
    decode and its routes' projections), run by 16 worker threads.  It is timed
    on routing seed 1000 (the faster of two runs each): with no expert owned (the fixed part) and
    owning as many experts as there are workers (one parallel wave of the
    whole layer's expert jobs), spaced evenly through the used experts ordered
    by route count (every expert's routes, so the projections keep their real
    row counts).  The layer estimate is fixed + (sampled run - fixed) x
    used / sampled."""
    from oracle import moe_oracle as O

    x, ids, w = work.host[0]
    experts = work.cfg.experts
    workers = min(16, len(os.sched_getaffinity(0)))
    sampled = workers
    used, counts = np.unique(ids.reshape(-1), return_counts=True)
    order = used[np.argsort(-counts, kind="stable")]
    pick = order[np.linspace(0, len(order) - 1, min(sampled, len(order))).round().astype(int)]
    pick = np.unique(pick)
    # a permutation of the expert ids that puts the sampled experts first
    rest = np.setdiff1d(np.arange(experts), pick)
    perm = np.empty(experts, np.int32)
    perm[pick] = np.arange(len(pick))
    perm[rest] = np.arange(len(pick), experts)
    pids = perm[ids].astype(np.int32)
    import torch

    index = torch.as_tensor(pick, dtype=torch.long, device=device)
    host = {k: work.tables[k].index_select(0, index).cpu().numpy() for k in TABLE_KEYS}
    none = {k: v[:0] for k, v in host.items()}

    def timed(tables):
        t0 = time.perf_counter()
        O.routed_experts(x, pids, w, **tables, num_experts=experts, expert_offset=0, workers=workers)
        return time.perf_counter() - t0

    fixed = min(timed(none) for _ in range(2))
    part = min(timed(host) for _ in range(2))  # the first call also pays the thread pool's start-up
    est = fixed + max(part - fixed, 0.0) * len(used) / len(pick)
    return {
        "value": est * 1e6,
        "unit": "us/layer",
        "cores": len(os.sched_getaffinity(0)),
        "threads": int(workers),
        "extrapolated": True,
        "extrapolation": f"measured on {len(pick)} of {len(used)} experts, scaled to all (value is an estimate)",
        "kind": "port",
        "sample": (f"numpy oracle (oracle/moe_oracle.py) on routing seed 1000: fixed part (grouping, restore, "
                   f"slot sum over all {ids.size} routes) {fixed:.2f} s, plus {len(pick)} of {len(used)} used "
                   f"experts (evenly spaced by route count, {int(counts[np.isin(used, pick)].sum())} routes) "
                   f"{part - fixed:.2f} s, scaled by {len(used)}/{len(pick)}; one expert per worker thread, "
                   f"{workers} workers, 1 BLAS thread each"),
        "measured_s": 2 * (part + fixed),
    }


def measure_shares(cfg, tables, device, steps, shares=8):
    """Every expert-parallel share of one layer (E/shares experts each) on this
    GPU, one after the other: each share's FP32 partial call (only its own
    routes planned and computed) replayed from one HIP graph, the sum of the
    shares' times against the whole layer's, and each share's algorithmic
    bytes (its selected experts' e4m3 tables and scales, the token rows and its
    FP32 partial)."""
    import torch

    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts_share

    work = Workload(cfg, tables, device, rotations=8)
    local = cfg.experts // shares
    h, i = cfg.hidden, cfg.intermediate
    per_expert = 3 * h * i + 3 * (h // 128) * (i // 128) * 4
    out = torch.empty((cfg.tokens, h), dtype=torch.float32, device=device)
    whole_ms, _ = graph_time(layer_body(work), steps, 3)
    rows = []
    for rank in range(shares):
        lo = rank * local
        share = [tables[k][lo:lo + local] for k in TABLE_KEYS]

        def body(j, share=share, lo=lo):
            x, ids, w = work.inputs[j % len(work.inputs)]
            routed_experts_share(x, ids, w, *share, num_experts=cfg.experts, expert_offset=lo, out=out)

        ms, _ = graph_time(body, steps, 3)
        owned = [((ids >= lo) & (ids < lo + local)) for _, ids, _ in work.host]
        distinct = float(np.mean([len(np.unique(ids[m])) for m, (_, ids, _) in zip(owned, work.host)]))
        nbytes = distinct * per_expert + cfg.tokens * h * 2 + cfg.tokens * h * 4
        rows.append({"rank": rank, "experts": [lo, lo + local], "us": ms * 1e3,
                     "owned_routes": float(np.mean([m.sum() for m in owned])), "distinct_experts": distinct,
                     "algorithmic_bytes": nbytes, "hbm_gbs": nbytes / (ms * 1e-3) / 1e9})
    whole_bytes = float(np.mean(work.bytes_total))
    return {
        "shares": shares, "local_experts": local, "whole_layer_us": whole_ms * 1e3,
        "whole_layer_bytes": whole_bytes,
        "share_us": [r["us"] for r in rows], "sum_of_shares_us": float(sum(r["us"] for r in rows)),
        "mean_share_frac_of_layer_time": float(np.mean([r["us"] for r in rows]) / (whole_ms * 1e3)),
        "mean_share_frac_of_layer_bytes": float(np.mean([r["algorithmic_bytes"] for r in rows]) / whole_bytes),
        "per_share": rows,
        "note": ("glm_moe_routed_experts_share on one GPU holding the share's tables (views of the layer's): "
                 "route plan over every route, tiles and projections for the share's experts only, FP32 "
                 "partial out; the sum over the expert axis and the epilogue are not timed"),
    }


def measure_secondary(scfg, tables, device, activations, mode, steps, cpu=True):
    """Layer time, stage times, full layer and (FP8 mode) error of one secondary config."""
    swork = Workload(scfg, tables, device, rotations=8, activations=activations)
    body = layer_body(swork)
    sms_eager, _ = eager_time(body, steps, 3)
    sms, _ = graph_time(body, steps, 3)
    _, sstages, sorder = stage_times(swork, steps, 3)
    s = summarize(swork, sms, sstages, sorder)
    s["us_per_layer_eager"] = sms_eager * 1e3
    s["hbm_frac"] = s["layer_hbm_gbs"] / HBM_PEAK_GBS
    s["bf16_mfma_frac"] = s["layer_tflops"] / BF16_PEAK_TFLOPS
    s["roofline"] = dominant_roofline(scfg, s, mode)
    with_full_layer(s, swork, steps)
    if mode != "fp8":
        with_router(s, scfg, device)
    if mode != "fp8" and cpu and scfg.tokens * scfg.top_k > DECODE_PATH_MAX_ROUTES:
        print(f"[bench] CPU baseline of {scfg.name} (sampled numpy oracle)", file=sys.stderr, flush=True)
        s["cpu_baseline"] = cpu_baseline_sampled(swork, device)
    if mode == "fp8":
        s["activations"] = "float8_e4m3fn (native FP8 MFMA mode)"
        s["fp8_mfma_frac"] = s["layer_tflops"] / FP8_PEAK_TFLOPS
        s["error_vs_reference"] = fp8_error(swork, device)
    del swork
    return s


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only; the multi-GPU (expert-parallel) "
                                   "design is documented, not measured", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from glm_moe import synthetic as S

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    device = torch.device("cuda:0")
    base, _, mode = args.config.partition(":")
    if mode not in ("", "fp8"):
        raise SystemExit(f"unknown mode {mode!r}: a config takes no suffix or ':fp8'")
    cfg = S.CONFIGS[base]
    activations = "float8_e4m3fn" if mode == "fp8" else "bfloat16"
    print(f"[bench] generating {cfg.experts} experts of {cfg.name} weights on {device}", file=sys.stderr, flush=True)
    tables = S.device_expert_tables(cfg, seed=0, device=device)
    torch.cuda.synchronize()
    work = Workload(cfg, tables, device, activations=activations)
    print(f"[bench] timing {args.steps} steps after {args.warmup} warmups", file=sys.stderr, flush=True)
    # headline: the K steps replayed from one HIP graph (the eager loop beside it);
    # per-kernel times: an eager loop with HIP events the kernels record on the
    # launch stream around every stage
    body = layer_body(work)
    ms_eager, eager_batches = eager_time(body, args.steps, args.warmup)
    timing_note = None
    try:
        ms, graph_batches = graph_time(body, args.steps, args.warmup)
    except Exception as exc:  # keep a measurement: the eager loop, labelled as such
        print(f"[bench] graph replay failed: {exc!r}; reporting the eager loop", file=sys.stderr, flush=True)
        ms, graph_batches = ms_eager, eager_batches
        timing_note = f"eager loop (graph replay failed: {exc!r})"
    ms_ev, stages, order = stage_times(work, args.steps, args.warmup)
    head = summarize(work, ms, stages, order)
    head["us_per_layer_eager"] = ms_eager * 1e3
    head["us_per_layer_with_stage_events"] = ms_ev * 1e3

    if not args.headline_only:
        with_full_layer(head, work, args.steps)
        with_router(head, cfg, device)
        with_mlp_from_logits(head, work, args.steps)
    roofline = dominant_roofline(cfg, head, mode)
    if args.copy_calibration:
        copy_calibration(device)

    secondary = {}
    for name in [s for s in args.secondary.split(",") if s]:
        if name == args.config:
            continue
        base, _, mode = name.partition(":")
        scfg = S.CONFIGS[base]
        activations = "float8_e4m3fn" if mode == "fp8" else "bfloat16"
        print(f"[bench] secondary {name}", file=sys.stderr, flush=True)
        try:
            if mode == "share8":
                secondary[name] = measure_shares(scfg, tables, device, args.secondary_steps)
            else:
                secondary[name] = measure_secondary(scfg, tables, device, activations, mode, args.secondary_steps,
                                                    cpu=not args.no_cpu_baseline)
        except Exception as exc:  # a secondary figure: report it, keep the headline
            print(f"[bench] secondary {name} failed: {exc!r}", file=sys.stderr, flush=True)
            secondary[name] = {"error": repr(exc)}

    baseline = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline (numpy oracle)", file=sys.stderr, flush=True)
        baseline = cpu_baseline(work, device)

    line = {
        "metric": "us per routed-expert MoE layer (decode T=1, E=256, H=6144, I=2048, top-8)"
        if args.config == "decode_t1" else f"us per routed-expert MoE layer ({args.config})",
        "value": head["us_per_layer"],
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 e4m3 x e4m3 (native FP8 mode)" if mode == "fp8" else "bf16",
        "data": "synthetic (seeded N(0,1) activations and router logits, N(0,0.02) e4m3fn weights with "
                "128x128 FP32 block scales, generated on the GPU)",
        "config": {
            "workload": f"{cfg.name}: T={cfg.tokens} E={cfg.experts} H={cfg.hidden} I={cfg.intermediate} "
                        f"top-{cfg.top_k}, all experts resident, {ROTATIONS} rotated routings",
            "tokens": cfg.tokens, "experts": cfg.experts, "hidden": cfg.hidden,
            "intermediate": cfg.intermediate, "top_k": cfg.top_k,
        },
        "full_layer_us": head.get("full_layer_us"),
        "full_layer_hbm_gbs": head.get("full_layer_hbm_gbs"),
        "full_layer_note": head.get("full_layer_note", head.get("full_layer_error")),
        "router": head.get("router"),
        "mlp_from_logits": head.get("mlp_from_logits"),
        "layer_hbm_gbs": head["layer_hbm_gbs"],
        "layer_hbm_frac": head["layer_hbm_gbs"] / HBM_PEAK_GBS,
        "stage_us": head["stage_us"],
        "us_per_layer_eager": head["us_per_layer_eager"],
        "us_per_layer_with_stage_events": head["us_per_layer_with_stage_events"],
        "timing": timing_note or (f"value: median over {len(graph_batches)} timed replays (each between two "
                                  f"synchronisations, {len(graph_batches) * args.steps} calls in all) of one HIP "
                                  f"graph of the K layer calls, after untimed replays for >= {WARM_SECONDS} s; "
                                  f"us_per_layer_eager: the same K calls launched one by one from Python, timed "
                                  f"the same way"),
        "timed_batches_us": [round(b * 1e3, 3) for b in graph_batches],
        "eager_batches_us": [round(b * 1e3, 3) for b in eager_batches],
        "distinct_experts": head["distinct_experts"],
        "roofline": roofline,
        "cpu_baseline": baseline,
        "secondary": secondary,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
