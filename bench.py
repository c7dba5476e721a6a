#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X: Qwen3-30B-A3B-shaped layers, seeded random weights.

    python bench.py [--steps K] [--warmup W]
                    [--workload prefill512|decode|prefill4096|prefill4096_zipf|dsv2_mixed|stack48|runtime_decode|
                                runtime_prefill512]

Inputs and weights are resident in HBM when timing starts.  A prefill step
is one MoE layer forward over one batch of synthetic tokens: route (K1) ->
pack with the balanced tile schedule (K2) -> grouped SwiGLU gate/up + down
(K3) -> merge (K5).  A decode step is one token through 16 layer copies: one
replay of a hipGraph of 16 single-launch layers (route + top-k + gate/up +
down + merge in one launch each); its throughput counts the 16 layer
launches.  Steps rotate over several independently seeded layer copies so the
256 MB Infinity Cache cannot hold the streamed weights between steps.

The default workload is the T = 1 decode layer (128 experts, top-8, all
resident), the configuration the metric is quoted on.  The same JSON line
also carries the T = 512 prefill (uniform routing), the T = 4096 prefill on
the Zipf(1.1)-biased routing with every expert resident (the grouped SwiGLU
the T = 4096 target names; the uniform routing beside it), the T = 4096
Zipf-skewed layer with 32 resident experts and 8 demand staging slots
through the runtime, the runtime's T = 1 and T = 512 layer calls with every
expert resident (their host cost around the kernels), and the DeepSeek-V2-Lite
mixed-batch results
("workloads"), each with its own roofline figure, and CPU baselines: the
AVX2 bf16 SwiGLU expert kernel under oracle/ (a stand-in for ktransformers'
AVX2BF16_MOE, which is not available offline) timed on this host's cores on
the same layers and routings, each over a sample of about CPU_SAMPLE_S
seconds of CPU work.

Roofline: ``achieved`` is algorithmic bytes (or useful flops) of the dominant
kernel per launch divided by its mean duration, measured with HIP events on
the launch stream during the timed steps (for T = 4096: both grouped
launches against the layer's useful flops).  ``traffic`` is read from the
committed rocprofv3 counter summary of the same command under profiles/.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

METRIC = "MoE layer tok/s at T=1 and T=4096; HBM GB/s and MFMA util vs peak"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
H, I, E, K_TOP = 2048, 768, 128, 8
EXPERT_BYTES = 3 * I * H * 2   # 9 437 184
ROUTER_BYTES = E * H * 2
CPU_SAMPLE_S = 10.0            # seconds of CPU work per CPU-baseline sample


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="decode",
                    choices=["prefill512", "decode", "prefill4096", "prefill4096_zipf", "dsv2_mixed", "stack48",
                             "runtime_decode", "runtime_prefill512"])
    ap.add_argument("--no-extra", action="store_true",
                    help="only the main workload (for prefill4096: without the uniform-routing comparison)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0: physical cores of this process's CPUs (at most 16, one GPU's share) - 1")
    ap.add_argument("--cpu-seconds", type=float, default=CPU_SAMPLE_S,
                    help="CPU work per CPU-baseline sample (after two warm-up runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 5 device copies of 1 GiB (calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--calibrate-costs", metavar="PATH",
                    help="only measure the per-expert cost table of the placement planner and write it to PATH")
    return ap.parse_args()


def calibrate_copy():
    """Five dst.copy_(src) of 1 GiB each: a kernel with known HBM traffic
    (1 GiB read + 1 GiB written per dispatch) for counter calibration."""
    import torch
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "dispatches": 5}))


def calibrate_costs(path, device, threads, reps=15, group=32, copies=40):
    """Per-expert completion times by routed token count on this host, in the
    FileCosts format (benchmarks/pdscope_compare.py:55-85; the loads of the
    reference's costs/cost_table.json):
      cpu_ms  one expert's n rows on the host's AVX2 stand-in CPU kernel
              (oracle/cpu_moe_avx2.c, `threads` threads), its weights rotated
              through `copies` host copies so DRAM serves them, median;
      gpu_ms  one expert's share of a resident grouped launch: the gate/up and
              down launches over `group` experts of n rows each, HIP events,
              divided by `group` (the runtime launches its GPU experts together),
              median;
      h2d_ms  its 9 MiB gate|up|down block copied from pinned host memory into
              an HBM slot (median) plus gpu_ms.
    """
    import numpy as np
    import torch
    from oracle import oracle as orc
    from pdscope_amd import ops, synthetic
    loads = (1, 4, 16, 64, 128, 256, 1024, 4096)
    T = 4096
    lay = synthetic.make_layer(H, I, E, K_TOP, True, seed=20261013, device=device)
    x = synthetic.make_tokens(T, H, seed=20261014, device=device)
    slots = ops.slot_table([lay.experts[e] for e in range(E)], device)
    host = torch.empty((4, EXPERT_BYTES), dtype=torch.uint8, pin_memory=True)
    host.copy_(lay.experts[:4].view(torch.uint8).reshape(4, -1).cpu())
    slot = torch.empty(EXPERT_BYTES, dtype=torch.uint8, device=device)
    rows_max = group * loads[-1]
    h_ws = torch.empty(rows_max * I, dtype=torch.bfloat16, device=device)
    y = torch.empty(rows_max * H, dtype=torch.bfloat16, device=device)
    i32 = dict(dtype=torch.int32, device=device)
    sel_all = torch.arange(E, **i32)
    tile_start = torch.empty(E + 1, **i32)
    order = torch.empty(E, **i32)
    stream = torch.cuda.current_stream(device)
    copy_ms = []
    for r in range(reps + 2):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        slot.copy_(host[r % 4], non_blocking=True)
        b.record(stream)
        torch.cuda.synchronize(device)
        if r >= 2:
            copy_ms.append(a.elapsed_time(b))
    copy_med = statistics.median(copy_ms)
    experts_host = u16(lay.experts[:4])
    pool = [np.ascontiguousarray(experts_host[i % 4]) for i in range(copies)]
    x_host = u16(x)
    points = {}
    for n in loads:
        counts = torch.zeros(E, **i32)
        counts[:group] = n
        offsets = torch.zeros(E + 1, **i32)
        offsets[1:] = torch.cumsum(counts, 0)
        perm = torch.arange(group * n, **i32) % T
        bm = ops.grouped_block_m(n, n)
        ops.schedule(counts, sel_all, bm, out=tile_start, order=order)
        max_tiles = group * ((n + bm - 1) // bm)
        gpu = []
        for r in range(reps + 2):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            ops.swiglu_grouped(x, perm, offsets, order, tile_start, max_tiles, bm, slots, H, I, h_ws, y)
            b.record(stream)
            torch.cuda.synchronize(device)
            if r >= 2:
                gpu.append(a.elapsed_time(b) / group)
        rows = np.ascontiguousarray(x_host[np.arange(n) % T])
        sel = np.zeros(n, np.int64)
        coeff = np.ones(n, np.float32)
        cpu = []
        for r in range(2 + (5 if n >= 1024 else 9)):
            ptrs = [pool[r % copies].ctypes.data] * 4
            t0 = time.perf_counter()
            orc.cpu_moe_rows(rows, sel, coeff, ptrs, H, I, threads)
            if r >= 2:
                cpu.append((time.perf_counter() - t0) * 1e3)
        g = statistics.median(gpu)
        points[str(n)] = dict(cpu_ms=statistics.median(cpu), gpu_ms=g, h2d_ms=copy_med + g)
        log(f"[costs] n={n}: {points[str(n)]}")
    table = dict(schema_version=1, kind="pdscope_cost_table",
                 model="Qwen3-30B-A3B-shaped expert (H 2048, I 768), bf16",
                 platform=f"AMD Instinct MI355X + {cpu_model()}",
                 native_operator="AVX2 bf16 SwiGLU stand-in kernel (oracle/cpu_moe_avx2.c)", workers=threads,
                 loads=list(loads), points=points,
                 scope=f"per-expert completion time by routed token count: CPU stand-in path (weights from DRAM), "
                       f"one expert's share of a grouped launch over {group} resident experts, and pinned H2D copy "
                       f"({copy_med:.3f} ms per 9 MiB) plus that share; measured by bench.py --calibrate-costs. "
                       f"Recalibrate per machine.")
    with open(path, "w") as f:
        json.dump(table, f, indent=2)
        f.write("\n")
    print(json.dumps(dict(calibration="costs", path=path, loads=list(loads))))


def traffic_from_profiles(name):
    """HBM bytes per launch of the dominant kernel, from the committed counter
    summary profiles/<name> (line 'traffic_bytes_per_launch: N'), or None."""
    import re
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    except OSError:
        return None
    return float(m.group(1)) if m else None


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ----------------------------------------------------------------------------- GPU legs

def build_layers(n, device, seed0):
    from pdscope_amd import ops, synthetic
    layers = []
    for i in range(n):
        lay = synthetic.make_layer(H, I, E, K_TOP, True, seed=seed0 + 1000 * i, device=device)
        slots = ops.slot_table([lay.experts[e] for e in range(E)], device)
        layers.append((lay, slots))
    return layers


def run_prefill(T, steps, warmup, n_layers, device, seed0, bias=None):
    """Eager launches; HIP events bracket the grouped gate/up and down kernels
    in every timed step.  bias: the router's fp32 logit bias (the Zipf
    workload).  Each layer copy's row tile comes from its own routing's mean
    and largest expert rows, as the runtime chooses it for a resident launch."""
    import torch
    from pdscope_amd import layer, ops, synthetic
    layers = build_layers(n_layers, device, seed0)
    xs = [synthetic.make_tokens(T, H, seed=seed0 + 7 + 1000 * i, device=device) for i in range(n_layers)]
    ws = layer.MoEWorkspace(T, H, I, E, K_TOP, device)
    n = T * K_TOP
    _, _, _, packed = ws.views(T)
    stream = torch.cuda.current_stream(device)
    tiles = {}

    def step(i, ev=None):
        lay, slots = layers[i % n_layers]
        x = xs[i % n_layers]
        logits, ids, w = layer.route(x, lay.gate, ws, bias=bias)
        bm = tiles.get(i % n_layers, ops.grouped_block_m(n // E))
        max_tiles = (n + bm - 1) // bm + E
        # the down launch has its own row tile (layer.down_block_m); the pack
        # launch writes the balanced schedule for both
        bmd = layer.down_block_m(bm, H, I)
        ts_d = ws.tile_start_down if bmd != bm else ws.tile_start
        ops.pack(ids, E, out=packed, workspace=ws.pack_ws,
                 schedule=(ws.sel_all, bm, ws.sel_order, ws.tile_start) + ((bmd, ts_d) if bmd != bm else ()))
        if ev is not None:
            ev[0].record(stream)
        ops.swiglu_grouped_gateup(x, packed.perm_token, packed.offsets, ws.sel_order, ws.tile_start, max_tiles, bm,
                                  slots, H, I, ws.h_ws)
        if ev is not None:
            ev[1].record(stream)
        ops.swiglu_grouped_down(ws.h_ws, packed.offsets, ws.sel_order, ts_d, (n + bmd - 1) // bmd + E, bmd, slots,
                                H, I, ws.y)
        if ev is not None:
            ev[2].record(stream)
        ops.merge(ws.y, packed.row_of, w, ws.out[:T])

    # experts touched per layer (for algorithmic bytes) and each copy's row
    # tile, from its routing and grouping alone (no grouped launch on a tile
    # the timed steps do not use)
    touched, max_rows = [], []
    for i in range(n_layers):
        _, ids, _ = layer.route(xs[i], layers[i][0].gate, ws, bias=bias)
        ops.pack(ids, E, out=packed, workspace=ws.pack_ws)
        torch.cuda.synchronize(device)
        counts = ws.counts.cpu()
        live = counts[counts > 0]
        touched.append(int(live.numel()))
        max_rows.append(int(live.max()))
        tiles[i] = ops.grouped_block_m(int(live.sum()) // int(live.numel()), int(live.max()))
    for i in range(warmup):
        step(i)
    # the measured pass (no events: an event between launches costs the
    # stream a few microseconds), then a pass with events around the two
    # grouped launches of every step for their times
    torch.cuda.synchronize(device)
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - t0
    events = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(steps)]
    for i in range(steps):
        step(i, events[i])
    torch.cuda.synchronize(device)
    gateup_ms = [a.elapsed_time(b) for a, b, _ in events]
    down_ms = [b.elapsed_time(c) for _, b, c in events]
    grouped_ms = [g + d for g, d in zip(gateup_ms, down_ms)]
    mean_touched = sum(touched[i % n_layers] for i in range(steps)) / steps
    bmm = vendor_bmm_ms(n // E, device) if bias is None and n % E == 0 and n // E >= 128 else None
    return dict(T=T, wall_s=wall, ms_per_step=wall / steps * 1e3, tok_s=T * steps / wall,
                gateup_ms_mean=statistics.mean(gateup_ms), gateup_ms_median=statistics.median(gateup_ms),
                down_ms_mean=statistics.mean(down_ms), down_ms_median=statistics.median(down_ms),
                grouped_ms_mean=statistics.mean(grouped_ms), grouped_ms_median=statistics.median(grouped_ms),
                vendor_bmm=bmm, touched=mean_touched, max_rows=max(max_rows),
                block_m=sorted(set(tiles.values())), routing="zipf(1.1) bias" if bias is not None else "uniform",
                layers=n_layers, steps_run=steps, first_layer=layers[0], first_x=xs[0], ws=ws, bias=bias)


def vendor_bmm_ms(rows, device, reps=20):
    """The layer's expert GEMMs as the BLAS library runs them at their mean
    size: torch.bmm over E experts of `rows` rows each, gate|up
    ([rows, H] x [H, 2I]) and down ([rows, I] x [I, H]), contiguous operands.
    A library reference for the two grouped launches (which also gather the
    routed rows, apply SwiGLU and cover ragged per-expert row counts)."""
    import torch
    a = torch.randn(E, rows, H, dtype=torch.bfloat16, device=device)
    w1 = torch.randn(E, H, 2 * I, dtype=torch.bfloat16, device=device)
    h = torch.randn(E, rows, I, dtype=torch.bfloat16, device=device)
    w2 = torch.randn(E, I, H, dtype=torch.bfloat16, device=device)
    out = {}
    for name, fn in (("gateup", lambda: torch.bmm(a, w1)), ("down", lambda: torch.bmm(h, w2))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize(device)
        ms = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize(device)
            ms.append(e0.elapsed_time(e1))
        out[f"{name}_ms"] = statistics.median(ms)
    del a, w1, h, w2
    out["what"] = f"torch.bmm over {E} experts x {rows} rows (BLAS), gate|up then down"
    return out


def run_decode(steps, warmup, n_layers, device, seed0):
    """All layer copies captured in ONE hipGraph (as a decode step over a stack
    of resident layers replays them).  A step is one replay: one token through
    the n_layers layers.  Exactly `steps` replays are timed after `warmup`
    untimed ones between a HIP event on the replay stream before the first and
    one after the last; the layer time is their span over steps * n_layers
    launches, and both the throughput and the roofline come from it (the
    spread over replays comes from a second pass with an event after each).
    The same is done for the three-launch path (route + decode GEMV +
    down/merge) for reference."""
    import torch
    from pdscope_amd import layer, ops, synthetic
    layers = build_layers(n_layers, device, seed0)
    xs = [synthetic.make_tokens(1, H, seed=seed0 + 7 + 1000 * i, device=device) for i in range(n_layers)]
    wss = [layer.MoEWorkspace(1, H, I, E, K_TOP, device) for _ in range(n_layers)]
    stream = torch.cuda.current_stream(device)

    def capture(fused):
        side = torch.cuda.Stream(device)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(n_layers):
                layer.moe_forward(xs[i], layers[i][0].gate, layers[i][1], wss[i], fused_decode=fused)
        stream.wait_stream(side)
        torch.cuda.synchronize(device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n_layers):
                layer.moe_forward(xs[i], layers[i][0].gate, layers[i][1], wss[i], fused_decode=fused)
        torch.cuda.synchronize(device)
        return g

    def timed(g, nsteps, nwarm):
        # graph replay must equal eager execution, layer by layer
        eager = []
        for i in range(n_layers):
            layer.moe_forward(xs[i], layers[i][0].gate, layers[i][1], wss[i])
            eager.append(wss[i].out[:1].clone())
        g.replay()
        torch.cuda.synchronize(device)
        for i in range(n_layers):
            if not torch.equal(wss[i].out[:1], eager[i]):
                raise AssertionError("decode graph replay differs from eager execution")
        for _ in range(nwarm):
            g.replay()
        # the measured pass: exactly nsteps replays between two
        # synchronisations, a HIP event before the first and after the last
        # (an event between replays costs the stream a few microseconds)
        first, last = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        first.record(stream)
        for r in range(nsteps):
            g.replay()
        last.record(stream)
        torch.cuda.synchronize(device)
        wall = time.perf_counter() - t0
        # the spread over replays, from a second pass with an event after each
        events = [torch.cuda.Event(enable_timing=True) for _ in range(nsteps + 1)]
        events[0].record(stream)
        for r in range(nsteps):
            g.replay()
            events[r + 1].record(stream)
        torch.cuda.synchronize(device)
        replay_ms = [events[r].elapsed_time(events[r + 1]) for r in range(nsteps)]
        return wall, replay_ms, first.elapsed_time(last)

    fused = ops.decode_layer_supported(H, I, E, K_TOP, device)
    g = capture(True)
    wall, replay_ms, total_ms = timed(g, steps, warmup)
    if fused and ops.decode_workspace_error(device, H):
        raise AssertionError("a bounded wait of the fused decode kernel gave up")
    g3 = capture(False)
    _, replay_ms3, _ = timed(g3, min(steps, 200), 20)
    chain = run_decode_chain(layers, device, seed0, reps=max(20, min(steps, 500) // 4)) if fused else None
    read_ms = plain_read_ms(K_TOP * EXPERT_BYTES + ROUTER_BYTES, n_layers, device)
    kernel = ("decode_layer_kernel (route + top-k + gate/up + down/merge in one launch), "
              f"{n_layers} layers per hipGraph" if fused else
              f"route_gemv + decode_gateup + decode_down, {n_layers} layers per hipGraph")
    launches = steps * n_layers
    layer_ms = [ms / n_layers for ms in replay_ms]
    return dict(T=1, wall_s=wall, event_s=total_ms / 1e3, ms_per_step=total_ms / steps,
                tok_s=launches / (total_ms / 1e3), wall_tok_s=launches / wall, kernel=kernel,
                layer_ms_mean=total_ms / launches, layer_ms_median=statistics.median(layer_ms),
                layer_ms_min=min(layer_ms), layer_ms_max=max(layer_ms),
                three_launch_layer_ms=statistics.median(replay_ms3) / n_layers, steps_run=steps,
                layer_launches=launches, chain=chain, plain_read_layer_ms=read_ms, layers=n_layers,
                first_layer=layers[0], first_x=xs[0], ws=wss[0])


def run_decode_chain(layers, device, seed0, reps):
    """The same layers chained as a decode step runs them, in one hipGraph:
    layer l takes the previous output plus the residual stream
    (x_eff = bf16(x + resid)) and predicts layer l+1's experts from its own
    input (the gate-fallback predictor, fused into the launch).  Returns the
    per-layer time and how many predicted experts layer l+1 then selected."""
    import torch
    from pdscope_amd import ops, synthetic
    n = len(layers)
    x0 = synthetic.make_tokens(1, H, seed=seed0 + 11, device=device)
    r0 = synthetic.make_tokens(1, H, seed=seed0 + 12, device=device)
    bufs = [dict(out=torch.empty((1, H), dtype=torch.bfloat16, device=device),
                 x_out=torch.empty((1, H), dtype=torch.bfloat16, device=device),
                 logits=torch.empty((1, E), dtype=torch.bfloat16, device=device),
                 ids=torch.empty((1, K_TOP), dtype=torch.int32, device=device),
                 weights=torch.empty((1, K_TOP), dtype=torch.bfloat16, device=device),
                 h_ws=torch.empty(K_TOP * I, dtype=torch.bfloat16, device=device),
                 pred=torch.full((K_TOP,), -1, dtype=torch.int32, device=device)) for _ in range(n)]

    def step():
        x, r = x0, r0
        for l, (lay, slots) in enumerate(layers):
            b = bufs[l]
            extra = dict(next_gate=layers[l + 1][0].gate, pred_out=b["pred"]) if l + 1 < n else {}
            ops.decode_layer(x, lay.gate, slots, I, K_TOP, True, out=b["out"], logits=b["logits"], ids=b["ids"],
                             weights=b["weights"], h_ws=b["h_ws"], resid=r, x_out=b["x_out"], **extra)
            x, r = b["out"], b["x_out"]

    stream = torch.cuda.current_stream(device)
    side = torch.cuda.Stream(device)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        step()
    stream.wait_stream(side)
    torch.cuda.synchronize(device)
    eager = [b["out"].clone() for b in bufs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    g.replay()
    torch.cuda.synchronize(device)
    if not all(torch.equal(b["out"], e) for b, e in zip(bufs, eager)):
        raise AssertionError("chained decode graph replay differs from eager execution")
    hits = sum(len(set(bufs[l]["pred"].tolist()) & set(bufs[l + 1]["ids"][0].tolist())) for l in range(n - 1))
    for _ in range(5):
        g.replay()
    # timed as the plain decode step: HIP events before the first replay and
    # after the last
    first, last = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    torch.cuda.synchronize(device)
    first.record(stream)
    for k in range(reps):
        g.replay()
    last.record(stream)
    torch.cuda.synchronize(device)
    return dict(layer_ms_mean=first.elapsed_time(last) / (reps * n), predictor_hits=hits,
                predictor_total=K_TOP * (n - 1),
                what="residual sum + next-layer gate-fallback prediction fused into each layer's launch")


def plain_read_ms(nbytes, n_regions, device, reps=12):
    """Time of a vendor GEMV reading `nbytes` once: torch.mv of a [nbytes / 4096, 2048]
    bf16 matrix (the BLAS library's matrix-vector kernel), over distinct
    matrices, one per layer copy, so that the 256 MB Infinity Cache holds
    none of them: a library reference for one launch streaming that many bytes."""
    import torch
    rows = nbytes // (2 * H)
    mats = torch.empty((n_regions, rows, H), dtype=torch.bfloat16, device=device).normal_()
    v = torch.ones(H, dtype=torch.bfloat16, device=device)
    out = torch.empty((n_regions, rows), dtype=torch.bfloat16, device=device)
    for r in range(n_regions):
        torch.mv(mats[r], v, out=out[r])
    torch.cuda.synchronize(device)
    ms = []
    for _ in range(reps):   # the copies back to back between two events, as the decode graph is timed
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for r in range(n_regions):
            torch.mv(mats[r], v, out=out[r])
        e1.record()
        torch.cuda.synchronize(device)
        ms.append(e0.elapsed_time(e1) / n_regions)
    del mats, out
    return statistics.median(ms[2:])


def run_zipf_staged(steps, warmup, n_layers, device, seed0):
    """T = 4096 prefill through the drop-in runtime (PDScopeCudaRuntime.forward)
    with a Zipf(1.1) router bias: per layer the 32 hottest experts are resident
    in the cache pool and every other touched expert is copied from pinned
    host memory into one of 8 demand staging slots, its grouped launch
    following its copy while the next copies stream.  A step is one whole
    layer call (host-synchronous, as the runtime is), timed by wall clock."""
    import torch
    from pdscope_amd import ops, synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.executor import masters_from_block
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    T = 4096
    bias, perm = synthetic.zipf_bias(E, 1.1, seed=seed0, device=device)
    hottest = sorted(range(E), key=lambda e: int(perm[e]))[:32]
    gates, masters, hot = [], {}, []
    for i in range(n_layers):
        lay = synthetic.make_layer(H, I, E, K_TOP, True, seed=seed0 + 9000 + 1000 * i, device=device)
        masters.update(masters_from_block(i, lay.experts, E, H, I))
        gates.append(lay.gate)
        hot += [ExpertKey(i, e, "bf16") for e in hottest]
        if i == 0:
            lay0 = lay
        del lay
    torch.cuda.empty_cache()
    xs = [synthetic.make_tokens(T, H, seed=seed0 + 9007 + 1000 * i, device=device) for i in range(n_layers)]
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, demand_slots=8, device=device,
                            diagnostics=False)
    try:
        def step(i):
            # one request per pass over the rotated layers (the ledger orders events per request)
            return rt.forward(xs[i % n_layers], gates[i % n_layers], layer=i % n_layers, step=0, top_k=K_TOP,
                              request=f"bench{i // n_layers}", bias=bias, prefetch=False)

        warmup = -(-warmup // n_layers) * n_layers  # whole passes, so timed passes start at layer 0
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize(device)
        rows, times = [], []
        t0 = time.perf_counter()
        for i in range(warmup, warmup + steps):
            a = time.perf_counter()
            _, _, row = step(i)
            torch.cuda.synchronize(device)
            times.append(time.perf_counter() - a)
            rows.append(row)
        wall = time.perf_counter() - t0
        n_demand = [len(r["decision"]["on_demand_queue"]) for r in rows]
        n_touched = [len(r["token_counts"]) for r in rows]
        h2d = [r["counters"].get("h2d_bytes_completed", 0) for r in rows]
        max_rows = max(max(r["token_counts"].values()) for r in rows)
        # the copy engine alone: the same number of expert blocks, back to back, into the staging slots
        srcs = [masters[ExpertKey(0, e, "bf16")].flat for e in range(E) if e not in hottest]
        nc = len(srcs)
        copy_gbs = copy_engine_gbs(rt, srcs, device)
    finally:
        rt.close()
    t = statistics.mean(times)
    h2d_mean = statistics.mean(h2d)
    pcie = dict(bound="pcie_h2d", achieved=h2d_mean / t / 1e9, peak=copy_gbs, unit="GB/s",
                peak_kind="measured back-to-back expert copies on this host")
    pcie["frac"] = pcie["achieved"] / pcie["peak"]
    flops = 2.0 * T * K_TOP * 3 * I * H
    return dict(tok_s=T * steps / wall, ms_per_step=wall / steps * 1e3, kernel="whole layer through the runtime",
                kernel_ms_mean=t * 1e3, kernel_ms_median=statistics.median(times) * 1e3,
                resident_experts=len(hottest), demand_slots=8, experts_touched=statistics.mean(n_touched),
                demand_experts=statistics.mean(n_demand), h2d_bytes_per_layer=h2d_mean,
                max_rows_per_expert=max_rows, pcie=pcie, layer_tflops=flops / t / 1e12,
                layers_rotated=n_layers, copy_only_ms=nc * EXPERT_BYTES / copy_gbs / 1e6,
                first_layer=(lay0, None), first_x=xs[0], bias=bias)


def run_stack(n_layers, device, seed0, T_prefill=2048, n_decode=64, cap_gib=24, hot_per_layer=40, demand_slots=8):
    """48 Qwen3-30B-A3B-shaped MoE blocks through the drop-in runtime
    (pdscope_amd.stack): the expert masters live in pinned host memory
    (48 x 128 x 9 MiB); the process's device memory stays within cap_gib
    (allocator capped 1 GiB below it, expert slots sized within the cap: a
    static hot set chosen by calibration routing, speculative prefetch slots
    and 8 demand staging slots); the gate-fallback predictor (layer l+1 gate
    on the layer-l activation) prefetches, and decode layers replay their
    captured single-launch graph over the resident set.  Prefill 2048
    tokens, then 64 decode steps.  The run raises if the ledger does not
    close or the device footprint exceeds the cap."""
    from pdscope_amd import stack
    t_setup = time.perf_counter()
    model = stack.build_stack(n_layers, device, seed0=seed0, hot_per_layer=hot_per_layer)
    session = stack.StackSession(model, device, stack.StackBudget(device_total=cap_gib << 30,
                                                                  demand_slots=demand_slots))
    setup_s = time.perf_counter() - t_setup
    try:
        res = session.run(T_prefill, n_decode)
        copy_gbs = copy_engine_gbs(session.runtime, [model.expert_block(0, e) for e in range(E)], device)
    finally:
        session.close()
    prefill, decode = res["prefill"], res["decode"]
    pcie = dict(bound="pcie_h2d", achieved=prefill["h2d_gbs"], peak=copy_gbs, unit="GB/s",
                peak_kind="measured back-to-back expert copies on this host", phase="prefill")
    pcie["frac"] = pcie["achieved"] / pcie["peak"]
    del model, session
    return dict(tok_s=decode["tok_s"], ms_per_step=1e3 / decode["tok_s"], kernel="48-layer stack through the runtime",
                kernel_ms_mean=1e3 * decode["wall_s"] / n_decode, prefill=prefill, decode=decode,
                predictor=res["predictor"], memory=res["memory"], closure=res["closure"], layers=n_layers,
                setup_s=setup_s, tokens_prefill=T_prefill, decode_steps=n_decode, pcie=pcie, steps_run=n_decode)


def run_runtime_decode(steps, warmup, n_layers, device, seed0, T=1):
    """Layer calls through the drop-in runtime with every expert resident.
    T=1 (decode): one token per PDScopeCudaRuntime.forward call, each layer
    served by its bound single-launch kernel (with the next layer's
    prediction), the routing read back for the ledger's reveal, acquire /
    release of the routed experts and the trace row.  T>1 (prefill, step 0
    of a new request per pass): the whole resident layer launched before the
    counts come back, the demand revealed while it runs.  A step is one
    layer call, timed by wall clock: the host cost of the runtime around the
    layer's kernels."""
    import torch
    from pdscope_amd import synthetic
    from pdscope_amd.cache import ExpertKey
    from pdscope_amd.executor import masters_from_block
    from pdscope_amd.pdscope_runtime import PDScopeCudaRuntime
    gates, masters, hot = [], {}, []
    for l in range(n_layers):
        lay = synthetic.make_layer(H, I, E, K_TOP, True, seed=seed0 + 40000 + 1000 * l, device=device)
        masters.update(masters_from_block(l, lay.experts, E, H, I))
        gates.append(lay.gate)
        hot += [ExpertKey(l, e, "bf16") for e in range(E)]
        del lay
    torch.cuda.empty_cache()
    rt = PDScopeCudaRuntime(masters, hot_keys=hot, speculative_slots=0, demand_slots=8, resident_graphs=True,
                            device=device, diagnostics=False)
    x = synthetic.make_tokens(T, H, seed=seed0 + 40999, device=device)
    try:
        def pass_(step):
            for l in range(n_layers):
                # decode steps continue one request; a prefill is step 0 of a request of its own
                rt.forward(x, gates[l], layer=l, step=step if T == 1 else 0,
                           request="runtime_decode" if T == 1 else f"runtime_prefill_{step}", top_k=K_TOP,
                           next_gate=gates[l + 1] if l + 1 < n_layers else None)
        n_warm = max(1, -(-warmup // n_layers))
        n_timed = max(1, steps // n_layers)
        for p in range(n_warm):
            pass_(1 + p)
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        for p in range(n_timed):
            pass_(1 + n_warm + p)
        torch.cuda.synchronize(device)
        wall = time.perf_counter() - t0
    finally:
        rt.close()
    calls = n_timed * n_layers
    t = wall / calls
    touched = min(E, T * K_TOP)
    layer_bytes = touched * EXPERT_BYTES + ROUTER_BYTES + 2 * T * H * 2
    hbm = dict(bound="hbm", achieved=layer_bytes / t / 1e9, peak=HBM_PEAK_GBS, unit="GB/s")
    hbm["frac"] = hbm["achieved"] / hbm["peak"]
    return dict(tok_s=T / t, ms_per_step=t * 1e3,
                kernel=f"PDScopeCudaRuntime.forward, T={T}, all experts resident",
                kernel_ms_mean=t * 1e3, host_us_per_layer_call=t * 1e6, layers_rotated=n_layers, hbm=hbm,
                steps_run=calls)


def copy_engine_gbs(rt, srcs, device):
    """Back-to-back expert copies from pinned host memory into the runtime's
    staging slots on a side stream: the H2D rate the staging path can reach."""
    import torch
    from pdscope_amd import ops
    dst = rt.executor.staging
    s = torch.cuda.Stream(device)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for j, src in enumerate(srcs):
        ops.stage_expert(dst[j % len(dst)][:EXPERT_BYTES], src.view(torch.uint8), stream=s)
    e1.record(s)
    torch.cuda.synchronize(device)
    return len(srcs) * EXPERT_BYTES / (e0.elapsed_time(e1) / 1e3) / 1e9


def run_dsv2_mixed(steps, warmup, n_layers, device, seed0):
    """DeepSeek-V2-Lite layer (64 routed experts of 1408, top-6 without
    renormalisation, 2 shared experts as one 2816 MLP) on one mixed ragged
    batch: 48 decode tokens + chunked-prefill segments of 256 and 1000 tokens
    in one launch (the MoE math is per token, so segments only set T)."""
    import torch
    from pdscope_amd import layer, ops, synthetic
    cfg = synthetic.DSV2
    Hd, Id, Ed, kd, Is = cfg["H"], cfg["I"], cfg["E"], cfg["k"], cfg["shared_I"]
    T = 48 + 256 + 1000
    lays = []
    for i in range(n_layers):
        lay = synthetic.make_layer(Hd, Id, Ed, kd, False, seed=seed0 + 5000 + 1000 * i, device=device, shared_I=Is)
        lays.append((lay, ops.slot_table([lay.experts[e] for e in range(Ed)], device),
                     ops.slot_table([lay.shared], device)))
    xs = [synthetic.make_tokens(T, Hd, seed=seed0 + 5007 + 1000 * i, device=device) for i in range(n_layers)]
    ws = layer.MoEWorkspace(T, Hd, Id, Ed, kd, device, shared_I=Is)
    stream = torch.cuda.current_stream(device)

    def step(i):
        lay, slots, shared = lays[i % n_layers]
        layer.moe_forward(xs[i % n_layers], lay.gate, slots, ws, normalize=False, shared_slot=shared)

    touched = []
    for i in range(n_layers):
        step(i)
        torch.cuda.synchronize(device)
        touched.append(int((ws.counts > 0).sum().item()))
    for i in range(warmup):
        step(i)
    # the measured pass, HIP events before the first step and after the last
    # (an event between steps costs the stream a few microseconds); then the
    # spread over steps from a pass with an event after each
    first, last = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    torch.cuda.synchronize(device)
    t0 = time.perf_counter()
    first.record(stream)
    for i in range(steps):
        step(i)
    last.record(stream)
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - t0
    mean_ms = first.elapsed_time(last) / steps
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    events[0].record(stream)
    for i in range(steps):
        step(i)
        events[i + 1].record(stream)
    torch.cuda.synchronize(device)
    layer_ms = [events[i].elapsed_time(events[i + 1]) for i in range(steps)]
    mean_touched = sum(touched[i % n_layers] for i in range(steps)) / steps
    expert = 3 * Id * Hd * 2
    layer_bytes = mean_touched * expert + 3 * Is * Hd * 2 + Ed * Hd * 2 + 2 * T * Hd * 2
    layer_flops = 2.0 * T * kd * 3 * Id * Hd + 2.0 * T * 3 * Is * Hd + 2.0 * T * Ed * Hd
    t = mean_ms / 1e3
    hbm = dict(bound="hbm", achieved=layer_bytes / t / 1e9, peak=HBM_PEAK_GBS, unit="GB/s")
    hbm["frac"] = hbm["achieved"] / hbm["peak"]
    return dict(tok_s=T * steps / wall, ms_per_step=wall / steps * 1e3,
                kernel="whole layer (events around the measured steps)",
                kernel_ms_mean=mean_ms, kernel_ms_median=statistics.median(layer_ms),
                experts_touched=mean_touched, tokens=T, layers_rotated=n_layers, hbm=hbm,
                layer_tflops=layer_flops / t / 1e12, layer_bytes=layer_bytes,
                shape=dict(hidden=Hd, experts=Ed, intermediate=Id, top_k=kd, shared_intermediate=Is))


# ----------------------------------------------------------------------------- CPU baseline

CPU_SHARE = 16   # host CPUs that one GPU's work may occupy


def host_cores():
    """Logical CPUs this process may run on, the physical cores among them
    (distinct (package, core) pairs from sysfs) and the CPU model."""
    try:
        aff = sorted(os.sched_getaffinity(0))
    except AttributeError:
        aff = list(range(os.cpu_count() or 2))
    cores = set()
    for c in aff:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            cores.add((open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip()))
        except OSError:
            cores.add(("?", str(c)))
    return dict(logical_cpus=len(aff), physical_cores=len(cores), share=CPU_SHARE, model=cpu_model())


def cpu_threads(requested):
    """Worker threads of the CPU baseline: one per physical core of the
    process's CPUs, within one GPU's share of the host, minus one for the
    control thread (the reference's README.md:142 and docs/REPRODUCE.md:38-41)."""
    if requested > 0:
        return requested
    hc = host_cores()
    return max(1, min(hc["physical_cores"], hc["logical_cpus"], CPU_SHARE) - 1)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def u16(t):
    import numpy as np
    import torch
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def timed_sample(run, budget_s, warm=2, min_runs=3):
    """run(r) repeated after `warm` untimed calls until `budget_s` seconds of
    timed work (and at least min_runs runs) have passed; the per-run times."""
    for r in range(warm):
        run(r)
    times = []
    r = warm
    while len(times) < min_runs or sum(times) < budget_s:
        t0 = time.perf_counter()
        run(r)
        times.append(time.perf_counter() - t0)
        r += 1
    return times


def cpu_baseline_prefill(lay, x, threads, budget_s, *, bias=None, what="", warm=2):
    """The full expert work of one layer's routing (all T*k rows, each through
    its expert, scaled by its routing weight) on the host cores, repeated for
    about budget_s seconds; tokens per second of CPU time."""
    import numpy as np
    from oracle import oracle as orc
    from pdscope_amd import layer
    T = x.shape[0]
    ws = layer.MoEWorkspace(T, H, I, E, K_TOP, x.device, route_only=True)
    layer.route(x, lay.gate, ws, bias=bias)
    ids = ws.ids[:T].cpu().numpy()
    w = ws.weights[:T].float().cpu().numpy()
    x_host = u16(x)
    experts = np.ascontiguousarray(u16(lay.experts))
    ptrs = [experts[e].ctypes.data for e in range(E)]
    rows = np.ascontiguousarray(np.repeat(x_host, K_TOP, axis=0))
    sel = ids.reshape(-1).astype(np.int64)
    coeff = w.reshape(-1).astype(np.float32)
    times = timed_sample(lambda r: orc.cpu_moe_rows(rows, sel, coeff, ptrs, H, I, threads), budget_s, warm=warm)
    total = sum(times)
    return dict(value=T * len(times) / total, unit="tok/s", cores=threads, kind="port",
                sample=f"{what}T={T} layer, full expert work of its routing ({T * K_TOP} rows through "
                       f"{int((np.bincount(sel, minlength=E) > 0).sum())} experts), {len(times)} runs "
                       f"({total:.1f} s of CPU work) after {warm} warm-ups, {threads} threads, {cpu_model()}",
                median_s=statistics.median(times))


def cpu_baseline_decode(lay, x, threads, budget_s, copies=8, warm=2):
    """One T=1 token through its 8 routed experts on the host cores, repeated
    for about budget_s seconds; the 8 experts' weights rotate through
    `copies` distinct host copies (copies x 75 MB, more than a last-level
    cache holds) so DRAM serves them, as it serves a CPU decode step."""
    import ctypes
    import numpy as np
    from oracle import oracle as orc
    from pdscope_amd import layer
    ws = layer.MoEWorkspace(1, H, I, E, K_TOP, x.device, route_only=True)
    layer.route(x, lay.gate, ws)
    ids = np.ascontiguousarray(ws.ids[:1].cpu().numpy().reshape(-1), dtype=np.int32)
    w = np.ascontiguousarray(u16(ws.weights[:1]).reshape(-1))
    x_host = np.ascontiguousarray(u16(x).reshape(-1))
    experts = u16(lay.experts)
    u16p = ctypes.POINTER(ctypes.c_uint16)
    bufs, tables = [], []
    for _ in range(copies):
        c = np.ascontiguousarray(experts[ids].copy())
        bufs.append(c)
        ptrs = [ctypes.cast(experts[0].ctypes.data, u16p)] * E
        for s, e in enumerate(ids):
            ptrs[e] = ctypes.cast(c[s].ctypes.data, u16p)
        tables.append((u16p * E)(*ptrs))
    out = np.empty(H, np.uint16)
    L = orc.lib()

    def run(r):
        rc = L.cpu_moe_decode(x_host.ctypes.data_as(u16p), ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                              w.ctypes.data_as(u16p), K_TOP, tables[r % copies], H, I, out.ctypes.data_as(u16p),
                              threads)
        if rc:
            raise RuntimeError("cpu_moe_decode unavailable (needs AVX2+FMA)")
    times = timed_sample(run, budget_s, warm=warm)
    total = sum(times)
    return dict(value=len(times) / total, unit="tok/s", cores=threads, kind="port",
                sample=f"T=1 tokens through their 8 routed experts of one layer, {len(times)} tokens "
                       f"({total:.1f} s of CPU work) after {warm} warm-ups, weights rotated over {copies} host "
                       f"copies, {threads} threads, {cpu_model()}",
                median_s=statistics.median(times), dram_gbs=K_TOP * EXPERT_BYTES * len(times) / total / 1e9)


# ----------------------------------------------------------------------------- reporting

def prefill_record(res):
    """Roofline figures of the grouped SwiGLU: `mfma` counts both launches
    (gate/up + down) against the layer's useful flops 2*T*k*3*I*H (no tile
    padding); `hbm` is the gate/up launch's algorithmic bytes (the HBM-bound
    launch at T=512) over its own time."""
    T, touched = res["T"], res["touched"]
    n = T * K_TOP
    gateup_bytes = touched * 2 * I * H * 2 + T * H * 2 + n * I * 2
    grouped_flops = 2.0 * n * 3 * I * H
    t_gu = res["gateup_ms_mean"] / 1e3
    t_grp = res["grouped_ms_mean"] / 1e3
    layer_bytes = touched * EXPERT_BYTES + ROUTER_BYTES + 2 * T * H * 2
    layer_flops = grouped_flops + 2.0 * T * E * H
    hbm = dict(bound="hbm", achieved=gateup_bytes / t_gu / 1e9, peak=HBM_PEAK_GBS, unit="GB/s",
               kernel="grouped_kernel<gateup>")
    hbm["frac"] = hbm["achieved"] / hbm["peak"]
    mfma = dict(bound="mfma", achieved=grouped_flops / t_grp / 1e12, peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                kernel="grouped_kernel<gateup> + grouped_kernel<down>", flops=grouped_flops)
    mfma["frac"] = mfma["achieved"] / mfma["peak"]
    gu_flops = 2.0 * n * H * 2 * I
    layer_s = res["ms_per_step"] / 1e3
    return dict(tok_s=res["tok_s"], ms_per_step=res["ms_per_step"], routing=res["routing"],
                kernel="grouped_kernel<gateup> + grouped_kernel<down>",
                kernel_ms_mean=res["grouped_ms_mean"], kernel_ms_median=res["grouped_ms_median"],
                gateup_ms_mean=res["gateup_ms_mean"], gateup_ms_median=res["gateup_ms_median"],
                down_ms_mean=res["down_ms_mean"], down_ms_median=res["down_ms_median"],
                gateup_mfma_frac=gu_flops / t_gu / 1e12 / BF16_PEAK_TFLOPS, vendor_bmm=res["vendor_bmm"],
                gateup_bytes=gateup_bytes, grouped_flops=grouped_flops, experts_touched=touched,
                max_rows_per_expert=res["max_rows"], block_m=res["block_m"], layers_rotated=res["layers"],
                hbm=hbm, mfma=mfma, layer_hbm_gbs=layer_bytes / layer_s / 1e9,
                layer_mfma_tflops=layer_flops / layer_s / 1e12)


def decode_record(res):
    layer_bytes = K_TOP * EXPERT_BYTES + ROUTER_BYTES + 2 * H * 2
    t = res["layer_ms_mean"] / 1e3
    hbm = dict(bound="hbm", achieved=layer_bytes / t / 1e9, peak=HBM_PEAK_GBS, unit="GB/s")
    hbm["frac"] = hbm["achieved"] / hbm["peak"]
    read_ms = res["plain_read_layer_ms"]
    return dict(tok_s=res["tok_s"], ms_per_step=res["ms_per_step"], kernel=res["kernel"],
                clock="HIP events on the replay stream over the timed replays (throughput and roofline)",
                wall_tok_s=res["wall_tok_s"], layer_launches=res["layer_launches"],
                kernel_ms_mean=res["layer_ms_mean"], kernel_ms_median=res["layer_ms_median"],
                kernel_ms_min=res["layer_ms_min"], kernel_ms_max=res["layer_ms_max"],
                three_launch_layer_ms=res["three_launch_layer_ms"],
                kernel_bytes=layer_bytes, layers_rotated=res["layers"], hbm=hbm,
                vendor_gemv=dict(ms=read_ms, gbs=layer_bytes / (read_ms / 1e3) / 1e9,
                                 layer_over_gemv=res["layer_ms_mean"] / read_ms,
                                 what="torch.mv (BLAS GEMV) reading the layer's byte count once per launch, "
                                      "launches back to back over distinct matrices"),
                chained_step=res["chain"])


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the MoE layer path here is "
              "single-GPU and multi-GPU figures are not measured", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return
    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from pdscope_amd import _lib, synthetic
    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    threads = cpu_threads(args.cpu_threads)
    if args.calibrate_costs:
        calibrate_costs(args.calibrate_costs, device, threads)
        return

    plan = {"prefill512": ("prefill", 512, 4), "decode": ("decode", 1, 16), "prefill4096": ("prefill", 4096, 2),
            "prefill4096_zipf": ("zipf", 4096, 2), "dsv2_mixed": ("dsv2", 1304, 4), "stack48": ("stack", 2048, 48),
            "runtime_decode": ("rtdecode", 1, 4), "runtime_prefill512": ("rtdecode", 512, 4)}
    # the 48-layer stack pins 58 GB of host masters: it runs only when asked for
    order = [args.workload] + ([] if args.no_extra else [w for w in plan if w not in (args.workload, "stack48")])
    records, raw = {}, {}
    for wl in order:
        kind, T, nl = plan[wl]
        main_leg = wl == args.workload
        # extra legs: enough warm-up for the weight pages of every layer copy
        # to be mapped, and steps enough for a stable mean (a few seconds each)
        steps = args.steps if main_leg else {"prefill512": 400, "decode": 500, "prefill4096": 200, "prefill4096_zipf": 20,
                                                       "dsv2_mixed": 300, "runtime_decode": 800,
                                                       "runtime_prefill512": 200}[wl]
        warmup = args.warmup if main_leg else {"prefill512": 100, "decode": 200, "prefill4096": 50, "prefill4096_zipf": 2,
                                                        "dsv2_mixed": 50, "runtime_decode": 80,
                                                        "runtime_prefill512": 20}[wl]
        if kind == "decode":
            steps = max(steps, 1)
        log(f"[bench] {wl}: T={T} layers={nl} steps={steps} warmup={warmup}")
        if kind == "prefill" and T == 4096:
            # the staged T=4096 layer's weights, tokens and Zipf(1.1) router bias with every
            # expert resident: the grouped SwiGLU whose MFMA fraction the record reports;
            # the uniform routing of the same shape is recorded beside it
            bias, _ = synthetic.zipf_bias(E, 1.1, seed=20261011, device=device)
            res = run_prefill(T, steps, warmup, nl, device, 20261011 + 9000, bias=bias)
            rec = prefill_record(res)
            if not args.no_extra:
                uni = run_prefill(T, max(20, steps // 2), max(5, warmup // 2), nl, device, 20261011)
                rec["uniform_routing"] = {kk: v for kk, v in prefill_record(uni).items()
                                          if kk in ("tok_s", "kernel_ms_mean", "gateup_ms_mean", "down_ms_mean",
                                                    "gateup_mfma_frac", "mfma", "vendor_bmm", "block_m")}
                for kk in ("first_layer", "first_x", "ws", "bias"):
                    uni.pop(kk, None)
        elif kind == "prefill":
            res = run_prefill(T, steps, warmup, nl, device, 20261011)
            rec = prefill_record(res)
        elif kind == "dsv2":
            res = run_dsv2_mixed(steps, warmup, nl, device, 20261011)
            rec = dict(res)
        elif kind == "zipf":
            res = run_zipf_staged(steps, warmup, nl, device, 20261011)
            rec = dict(res)
        elif kind == "stack":
            res = run_stack(nl, device, 20261011)
            rec = dict(res)
        elif kind == "rtdecode":
            res = run_runtime_decode(steps, warmup, nl, device, 20261011, T=T)
            rec = dict(res)
        else:
            res = run_decode(steps, warmup, nl, device, 20261011)
            rec = decode_record(res)
        rec["steps"], rec["warmup"] = res.get("steps_run", steps), warmup
        bw = rec.get("hbm") or rec["pcie"]
        log(f"[bench] {wl}: {rec['tok_s']:.1f} tok/s, {rec['ms_per_step']:.4f} ms/step, kernel "
            f"{rec['kernel_ms_mean']:.4f} ms, {bw['achieved']:.0f} GB/s ({bw['bound']})")
        records[wl] = rec
        raw[wl] = res
        if not args.no_cpu_baseline and wl in ("prefill512", "decode", "prefill4096", "prefill4096_zipf"):
            log(f"[bench] {wl}: CPU baseline on {threads} threads, ~{args.cpu_seconds:.0f} s")
            lay0 = res["first_layer"][0]
            if kind == "decode":
                cb = cpu_baseline_decode(lay0, res["first_x"], threads, args.cpu_seconds)
                # thread sweep (docs/REPRODUCE.md:50-52 of the reference), a short sample per count
                sweep = []
                for nt in sorted({1, 2, 4, 8, threads}):
                    s = cpu_baseline_decode(lay0, res["first_x"], nt, 1.5, warm=1)
                    sweep.append(dict(threads=nt, tok_s=s["value"], dram_gbs=s["dram_gbs"]))
                cb["thread_sweep"] = sweep
            elif res.get("bias") is not None:
                cb = cpu_baseline_prefill(lay0, res["first_x"], threads, args.cpu_seconds, bias=res["bias"],
                                          what="Zipf(1.1)-biased ")
            else:
                cb = cpu_baseline_prefill(lay0, res["first_x"], threads, args.cpu_seconds)
            hc = cb["host"] = host_cores()
            cb["sample"] += (f"; host: {hc['logical_cpus']} logical CPUs and {hc['physical_cores']} physical cores "
                             f"in this process's affinity, {threads} workers = min(physical cores, "
                             f"{CPU_SHARE}-CPU share of one GPU) - 1 for the control thread")
            rec["cpu_baseline"] = cb
            log(f"[bench] {wl}: CPU baseline {cb['value']:.2f} tok/s")
        for k in ("first_layer", "first_x", "ws", "bias"):
            res.pop(k, None)
            rec.pop(k, None)
        torch.cuda.empty_cache()

    main = records[args.workload]
    if args.workload == "prefill4096":
        roof = dict(main["mfma"])
    elif args.workload in ("prefill4096_zipf", "stack48"):
        roof = dict(main["pcie"])
    else:
        roof = dict(main["hbm"])
    roof.setdefault("kernel", main["kernel"])
    # committed counter summary of the main workload's dominant launches (none for the copy-bound legs)
    traffic_profile = {"decode": "decode_traffic.md", "prefill512": "prefill512_traffic.md",
                       "prefill4096": "prefill4096_zipf_traffic.md",
                       "dsv2_mixed": "dsv2_mixed_traffic.md"}.get(args.workload)
    roof["traffic"] = traffic_from_profiles(traffic_profile) if traffic_profile else None
    roof["traffic_source"] = (f"profiles/{traffic_profile}: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this "
                              "workload's command, committed; not measured in this run"
                              if roof["traffic"] is not None else None)
    cfg_name = {"dsv2_mixed": "DeepSeek-V2-Lite-shaped MoE layer (64 x 1408 routed top-6, 2 shared), mixed batch "
                              "48 decode + 256 + 1000 prefill tokens",
                "prefill512": "Qwen3-30B-A3B-shaped MoE layer, prefill T=512 uniform routing, 128 experts resident",
                "decode": "Qwen3-30B-A3B-shaped MoE layer, decode T=1, 128 experts resident; a step is one token "
                          "through 16 layer copies (one hipGraph replay of 16 single-launch layers)",
                "prefill4096": "Qwen3-30B-A3B-shaped MoE layer, prefill T=4096 with a Zipf(1.1) router bias (the "
                               "T=4096 layer's routing), all 128 experts resident: the grouped SwiGLU",
                "prefill4096_zipf": "Qwen3-30B-A3B-shaped MoE layer, prefill T=4096 with a Zipf(1.1) router bias, "
                                    "32 experts resident, the rest staged through 8 demand slots",
                "runtime_prefill512": "Qwen3-30B-A3B-shaped MoE layers through PDScopeCudaRuntime.forward, prefill "
                                      "T=512, all 128 experts resident (launched before the counts come back); a step "
                                      "is one layer call (host cost of the runtime included)",
                "runtime_decode": "Qwen3-30B-A3B-shaped MoE layers through PDScopeCudaRuntime.forward, decode T=1, "
                                  "all 128 experts resident, bound single-launch layer with next-layer prediction; a step is "
                                  "one layer call (host cost of the runtime included)",
                "stack48": "48 Qwen3-30B-A3B-shaped MoE blocks (identity attention + RMSNorm), prefill 2048 then 64 "
                           "decode steps, 24 GiB expert-slot cap, gate-fallback prefetch, bound single-launch decode; "
                           "value is decode tok/s"}
    kind, T, nl = plan[args.workload]
    line = {
        "metric": METRIC,
        "value": round(main["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": main["steps"],
        "warmup": main["warmup"],
        "ms_per_step": round(main["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random bf16 weights ~N(0,0.02), activations ~N(0,1))",
        "config": {"workload": cfg_name[args.workload], "tokens": T,
                   **main.get("shape", dict(hidden=H, experts=E, intermediate=I, top_k=K_TOP)),
                   "layers_rotated": nl, "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": {k: v for k, v in main.get("cpu_baseline", {}).items() if k in
                         ("value", "unit", "cores", "kind", "sample")} or None,
        "workloads": records,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
