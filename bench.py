#!/usr/bin/env python3
"""Benchmark of the MI355X W4A16 MoE expert path (one GPU).

Headline (the JSON ``value``): one MoE layer at decode, 1 token, hidden 2048,
512 experts, top-10, moe_intermediate 512, int4 weights with bf16 group-128
scales — HBM GB/s of algorithmic bytes (10 experts' int4 weights + scales, x,
router logits, output: 16,229,376 B per layer) over the measured time per
layer. A "step" is one such layer. Every step uses another layer of a cold
pool (distinct weights, >= 6 GiB in total) and its own token, so the touched
experts are not resident in the 256 MB Infinity Cache; the K steps are
captured in one HIP graph and replayed (host launch cost would otherwise
dominate a microsecond-scale layer).

The per-step time is the wall clock of one replay of the K-step graph,
synchronised on both sides, with nothing else in the timed region.

Also reported in the same JSON line: the dominant kernel's roofline (the
single fused decode kernel that carries the whole layer, timed live with
events on the stream it runs on, over a second replay of the same graph), the CPU
oracle timed on this host on a bounded sample, the 4096-token prefill layer
in TFLOP/s against the bf16 MFMA peak, the 512-token prefill layer with Zipf
routing in GB/s over the routed experts and TFLOP/s, the 48-layer batch-4
decode step in streaming GB/s, the single projection in GB/s, the whole MoE
block at decode (shared expert and router projection plus the experts) and
at the 4096-token prefill shape (with the shared/router projections'
TFLOP/s), a W8A16 dense projection (decode GB/s and 512-row TFLOP/s), the
load-time LQP -> int4pack conversion of one layer in GB/s, the decode
layer read from the plain int4pack container (no decode tiles), and, at the
reference model's expert shape (H2560, MI640, g64), the one-token decode
layer, the 128- and 512-token prefill layers and the weighted combine of
8192 tokens.
Inputs are synthetic (seeded, generated on the device) and resident in HBM
before timing starts.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "qwen-ascend_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "W4A16 MoE layer µs + HBM GB/s (decode B=1); grouped-GEMM TFLOP/s (prefill)"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
# Secondary lines time at least this many calls (microsecond-scale ones) or
# layers (prefill) per graph replay, whatever --steps is: one replay's launch
# and the first calls' ramp would otherwise weigh on a 20-step run (the
# headline times exactly --steps steps).
MIN_CALLS = 200
MIN_LAYERS = 10


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def per_expert_bytes(H, MI, gs):
    return (H * 2 * MI + MI * H) // 2 + (H // gs * 2 * MI + MI // gs * H) * 2


def graph_of(fn, n):
    """Capture n calls of fn(i) in one CUDA/HIP graph (after one eager call)."""
    import torch
    fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    return g


def time_graph(g, reps=1):
    """Wall time of `reps` replays (synchronised on both sides, nothing else in
    the timed region), then the event time of `reps` further replays. The
    event records stay out of the wall-timed region: their host calls, made
    while the GPU waits for the replay, cost ~10 us per replay (0.5 us per
    step of a 20-step decode graph)."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return t1 - t0, e0.elapsed_time(e1) / 1e3


def bench_decode_b1(args, dev):
    """The headline workload plus the dominant-kernel roofline."""
    import torch
    from qmoe import moe_decode
    from qmoe.workload import device_layer
    H, MI, E, k, gs = 2048, 512, 512, 10, 128
    L = args.pool_layers
    log(f"decode B=1: building a cold pool of {L} layers ({L * 0.774:.1f} GiB, and as much again of decode tiles)")
    pool = [device_layer(H, MI, E, gs, 1000 + 10 * l, dev) for l in range(L)]
    for gu, dn in pool:  # load-time decode tiles (ExpW4.decode_tiles), before any capture
        gu.decode_tiles("gate_up")
        dn.decode_tiles("down")
    K, W = args.steps, args.warmup
    g = torch.Generator(device=dev)
    g.manual_seed(1001)
    xs = torch.randn((K, 1, H), generator=g, device=dev).to(torch.bfloat16)
    lgs = torch.randn((K, 1, E), generator=g, device=dev).to(torch.bfloat16)

    def step(i):
        gu, dn = pool[i % L]
        moe_decode(xs[i], lgs[i], gu, dn, k)

    for i in range(W):
        step(i)
    torch.cuda.synchronize()
    log(f"decode B=1: capturing {K} steps")
    graph = graph_of(step, K)
    time_graph(graph)                      # untimed replay (warm instruction caches, graph upload)
    wall, ev = time_graph(graph)
    layer_bytes = k * per_expert_bytes(H, MI, gs) + H * 2 + E * 2 + H * 2
    sec_per_step = wall / K
    res = {
        "ms_per_step": sec_per_step * 1e3,
        "us_per_layer": sec_per_step * 1e6,
        "event_us_per_layer": ev / K * 1e6,
        "value": layer_bytes / sec_per_step / 1e9,
        "tokens_per_s": 1.0 / sec_per_step,
        "layer_bytes": layer_bytes,
    }
    # dominant kernel: the whole layer is one launch of the fused decode kernel
    # (routing, gate_up, SwiGLU, down, weighted combine), so its average launch
    # period is the graph's event time over the K launches
    kern_s = ev / K
    achieved = layer_bytes / kern_s / 1e9
    res["roofline"] = {"kernel": DECODE_KERNEL, "bound": "hbm", "achieved": achieved,
                       "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                       "traffic": traffic_of(DECODE_KERNEL), "bytes_per_launch": layer_bytes,
                       "us_per_launch": kern_s * 1e6}
    res["layer_roofline_frac"] = res["value"] / HBM_PEAK_GBS
    # the same K steps reading the int4pack container itself (no decode tiles)
    log("decode B=1: the same steps without decode tiles")

    def step_plain(i):
        gu, dn = pool[i % L]
        moe_decode(xs[i], lgs[i], gu, dn, k, tiles=False)

    graph_p = graph_of(step_plain, K)
    time_graph(graph_p)
    wall_p, ev_p = time_graph(graph_p)
    res["int4pack_only"] = {"us_per_layer": wall_p / K * 1e6, "event_us_per_layer": ev_p / K * 1e6,
                            "GB_s": layer_bytes / (wall_p / K) / 1e9,
                            "kernel": DECODE_KERNEL.replace("true", "false")}
    del graph_p, pool
    torch.cuda.empty_cache()
    return res


# the one-token decode launch: the XCD-group kernel (routing over 8 logits per lane, 16 gate_up rows per lane,
# weights from decode tiles)
DECODE_KERNEL = "moe_decode_xcd_kernel<8, 16, true>"
# the one-token projections: the W4A16 split-K GEMV on narrow tiles (128-row
# slices), the W8A16 split-K GEMV
PROJ_KERNEL = "w4a16_gemv_narrow_kernel<true, 16>"
W8_GEMV_KERNEL = "w8a16_gemv_kernel<1, 16>"


def traffic_of(kernel):
    """HBM bytes per launch measured by the committed rocprofv3 counter runs."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get("kernels", {}).get(kernel, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


COPY_BYTES = 256 << 20
READ_COUNTERS = "TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_32B_sum TCC_EA0_RDREQ_128B_sum"


def _short_name(name):
    import re
    m = re.match(r"_ZN12_GLOBAL__N_1(\d+)", name)
    if m:  # a mangled name of an anonymous-namespace kernel: its length-prefixed identifier
        return name[m.end():m.end() + int(m.group(1))]
    n = name.replace("(anonymous namespace)::", "").replace("void ", "")
    return re.sub(r"\(.*", "", n)


def _counter_means(csv_path):
    """Per kernel (short name) and counter: the mean value per dispatch."""
    import csv
    acc = {}
    with open(csv_path) as fh:
        for r in csv.DictReader(fh):
            d = acc.setdefault(_short_name(r["Kernel_Name"]), {})
            d.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in acc.items()}


def _read_bytes(c):
    """Bytes the L2 read from memory: gfx950 issues 32-, 64- and 128-byte
    requests (rocprof's FETCH_SIZE counts the 128-byte ones as 64)."""
    n, n32, n128 = c["TCC_EA0_RDREQ_sum"], c["TCC_EA0_RDREQ_32B_sum"], c["TCC_EA0_RDREQ_128B_sum"]
    return 32 * n32 + 128 * n128 + 64 * (n - n32 - n128)


TRAFFIC_KERNELS = ("moe_decode", "w4a16_gemv", "w8a16_gemv")


def counters_summary(dirs):
    """Turn rocprofv3 --pmc runs (read requests / WRITE_SIZE of the
    HBM-bound benches, then of the 256 MiB copy) into profiles/traffic.json.
    The first two arguments may each list several run directories, comma
    separated (the decode run and the --only-projection run)."""
    crd, cwr = (Path(d) / "run_counter_collection.csv" for d in dirs[2:])
    copy_r = [v for k, v in _counter_means(crd).items() if "copyBuffer" in k][0]
    copy_w = [v for k, v in _counter_means(cwr).items() if "copyBuffer" in k][0]
    f_read = COPY_BYTES / _read_bytes(copy_r)
    f_write = COPY_BYTES / (copy_w["WRITE_SIZE"] * 1024)
    reads, writes = {}, {}
    for d in dirs[0].split(","):
        reads.update(_counter_means(Path(d) / "run_counter_collection.csv"))
    for d in dirs[1].split(","):
        writes.update(_counter_means(Path(d) / "run_counter_collection.csv"))
    out = {"calibration": {"copy_bytes": COPY_BYTES, "read_factor": f_read, "write_factor": f_write,
                           "fetch_size_kib_reads_as": copy_r.get("FETCH_SIZE")},
           "kernels": {}}
    for k in reads:
        if not any(t in k for t in TRAFFIC_KERNELS) or k not in writes:
            continue
        rb, wb = _read_bytes(reads[k]) * f_read, writes[k]["WRITE_SIZE"] * 1024 * f_write
        out["kernels"][k] = {"read_bytes_per_launch": rb, "write_bytes_per_launch": wb,
                             "hbm_bytes_per_launch": rb + wb}
    (ROOT / "profiles" / "traffic.json").write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out, indent=1))


LIB_KERNELS = ("moe_decode", "grouped_gemm", "w4a16_gemv", "slot_reduce", "rows_to_f16", "route_", "router_topk",
               "bf16_gemv", "bf16_gemm", "w8a16", "lqp_", "swiglu", "shared_gate", "expert_gather", "weighted_reduce",
               "epilogue", "merge", "decode_tiles", "xcc_probe", "tiles_from_ends")


def trace_summary(d):
    """rocprofv3 --kernel-trace output dir -> markdown table of this library's
    kernels, one line per (kernel, grid): dispatches and durations in us."""
    import csv
    groups = {}
    with open(Path(d) / "run_kernel_trace.csv") as fh:
        for r in csv.DictReader(fh):
            name = _short_name(r["Kernel_Name"])
            if "rocprim" in name or not any(k in name for k in LIB_KERNELS):
                continue
            wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
            grid = tuple(int(r[f"Grid_Size_{a}"]) // max(1, int(r[f"Workgroup_Size_{a}"])) for a in "XYZ")
            key = (name, "x".join(str(g) for g in grid if g > 1) or "1", wg)
            groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = ["| kernel | workgroups x threads | dispatches | avg us | min us | max us |",
             "|---|---|---:|---:|---:|---:|"]
    for (name, grid, wg), ds in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| {name} | {grid} x {wg} | {len(ds)} | {sum(ds) / len(ds):.2f} | {min(ds):.2f} | {max(ds):.2f} |")
    print("\n".join(lines))


def bench_decode_ref_shape(args, dev):
    """The one-token decode layer at the reference model's expert shape (H2560,
    MI640, 512 experts, top-10, g64: fnx/engine.py:23,40-42, fnx/load.py:74),
    decode tiles, a cold pool of 4 layers. The XCD-group launch has 1760
    workgroups here (5 act tiles per slot, 20 K-slices), more than the 1024 that
    are resident at once. The reference's own figures at this shape are per
    component: gather + gate_up 52.61 us (docs/r138-expert-gather.md:35) and
    down + epilogue 49.68 us (docs/r156-moe-kmajor.md:13-17)."""
    import torch
    from qmoe import moe_decode
    from qmoe.workload import device_layer
    H, MI, E, k, gs, L = 2560, 640, 512, 10, 64, 4
    pool = [device_layer(H, MI, E, gs, 6000 + 10 * l, dev) for l in range(L)]
    for gu, dn in pool:
        gu.decode_tiles("gate_up")
        dn.decode_tiles("down")
    K = max(args.steps, MIN_CALLS)
    g = torch.Generator(device=dev)
    g.manual_seed(6001)
    xs = torch.randn((K, 1, H), generator=g, device=dev).to(torch.bfloat16)
    lgs = torch.randn((K, 1, E), generator=g, device=dev).to(torch.bfloat16)
    graph = graph_of(lambda i: moe_decode(xs[i], lgs[i], pool[i % L][0], pool[i % L][1], k), K)
    time_graph(graph)
    wall, ev = time_graph(graph)
    b = k * per_expert_bytes(H, MI, gs) + H * 2 + E * 2 + H * 2
    del graph, pool
    torch.cuda.empty_cache()
    return {"workload": "moe_decode_b1_h2560_e512_mi640_top10_g64", "us_per_layer": wall / K * 1e6,
            "event_us_per_layer": ev / K * 1e6, "GB_s": b / (wall / K) / 1e9, "bytes_per_layer": b}


def bench_weighted_reduce(args, dev):
    """The ordered weighted combine with the inverse gather at the reference's
    production chunk (fnx/weighted_reduce.py, 8192 tokens x top-10, width 2560,
    expert-major products): out[t] = bf16(sum_j bf16(x[inv[t k + j]] w[t, j])).
    The reference measured 0.7493 ms for this subgraph (docs/r119-weighted-reduce.md:39)."""
    import torch
    from qmoe.weighted_reduce import reduce
    T, k, H = 8192, 10, 2560
    g = torch.Generator(device=dev)
    g.manual_seed(7001)
    x = torch.randn((T * k, H), generator=g, device=dev).to(torch.bfloat16)
    w = torch.rand((T, k), generator=g, device=dev).to(torch.bfloat16)
    inv = torch.randperm(T * k, generator=g, device=dev)
    n = max(MIN_LAYERS, args.steps // 20)
    graph = graph_of(lambda i: reduce(x, w, inverse=inv), n)
    time_graph(graph)
    wall, ev = time_graph(graph)
    s = ev / n
    b = T * k * H * 2 + T * k * 8 + T * k * 2 + T * H * 2
    del graph, x
    torch.cuda.empty_cache()
    return {"workload": "weighted_reduce_inverse_t8192_k10_h2560", "ms_per_call": s * 1e3, "GB_s": b / s / 1e9,
            "bytes_per_call": b}


def bench_projection(args, dev):
    """Single W4A16 projection [1,2048] x [2048 -> 4096], g128, cold pool of weights."""
    import torch
    from qmoe import weight_quant_batchmatmul
    from qmoe.workload import device_int4_words, device_scales
    K_, N, gs = 2048, 4096, 128
    copies = 256                                      # 256 x 4.1 MB > 1 GiB
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    ws = [device_int4_words((K_, N // 8), g, dev) for _ in range(copies)]
    ss = [device_scales((K_ // gs, N), g, dev) for _ in range(copies)]
    n = max(args.steps, MIN_CALLS)
    xs = torch.randn((n, 1, K_), generator=g, device=dev).to(torch.bfloat16)
    graph = graph_of(lambda i: weight_quant_batchmatmul(xs[i], ws[i % copies], ss[i % copies],
                                                        antiquant_group_size=gs), n)
    time_graph(graph)
    wall, ev = time_graph(graph)
    b = K_ * N // 2 + K_ // gs * N * 2 + K_ * 2 + N * 2
    return {"workload": "w4a16_proj_2048x4096_g128", "us_per_call": ev / n * 1e6, "GB_s": b / (ev / n) / 1e9,
            "bytes_per_call": b, "kernel": PROJ_KERNEL, "traffic": traffic_of(PROJ_KERNEL)}


def bench_layers48(args, dev):
    """Batch-4 decode step over 48 distinct layers (streaming, weights cold)."""
    import torch
    from qmoe import moe_decode
    from qmoe.workload import device_layer
    H, MI, E, k, gs, B, NL = 2048, 512, 512, 10, 128, 4, 48
    log("48-layer decode: generating 48 layers (37 GiB, and as much again of decode tiles) on the device")
    layers = [device_layer(H, MI, E, gs, 3000 + 10 * l, dev) for l in range(NL)]
    for gu, dn in layers:  # load-time decode tiles, read by the per-pair launch of 2-4 tokens
        gu.decode_tiles("gate_up")
        dn.decode_tiles("down")
    g = torch.Generator(device=dev)
    g.manual_seed(3001)
    steps = max(4, args.steps // 50)
    xs = torch.randn((steps, NL, B, H), generator=g, device=dev).to(torch.bfloat16)
    lgs = torch.randn((steps, NL, B, E), generator=g, device=dev).to(torch.bfloat16)
    idx_keep = []

    def step(i):
        for l in range(NL):
            out, idx, _ = moe_decode(xs[i, l], lgs[i, l], layers[l][0], layers[l][1], k)
            idx_keep.append(idx)

    graph = graph_of(step, steps)
    time_graph(graph)
    wall, ev = time_graph(graph)
    # distinct experts per (step, layer): read once each
    idxs = idx_keep[-steps * NL:]
    distinct = sum(int(torch.unique(t).numel()) for t in idxs)
    b = distinct * per_expert_bytes(H, MI, gs) + steps * NL * (B * H * 2 * 2 + B * E * 2)
    del layers
    torch.cuda.empty_cache()
    return {"workload": "moe_decode_b4_48layers_h2048_e512_mi512_top10_g128", "ms_per_step": ev / steps * 1e3,
            "GB_s": b / ev / 1e9, "distinct_experts_per_layer": distinct / (steps * NL)}


def bench_prefill(args, dev):
    """4096-token prefill layer, H3072/MI768/g64, 512 experts, top-10, uniform routing."""
    import torch
    from qmoe import moe_prefill
    from qmoe.workload import device_layer
    T, H, MI, E, k, gs = 4096, 3072, 768, 512, 10, 64
    gu, dn = device_layer(H, MI, E, gs, 4000, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4001)
    n = max(MIN_LAYERS, args.steps // 20)
    xs = torch.randn((2, T, H), generator=g, device=dev).to(torch.bfloat16)
    lgs = torch.randn((2, T, E), generator=g, device=dev).to(torch.bfloat16)
    graph = graph_of(lambda i: moe_prefill(xs[i % 2], lgs[i % 2], gu, dn, k), n)
    time_graph(graph)
    wall, ev = time_graph(graph)
    flop = 2 * T * k * (H * 2 * MI + MI * H)
    s = ev / n
    tf = flop / s / 1e12
    return {"workload": "moe_prefill_t4096_h3072_e512_mi768_top10_g64", "ms_per_layer": s * 1e3, "TFLOP_s": tf,
            "mfma_frac": tf / MFMA_BF16_PEAK_TFLOPS, "tokens_per_s": T / s}


def bench_prefill_zipf(args, dev):
    """512-token prefill layer with skewed (Zipf 1.1) routing, H2048/MI512/g128,
    512 experts, top-10: the small-batch grouped path with empty and
    lightly loaded experts. Reported as GB/s over the experts actually routed
    to and as TFLOP/s."""
    import torch
    from qmoe import moe_prefill, router_topk
    from qmoe.workload import device_layer, zipf_logits
    T, H, MI, E, k, gs = 512, 2048, 512, 512, 10, 128
    gu, dn = device_layer(H, MI, E, gs, 5000, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(5001)
    n = max(MIN_LAYERS, args.steps // 20)
    xs = torch.randn((2, T, H), generator=g, device=dev).to(torch.bfloat16)
    lgs = torch.stack([torch.from_numpy(zipf_logits(T, E, 1.1, 5002 + i).view("int16")).view(torch.bfloat16)
                       for i in range(2)]).to(dev)
    graph = graph_of(lambda i: moe_prefill(xs[i % 2], lgs[i % 2], gu, dn, k), n)
    time_graph(graph)
    wall, ev = time_graph(graph)
    s = ev / n
    uniq = sum(int(torch.unique(router_topk(lgs[i], k)[0]).numel()) for i in range(2)) / 2
    b = uniq * per_expert_bytes(H, MI, gs) + T * H * 2 * 2 + T * E * 2
    flop = 2 * T * k * (H * 2 * MI + MI * H)
    return {"workload": "moe_prefill_t512_zipf1.1_h2048_e512_mi512_top10_g128", "ms_per_layer": s * 1e3,
            "GB_s": b / s / 1e9, "TFLOP_s": flop / s / 1e12, "distinct_experts": uniq, "tokens_per_s": T / s}


def bench_prefill_ref_shape(args, dev):
    """Prefill layers at the reference model's expert shape (H2560, MI640, 512
    experts, top-10, g64), 128 and 512 tokens, uniform routing: the grouped
    expert path alone. The reference measured its grouped-GEMM prefill MoE
    layer at 7.5 ms (128 tokens) and 11.1 ms (512 tokens)
    (docs/Qwen3.8-Flash-Next-第50轮优化记录.md:18-19)."""
    import torch
    from qmoe import moe_prefill
    from qmoe.workload import device_layer
    H, MI, E, k, gs = 2560, 640, 512, 10, 64
    gu, dn = device_layer(H, MI, E, gs, 6100, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(6101)
    n = max(MIN_LAYERS, args.steps // 20)
    res = {"workload": "moe_prefill_h2560_e512_mi640_top10_g64"}
    for T in (128, 512):
        xs = torch.randn((2, T, H), generator=g, device=dev).to(torch.bfloat16)
        lgs = torch.randn((2, T, E), generator=g, device=dev).to(torch.bfloat16)
        graph = graph_of(lambda i: moe_prefill(xs[i % 2], lgs[i % 2], gu, dn, k), n)
        time_graph(graph)
        _, ev = time_graph(graph)
        s = ev / n
        res[f"t{T}_ms_per_layer"] = s * 1e3
        res[f"t{T}_TFLOP_s"] = 2 * T * k * (H * 2 * MI + MI * H) / s / 1e12
        del graph
    del gu, dn
    torch.cuda.empty_cache()
    return res


def bench_w8(args, dev):
    """W8A16 dense projection (DenseW8's op) 2048 -> 8192, g128: one token from
    a cold pool of weights (GB/s), and 512 rows (TFLOP/s)."""
    import torch
    from qmoe import weight_quant_batchmatmul
    K_, N, gs = 2048, 8192, 128
    copies = 64                                       # 64 x 16.8 MB > 1 GiB
    g = torch.Generator(device=dev)
    g.manual_seed(8001)
    ws = [torch.randint(-128, 128, (K_, N), dtype=torch.int8, device=dev, generator=g) for _ in range(copies)]
    ss = [(torch.rand((K_ // gs, N), generator=g, device=dev) * 0.004).to(torch.bfloat16) for _ in range(copies)]
    n = max(args.steps, MIN_CALLS)
    xs = torch.randn((n, 1, K_), generator=g, device=dev).to(torch.bfloat16)
    graph = graph_of(lambda i: weight_quant_batchmatmul(xs[i], ws[i % copies], ss[i % copies],
                                                        antiquant_group_size=gs), n)
    time_graph(graph)
    wall, ev = time_graph(graph)
    b = K_ * N + K_ // gs * N * 2 + K_ * 2 + N * 2
    out = {"workload": "w8a16_proj_2048x8192_g128", "us_per_call": ev / n * 1e6, "GB_s": b / (ev / n) / 1e9,
           "bytes_per_call": b, "kernel": W8_GEMV_KERNEL, "traffic": traffic_of(W8_GEMV_KERNEL)}
    M = 512
    xm = torch.randn((M, K_), generator=g, device=dev).to(torch.bfloat16)
    reps = 20
    graph = graph_of(lambda i: weight_quant_batchmatmul(xm, ws[i % copies], ss[i % copies],
                                                        antiquant_group_size=gs), reps)
    time_graph(graph)
    wall, ev = time_graph(graph)
    out["prefill_m512_us"] = ev / reps * 1e6
    out["prefill_m512_TFLOP_s"] = 2 * M * K_ * N / (ev / reps) / 1e12
    del ws, ss
    torch.cuda.empty_cache()
    return out


def bench_block_decode(args, dev):
    """The whole MoE block at decode, 1 token: shared expert and router
    projection (bf16 [2MI+1+E, H] and [H, MI]) then the experts, H2048/MI512,
    512 experts, top-10, g128, from a cold pool of 8 layers, in two launches
    (the projection; the experts with the shared down projection). GB/s over
    the expert bytes of the 10 routed experts plus the dense weights."""
    import torch
    from qmoe.shared import moe_block
    from qmoe.workload import device_layer
    H, MI, E, k, gs, L = 2048, 512, 512, 10, 128, 8
    g = torch.Generator(device=dev)
    g.manual_seed(7001)
    pool = []
    for l in range(L):
        gu, dn = device_layer(H, MI, E, gs, 7000 + 10 * l, dev)
        gu.decode_tiles("gate_up")
        dn.decode_tiles("down")
        sh_gu = (torch.randn((2 * MI + 1 + E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        sh_dn = (torch.randn((H, MI), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        pool.append((gu, dn, sh_gu, sh_dn))
    n = max(args.steps, MIN_CALLS)
    xs = torch.randn((n, 1, H), generator=g, device=dev).to(torch.bfloat16)

    def step(i):
        gu, dn, sh_gu, sh_dn = pool[i % L]
        moe_block(xs[i], sh_gu, sh_dn, gu, dn, k)

    graph = graph_of(step, n)
    time_graph(graph)
    wall, ev = time_graph(graph)
    s = ev / n
    dense = ((2 * MI + 1 + E) * H + H * MI) * 2
    b = k * per_expert_bytes(H, MI, gs) + dense + H * 2 * 2
    del pool
    torch.cuda.empty_cache()
    return {"workload": "moe_block_decode_b1_h2048_e512_mi512_top10_g128_shared", "us_per_layer": s * 1e6,
            "GB_s": b / s / 1e9, "bytes_per_layer": b, "launches_per_layer": 2}


def bench_block_prefill(args, dev):
    """The whole MoE block at the 4096-token prefill shape (H3072, MI768, 512
    experts, top-10, g64): the shared expert and router projections on the
    hand-written bf16 MFMA GEMM (sh_gu [2MI+1+E, H], sh_down [H, MI]), then the
    grouped expert path. Reports the whole block and, timed alone, the
    shared/router part in TFLOP/s of its two GEMMs."""
    import torch
    from qmoe.shared import moe_block, shared_router
    from qmoe.workload import device_layer
    T, H, MI, E, k, gs = 4096, 3072, 768, 512, 10, 64
    gu, dn = device_layer(H, MI, E, gs, 4000, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4101)
    sh_gu = (torch.randn((2 * MI + 1 + E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    sh_dn = (torch.randn((H, MI), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    xs = torch.randn((2, T, H), generator=g, device=dev).to(torch.bfloat16)
    n = max(MIN_LAYERS, args.steps // 20)
    graph = graph_of(lambda i: moe_block(xs[i % 2], sh_gu, sh_dn, gu, dn, k), n)
    time_graph(graph)
    _, ev = time_graph(graph)
    s_block = ev / n
    graph = graph_of(lambda i: shared_router(xs[i % 2], sh_gu, sh_dn, MI), n)
    time_graph(graph)
    _, ev = time_graph(graph)
    s_sh = ev / n
    flop_sh = 2 * T * H * (2 * MI + 1 + E) + 2 * T * MI * H
    flop_exp = 2 * T * k * (H * 2 * MI + MI * H)
    del gu, dn
    torch.cuda.empty_cache()
    return {"workload": "moe_block_prefill_t4096_h3072_e512_mi768_top10_g64_shared", "ms_per_block": s_block * 1e3,
            "tokens_per_s": T / s_block, "TFLOP_s": (flop_sh + flop_exp) / s_block / 1e12,
            "shared_router_ms": s_sh * 1e3, "shared_router_TFLOP_s": flop_sh / s_sh / 1e12,
            "shared_router_mfma_frac": flop_sh / s_sh / 1e12 / MFMA_BF16_PEAK_TFLOPS}


def bench_artifact(args, dev):
    """Load-time conversion of one layer's experts from the LQP layout (v2o,
    int4 packed along K) to the expert-major int4pack container: 512 experts,
    H2048/MI512 (gate_up v2o [512, 1024, 1024] and down [512, 2048, 256]
    uint8). GB/s over the bytes read plus written."""
    import torch
    from qmoe.artifact import lqp_to_int4pack
    E, H, MI = 512, 2048, 512
    g = torch.Generator(device=dev)
    g.manual_seed(6001)
    v_gu = torch.randint(0, 256, (E, 2 * MI, H // 2), dtype=torch.uint8, device=dev, generator=g)
    v_dn = torch.randint(0, 256, (E, H, MI // 2), dtype=torch.uint8, device=dev, generator=g)
    outs = []

    def conv():
        outs.clear()
        outs.append(lqp_to_int4pack(v_gu, expert_major=True))
        outs.append(lqp_to_int4pack(v_dn, expert_major=True))

    conv()
    torch.cuda.synchronize()
    n = 5
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        conv()
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) / 1e3 / n
    b = 2 * (v_gu.numel() + v_dn.numel())
    del v_gu, v_dn, outs
    torch.cuda.empty_cache()
    return {"workload": "lqp_v2o_to_int4pack_em_e512_h2048_mi512", "ms_per_layer": s * 1e3, "GB_s": b / s / 1e9,
            "hbm_frac": b / s / 1e9 / HBM_PEAK_GBS}


def copy_calibration(args, dev):
    """A device-to-device copy of 256 MiB, repeated: each dispatch reads and
    writes exactly 268,435,456 bytes, which is what the FETCH_SIZE and
    WRITE_SIZE counters of one dispatch are scaled against."""
    import torch
    n = 256 << 20
    src = torch.empty(n // 2, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    for _ in range(max(3, args.steps // 20)):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_dispatch": n, "dispatches": max(3, args.steps // 20)}), flush=True)


def _blas_threads():
    """Threads numpy's BLAS runs the oracle's matmuls on (the host's cores)."""
    try:
        from threadpoolctl import threadpool_info
        return max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
    except Exception:  # noqa: BLE001
        return len(os.sched_getaffinity(0))


def cpu_baseline(args):
    """The numpy oracle of the decode layer on this host's cores, bounded sample."""
    from oracle import qmoe_oracle as O
    from qmoe import workload as Wk
    H, MI, E, k, gs = 2048, 512, 512, 10, 128
    lay = Wk.moe_layer(H, MI, E, gs, 1000)
    cores = len(os.sched_getaffinity(0))
    blas = _blas_threads()
    n, t0 = 0, time.perf_counter()
    while True:
        x = Wk.normal_bf16((1, H), 5000 + n)
        lg = Wk.normal_bf16((1, E), 6000 + n)
        O.moe_decode(x, lg, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
        n += 1
        el = time.perf_counter() - t0
        if (el >= args.cpu_seconds and n >= 3) or n >= 1000:
            break
    s = el / n
    layer_bytes = k * per_expert_bytes(H, MI, gs) + H * 2 + E * 2 + H * 2
    return {"value": layer_bytes / s / 1e9, "unit": "GB/s", "cores": blas, "kind": "port",
            "us_per_layer": s * 1e6,
            "sample": f"{n} decode layers (1 token, 512 experts, top-10) through the numpy oracle "
                      f"(int4 unpack, fp32 dequant, fp32 matmul, bf16 rounding points); host has {cores} cores"}


def cpu_baseline_configs(args):
    """The numpy oracle on the other workloads, on this host's cores, each on a
    bounded sample: the single projection (repeated calls), the 48-layer
    batch-4 decode step (whole layers of four tokens, scaled), the 512-token
    Zipf prefill layer (one whole layer) and the 4096-token prefill layer
    (the experts of one eighth of the layer with the rows routed to them: the
    grouped gate_up GEMM, SwiGLU and grouped down GEMM, timed and scaled by 8;
    the ordered slot reduction, under 1% of the CPU time, is left out)."""
    from oracle import qmoe_oracle as O
    from qmoe import workload as Wk
    cores = _blas_threads()
    out = {}
    # single projection [1, 2048] x [2048 -> 4096], g128
    K_, N, gs = 2048, 4096, 128
    w, sc, x = Wk.int4_words((K_, N // 8), 11), Wk.scales((K_ // gs, N), 12), Wk.normal_bf16((1, K_), 13)
    n, t0 = 0, time.perf_counter()
    while True:
        O.w4a16_gemm(x, w, sc, gs)
        n += 1
        el = time.perf_counter() - t0
        if (el >= min(3.0, args.cpu_seconds) and n >= 3) or n >= 10000:
            break
    b = K_ * N // 2 + K_ // gs * N * 2 + K_ * 2 + N * 2
    out["projection"] = {"cores": cores, "value": b / (el / n) / 1e9, "unit": "GB/s", "us_per_call": el / n * 1e6, "kind": "port",
                         "sample": f"{n} calls of the oracle's W4A16 GEMM, 2048 -> 4096 g128"}
    # 48-layer batch-4 decode step: four tokens per layer through the oracle's
    # decode (one layer's weights; the CPU cost does not depend on which
    # layer's), timed over whole layers and scaled to 48
    H, MI, E, k, gs, B, NL = 2048, 512, 512, 10, 128, 4, 48
    lay = Wk.moe_layer(H, MI, E, gs, 3000)
    n, distinct, t0 = 0, 0, time.perf_counter()
    while True:
        x, lg = Wk.normal_bf16((B, H), 3100 + n), Wk.normal_bf16((B, E), 3200 + n)
        ids = set()
        for t in range(B):
            ids.update(O.moe_decode(x[t], lg[t], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)["idx"][0].tolist())
        distinct += len(ids)
        n += 1
        el = time.perf_counter() - t0
        if (el >= min(3.0, args.cpu_seconds) and n >= 2) or n >= NL:
            break
    step_s = el / n * NL
    b = distinct / n * NL * per_expert_bytes(H, MI, gs) + NL * (B * H * 2 * 2 + B * E * 2)
    out["decode_48_layers"] = {"cores": cores, "value": b / step_s / 1e9, "unit": "GB/s", "ms_per_step": step_s * 1e3,
                               "kind": "port",
                               "sample": f"{n} layers of four tokens through the oracle's decode; time x {NL}/{n}"}
    del lay
    # 512-token prefill layer, Zipf(1.1) routing, H2048/MI512/g128
    T, H, MI, E, k, gs = 512, 2048, 512, 512, 10, 128
    lay = Wk.moe_layer(H, MI, E, gs, 5000)
    x, lg = Wk.normal_bf16((T, H), 5003), Wk.zipf_logits(T, E, 1.1, 5002)
    t0 = time.perf_counter()
    O.moe_prefill(x, lg, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
    el = time.perf_counter() - t0
    out["prefill_zipf_t512"] = {"cores": cores, "value": T / el, "unit": "tokens/s", "ms_per_layer": el * 1e3, "kind": "port",
                                "sample": "one whole layer through the oracle (router, grouping, grouped GEMMs, "
                                          "SwiGLU, ordered weighted reduce)"}
    del lay
    # 4096-token prefill layer, H3072/MI768/g64, uniform routing: 1/8 of the experts
    T, H, MI, E, k, gs = 4096, 3072, 768, 512, 10, 64
    part = E // 8
    x, lg = Wk.normal_bf16((T, H), 4001), Wk.normal_bf16((T, E), 4002)
    idx, _ = O.router(lg, k)
    _, ends, order, _ = O.group_routing(idx, E)
    lay = Wk.moe_layer(H, MI, part, gs, 4000)
    rows = int(ends[part - 1])
    t0 = time.perf_counter()
    gu = O.grouped_gemm(x[order[:rows] // k], lay["gu_w"], lay["gu_s"], ends[:part])
    act = O.swiglu(gu)
    O.grouped_gemm(act, lay["dn_w"], lay["dn_s"], ends[:part])
    el = (time.perf_counter() - t0) * (E / part)
    flop = 2 * T * k * (H * 2 * MI + MI * H)
    out["prefill_t4096"] = {"cores": cores, "value": flop / el / 1e12, "unit": "TFLOP/s", "ms_per_layer": el * 1e3,
                            "tokens_per_s": T / el, "kind": "port",
                            "sample": f"experts 0..{part - 1} of the layer with their {rows} routed rows through the "
                                      f"oracle's grouped gate_up GEMM, SwiGLU and grouped down GEMM; time x {E // part}"}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pool-layers", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-decode", action="store_true", help="skip the secondary workloads")
    ap.add_argument("--only-projection", action="store_true",
                    help="only the one-token W4A16 (2048 -> 4096) and W8A16 (2048 -> 8192) projections (for "
                         "counter runs): print their lines")
    ap.add_argument("--only-prefill", action="store_true",
                    help="only the 4096-token prefill layer (for counter runs of the grouped GEMM): print its "
                         "line and exit")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy (the reference for HBM counter scaling)")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="rocprofv3 --kernel-trace output dir: print this library's kernels per grid and exit")
    ap.add_argument("--counters-summary", nargs=4, metavar="DIR",
                    help="rocprofv3 output dirs of the read-request runs (decode and --only-projection, comma "
                         "separated), their WRITE_SIZE runs (likewise), and the same two for --copy-calibration: "
                         "write profiles/traffic.json and exit")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.counters_summary:
        counters_summary(args.counters_summary)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU; multi-GPU runs are not part of this build "
              "(the expert path would shard by experts, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(args, dev)
        return
    if args.only_prefill:
        print(json.dumps(bench_prefill(args, dev)), flush=True)
        return
    if args.only_projection:
        print(json.dumps({"projection": bench_projection(args, dev), "w8a16_projection": bench_w8(args, dev)}),
              flush=True)
        return
    res = bench_decode_b1(args, dev)
    extra = {}
    if not args.only_decode:
        extra["projection"] = bench_projection(args, dev)
        extra["prefill"] = bench_prefill(args, dev)
        extra["prefill_zipf_t512"] = bench_prefill_zipf(args, dev)
        extra["decode_48_layers"] = bench_layers48(args, dev)
        extra["moe_block_decode"] = bench_block_decode(args, dev)
        extra["moe_block_prefill"] = bench_block_prefill(args, dev)
        extra["w8a16_projection"] = bench_w8(args, dev)
        extra["artifact_conversion"] = bench_artifact(args, dev)
        extra["decode_reference_shape"] = bench_decode_ref_shape(args, dev)
        extra["weighted_reduce_t8192"] = bench_weighted_reduce(args, dev)
        extra["prefill_reference_shape"] = bench_prefill_ref_shape(args, dev)
    line = {
        "metric": METRIC,
        "value": res["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded, generated on the device)",
        "config": {"workload": "moe_decode_b1_h2048_e512_mi512_top10_g128", "tokens": 1, "hidden": 2048,
                   "experts": 512, "top_k": 10, "moe_intermediate": 512, "group_size": 128,
                   "cold_pool_layers": args.pool_layers, "parallelism": "single GPU"},
        "us_per_layer": res["us_per_layer"],
        "tokens_per_s": res["tokens_per_s"],
        "layer_roofline_frac": res["layer_roofline_frac"],
        "roofline": res["roofline"],
        "decode_int4pack_only": res["int4pack_only"],
    }
    line.update(extra)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args)
        if not args.only_decode:
            line["cpu_baseline_configs"] = cpu_baseline_configs(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
