#!/usr/bin/env python
"""MoE-layer decode benchmark (BASELINE.json metric) on one MI355X.

Workload: Qwen3-30B-A3B-shaped MoE layer -- hidden
2048, 128 experts, top-8 softmax router with renormalised weights, expert
intermediate 768, affine 4-bit group-64 weights from N(0, 0.02); 48
independent layer copies (16.3 GB) rotated so the 256 MB Infinity Cache
cannot hold the working set.  Decode batch B (default 1) of bf16 N(0,1)
tokens; synthetic, seeded data.

A step = one pass of the MoE block over the batch through all 48 layer copies
(48 layer calls, replayed from one HIP graph).  Reported:
  value       us per token per layer call at B (lower is better)
  gbps        algorithmic HBM bytes per layer call / layer time
  roofline    of the dominant kernel -- the single-launch layer kernel
              k_moe_decode1x (XCD-partitioned), one launch per layer call --
              from HIP events on the stream it runs on, around the timed
              region; `traffic` is the measured HBM bytes per launch from the
              committed rocprofv3 counter summary
              (profiles/k_moe_decode1x_qwen3_b1_counters.json)
  cpu_baseline  this repo's C++/OpenMP restatement of the unpatched MLX path
              (MLX is not installable offline) on the host cores, rank 0.
  batches     B = 4 and 16 decode lines, the 512-token prefill line
              (config 4) and, unless --no-other-configs, the LFM2, GLM-mxfp4
              and DeepSeek-V3 lines (configs 0, 2, 4).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B]
       python bench.py --no-other-configs     # Qwen3 lines only
       python bench.py --profile-run [--batch B]   # short run for rocprofv3 --pmc
       python bench.py --summarize-pmc OUT FETCH_DIR WRITE_DIR [MFMA_DIR]
       python bench.py --phase-trace          # per-phase stamps of the B=1 kernel
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import sys
import time
from pathlib import Path

METRIC = "MoE-layer decode µs/token + HBM GB/s (% roofline), Qwen3-30B-A3B shape 4-bit"
HBM_PEAK_GBPS = 8000.0

H, E, K, I, GS = 2048, 128, 8, 768, 64
LAYERS = 48
ROOT = Path(__file__).resolve().parent
COPY_BYTES = 256 << 20  # calibration copy of --profile-run: reads and writes this many bytes
# the single-launch kernel of each decode batch (rocprofv3 kernel names)
DECODE_KERNELS = {1: "zmoe::k_moe_decode1x<0, 2, 768, 1, 8, false>"}
# committed rocprofv3 counter summaries (profiles/<name>.json) of the decode lines
COUNTER_FILES = {1: "k_moe_decode1x_qwen3_b1_counters"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def per_expert_bytes(h=H, i=I, gs=GS) -> int:
    """Packed gate+up+down nibbles plus bf16 scale and bias per group."""
    gate_up = 2 * i * (h // 2 + (h // gs) * 4)
    down = h * (i // 2 + (i // gs) * 4)
    return gate_up + down


def build_layers(dev, n_layers: int, seed: int = 0):
    import torch

    from zmlx_amd.layer import QuantizedMoELayer, QuantProj
    from zmlx_amd.quant import quantize_affine

    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def bank(n_out, n_in):
        ws, ss, bs = [], [], []
        for e0 in range(0, E, 16):
            w = (torch.randn((16, n_out, n_in), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            q, s, b = quantize_affine(w, GS)
            ws.append(q), ss.append(s), bs.append(b)
        return torch.cat(ws), torch.cat(ss), torch.cat(bs)

    base = {"gate": bank(I, H), "up": bank(I, H), "down": bank(H, I)}
    torch.cuda.synchronize()
    layers = []
    for li in range(n_layers):
        copy = {k: tuple(t.clone() for t in v) for k, v in base.items()}
        wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        layers.append(QuantizedMoELayer.for_family(
            "qwen3", wr, QuantProj(*copy["gate"]), QuantProj(*copy["up"]), QuantProj(*copy["down"]), top_k=K,
            group_size=GS))
    torch.cuda.synchronize()
    return layers, base


def capture_step(layers, x):
    """Capture one step (every layer copy once) into a HIP graph so replays
    measure the GPU, not Python/ctypes launch overhead."""
    import torch

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for layer in layers:  # allocate workspaces / outputs outside capture
            layer(x)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for layer in layers:
            layer(x)
    torch.cuda.synchronize()
    return graph


def time_layers(layers, x, steps: int, warmup: int, use_graph: bool = True, per_step: list | None = None) -> float:
    """Average ms per step (one call of every layer copy), from HIP events
    recorded on the stream the layer kernels run on (torch's current stream,
    where the graph is replayed).  If ``per_step`` is a list, the ms of each
    step is appended to it (events between steps)."""
    import torch

    if use_graph:
        graph = capture_step(layers, x)
        run = graph.replay
    else:
        def run():
            for layer in layers:
                layer(x)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    evs[0].record()
    for i in range(steps):
        run()
        evs[i + 1].record()
    torch.cuda.synchronize()
    if per_step is not None:
        per_step.extend(evs[i].elapsed_time(evs[i + 1]) for i in range(steps))
    return evs[0].elapsed_time(evs[-1]) / steps


def unique_experts(layers, x):
    import torch

    counts = []
    idxs = []
    for layer in layers:
        _, idx, _ = layer(x, return_routing=True)
        idxs.append(idx)
    torch.cuda.synchronize()
    for idx in idxs:
        counts.append(int(torch.unique(idx).numel()))
    return counts, idxs


def prefill_x(layer, B, gen, dev, skew=1.1, peak=3.0, seed=7):
    """x for the prefill line (config 4): N(0,1) tokens plus a shared
    component along the router rows that adds a Zipf-skewed logit offset
    peak * rank^-skew to the experts (ranks over a fixed random permutation),
    so expert loads are imbalanced."""
    import torch

    wr = layer._router_w.float()
    rank = torch.empty(E, device=dev)
    perm = torch.randperm(E, generator=torch.Generator().manual_seed(seed)).to(dev)
    rank[perm] = torch.arange(1, E + 1, device=dev, dtype=torch.float32)
    off = peak * rank.pow(-skew)
    v = ((off / (wr * wr).sum(1))[:, None] * wr).sum(0)
    z = torch.randn((B, H), generator=gen, device=dev)
    return (z + v[None, :]).to(torch.bfloat16)


def prefill_line(layers, B, gen, dev, steps, warmup):
    """Config 4: B tokens through every layer copy (grouped GEMMs on MFMA over
    the pairs sorted by expert), graph-replayed like the decode lines."""
    x = prefill_x(layers[0], B, gen, dev)
    counts, idxs = unique_experts(layers, x)
    import torch

    loads = torch.bincount(idxs[0].reshape(-1).long(), minlength=E).cpu().tolist()
    ms = time_layers(layers, x, steps, warmup)
    layer_us = ms * 1e3 / len(layers)
    avg_unique = sum(counts) / len(counts)
    alg_bytes = avg_unique * per_expert_bytes() + E * H * 2 + 4 * B * H
    flops = B * K * 6 * H * I + 2 * B * E * H
    gbps = alg_bytes / (layer_us * 1e-6) / 1e9
    return {"tokens": B, "us_per_layer_call": round(layer_us, 3), "us_per_token": round(layer_us / B, 4),
            "gbps": round(gbps, 1), "roofline_frac": round(gbps / HBM_PEAK_GBPS, 4),
            "tflops": round(flops / (layer_us * 1e-6) / 1e12, 2), "mfma_frac_bf16": round(flops / (layer_us * 1e-6) / 2.5e15, 4),
            "unique_experts": round(avg_unique, 2), "max_expert_rows": max(loads), "min_expert_rows": min(loads),
            "alg_bytes_per_call": int(alg_bytes), "steps": steps, "counters": prefill_counters()}


def profile_run(args) -> int:
    """Short run for `rocprofv3 --pmc`: one calibration copy of COPY_BYTES
    (torch's copy kernel), then graph replays of the B=1 workload."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    layers, _ = build_layers(dev, args.layers)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    if args.batch >= 32:  # the prefill line's Zipf-skewed tokens
        x = prefill_x(layers[0], args.batch, gen, dev)
    else:
        x = torch.randn((args.batch, H), generator=gen, device=dev).to(torch.bfloat16)
    ms = time_layers(layers, x, args.steps, args.warmup)
    log(f"profile run: B={args.batch} {ms * 1e3 / len(layers):.2f} us per layer call")
    return 0


def _pmc_rows(d: str):
    """(kernel name, counter, value) rows of a rocprofv3 --pmc CSV run."""
    for path in Path(d).rglob("*counter_collection.csv"):
        with open(path) as f:
            for row in csv.DictReader(f):
                yield row["Kernel_Name"], row.get("Counter_Name"), float(row["Counter_Value"])


def _short_kernel(name: str) -> str:
    """Kernel name without its return type and parameter list (template
    arguments kept)."""
    name = name.replace("void ", "", 1)
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def summarize_pmc(out_path: str, fetch_dir: str, write_dir: str, mfma_dir: str | None = None) -> int:
    """Turns rocprofv3 --pmc runs of --profile-run into per-kernel HBM bytes
    per dispatch: FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled by
    the factor that makes the run's calibration copy move exactly COPY_BYTES.
    With a third run of SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE and
    SQ_INSTS_VALU_MFMA_MOPS_BF16 it adds each kernel's MFMA utilisation
    (rocprofv3's MfmaUtil: busy cycles summed over SIMDs / (GUI-active cycles
    x SIMDs)) and the bf16 MFMA flops it executed (MOPS x 512)."""
    out: dict = {"kernels": {}}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        vals: dict = {}
        for k, c, v in _pmc_rows(d):
            if c in (None, counter):
                vals.setdefault(k, []).append(v)
        copy = [v for k, vs in vals.items() if "copy" in k.lower() or "elementwise" in k.lower() for v in vs]
        if not copy:
            print(f"no calibration copy for {counter} in {d}", file=sys.stderr)
            return 1
        factor = (COPY_BYTES / 1024.0) / max(copy)
        out[counter + "_calibration"] = {"copy_kib": max(copy), "factor": factor}
        for k, vs in vals.items():
            if not k.lstrip("void ").startswith("zmoe::"):
                continue
            rec = out["kernels"].setdefault(_short_kernel(k), {})
            rec[counter.lower() + "_bytes"] = sum(vs) / len(vs) * 1024.0 * factor
            rec["dispatches"] = len(vs)
    for rec in out["kernels"].values():
        rec["bytes"] = rec.get("fetch_size_bytes", 0.0) + rec.get("write_size_bytes", 0.0)
    if mfma_dir:
        simds = 4 * 256  # MI355X: 256 CUs x 4 SIMDs
        acc: dict = {}
        for k, c, v in _pmc_rows(mfma_dir):
            if k.lstrip("void ").startswith("zmoe::"):
                acc.setdefault(_short_kernel(k), {}).setdefault(c, []).append(v)
        for k, cs in acc.items():
            rec = out["kernels"].setdefault(k, {})
            busy = sum(cs.get("SQ_VALU_MFMA_BUSY_CYCLES", [0])) / max(1, len(cs.get("SQ_VALU_MFMA_BUSY_CYCLES", [1])))
            gui = sum(cs.get("GRBM_GUI_ACTIVE", [0])) / max(1, len(cs.get("GRBM_GUI_ACTIVE", [1])))
            mops = sum(cs.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [0])) / max(1, len(cs.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [1])))
            rec["mfma_busy_cycles"] = busy
            rec["gui_active_cycles"] = gui
            rec["mfma_util"] = busy / (gui * simds) if gui else None
            rec["mfma_bf16_flops"] = mops * 512
    with open(out_path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))
    return 0


# Phase stamps of the XCD-partitioned one-token kernel (k_moe_decode1x), by
# trace slot: thread 0 of each workgroup, 100 MHz realtime counter.
PHASES = [
    (0, "kernel start (workgroup running)"),
    (1, "R: router rows of this XCD computed and stored, x tile written"),
    (3, "T: the XCD's logits polled from L2"),
    (4, "T: softmax and ranking done"),
    (5, "T: after the workgroup barrier (unit known)"),
    (13, "A: gate/up loads issued"),
    (6, "A: gate/up rows computed"),
    (7, "A: down-projection loads issued, act words stored"),
    (8, "D: act row staged in LDS from L2"),
    (9, "D: after the workgroup barrier"),
    (11, "D: down rows computed"),
    (10, "D: unit outputs stored (device scope)"),
    (12, "C: combine done (combining workgroups) / exit"),
]



def phase_trace(args) -> int:
    """Per-phase timing of the B=1 layer kernel: the untraced per-call time,
    then one traced graph replay whose stamps give, per phase, the median
    over workgroups and the latest workgroup (median over the 48 layer
    calls), relative to the earliest workgroup start of each call."""
    import statistics as st

    import torch

    from zmlx_amd import _native as N

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    B = args.batch
    if B != 1:
        print("--phase-trace: B=1 (the one-token kernels) only", file=sys.stderr)
        return 2
    if args.phase_config:
        if args.phase_config not in OTHER_CONFIGS:
            print(f"--phase-config: one of {sorted(OTHER_CONFIGS)}", file=sys.stderr)
            return 2
        layers = build_config_layers(args.phase_config, dev, gen)
        hidden = OTHER_CONFIGS[args.phase_config][1]
    else:
        layers, _ = build_layers(dev, args.layers)
        hidden = H
    print(f"config: {args.phase_config or 'qwen3_30b_a3b'}")
    x = torch.randn((B, hidden), generator=gen, device=dev).to(torch.bfloat16)
    phases = PHASES
    ms = time_layers(layers, x, args.steps, args.warmup)
    print(f"B={B} untraced: {ms * 1e3 / len(layers):.2f} us per layer call")
    for layer in layers:
        layer.desc.flags |= N.LAYER_TRACE
    ms_t = time_layers(layers, x, args.steps, args.warmup)
    print(f"traced:   {ms_t * 1e3 / len(layers):.2f} us per layer call")
    med: dict = {}
    last: dict = {}
    ends = []
    for layer in layers:
        t = layer.phase_trace(B).cpu()
        t0 = int(t[:, 0].min())
        ends.append((int(t.max()) - t0) * 0.01)
        for slot, _ in phases:
            col = [(int(v) - t0) * 0.01 for v in t[:, slot].tolist() if int(v) >= t0]
            if col:
                med.setdefault(slot, []).append(st.median(col))
                last.setdefault(slot, []).append(max(col))
    print("| slot | phase | median workgroup (us) | latest workgroup (us) |")
    print("|---|---|---|---|")
    for slot, name in phases:
        if slot in med:
            print(f"| {slot} | {name} | {st.median(med[slot]):.2f} | {st.median(last[slot]):.2f} |")
    print(f"| | last workgroup done | | {st.median(ends):.2f} |")
    errs = sum(layer.sync_error() for layer in layers)
    print(f"sticky error words: {errs}")
    return 0


def prefill_counters():
    """Per-kernel HBM bytes and MFMA activity of the prefill line's grouped
    GEMMs from the committed rocprofv3 counter summary
    (profiles/k_grouped_qmm_qwen3_prefill512_counters.json), or None."""
    prof = load_profile("k_grouped_qmm_qwen3_prefill512_counters")
    if not prof:
        return None
    out = {}
    for k, rec in prof.get("kernels", {}).items():
        if "k_grouped_qmm" not in k:
            continue
        out[k] = {"hbm_bytes": int(rec["bytes"]) if "bytes" in rec else None,
                  "mfma_util": round(rec["mfma_util"], 4) if rec.get("mfma_util") is not None else None,
                  "mfma_bf16_flops": rec.get("mfma_bf16_flops")}
    return out


def load_profile(name: str):
    """A committed counter summary (profiles/<name>.json), or None."""
    try:
        with open(ROOT / "profiles" / f"{name}.json") as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def cpu_baseline(base, layer0, x_host, budget_s: float = 12.0, max_tokens: int = 4096):
    """C++/OpenMP restatement of the unpatched path on the host cores, on a
    bounded sample of the same workload (one layer copy, single-token calls)."""
    import numpy as np
    import torch

    from oracle import ref_lib

    threads = min(len(os.sched_getaffinity(0)), 16)
    ref_lib.lib().oref_set_threads(threads)

    def bits(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    def words(t):
        return np.ascontiguousarray(t.contiguous().view(torch.int32).cpu().numpy().view(np.uint32))

    banks = {k: (words(v[0]), bits(v[1]), bits(v[2])) for k, v in base.items()}
    wr = bits(layer0._router_w)
    x16 = bits(x_host)
    # warm-up (page in the 340 MB layer)
    ref_lib.moe_layer_qwen_bits(x16[:1], wr, banks["gate"], banks["up"], banks["down"], k=K)
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s and n < max_tokens:
        ref_lib.moe_layer_qwen_bits(x16[n % x16.shape[0]:][:1], wr, banks["gate"], banks["up"], banks["down"], k=K)
        n += 1
    dt = time.perf_counter() - t0
    alg = K * per_expert_bytes() + E * H * 2 + 4 * H
    return {
        "value": round(dt * 1e6 / n, 2),
        "unit": "us/token",
        "gbps": round(alg * n / dt / 1e9, 2),
        "cores": threads,
        "kind": "port",
        "sample": f"{n} single-token calls of one Qwen3-shaped layer copy (B=1), "
                  f"C++/OpenMP restatement of the unpatched MLX path (MLX unavailable offline; AVX2, one "
                  f"parallel region per token), {dt:.1f}s",
    }


# The other BASELINE configs (measured with --all-configs; not the headline
# value): name -> (family, H, E, K, I, quant mode, group size, shared I,
# router kwargs, batches, layer copies).  Copies are clones of one generated
# bank, so every call reads its own weights from HBM (>= 8 copies, working
# sets well above the 256 MB Infinity Cache).
OTHER_CONFIGS = {
    "lfm2_8b_a1b": ("lfm2", 2048, 32, 4, 1792, "affine", 64, 0, {}, (1,), 8),
    "glm_4.7_flash_mxfp4": ("glm", 2048, 64, 4, 1536, "mxfp4", 32, 1536, {"routed_scaling_factor": 1.8}, (1, 8), 8),
    "deepseek_v3": ("deepseek", 7168, 256, 8, 2048, "affine", 64, 2048,
                    {"n_group": 8, "topk_group": 4, "routed_scaling_factor": 2.5}, (1, 64), 8),
}


def expert_bytes(h, i, mode, gs) -> int:
    if mode == "affine":
        return 2 * i * (h // 2 + (h // gs) * 4) + h * (i // 2 + (i // gs) * 4)
    return 2 * i * (h // 2 + h // 32) + h * (i // 2 + i // 32)


def build_config_layers(name: str, dev, g):
    """The layer copies of one of OTHER_CONFIGS (random weights from g)."""
    import torch

    from zmlx_amd.layer import QuantizedMoELayer, QuantProj
    from zmlx_amd.quant import quantize_affine, quantize_mxfp4

    fam, h, e, k, i, mode, gs, shi, kw, _, copies = OTHER_CONFIGS[name]
    log(f"{name}: building {copies} layer copies")

    def bank(n_exp, n_out, n_in):
        ws, ss, bs = [], [], []
        for e0 in range(0, n_exp, 16):
            w = (torch.randn((min(16, n_exp - e0), n_out, n_in), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            if mode == "affine":
                q, sc, bi = quantize_affine(w, gs)
            else:
                (q, sc), bi = quantize_mxfp4(w), None
            ws.append(q), ss.append(sc), bs.append(bi)
        return torch.cat(ws), torch.cat(ss), (torch.cat(bs) if bs[0] is not None else None)

    base = {"gate": bank(e, i, h), "up": bank(e, i, h), "down": bank(e, h, i)}
    sh = {"gate": bank(1, shi, h), "up": bank(1, shi, h), "down": bank(1, h, shi)} if shi else None
    layers = []
    for _ in range(copies):
        cp = {n: tuple(None if t is None else t.clone() for t in v) for n, v in base.items()}
        shared = None
        if sh is not None:
            shared = tuple(QuantProj(v[0][0].clone(), v[1][0].clone(), None if v[2] is None else v[2][0].clone())
                           for v in (sh["gate"], sh["up"], sh["down"]))
        wr = (torch.randn((e, h), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        bias = (torch.randn((e,), generator=g, device=dev) * 0.05) if fam in ("glm", "deepseek") else None
        layers.append(QuantizedMoELayer.for_family(
            fam, wr, *(QuantProj(*cp[n]) for n in ("gate", "up", "down")), top_k=k, router_bias=bias,
            group_size=gs, mode=mode, shared=shared, **kw))
    del base, sh
    torch.cuda.synchronize()
    return layers


def other_config_lines(dev, steps: int, warmup: int) -> dict:
    """Per-config lines: us per layer call, algorithmic GB/s and the fraction
    of the 8 TB/s roofline at each of the config's batch sizes."""
    import torch

    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    for name, (fam, h, e, k, i, mode, gs, shi, kw, batches, copies) in OTHER_CONFIGS.items():
        layers = build_config_layers(name, dev, g)
        for B in batches:
            x = torch.randn((B, h), generator=g, device=dev).to(torch.bfloat16)
            uniq = []
            for layer in layers:
                _, idx, _ = layer(x, return_routing=True)
                uniq.append(int(torch.unique(idx).numel()))
            ms = time_layers(layers, x, steps, warmup)
            us = ms * 1e3 / len(layers)
            avg_u = sum(uniq) / len(uniq)
            alg = avg_u * expert_bytes(h, i, mode, gs) + (expert_bytes(h, shi, mode, gs) if shi else 0) \
                + e * h * 2 + 4 * B * h
            gbps = alg / (us * 1e-6) / 1e9
            out[f"{name}_b{B}"] = {"us_per_layer_call": round(us, 3), "us_per_token": round(us / B, 3),
                                   "gbps": round(gbps, 1), "roofline_frac": round(gbps / HBM_PEAK_GBPS, 4),
                                   "unique_experts": round(avg_u, 2), "alg_bytes_per_call": int(alg),
                                   "layer_copies": copies, "steps": steps}
            log(f"{name} B={B}: {out[f'{name}_b{B}']}")
        del layers
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--extra-batches", default="4,16")
    ap.add_argument("--prefill", type=int, default=512,
                    help="tokens of the prefill line (config 4; 0 skips it)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the other BASELINE configs (LFM2, GLM-mxfp4, DeepSeek-V3)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--profile-run", action="store_true", help="short run for rocprofv3 counter passes")
    ap.add_argument("--phase-trace", action="store_true", help="per-phase stamps of the B=1 layer kernel")
    ap.add_argument("--phase-config", default="", help="with --phase-trace: one of the other configs "
                    "(e.g. lfm2_8b_a1b) instead of the Qwen3 layer")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="PATH",
                    help="OUT_JSON FETCH_DIR WRITE_DIR [MFMA_DIR]: per-kernel counter summary")
    args = ap.parse_args()
    if args.summarize_pmc:
        if len(args.summarize_pmc) not in (3, 4):
            ap.error("--summarize-pmc OUT_JSON FETCH_DIR WRITE_DIR [MFMA_DIR]")
        return summarize_pmc(*args.summarize_pmc)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the decode MoE layer on one MI355X); "
              "--gpus must be 1", file=sys.stderr)
        return 2

    import torch

    import zmlx_amd  # noqa: F401  (fails loudly if the HIP library is missing)

    if args.profile_run:
        return profile_run(args)
    if args.phase_trace:
        return phase_trace(args)
    dev = torch.device("cuda:0")
    log(f"building {args.layers} layer copies (this takes a few seconds)")
    layers, base = build_layers(dev, args.layers)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    batches = [args.batch] + [int(b) for b in args.extra_batches.split(",") if b and int(b) != args.batch]
    per_b = {}
    main_rec = None
    for B in batches:
        x = torch.randn((B, H), generator=gen, device=dev).to(torch.bfloat16)
        counts, idxs = unique_experts(layers, x)
        steps = args.steps if B == args.batch else max(5, args.steps // 4)
        log(f"B={B}: timing {steps} steps x {len(layers)} layers")
        step_ms: list = []
        ms = time_layers(layers, x, steps, args.warmup, use_graph=not args.no_graph, per_step=step_ms)
        layer_us = ms * 1e3 / len(layers)
        q = sorted(v * 1e3 / len(layers) for v in step_ms)
        pct = {f"p{p}": round(q[min(len(q) - 1, int(p / 100 * len(q)))], 3) for p in (10, 50, 90)}
        avg_unique = sum(counts) / len(counts)
        alg_bytes = avg_unique * per_expert_bytes() + E * H * 2 + 4 * B * H
        gbps = alg_bytes / (layer_us * 1e-6) / 1e9
        rec = {"us_per_token": round(layer_us / B, 3), "us_per_layer_call": round(layer_us, 3),
               "gbps": round(gbps, 1), "roofline_frac": round(gbps / HBM_PEAK_GBPS, 4),
               "unique_experts": round(avg_unique, 2), "alg_bytes_per_call": int(alg_bytes), "steps": steps,
               "ms_per_step": round(ms, 4), "us_per_layer_call_pct": pct}
        per_b[str(B)] = rec
        if B == args.batch:
            main_rec = rec
            # B=1: one k_moe_decode1x launch per layer call, so the timed
            # region holds steps x layers launches and nothing else; other
            # batches run a kernel sequence, priced per layer call
            kname = DECODE_KERNELS.get(B)
            tr = (load_profile(COUNTER_FILES.get(B, "")) or {}).get("kernels", {}).get(kname) if kname else None
            roof = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(gbps / HBM_PEAK_GBPS, 4),
                    "traffic": int(tr["bytes"]) if tr else None,
                    "kernel": kname or "kernel sequence (k_dense_logits, k_route_rows, k_gather_qmv x2, "
                                       "k_moe_combine; or k_grouped_qmm from 32 tokens)",
                    ("avg_launch_us" if kname else "avg_call_us"): round(layer_us, 3),
                    ("alg_bytes_per_launch" if kname else "alg_bytes_per_call"): int(alg_bytes)}
        log(f"B={B}: {rec}")

    if args.prefill > 0:
        per_b["prefill"] = prefill_line(layers, args.prefill, gen, dev, max(3, args.steps // 10), args.warmup)
        log(f"prefill: {per_b['prefill']}")

    n_copies = len(layers)
    if not args.no_other_configs:
        layers = layers[:1]  # the CPU baseline reads the first copy
        torch.cuda.empty_cache()
        per_b["configs"] = other_config_lines(dev, max(5, args.steps // 5), args.warmup)

    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (C++ restatement) ...")
        x_host = torch.randn((64, H), generator=gen, device=dev).to(torch.bfloat16)
        cpu = cpu_baseline(base, layers[0], x_host, budget_s=args.cpu_budget)
        log(f"CPU baseline: {cpu}")

    out = {
        "metric": METRIC,
        "value": main_rec["us_per_token"],
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_rec["ms_per_step"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "qwen3-30b-a3b-moe-layer-decode", "hidden": H, "experts": E, "top_k": K,
                   "inter": I, "quant": "affine4-g64", "batch": args.batch, "layer_copies": n_copies,
                   "parallelism": "none (1 GPU)"},
        "gbps": main_rec["gbps"],
        "roofline": roof,
        "cpu_baseline": cpu,
        "batches": per_b,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
