"""Benchmark of the fused Token-Union W4A16 MoE layer on one MI355X.

Metric: fused W4A16 MoE layer time and achieved HBM GB/s at
M=1 (configs[1], the headline ``value``) and M=7 (configs[2], reported beside
it), Gemma-4-26B-A4B expert shapes: hidden 2816, 128 experts, top-8,
intermediate 704, int4 weights with bf16 scales per group of 128 (the down
projection has 6 groups, the last 64 rows wide).

A step is one layer: router top-8 softmax + Token-Union alignment + gate_up +
gelu_tanh*up + down + routing-weighted combine, as ONE kernel launch
(gi_moe_layer_from_logits) from N(0,1) fp32 router logits.

Measurement:
  * Weights: 4 independent copies of the full 128-expert layer (1.57 GB).
    Each step's N(0,1) logits are relabelled (a permutation of expert ids,
    values unchanged) so that every copy's experts are visited in rotation:
    >= 1 GB of other weights is read between two reads of the same expert
    bytes inside the timed replay, so the 256 MB MALL cannot serve them.
  * W warmup steps, then K steps captured in one HIP graph, replayed once
    untimed (the graph's upload), then replayed between HIP events on the
    launch stream (synchronised on both sides); us_per_layer = elapsed / K.
    Between two reads of the same bytes more than all caches together
    (256 MB MALL + 32 MB L2) must be read: the untimed replay's own steps
    count, and where they fall short (the 4 MB steps of configs[0]) 1 GiB of
    other memory is read before the timed replay.  The realised minimum
    reuse distance (untimed replay and flush included) is reported.  Hot-cache (same weights every step) and
    stream-launched (no graph, Python ctypes per call) figures are reported
    separately; neither is ``value``.
  * Algorithmic bytes per layer = unique experts x 3,069,440 B (packed
    gate_up + down words and their bf16 scales), activations excluded.
  * cpu_baseline: the reference's PyTorch CPU dequant+matmul path
    (oracle/cpu_baseline.py), timed on this host's cores on a bounded sample.
  * The default line also carries every other BASELINE config under the
    same clock (``configs``): the W4A16 linear, the prefill
    layer at M=512 and the lm_head at M=6.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from gemmainfer_amd import _lib as L  # noqa: E402
from gemmainfer_amd import synth  # noqa: E402

METRIC = "fused W4A16 MoE layer us + achieved HBM GB/s at M=1 and M=7 (1 GPU)"
E, H, I, TOP_K, GS = 128, 2816, 704, 8, 128
COPIES = 4
PEAK_GBPS = 8000.0


def expert_bytes(h=H, i=I, gs=None) -> int:
    """Packed words + bf16 scales of one expert (gate_up and down)."""
    gs = GS if gs is None else gs
    gu = (h // 8) * 2 * i * 4 + math.ceil(h / gs) * 2 * i * 2
    dn = (i // 8) * h * 4 + math.ceil(i / gs) * h * 2
    return gu + dn


def first_occurrence_unique(idx_row_major):
    seen, out = set(), []
    for e in idx_row_major:
        if e not in seen:
            seen.add(e)
            out.append(e)
    return out


def make_steps(m, noise, seed, n_desc):
    """Per-step (copy, logits, unique experts) with expert ids relabelled so
    that each copy's experts are used in rotation."""
    cursor = [0] * COPIES
    steps = []
    for s in range(n_desc):
        c = s % COPIES
        logits = synth.router_logits(m, E, seed=seed * 100003 + s, verify_noise=noise)
        top = torch.topk(logits, TOP_K, dim=-1).indices.reshape(-1).tolist()
        uniq = first_occurrence_unique(top)
        block = [(cursor[c] + j) % E for j in range(len(uniq))]
        cursor[c] = (cursor[c] + len(uniq)) % E
        rest_src = [e for e in range(E) if e not in set(uniq)]
        rest_dst = [e for e in range(E) if e not in set(block)]
        perm = [0] * E  # perm[old] = new
        for o, n in zip(uniq, block):
            perm[o] = n
        for o, n in zip(rest_src, rest_dst):
            perm[o] = n
        new = torch.empty_like(logits)
        new[:, torch.tensor(perm)] = logits
        steps.append({"copy": c, "logits": new, "unique": sorted(block), "U": len(uniq)})
    return steps


def min_reuse_distance_bytes(steps, order, gs=None, prior=(), gap_bytes=0):
    """Smallest number of bytes read between a read of one expert's weights in
    the timed ``order`` and the previous read of the same bytes: earlier reads
    in ``order`` or in ``prior`` (the steps run before the timed region: the
    launch before capture and the graph's upload replay), with ``gap_bytes``
    of other reads (the cache flush) between ``prior`` and ``order``."""
    eb = expert_bytes(gs=gs)
    last, touched, best = {}, 0, None

    def visit(s, timed):
        nonlocal touched, best
        st = steps[s]
        for e in st["unique"]:
            key = (st["copy"], e)
            if timed and key in last:
                d = touched - last[key]
                best = d if best is None else min(best, d)
        for e in st["unique"]:
            last[(st["copy"], e)] = touched
        touched += st["U"] * eb

    for s in prior:
        visit(s, False)
    touched += gap_bytes
    for s in order:
        visit(s, True)
    return best


# Cache hygiene between a graph's untimed upload replay and its timed
# replay: two reads of the same weight bytes must have more than every cache
# together between them (the 256 MB MALL and 8 x 4 MB of L2).  Where the
# steps of the replays do not provide that themselves (configs[0]: 4 MB per
# step), FLUSH_BYTES of other memory are read in between.  A flush where the
# steps already provide it only cools the TLB for the first timed launches.
CACHE_BYTES = (256 + 32) << 20
FLUSH_BYTES = 1 << 30
_FLUSH = {}


def flush_caches(device):
    buf = _FLUSH.get(device)
    if buf is None:
        buf = _FLUSH[device] = torch.zeros(FLUSH_BYTES // 8, dtype=torch.int64, device=device)
    buf.max()  # reads every byte once


class LayerRunner:
    """Direct C-ABI launches of gi_moe_layer_from_logits with fixed buffers."""

    def __init__(self, m, steps, copies, device, gs=None):
        self.lib = L.load()
        self.m = m
        self.gs = GS if gs is None else gs
        self.dev = device
        self.copies = copies
        self.x = synth.activations(m, H, seed=7).to(device)
        self.logits = [st["logits"].to(device).contiguous() for st in steps]
        self.copy_of = [st["copy"] for st in steps]
        self.out = torch.empty(m, H, dtype=torch.bfloat16, device=device)
        self.idx = torch.empty(m, TOP_K, dtype=torch.int32, device=device)
        self.w = torch.empty(m, TOP_K, dtype=torch.bfloat16, device=device)
        nbytes = self.lib.gi_fused_moe_workspace_bytes(m, TOP_K, H, I, E)
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        torch.cuda.synchronize()

    def launch(self, s):
        W = self.copies[self.copy_of[s]]
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        st = self.lib.gi_moe_layer_from_logits(
            p(self.x), L.DTYPE_BF16, p(self.logits[s]), L.DTYPE_FP32, None,
            p(W["gate_up_packed"]), p(W["gate_up_scales"]), W["gate_up_scales"].shape[1],
            p(W["down_packed"]), p(W["down_scales"]), W["down_scales"].shape[1],
            p(self.out), p(self.idx), p(self.w), self.m, H, I, E, TOP_K, self.gs,
            p(self.ws), self.ws.numel(), 0, stream)
        L.check(st, "gi_moe_layer_from_logits")

    def status(self):
        v = ctypes.c_int32(0)
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        L.check(self.lib.gi_workspace_status(ctypes.c_void_p(self.ws.data_ptr()), self.ws.numel(),
                                             ctypes.byref(v), stream), "status")
        return v.value


def time_graph(runner, order, device, flush=False):
    """Capture launches in `order` into one graph; return us per launch
    (flush: FLUSH_BYTES read between the upload replay and the timed one)."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        runner.launch(order[0])  # launch once on the capture stream before capturing
    torch.cuda.current_stream(device).wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        for i in order:
            runner.launch(i)
    torch.cuda.synchronize()
    g.replay()  # untimed replay: first replay uploads the graph
    if flush:
        flush_caches(device)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / len(order)


def time_stream(runner, order):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in order:
        runner.launch(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / len(order)


def bench_config(m, noise, seed, copies, steps, warmup, device, gs=None):
    # one descriptor per executed step, so the expert rotation never wraps
    gs = GS if gs is None else gs
    n_desc = warmup + steps
    desc = make_steps(m, noise, seed, n_desc)
    runner = LayerRunner(m, desc, copies, device, gs)
    for i in range(warmup):
        runner.launch(i)
    torch.cuda.synchronize()
    order = [warmup + i for i in range(steps)]
    natural = min_reuse_distance_bytes(desc, order, gs, prior=[order[0]] + order)
    flush = natural is None or natural <= CACHE_BYTES
    us = time_graph(runner, order, device, flush=flush)
    hot_us = time_graph(runner, [order[0]] * min(steps, 200), device)
    stream_us = time_stream(runner, order[: min(steps, 200)])
    if runner.status() != 0:
        raise RuntimeError("device status word set during the benchmark")
    mean_u = statistics.fmean(desc[i]["U"] for i in order)
    nbytes = mean_u * expert_bytes(gs=gs)
    return {
        "M": m,
        "group_size": gs,
        "us_per_layer": us,
        "gbps": nbytes / (us * 1e-6) / 1e9,
        "unique_experts_mean": mean_u,
        "unique_experts_range": [min(desc[i]["U"] for i in order), max(desc[i]["U"] for i in order)],
        "algorithmic_bytes_per_layer": nbytes,
        "min_reuse_distance_bytes": min_reuse_distance_bytes(desc, order, gs, prior=[order[0]] + order,
                                                             gap_bytes=FLUSH_BYTES if flush else 0),
        "cache_flush_bytes": FLUSH_BYTES if flush else 0,
        "hot_cache_us_per_layer": hot_us,
        "stream_launched_us_per_layer": stream_us,
    }


class DtypeRunner:
    """gi_fused_batched_moe with fp16 or fp32 activations and scales (the
    reference's other dtypes, marlin.cu:694-700): ids and weights routed on
    the host from each step's logits (gemma.py:77-80), out accumulated into."""

    def __init__(self, m, steps, copies, device, dt, gs=None):
        self.lib = L.load()
        self.m, self.dev, self.copies, self.dt = m, device, copies, dt
        self.gs = GS if gs is None else gs
        self.code = L.DTYPE_FP16 if dt == torch.float16 else L.DTYPE_FP32
        self.x = synth.activations(m, H, seed=7).to(dt).to(device)
        self.idx, self.w = [], []
        for st in steps:
            top, ix = torch.topk(st["logits"], TOP_K, dim=-1)
            self.idx.append(ix.to(torch.int32).contiguous().to(device))
            self.w.append(torch.softmax(top, dim=-1, dtype=torch.float32).to(dt).contiguous().to(device))
        self.copy_of = [st["copy"] for st in steps]
        self.out = torch.zeros(m, H, dtype=dt, device=device)
        nbytes = self.lib.gi_fused_moe_workspace_bytes(m, TOP_K, H, I, E)
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        torch.cuda.synchronize()

    def launch(self, s):
        W = self.copies[self.copy_of[s]]
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        st = self.lib.gi_fused_batched_moe(
            p(self.x), self.code, p(W["gate_up_packed"]), p(W["gate_up_scales"]), W["gate_up_scales"].shape[1],
            p(W["down_packed"]), p(W["down_scales"]), W["down_scales"].shape[1], p(self.idx[s]), L.DTYPE_INT32,
            p(self.w[s]), self.code, p(self.out), self.m, H, I, E, TOP_K, self.gs, p(self.ws), self.ws.numel(), 0,
            stream)
        L.check(st, "gi_fused_batched_moe (fp16/fp32)")


def bench_dtype(dt, steps, warmup, device):
    """The MoE layer at M=1 and M=7 (configs[1], [2] routing) with fp16 or fp32
    activations and scales: the same rotated weight words, scales in the dtype."""
    copies = []
    for c in range(COPIES):
        Wc = synth.device_moe_weights(E, H, I, GS, device, seed=100 + c)
        Wc["gate_up_scales"] = Wc["gate_up_scales"].to(dt)
        Wc["down_scales"] = Wc["down_scales"].to(dt)
        copies.append(Wc)
    torch.cuda.synchronize()
    rows = {}
    for m, noise, seed in ((1, 0.0, 1), (7, 0.5, 2)):
        desc = make_steps(m, noise, seed, warmup + steps)
        runner = DtypeRunner(m, desc, copies, device, dt)
        for i in range(warmup):
            runner.launch(i)
        torch.cuda.synchronize()
        order = [warmup + i for i in range(steps)]
        us = time_graph(runner, order, device)
        mean_u = statistics.fmean(desc[i]["U"] for i in order)
        sb = 2 if dt == torch.float16 else 4
        nbytes = mean_u * (expert_bytes() + (sb - 2) * (math.ceil(H / GS) * 2 * I + math.ceil(I / GS) * H))
        rows[f"M{m}"] = {"us_per_layer": us, "gbps": nbytes / (us * 1e-6) / 1e9, "unique_experts_mean": mean_u,
                         "algorithmic_bytes_per_layer": nbytes}
    return rows


class StreamRunner:
    """gi_probe_stream_read over the bytes one layer launch of each step reads
    (the packed gate_up and down words and the scales of the step's unique
    experts, on the step's weight copy): the attainable pure-read time for
    exactly the layer's algorithmic bytes, with the same rotation past the
    MALL."""

    def __init__(self, steps, copies, device, lpt):
        self.lib = L.load()
        self.dev, self.lpt = device, lpt
        self.sink = torch.zeros(4, dtype=torch.int32, device=device)
        self.segs = []
        for st in steps:
            W = copies[st["copy"]]
            ptrs, sizes = [], []
            for e in st["unique"]:
                for name in ("gate_up_packed", "gate_up_scales", "down_packed", "down_scales"):
                    t = W[name]
                    ptrs.append(t.data_ptr() + e * t.stride(0) * t.element_size())
                    sizes.append(t[e].numel() * t.element_size())
            n = len(ptrs)
            self.segs.append(((ctypes.c_void_p * n)(*ptrs), (ctypes.c_uint64 * n)(*sizes), n))

    def launch(self, s):
        ptrs, sizes, n = self.segs[s]
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        L.check(self.lib.gi_probe_stream_read(ptrs, sizes, n, self.lpt, ctypes.c_void_p(self.sink.data_ptr()),
                                              stream), "gi_probe_stream_read")


STREAM_LPT = (2, 4, 8, 16)


def bench_stream(m, noise, seed, copies, steps, warmup, device, gs=None):
    """Pure-read ceiling for the byte set of the M-row layer: the same steps
    (copy, unique experts) as bench_config, timed the same way, for every
    loads-per-thread setting of the probe; the fastest is the ceiling."""
    gs = GS if gs is None else gs
    desc = make_steps(m, noise, seed, warmup + steps)
    order = [warmup + i for i in range(steps)]
    mean_u = statistics.fmean(desc[i]["U"] for i in order)
    nbytes = mean_u * expert_bytes(gs=gs)
    sweep = {}
    for lpt in STREAM_LPT:
        runner = StreamRunner(desc, copies, device, lpt)
        for i in range(warmup):
            runner.launch(i)
        torch.cuda.synchronize()
        sweep[lpt] = time_graph(runner, order, device)
    best = min(sweep, key=sweep.get)
    us = sweep[best]
    return {"M": m, "group_size": gs, "us_per_read": us, "gbps": nbytes / (us * 1e-6) / 1e9,
            "bytes_per_read": nbytes, "unique_experts_mean": mean_u,
            "loads_per_thread": best, "sweep_us": {str(k): v for k, v in sweep.items()},
            "probe": "gi_probe_stream_read: 256-thread workgroups, 4 KB x loads_per_thread contiguous "
                     "bytes of one segment each, non-temporal 16-byte loads all issued before use"}


D1_ROUTING_PHASES = ["routing inputs landed (wave 0)", "wave 0 routing work done", None, None,
                     "x staged (wave 1)", "previous footprint cleared", "logit keys in LDS (wave 0)",
                     "top-k selected (wave 0)", None, "softmax (wave 0)"]
TIMELINE_PHASES = {
    # decode kernel (up to 8 rows per launch): roles by whether the workgroup holds gate/up items
    (1, "item"): ["start", "routing and tables", "x in LDS", "weight loads issued", "gate/up items done",
                  "activations staged", "down products", "sums over waves", "output / partial sums", "end",
                  "first item's first k block's words landed (wave 0)",
                  "first item's last k block's words landed (wave 0)",
                  "second item's first k block's words landed (wave 0)",
                  "second item's last k block's words landed (wave 0)",
                  "first down batch's words landed (wave 0)",
                  "top-k and softmax of token 0 (wave 0)", "all tokens routed (barrier)",
                  "Token-Union tables built (wave 0)", "work split computed (wave 0)",
                  "x written to LDS (wave 0)"],
    (1, "down"): ["start", "routing and tables", "x in LDS", "weight loads issued", "gate/up items done",
                  "activations staged", "down products", "sums over waves", "output / partial sums", "end"],
    # one-token kernel: item and unit workgroups
    (2, "item"): ["start", "routing", "weight loads issued", None, "gate/up products",
                  "activations published", "folded partial sums published",
                  "folded unit output written (items 0-7)", None, "end", *D1_ROUTING_PHASES,
                  "first k block's words landed (wave 0)", "last k block's words landed (wave 0)"],
    (2, "unit"): ["start", "routing", "weight loads issued", "words unpacked", "activations staged (wave 0)",
                  "down products", "unit output written", None, None, "end", *D1_ROUTING_PHASES,
                  "activations staged (last expert's wave)", "products issued (wave 0)",
                  "products done (wave 0)"],
    (2, "idle"): ["start", "routing", None, None, None, None, None, None, None, "end", *D1_ROUTING_PHASES],
}


def _timeline_role(kernel, v14):
    if kernel == 1:
        return "item" if v14 > 0 else "down"
    return {1: "item", 2: "unit"}.get(v14, "idle")


def bench_timeline(copies, steps, warmup, device, gs):
    """Phase stamps of the decode kernel (the timeline library only): for the
    M=1 and M=7 rotated steps, the graph-timed K launches each write every
    workgroup's stamps; per launch, times are taken from the earliest
    workgroup start, and per phase the median and the maximum over the
    workgroups of each role (gate/up items held or not) are reported as the
    median over the launches."""
    lib = L.load()
    slot = 1024 * 32
    res = {}
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for m, noise, seed in ((1, 0.0, 1), (7, 0.5, 2)):
        desc = make_steps(m, noise, seed, warmup + steps)
        runner = LayerRunner(m, desc, copies, device, gs)
        for i in range(warmup):
            runner.launch(i)
        torch.cuda.synchronize()
        buf = torch.zeros((steps + 1) * slot, dtype=torch.int64, device=device)
        L.check(lib.gi_probe_decode_timeline(p(buf), buf.numel() * 8), "gi_probe_decode_timeline")
        order = [warmup + i for i in range(steps)]
        us = time_graph(runner, order, device)  # slot 0: the launch before capture; 1..K: the graph
        L.check(lib.gi_probe_decode_timeline(None, 0), "gi_probe_decode_timeline")
        torch.cuda.synchronize()
        st = buf.view(steps + 1, 1024, 32)[1:].cpu()
        per = {}
        counts = {}
        spans = []
        kernel = None
        for k in range(steps):
            a = st[k]
            a = a[a[:, 0] != 0]
            kernel = int(a[0, 29])
            t0 = int(a[:, 0].min())
            rel = (a[:, :24] - t0).double() * 0.01  # 100 MHz -> us
            rel[a[:, :24] == 0] = float("nan")
            spans.append(float(rel[:, 9].max()))
            roles = [_timeline_role(kernel, int(v)) for v in a[:, 30]]
            for role in set(roles):
                mask = torch.tensor([r == role for r in roles])
                r = rel[mask]
                if k == 0:
                    counts[role] = int(mask.sum())
                row = []
                for i in range(24):
                    col = r[:, i][~torch.isnan(r[:, i])]
                    row.append((float(col.median()), float(col.max())) if col.numel() else (None, None))
                per.setdefault(role, []).append(row)
        roles_out = {}
        for role, rows in per.items():
            table = {}
            for i, name in enumerate(TIMELINE_PHASES[(kernel, role)]):
                med = [r[i][0] for r in rows if r[i][0] is not None]
                mx = [r[i][1] for r in rows if r[i][1] is not None]
                if name and med:
                    table[name] = {"median_us": statistics.median(med), "max_us": statistics.median(mx)}
            roles_out[role] = {"workgroups": counts.get(role, 0), "phases": table}
        roles = roles_out
        res[f"M{m}"] = {"us_per_layer_graph": us, "kernel_span_us_median": statistics.median(spans),
                        "kernel": "moe_decode1_kernel" if kernel == 2 else "moe_decode_kernel",
                        "roles": roles, "launches": steps}
        print(f"[timeline] M={m} graph {us:.2f} us, stamped span {statistics.median(spans):.2f} us",
              file=sys.stderr, flush=True)
    return res


class FrontEndRunner:
    """Router front-end of one MoE block (gemma.py:75-76) three ways, each step
    on one of COPIES gate copies in rotation: ``fused`` = gi_moe_router_logits
    (one launch); ``torch`` = the module's statements as the reference runs
    them on this build (the drop-in rmsnorm kernel, two bf16 elementwise
    products, the bf16 nn.Linear); ``layer`` = gi_moe_layer_from_hidden, the
    whole block (router launch + layer launch) on the expert weight copies."""

    def __init__(self, m, copies, device, mode, gs=None):
        import gemmainfer_csrc  # noqa: PLC0415  (the drop-in module)
        self.csrc = gemmainfer_csrc
        self.lib = L.load()
        self.m, self.dev, self.mode, self.copies = m, device, mode, copies
        self.gs = GS if gs is None else gs
        self.x = synth.activations(m, H, seed=9).to(device)
        self.R = []
        for c in range(COPIES):
            r = synth.router_weights(E, H, seed=200 + c)
            self.R.append({k: v.to(device) for k, v in r.items()})
        self.logits = torch.empty(m, E, dtype=torch.bfloat16, device=device)
        self.norm = torch.empty(m, H, dtype=torch.bfloat16, device=device)
        self.out = torch.empty(m, H, dtype=torch.bfloat16, device=device)
        self.idx = torch.empty(m, TOP_K, dtype=torch.int32, device=device)
        self.w = torch.empty(m, TOP_K, dtype=torch.bfloat16, device=device)
        self.es = [r["expert_scale"].float().contiguous() for r in self.R]
        nbytes = self.lib.gi_fused_moe_workspace_bytes(m, TOP_K, H, I, E)
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        torch.cuda.synchronize()

    def launch(self, s):
        r = self.R[s % COPIES]
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        if self.mode == "fused":
            L.check(self.lib.gi_moe_router_logits(p(self.x), L.DTYPE_BF16, p(r["router_scale"]),
                                                  p(r["gate"]), 1e-6, p(self.logits), self.m, H, E,
                                                  stream), "gi_moe_router_logits")
        elif self.mode == "torch":
            self.csrc.rmsnorm(self.x, torch.empty(0), self.norm, 1e-6, False)
            xn = self.norm * (r["router_scale"] * (H ** -0.5))
            self.logits = torch.nn.functional.linear(xn, r["gate"])
        else:
            W = self.copies[s % COPIES]
            L.check(self.lib.gi_moe_layer_from_hidden(
                p(self.x), L.DTYPE_BF16, p(r["router_scale"]), p(r["gate"]), 1e-6, p(self.logits),
                p(self.es[s % COPIES]), p(W["gate_up_packed"]), p(W["gate_up_scales"]),
                W["gate_up_scales"].shape[1], p(W["down_packed"]), p(W["down_scales"]),
                W["down_scales"].shape[1], p(self.out), p(self.idx), p(self.w), self.m, H, I, E,
                TOP_K, self.gs, p(self.ws), self.ws.numel(), 0, stream), "gi_moe_layer_from_hidden")


def bench_front_end(copies, steps, device, gs=None):
    """us per router front-end (fused launch vs the torch statements) at M=1
    and M=7, and the whole block from the hidden state at M=1."""
    res = {}
    n = min(steps, 200)
    for m in (1, 7, 512):
        row = {}
        for mode in ("fused", "torch"):
            runner = FrontEndRunner(m, copies, device, mode)
            for i in range(4):
                runner.launch(i)
            row[f"{mode}_us"] = time_graph(runner, list(range(n)), device)
        res[f"M{m}"] = row
    runner = FrontEndRunner(1, copies, device, "layer", gs)
    for i in range(4):
        runner.launch(i)
    res["layer_from_hidden_m1_us"] = time_graph(runner, list(range(n)), device)
    res["gate_bytes"] = E * H * 2
    return res


def prefill_flops(m, top_k=TOP_K, h=H, i=I):
    """Multiply-adds x 2 of the expert products over every (token, slot) pair."""
    return 2.0 * m * top_k * (h * 2 * i + i * h)


class ChunkedRunner:
    """The reference's chunked prefill (gemma.py:99-112): the layer on 8-row
    slices, one decode-path launch per slice, on the same logits."""

    def __init__(self, m, steps, copies, device):
        self.full = LayerRunner(m, steps, copies, device)
        self.lib = self.full.lib
        nbytes = self.lib.gi_fused_moe_workspace_bytes(8, TOP_K, H, I, E)
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        self.dev = device
        torch.cuda.synchronize()

    def launch(self, s):
        f = self.full
        W = f.copies[f.copy_of[s]]
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        for r0 in range(0, f.m, 8):
            st = self.lib.gi_moe_layer_from_logits(
                p(f.x[r0:r0 + 8]), L.DTYPE_BF16, p(f.logits[s][r0:r0 + 8]), L.DTYPE_FP32, None,
                p(W["gate_up_packed"]), p(W["gate_up_scales"]), W["gate_up_scales"].shape[1],
                p(W["down_packed"]), p(W["down_scales"]), W["down_scales"].shape[1],
                p(f.out[r0:r0 + 8]), p(f.idx[r0:r0 + 8]), p(f.w[r0:r0 + 8]), 8, H, I, E, TOP_K, GS,
                p(self.ws), self.ws.numel(), 0, stream)
            L.check(st, "gi_moe_layer_from_logits (8-row slice)")


def bench_prefill(steps, warmup, device):
    """the MoE layer at M=512 from i.i.d. N(0,1) router
    logits, on the grouped-GEMM prefill path, beside the same layer as 64
    decode-path launches of 8 rows (the reference's chunking)."""
    m = 512
    copies = [synth.device_moe_weights(E, H, I, GS, device, seed=100 + c) for c in range(COPIES)]
    torch.cuda.synchronize()
    desc = make_steps(m, 0.0, 3, warmup + steps)
    runner = LayerRunner(m, desc, copies, device)
    for i in range(warmup):
        runner.launch(i)
    torch.cuda.synchronize()
    order = [warmup + i for i in range(steps)]
    us = time_graph(runner, order, device)
    chunked = ChunkedRunner(m, desc, copies, device)
    ch_order = order[: max(4, steps // 10)]
    for i in range(2):
        chunked.launch(order[i])
    torch.cuda.synchronize()
    ch_us = time_graph(chunked, ch_order, device)
    mean_u = statistics.fmean(desc[i]["U"] for i in order)
    nbytes = mean_u * expert_bytes()
    gbps = nbytes / (us * 1e-6) / 1e9
    tflops = prefill_flops(m) / (us * 1e-6) / 1e12
    return {
        "metric": "chunked-prefill MoE layer us (M=512, configs[3]) + achieved HBM GB/s + MFMA utilisation (1 GPU)",
        "value": us, "unit": "us", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": us / 1000.0, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 activations, i.i.d. N(0,1) fp32 router logits, uniform int4 codes, "
                "|N(0,1)|*0.02 bf16 scales)",
        "config": {"workload": "MoE layer from logits at M=512: route + align + x reorder, grouped gate_up, "
                               "grouped down, combine (4 launches)", "M": m, "hidden": H, "experts": E, "top_k": TOP_K,
                   "moe_intermediate": I, "group_size": GS, "weight_copies_rotated": COPIES,
                   "timing": "HIP graph of K steps, HIP events"},
        "unique_experts_mean": mean_u,
        "algorithmic_bytes_per_layer": nbytes,
        "gbps": gbps,
        "tflops": tflops,
        "mfma_util": tflops * 1e12 / 2.5e15,
        "chunked_8row_us_per_layer": ch_us,
        "speedup_vs_chunked": ch_us / us,
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": gbps / PEAK_GBPS, "traffic": None},
    }


CALIB_BYTES = 256 << 20

# Dense W4A16 workloads (BASELINE configs 0 and 4): (M, K, N, group, softcap, copies)
LINEAR_WORKLOADS = {
    "linear": (1, 2816, 2816, 128, 0.0, 300),        # configs[0] shape, 4.09 MB per weight copy
    "lm_head": (6, 2816, 262144, 128, 30.0, 4),      # configs[4], 380.6 MB per copy
    "lm_head_m1": (1, 2816, 262144, 128, 30.0, 4),   # the same lm_head for one decoded token
}


def linear_bytes(k, n, gs):
    return (k // 8) * n * 4 + math.ceil(k / gs) * n * 2


class LinearRunner:
    """Direct C-ABI launches of gi_w4a16_linear over rotated weight copies."""

    def __init__(self, m, k, n, gs, softcap, copies, device):
        self.lib = L.load()
        self.m, self.k, self.n, self.gs, self.softcap = m, k, n, gs, softcap
        g = torch.Generator(device=device)
        g.manual_seed(0)
        self.B, self.S = [], []
        for _ in range(copies):
            self.B.append(torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), generator=g, device=device,
                                        dtype=torch.int64).to(torch.int32))
            self.S.append((torch.randn((math.ceil(k / gs), n), generator=g, device=device).abs() * 0.02)
                          .to(torch.bfloat16))
        self.A = synth.activations(m, k, seed=0).to(device)
        self.C = torch.empty(m, n, dtype=torch.bfloat16, device=device)
        nbytes = self.lib.gi_w4a16_workspace_bytes(m, k, n, gs)
        self.ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        self.dev = device
        torch.cuda.synchronize()

    def launch(self, i):
        c = i % len(self.B)
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        st = self.lib.gi_w4a16_linear(p(self.A), L.DTYPE_BF16, p(self.B[c]), p(self.S[c]), self.S[c].shape[0],
                                      p(self.C), self.m, self.k, self.n, self.gs, self.softcap,
                                      p(self.ws), self.ws.numel(), stream)
        L.check(st, "gi_w4a16_linear")


def cpu_baseline_linear(name, budget_s):
    """The reference's PyTorch CPU dequant+matmul (quant.py:67-75; + softcap for
    lm_head, gemma.py:351-357) on a bounded sample: the full configs[0]
    weight, or for lm_head a 16384-column slice of the vocabulary."""
    from oracle import cpu_baseline as CB

    m, k, n, gs, softcap, _ = LINEAR_WORKLOADS[name]
    n_s = n if n <= 16384 else 16384
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    B, S = synth.linear_weights(k, n_s, gs, seed=0)
    A = synth.activations(m, k, seed=0)
    run = (lambda: CB.lm_head_softcap(A, B, S, gs, softcap)) if softcap else \
        (lambda: CB.dequant_matmul(A, B, S, gs, n_s))
    run()
    times, t_start = [], time.perf_counter()
    while time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": linear_bytes(k, n_s, gs) / t / 1e9, "unit": "GB/s", "us_per_launch_sample": t * 1e6,
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} timed reps (median) of M={m}, K={k}, N={n_s} through "
                      f"oracle/cpu_baseline ({'lm_head_softcap' if softcap else 'dequant_matmul'}), "
                      f"restating quant.py:67-75; torch {torch.__version__}"}


def bench_linear(name, steps, warmup, device, cpu_budget_s=None):
    m, k, n, gs, softcap, copies = LINEAR_WORKLOADS[name]
    runner = LinearRunner(m, k, n, gs, softcap, copies, device)
    for i in range(warmup):
        runner.launch(i)
    torch.cuda.synchronize()
    order = [warmup + i for i in range(steps)]
    nbytes = linear_bytes(k, n, gs)
    # copy c % copies at step c: reuse after `copies` steps, or in the next replay
    natural = (min(len(order), copies) - 1) * nbytes
    flush = natural <= CACHE_BYTES
    us = time_graph(runner, order, device, flush=flush)
    hot_us = time_graph(runner, [order[0]] * min(steps, 200), device)
    gbps = nbytes / (us * 1e-6) / 1e9
    return {
        "metric": f"W4A16 linear us + achieved HBM GB/s ({name}: M={m}, K={k}, N={n}, gs={gs}"
                  + (f", softcap {softcap:g}" if softcap else "") + ", 1 GPU)",
        "value": gbps, "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": us / 1000.0, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (uniform int4 words, |N(0,1)|*0.02 bf16 scales, N(0,1) bf16 activations)",
        "config": {"workload": f"{name}: gi_w4a16_linear, one launch per step", "M": m, "K": k, "N": n,
                   "group_size": gs, "softcap": softcap, "weight_copies_rotated": copies,
                   "timing": "HIP graph of K steps, HIP events"},
        "us_per_launch": us, "hot_cache_us_per_launch": hot_us,
        "algorithmic_bytes_per_launch": nbytes,
        "min_reuse_distance_bytes": natural + (FLUSH_BYTES if flush else 0),
        "cache_flush_bytes": FLUSH_BYTES if flush else 0,
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": gbps / PEAK_GBPS, "traffic": None},
        "cpu_baseline": cpu_baseline_linear(name, cpu_budget_s) if cpu_budget_s else None,
    }


# Gemma-4-26B-A4B dense W4A16 linears of one decoder layer, (K, N), checkpoint
# group size 64 (attention.py:115-122, activations.py:26-28): a sliding-window
# layer has q, k, v, o and the shared MLP; a global layer's attention has
# q_global, k_global (= v) and o_global instead.
DENSE_PROJ = [
    ("q", 2816, 4096), ("k", 2816, 2048), ("v", 2816, 2048), ("o", 4096, 2816),
    ("mlp_gate", 2816, 2112), ("mlp_up", 2816, 2112), ("mlp_down", 2112, 2816),
    ("q_global", 2816, 8192), ("k_global", 2816, 1024), ("o_global", 8192, 2816),
]
DENSE_GS = 64
SLIDING = ("q", "k", "v", "o", "mlp_gate", "mlp_up", "mlp_down")


def bench_ingest(device):
    """gi_w4a16_ingest_batched of one MoE layer's experts (128 x gate, up, down
    at H=2816, I=704, gs 64) from checkpoint layout already in HBM: one launch
    per tensor kind (6 in all); bytes read + written per second between HIP
    events."""
    lib = L.load()
    g = torch.Generator(device=device)
    g.manual_seed(1)
    shapes = [(I, H, 0), (I, H, I), (H, I, 0)]  # (N, K, column offset): gate, up, down
    src = [(torch.randint(-(2 ** 31), 2 ** 31, (E, n, k // 8), generator=g, device=device, dtype=torch.int64)
            .to(torch.int32), torch.randn((E, n, k // DENSE_GS), generator=g, device=device).to(torch.bfloat16))
           for n, k, _ in shapes]
    gu = torch.empty((E, H // 8, 2 * I), dtype=torch.int32, device=device)
    gus = torch.empty((E, H // DENSE_GS, 2 * I), dtype=torch.bfloat16, device=device)
    dn = torch.empty((E, I // 8, H), dtype=torch.int32, device=device)
    dns = torch.empty((E, I // DENSE_GS, H), dtype=torch.bfloat16, device=device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    dst = [(gu, gus, 2 * I), (gu, gus, 2 * I), (dn, dns, H)]

    def one_layer():
        for (n, k, lo), (wp, ws), (dp, ds, ld) in zip(shapes, src, dst):
            L.check(lib.gi_w4a16_ingest_batched(
                ctypes.c_void_p(wp.data_ptr()), ctypes.c_void_p(ws.data_ptr()), L.DTYPE_BF16, E, n, k,
                k // DENSE_GS, n * (k // 8), n * (k // DENSE_GS), ctypes.c_void_p(dp.data_ptr() + 4 * lo),
                ctypes.c_void_p(ds.data_ptr() + 2 * lo), ld, dp.stride(0), ds.stride(0), stream),
                "gi_w4a16_ingest_batched")

    one_layer()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    one_layer()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0
    nbytes = 2 * E * sum(n * (k // 8) * 4 + n * (k // DENSE_GS) * 2 for n, k, _ in shapes)
    return {"us_per_moe_layer": us, "bytes_read_plus_written": nbytes, "gbps": nbytes / (us * 1e-6) / 1e9,
            "launches": 2 * len(shapes)}


class FusedDenseRunner:
    """A sliding-window layer's dense W4A16 work as this library's fused calls:
    q, k, v in one gi_w4a16_linear_multi, o, the shared MLP's gate/up with the
    gelu*up epilogue (gi_w4a16_gated_mlp) and down: 4 calls where the
    reference makes 7 linears plus a gelu and a product.  Weight copies are
    rotated past the MALL."""

    def __init__(self, m, device):
        self.lib = L.load()
        self.m, self.dev = m, device
        shp = {x[0]: (x[1], x[2]) for x in DENSE_PROJ}
        per_copy = sum(linear_bytes(*shp[x], DENSE_GS) for x in SLIDING)
        self.copies = max(2, math.ceil(600e6 / per_copy))
        g = torch.Generator(device=device)
        g.manual_seed(3)

        def mk(k, n):
            B = torch.randint(-(2 ** 31), 2 ** 31, (k // 8, n), generator=g, device=device,
                              dtype=torch.int64).to(torch.int32)
            S = (torch.randn((math.ceil(k / DENSE_GS), n), generator=g, device=device).abs() * 0.02).to(torch.bfloat16)
            return B, S
        self.W = [{x: mk(*shp[x]) for x in SLIDING} for _ in range(self.copies)]
        self.x = synth.activations(m, H, seed=1).to(device)
        self.q = torch.empty(m, 4096, dtype=torch.bfloat16, device=device)
        self.k = torch.empty(m, 2048, dtype=torch.bfloat16, device=device)
        self.v = torch.empty(m, 2048, dtype=torch.bfloat16, device=device)
        self.attn = synth.activations(m, 4096, seed=2).to(device)
        self.o = torch.empty(m, H, dtype=torch.bfloat16, device=device)
        self.act = torch.empty(m, 2112, dtype=torch.bfloat16, device=device)
        self.y = torch.empty(m, H, dtype=torch.bfloat16, device=device)
        nb = max([self.lib.gi_w4a16_workspace_bytes(m, shp[x][0], shp[x][1], DENSE_GS) for x in SLIDING] +
                 [self.lib.gi_w4a16_gated_mlp_workspace_bytes(m, H, 2112, DENSE_GS),
                  self.lib.gi_w4a16_linear_multi_workspace_bytes(3, (ctypes.c_int * 3)(4096, 2048, 2048), m, H,
                                                                 DENSE_GS)])
        self.ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=device)
        torch.cuda.synchronize()

    def launch(self, i):
        W = self.W[i % self.copies]
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        ws, wsn = p(self.ws), self.ws.numel()
        vp3 = lambda ts: (ctypes.c_void_p * 3)(*[t.data_ptr() for t in ts])  # noqa: E731
        L.check(self.lib.gi_w4a16_linear_multi(
            p(self.x), L.DTYPE_BF16, 3, vp3([W["q"][0], W["k"][0], W["v"][0]]),
            vp3([W["q"][1], W["k"][1], W["v"][1]]), (ctypes.c_int * 3)(*[W[x][1].shape[0] for x in "qkv"]),
            vp3([self.q, self.k, self.v]), (ctypes.c_int * 3)(4096, 2048, 2048), self.m, H, DENSE_GS, ws, wsn,
            stream), "qkv")
        L.check(self.lib.gi_w4a16_linear(p(self.attn), L.DTYPE_BF16, p(W["o"][0]), p(W["o"][1]), W["o"][1].shape[0],
                                         p(self.o), self.m, 4096, H, DENSE_GS, 0.0, ws, wsn, stream), "o")
        L.check(self.lib.gi_w4a16_gated_mlp(
            p(self.o), L.DTYPE_BF16, p(W["mlp_gate"][0]), p(W["mlp_gate"][1]), W["mlp_gate"][1].shape[0],
            p(W["mlp_up"][0]), p(W["mlp_up"][1]), W["mlp_up"][1].shape[0], p(self.act), self.m, H, 2112, DENSE_GS,
            ws, wsn, stream), "gated mlp")
        L.check(self.lib.gi_w4a16_linear(p(self.act), L.DTYPE_BF16, p(W["mlp_down"][0]), p(W["mlp_down"][1]),
                                         W["mlp_down"][1].shape[0], p(self.y), self.m, 2112, H, DENSE_GS, 0.0,
                                         ws, wsn, stream), "down")


def bench_dense(steps, warmup, device):
    res = {}
    for m in (1, 7):
        row = {}
        for name, k, n in DENSE_PROJ:
            nbytes = linear_bytes(k, n, DENSE_GS)
            copies = max(2, math.ceil(600e6 / nbytes))  # > the 256 MB MALL between reuses
            runner = LinearRunner(m, k, n, DENSE_GS, 0.0, copies, device)
            for i in range(min(warmup, 5)):
                runner.launch(i)
            us = time_graph(runner, list(range(min(steps, 200))), device)
            row[name] = {"K": k, "N": n, "us": us, "bytes": nbytes, "gbps": nbytes / (us * 1e-6) / 1e9}
            del runner
            torch.cuda.empty_cache()
        tot_us = sum(row[x]["us"] for x in SLIDING)
        tot_b = sum(row[x]["bytes"] for x in SLIDING)
        fr = FusedDenseRunner(m, device)
        for i in range(min(warmup, 5)):
            fr.launch(i)
        fused_us = time_graph(fr, list(range(min(steps, 200))), device)
        del fr
        torch.cuda.empty_cache()
        res[f"M{m}"] = {"sliding_layer_us": tot_us, "sliding_layer_gbps": tot_b / (tot_us * 1e-6) / 1e9,
                        "sliding_layer_bytes": tot_b, "per_projection": row,
                        "sliding_layer_fused_us": fused_us,
                        "sliding_layer_fused_gbps": tot_b / (fused_us * 1e-6) / 1e9}
        print(f"[bench] dense M={m}: fused calls (qkv, o, gated mlp, down) {fused_us:.1f} us", file=sys.stderr,
              flush=True)
        print(f"[bench] dense M={m}: sliding layer {tot_us:.1f} us, "
              f"{res[f'M{m}']['sliding_layer_gbps']:.0f} GB/s", file=sys.stderr, flush=True)
    ing = bench_ingest(device)
    m1 = res["M1"]
    return {
        "metric": "dense W4A16 projections of one Gemma-4-26B-A4B sliding-window layer (q, k, v, o, "
                  "shared MLP), us + achieved HBM GB/s at M=1 and M=7 (gs 64, 1 GPU)",
        "value": m1["sliding_layer_gbps"], "unit": "GB/s", "n_gpus": 1, "steps": min(steps, 200),
        "warmup": min(warmup, 5), "ms_per_step": m1["sliding_layer_us"] / 1000.0, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (uniform int4 words, N(0,1)*0.02 bf16 scales, N(0,1) bf16 activations)",
        "config": {"workload": "dense: gi_w4a16_linear per projection, one launch each, weight copies "
                               "rotated past the MALL", "group_size": DENSE_GS,
                   "timing": "HIP graph per projection, HIP events"},
        "roofline": {"bound": "hbm", "achieved": m1["sliding_layer_gbps"], "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": m1["sliding_layer_gbps"] / PEAK_GBPS, "traffic": None},
        "cpu_baseline": None,
        "M1": m1, "M7": res["M7"], "ingest": ing,
    }


def pmc_pass(copies, steps, warmup, device, m=1):
    """Eager launches for one rocprofv3 --pmc pass (FETCH_SIZE or WRITE_SIZE).

    First three float32 negations of a 256 MiB buffer (a plain streaming
    kernel that reads and writes exactly CALIB_BYTES each: the calibration
    for the counter), then W warmup + K rotated M-row layers (M=1, or M=7
    with the verify noise of configs[2]) launched one by
    one.  The profiler serialises dispatches; the rotation keeps >= 1 GB of
    other weights between reuses, as in the timed run.  Per-dispatch HBM
    bytes of the layer kernel = mean counter over the K layers after warmup,
    scaled by CALIB_BYTES / (mean counter of the calibration kernel).
    """
    src = torch.randn(CALIB_BYTES // 4, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    desc = make_steps(m, 0.0 if m == 1 else 0.5, 1 if m == 1 else 2, warmup + steps)
    runner = LayerRunner(m, desc, copies, device)
    for i in range(warmup + steps):
        runner.launch(i)
    torch.cuda.synchronize()
    if runner.status() != 0:
        raise RuntimeError("device status word set during the pmc pass")
    mean_u = statistics.fmean(desc[i]["U"] for i in range(warmup, warmup + steps))
    print(json.dumps({"pmc_pass": {"calibration_kernel": "neg float32", "calibration_bytes_read": CALIB_BYTES,
                                   "calibration_bytes_written": CALIB_BYTES, "calibration_dispatches": 3,
                                   "layer_dispatches": warmup + steps, "warmup": warmup, "M": m,
                                   "algorithmic_bytes_per_layer": mean_u * expert_bytes()}}))


def pmc_reduce(fetch_csv, write_csv, out_path, algorithmic_bytes=None):
    """Per-dispatch HBM bytes of the M=1 layer kernel from the counter CSVs of
    two --pmc-pass runs (FETCH_SIZE, then WRITE_SIZE; values in KiB per
    dispatch).  Each counter is scaled by CALIB_BYTES / its reading on the
    calibration kernel, which reads and writes exactly CALIB_BYTES."""
    import csv
    import collections

    def per_dispatch(path):
        vals, names = collections.defaultdict(float), {}
        with open(path) as f:
            for r in csv.DictReader(f):
                d = int(r["Dispatch_Id"])
                vals[d] += float(r["Counter_Value"])
                names[d] = r["Kernel_Name"]
        ids = sorted(vals)
        cal = [vals[d] for d in ids if "neg" in names[d].lower()][-3:]
        lay = [vals[d] for d in ids if any(k in names[d] for k in ("moe_decode1_kernel", "moe_decode_kernel", "fused_moe"))]
        if len(cal) != 3 or not lay:
            raise SystemExit(f"{path}: expected 3 calibration and >= 1 layer dispatches")
        return cal, lay

    res = {}
    for key, path in (("fetch", fetch_csv), ("write", write_csv)):
        cal, lay = per_dispatch(path)
        lay = lay[10:] if len(lay) > 10 else lay  # the pass's 10 warmup layers
        factor = (CALIB_BYTES / 1024.0) / statistics.fmean(cal)
        res[key] = {"counter_kib_mean": statistics.fmean(lay), "calibration_kib": cal,
                    "calibration_factor": factor, "bytes_per_dispatch": statistics.fmean(lay) * 1024.0 * factor,
                    "dispatches": len(lay)}
    res["hbm_bytes_per_launch"] = res["fetch"]["bytes_per_dispatch"] + res["write"]["bytes_per_dispatch"]
    res["algorithmic_bytes_per_launch"] = algorithmic_bytes if algorithmic_bytes else 8 * expert_bytes()
    Path(out_path).write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res))


def cpu_baseline(budget_s, max_reps, m=1, noise=0.0, seed=1, warmup=True, W=None):
    """The reference's PyTorch CPU path on the same workload (an M-row layer;
    the headline line uses M=1), bounded to about budget_s seconds of CPU work."""
    from oracle import cpu_baseline as CB

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    if W is None:
        W = synth.moe_weights(E, H, I, GS, seed=1)
    x = synth.activations(m, H, seed=seed)
    logits = synth.router_logits(m, E, seed=seed, verify_noise=noise)
    top, idx = torch.topk(logits, TOP_K, dim=-1)           # gemma.py:77-80
    w = torch.softmax(top, dim=-1, dtype=torch.float32).to(torch.bfloat16)
    args = (x, idx, w, W["gate_up_packed"], W["gate_up_scales"], W["down_packed"], W["down_scales"], GS)
    if warmup:
        CB.moe_forward(*args)
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        CB.moe_forward(*args)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    u = len(set(idx.reshape(-1).tolist()))
    nbytes = u * expert_bytes()
    try:
        model = [l for l in open("/proc/cpuinfo") if l.startswith("model name")][0].split(":")[1].strip()
    except Exception:
        model = platform.processor()
    return {
        "value": nbytes / t / 1e9,
        "unit": "GB/s",
        "us_per_layer": t * 1e6,
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} timed reps (median) of one M={m} layer (U={u}) through "
                   f"oracle/cpu_baseline.moe_forward, restating quant.py:67-75 + gemma.py:115-147; "
                   f"host {model}, torch {torch.__version__}"),
    }


def cpu_table(budget_s):
    """The reference's CPU path (oracle/cpu_baseline) on every BASELINE config,
    each bounded to about budget_s seconds: the MoE layer at M=1, 7 and 512
    (configs[1]-[3], the same routing draws as the GPU lines) and the W4A16
    linear at configs[0] and configs[4] (lm_head on a column sample)."""
    W = synth.moe_weights(E, H, I, GS, seed=1)
    rows = {}
    for key, m, noise, seed, warm in (("cfg1_M1", 1, 0.0, 1, True), ("cfg2_M7", 7, 0.5, 2, True),
                                      ("cfg3_M512", 512, 0.0, 3, False)):
        rows[key] = cpu_baseline(budget_s, 100000, m=m, noise=noise, seed=seed, warmup=warm, W=W)
        print(f"[cpu] {key} {rows[key]['us_per_layer']:.0f} us ({rows[key]['cores']} cores)",
              file=sys.stderr, flush=True)
    del W
    for key, name in (("cfg0_linear", "linear"), ("cfg4_lm_head", "lm_head")):
        rows[key] = cpu_baseline_linear(name, budget_s)
        print(f"[cpu] {key} {rows[key]['us_per_launch_sample']:.0f} us per sample launch",
              file=sys.stderr, flush=True)
    return {"cpu_table": rows}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--group-size", type=int, choices=[64, 128], default=128,
                    help="scale group size of the MoE weights of the headline line (configs[1]/[2] use 128; "
                         "the engine's checkpoints use 64, reported beside it in the default run)")
    ap.add_argument("--workload", choices=["moe", "prefill", "dense", "router", "stream", "timeline",
                                           "cpu_table", "fp16", "fp32", *LINEAR_WORKLOADS],
                    default="moe",
                    help="moe (default: the BASELINE metric, M=1 value with M=7 beside it), prefill "
                         "(configs[3], M=512) or a dense W4A16 shape (linear = configs[0], "
                         "lm_head = configs[4])")
    ap.add_argument("--pmc-reduce", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "OUT_JSON"),
                    help="reduce two --pmc-pass counter CSVs to per-launch HBM bytes (no GPU needed)")
    ap.add_argument("--pmc-m", type=int, choices=[1, 7], default=1,
                    help="rows of the --pmc-pass layers (7: configs[2])")
    ap.add_argument("--pmc-alg-bytes", type=float, default=None,
                    help="--pmc-reduce: algorithmic bytes per launch (the pass prints them; default 8 experts)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="eager calibration copy + rotated M=1 layers for a rocprofv3 --pmc run; no timing")
    args = ap.parse_args()
    if args.pmc_reduce:
        pmc_reduce(*args.pmc_reduce, algorithmic_bytes=args.pmc_alg_bytes)
        return
    if args.workload == "cpu_table":
        print(json.dumps(cpu_table(args.cpu_budget_s)))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's path runs on a single MI355X "
              f"(--gpus {args.gpus} is not supported: one process drives one GPU)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.workload == "prefill":
        print(json.dumps(bench_prefill(min(args.steps, 50), min(args.warmup, 5), device)))
        return
    if args.workload == "dense":
        print(json.dumps(bench_dense(args.steps, args.warmup, device)))
        return
    if args.workload in ("fp16", "fp32"):
        dt = torch.float16 if args.workload == "fp16" else torch.float32
        print(json.dumps({"workload": f"MoE layer with {args.workload} activations and scales",
                          "rows": bench_dtype(dt, min(args.steps, 100), args.warmup, device)}))
        return
    if args.workload not in ("moe", "router", "stream", "timeline"):
        print(json.dumps(bench_linear(args.workload, args.steps, args.warmup, device,
                                      None if args.no_cpu_baseline else args.cpu_budget_s)))
        return
    gs = args.group_size
    if args.workload == "timeline":
        from gemmainfer_amd import build as gbuild  # noqa: PLC0415
        L.LIB_PATH = gbuild.lib_path(timeline=True)  # before the first load
    copies = [synth.device_moe_weights(E, H, I, gs, device, seed=100 + c) for c in range(COPIES)]
    torch.cuda.synchronize()
    print(f"[bench] weights ready: {COPIES} x {E} experts, group size {gs}", file=sys.stderr, flush=True)
    if args.workload == "stream":
        rows = {}
        for m, noise, seed in ((1, 0.0, 1), (7, 0.5, 2)):
            rows[f"M{m}"] = bench_stream(m, noise, seed, copies, args.steps, args.warmup, device, gs)
            print(f"[bench] stream M={m} {rows[f'M{m}']['us_per_read']:.2f} us {rows[f'M{m}']['gbps']:.0f} GB/s",
                  file=sys.stderr, flush=True)
        r1 = rows["M1"]
        print(json.dumps({
            "metric": "pure-read ceiling: us and GB/s to read the bytes of one MoE layer launch at M=1 and M=7 "
                      "(1 GPU)",
            "value": r1["gbps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": r1["us_per_read"] / 1000.0, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u8", "data": "synthetic (the MoE benchmark's weight copies)",
            "config": {"workload": "gi_probe_stream_read over each step's unique-expert weight bytes, "
                                   "4 copies rotated", "group_size": gs,
                       "timing": "HIP graph of K steps, HIP events"},
            "roofline": {"bound": "hbm", "achieved": r1["gbps"], "peak": PEAK_GBPS, "unit": "GB/s",
                         "frac": r1["gbps"] / PEAK_GBPS, "traffic": None},
            "cpu_baseline": None, "stream": rows}))
        return
    if args.pmc_pass:
        pmc_pass(copies, args.steps, args.warmup, device, args.pmc_m)
        return
    if args.workload == "timeline":
        tl = bench_timeline(copies, min(args.steps, 100), args.warmup, device, gs)
        print(json.dumps({"timeline": tl, "group_size": gs,
                          "library": str(L.LIB_PATH.name),
                          "note": "phase stamps of the decode kernel (s_memrealtime, 100 MHz), from the "
                                  "earliest workgroup start of each launch; measurement build, not the "
                                  "product library"}))
        return
    if args.workload == "router":
        fe = bench_front_end(copies, args.steps, device, gs)
        print(json.dumps({
            "metric": "MoE router front-end us (gemma.py:75-76: router norm, router_scale, gate linear) "
                      "at M=1 and M=7, one launch vs the module's torch statements (1 GPU)",
            "value": fe["M1"]["fused_us"], "unit": "us", "n_gpus": 1, "steps": min(args.steps, 200),
            "warmup": 4, "ms_per_step": fe["M1"]["fused_us"] / 1000.0, "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (N(0,1) bf16 hidden states, router weights of gemmainfer_amd.synth)",
            "config": {"workload": "router: gi_moe_router_logits, one launch per step, 4 gate copies rotated",
                       "hidden": H, "experts": E, "timing": "HIP graph of K steps, HIP events"},
            "roofline": {"bound": "hbm", "achieved": fe["gate_bytes"] / (fe["M1"]["fused_us"] * 1e-6) / 1e9,
                         "peak": PEAK_GBPS, "unit": "GB/s",
                         "frac": fe["gate_bytes"] / (fe["M1"]["fused_us"] * 1e-6) / 1e9 / PEAK_GBPS,
                         "traffic": None},
            "cpu_baseline": None, "router_front_end": fe}))
        return
    m1 = bench_config(1, 0.0, 1, copies, args.steps, args.warmup, device, gs)
    print(f"[bench] M=1 {m1['us_per_layer']:.2f} us {m1['gbps']:.0f} GB/s", file=sys.stderr, flush=True)
    m7 = bench_config(7, 0.5, 2, copies, args.steps, args.warmup, device, gs)
    print(f"[bench] M=7 {m7['us_per_layer']:.2f} us {m7['gbps']:.0f} GB/s", file=sys.stderr, flush=True)
    fe = bench_front_end(copies, args.steps, device, gs)
    print(f"[bench] router front-end M=1 fused {fe['M1']['fused_us']:.2f} us, torch {fe['M1']['torch_us']:.2f} us; "
          f"block from hidden M=1 {fe['layer_from_hidden_m1_us']:.2f} us", file=sys.stderr, flush=True)
    # the pure-read ceiling of the same byte sets (same steps, same copies)
    ceiling = {}
    for key, (m, noise, seed, row) in {"M1": (1, 0.0, 1, m1), "M7": (7, 0.5, 2, m7)}.items():
        c = bench_stream(m, noise, seed, copies, args.steps, args.warmup, device, gs)
        row["attainable_gbps"] = c["gbps"]
        row["frac_of_attainable"] = row["gbps"] / c["gbps"]
        ceiling[key] = c
        print(f"[bench] stream ceiling M={m} {c['us_per_read']:.2f} us {c['gbps']:.0f} GB/s "
              f"(layer at {row['frac_of_attainable']:.2f} of it)", file=sys.stderr, flush=True)
    # the engine's group size (every real checkpoint is 64) beside the headline
    other = {}
    if gs == 128:
        del copies
        torch.cuda.empty_cache()
        copies = [synth.device_moe_weights(E, H, I, 64, device, seed=100 + c) for c in range(COPIES)]
        torch.cuda.synchronize()
        for key, (m, noise, seed) in {"m1": (1, 0.0, 1), "m7": (7, 0.5, 2)}.items():
            other[key] = bench_config(m, noise, seed, copies, args.steps, args.warmup, device, 64)
            print(f"[bench] group size 64 M={m} {other[key]['us_per_layer']:.2f} us "
                  f"{other[key]['gbps']:.0f} GB/s", file=sys.stderr, flush=True)
    # the other BASELINE configs on the same clock: configs[0] (W4A16 linear,
    # M=1), configs[3] (prefill, M=512) and configs[4] (lm_head, M=6)
    del copies
    torch.cuda.empty_cache()
    pf = bench_prefill(min(args.steps, 50), min(args.warmup, 5), device)
    print(f"[bench] prefill M=512 {pf['value']:.1f} us {pf['gbps']:.0f} GB/s "
          f"(8-row chunks {pf['chunked_8row_us_per_layer']:.0f} us)", file=sys.stderr, flush=True)
    torch.cuda.empty_cache()
    # configs[0] moves 4.09 MB per step: 200 steps over its 300 rotated copies
    # put 813 MB between two reads of a copy, more than every cache, with no
    # flush read (which would also cool the address translation of every one
    # of a short replay's ~4 us launches)
    lin = bench_linear("linear", max(args.steps, 200), args.warmup, device)
    print(f"[bench] linear M=1 {lin['us_per_launch']:.2f} us {lin['value']:.0f} GB/s", file=sys.stderr, flush=True)
    lmh = bench_linear("lm_head", args.steps, args.warmup, device)
    print(f"[bench] lm_head M=6 {lmh['us_per_launch']:.2f} us {lmh['value']:.0f} GB/s", file=sys.stderr, flush=True)
    torch.cuda.empty_cache()
    fp16 = bench_dtype(torch.float16, min(args.steps, 100), args.warmup, device)
    print(f"[bench] fp16 M=1 {fp16['M1']['us_per_layer']:.2f} us, M=7 {fp16['M7']['us_per_layer']:.2f} us",
          file=sys.stderr, flush=True)
    torch.cuda.empty_cache()

    def cfg_row(us, nbytes, **extra):
        gbps = nbytes / (us * 1e-6) / 1e9
        return {"us": us, "gbps": gbps, "frac": gbps / PEAK_GBPS, "algorithmic_bytes": nbytes, **extra}

    configs = {
        "cfg0_linear_M1": cfg_row(lin["us_per_launch"], lin["algorithmic_bytes_per_launch"]),
        "cfg1_moe_M1": cfg_row(m1["us_per_layer"], m1["algorithmic_bytes_per_layer"],
                               unique_experts_mean=m1["unique_experts_mean"]),
        "cfg2_moe_M7": cfg_row(m7["us_per_layer"], m7["algorithmic_bytes_per_layer"],
                               unique_experts_mean=m7["unique_experts_mean"]),
        "cfg3_prefill_M512": cfg_row(pf["value"], pf["algorithmic_bytes_per_layer"], mfma_util=pf["mfma_util"],
                                     chunked_8row_us=pf["chunked_8row_us_per_layer"]),
        "cfg4_lm_head_M6": cfg_row(lmh["us_per_launch"], lmh["algorithmic_bytes_per_launch"]),
    }
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_budget_s, 100000)
        print(f"[bench] cpu {cpu['us_per_layer']:.0f} us", file=sys.stderr, flush=True)
    traffic = None
    tfile = ROOT / "profiles" / "traffic_moe_layer_m1.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    res = {
        "metric": METRIC,
        "value": m1["gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": m1["us_per_layer"] / 1000.0,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) bf16 activations and fp32 router logits, uniform int4 codes, |N(0,1)|*0.02 bf16 scales)",
        "config": {
            "workload": "fused W4A16 MoE layer, decode M=1 (configs[1]): route+align+gate_up+gelu+down+combine, one launch",
            "M": 1, "hidden": H, "experts": E, "top_k": TOP_K, "moe_intermediate": I,
            "group_size": gs, "weight_copies_rotated": COPIES, "timing": "HIP graph of K steps, HIP events",
        },
        "us_per_layer": m1["us_per_layer"],
        "roofline": {
            "bound": "hbm",
            "achieved": m1["gbps"],
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": m1["gbps"] / PEAK_GBPS,
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "m1": m1,
        "m7": m7,
        "stream_ceiling": ceiling,
        "group_size_64": other or None,
        "router_front_end": fe,
        "configs": configs,
        "fp16_activations": fp16,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
