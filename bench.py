#!/usr/bin/env python3
"""RefineKV decode-attention benchmark on one MI355X.

Workload (the headline): a Llama-3.1-8B-shaped
attention stack -- 32 layers, 32 query / 8 KV heads, head_dim 128, bf16 --
at 131072 prompt tokens, block_size 32, eps 0.01, GQA "any", decoding 128
tokens; like the reference's protocol (speed/README.md:84-91) the timed
window is the last 125 of the 127 decode intervals, replayed as HIP graphs
(one graph = one decode step over all layers).  Each layer has its own KV
cache and summaries (17 GB in all), so the 256 MB Infinity Cache cannot hold
a step's data.  K/V are synthetic (refinekv.testing recipe drawn on the GPU:
N(0,1) keys/values, per-block key offsets, 2% of blocks with query-aligned
spikes); weights play no part in this op.

One JSON line on stdout: value = microseconds per decode step per layer.
"""

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "refinekv-release_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

METRIC = "decode attn µs/step/layer @128K ctx GQA32/8 d128; HBM GB/s vs peak"
PEAK_HBM_GBPS = 8000.0
# Kernels one rkv_decode call launches, in order, per decode path.
KERNELS = {"step": ("step",), "split": ("score", "attend", "merge")}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# BASELINE.json configs[1..3] as model stacks (random-init weights of the
# named architectures; uniform random prompt ids).
MODEL_CONFIGS = {
    "llama32k": dict(family="llama", prompt=32768, block=32, eps=0.01, reduction="any",
                     anchors=32, config_index=1),
    "llama128k": dict(family="llama", prompt=131072, block=32, eps=0.01, reduction="any",
                      anchors=0, config_index=2),
    "qwen64k": dict(family="qwen2", prompt=65536, block=64, eps=0.005, reduction="max",
                    anchors=64, config_index=3),
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=125)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--context", type=int, default=131072)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--group", type=int, default=4)
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--block", type=int, default=32)
    ap.add_argument("--eps", type=float, default=0.01)
    ap.add_argument("--reduction", default="any")
    ap.add_argument("--spikes", type=float, default=0.02)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-dense", action="store_true", help="skip the eps=0 dense baseline")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline (the reference's torch CPU backend)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy a 64 MiB buffer 5 times (scales rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE readings to bytes)")
    ap.add_argument("--summary-only", action="store_true",
                    help="only build the prefill summary of one layer (--heads, --context, "
                         "--dim, --block; N(0,1) bf16 K/V) three times (for profiler runs)")
    ap.add_argument("--path", choices=("step", "split"), default="step",
                    help="rkv_decode path: one launch per step (default) or three kernels")
    ap.add_argument("--graph-only", action="store_true",
                    help="only the graph-replay timing (for profiler runs)")
    ap.add_argument("--sweep", action="store_true",
                    help="the isolated-op sweep (BASELINE.json configs[4]): one JSON line per "
                         "(context, block, eps, spike fraction) point")
    ap.add_argument("--sweep-contexts", default="8192,32768,131072,524288",
                    help="--sweep: prompt lengths, comma-separated")
    ap.add_argument("--sweep-blocks", default="16,32,64",
                    help="--sweep: block sizes, comma-separated")
    ap.add_argument("--model", choices=sorted(MODEL_CONFIGS),
                    help="run a BASELINE.json model config as a random-init model stack "
                         "through RefineKV(cuda_graph=True) and report per-layer attention "
                         "time and expanded fractions")
    ap.add_argument("--new-tokens", type=int, default=128, help="--model: tokens to generate")
    ap.add_argument("--flip-query", action="store_true",
                    help="negate every layer's query at each decode step (inside the graph), so "
                         "consecutive steps expand different blocks")
    ap.add_argument("--speculation", choices=("auto", "off"), default="auto",
                    help="the one-launch step's speculation: a tile whose every block the "
                         "previous launch expanded issues its page rows before the decision "
                         "(off: always after it)")
    ap.add_argument("--phases", action="store_true",
                    help="phase timeline of the one-launch step (per-workgroup clock stamps from "
                         "librefinekv_hip_phases.so), then exit")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# HIP events through the runtime's C API (timing on the kernels' own stream)
# ---------------------------------------------------------------------------

class HipEvents:
    def __init__(self, n):
        self.rt = ctypes.CDLL("libamdhip64.so")
        self.rt.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.events = (ctypes.c_void_p * n)()
        for i in range(n):
            ev = ctypes.c_void_p()
            assert self.rt.hipEventCreate(ctypes.byref(ev)) == 0
            self.events[i] = ev

    def ptr(self, offset=0):
        return ctypes.cast(ctypes.byref(self.events, offset * ctypes.sizeof(ctypes.c_void_p)),
                           ctypes.c_void_p)

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        assert self.rt.hipEventElapsedTime(ctypes.byref(ms), self.events[a], self.events[b]) == 0
        return ms.value

    def close(self):
        for ev in self.events:
            self.rt.hipEventDestroy(ev)


# ---------------------------------------------------------------------------
# Workload
# ---------------------------------------------------------------------------

def make_layer(gen, a, capacity, device):
    """refinekv.testing.decode_inputs' recipe, drawn with a device generator."""
    H, G, D, P, B = a.heads, a.group, a.dim, a.context, a.block
    q = torch.randn(H, G, 1, D, generator=gen, device=device)
    keys = torch.randn(H, P + capacity, D, generator=gen, device=device)
    values = torch.randn(H, P + capacity, D, generator=gen, device=device)
    n = math.ceil(P / B)
    offset = torch.randn(H, n, D, generator=gen, device=device) * 0.5
    n_spikes = round(a.spikes * H * n)
    picks = torch.randperm(H * n, generator=gen, device=device)[:n_spikes]
    spike = torch.zeros(H * n, D, device=device)
    spike[picks] = 4.0 * q[:, :, 0].mean(1)[picks // n]
    offset += spike.view(H, n, D)
    keys[:, :P] += offset.repeat_interleave(B, dim=1)[:, :P]
    return (q.to(torch.bfloat16), keys.to(torch.bfloat16), values.to(torch.bfloat16))


def algorithmic_bytes(a, masks, counts, suffix):
    """Bytes each kernel of the decode step must move per layer-step, counted
    once in the reference's storage formats: score reads the key means and
    ellipsoids of every block; attend reads the value means of unexpanded
    blocks (the representatives), the value norms, the K/V tokens of expanded
    blocks and of the suffix, and writes the mask; merge writes the output.
    "step" (the one-launch kernel) and "decode" are their sum.  Intermediates (z, delta, partials) are not
    algorithmic bytes."""
    H, G, D = a.heads, a.group, a.dim
    n = counts.numel()
    sel = masks.float().mean(0)  # (H, N) fraction over layers
    expanded_tokens = (sel * counts.float()[None]).sum().item()
    unexpanded = ((1 - sel).sum()).item()
    q_bytes = H * G * D * 2
    score = 2 * H * n * D * 2 + q_bytes
    attend = (unexpanded * D * 2 + H * n * 4 + H * n + expanded_tokens * D * 2 * 2
              + H * suffix * D * 2 * 2 + q_bytes)
    merge = H * G * D * 2
    phases = dict(score=score, attend=attend, merge=merge)
    total = sum(phases.values())
    return dict(phases, step=total, decode=total)


def dense_bytes(a, suffix):
    """Algorithmic bytes of one dense decode: every visible key and value
    row, the query and the output."""
    H, G, D = a.heads, a.group, a.dim
    return H * (a.context + suffix) * D * 2 * 2 + 2 * H * G * D * 2


def main():
    a = parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported in this build "
              "(the path would shard by KV head: each GPU would run the op on its heads "
              "with no exchange inside it)", file=sys.stderr)
        sys.exit(2)
    if a.copy_calibration:
        copy_calibration()
        return
    if a.summary_only:
        summary_only(a)
        return
    if a.phases:
        phase_timeline(a)
        return
    if a.sweep:
        sweep(a)
        return
    if a.model:
        model_bench(a)
        return
    from refinekv import RefineKVConfig, build_summary, sparse_attention, _hip

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _hip.lib()
    _hip.set_decode_path(a.path)
    _hip.set_speculation(a.speculation)
    kernels = KERNELS[a.path]
    capacity = a.warmup + a.steps + 1
    cfg = RefineKVConfig(backend="hip", block_size=a.block, eps=a.eps,
                         gqa_reduction=a.reduction)
    dense_cfg = RefineKVConfig(backend="hip", block_size=a.block, eps=0.0,
                               gqa_reduction=a.reduction)

    # ---- layers, caches and prefill summaries ---------------------------
    gen = torch.Generator(device=dev).manual_seed(a.seed)
    layers = []
    t_sum = 0.0
    for i in range(a.layers):
        q, k, v = make_layer(gen, a, capacity, dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        summary = build_summary(k[:, :a.context], v[:, :a.context], cfg)
        torch.cuda.synchronize()
        t_sum += time.perf_counter() - t0
        layers.append(dict(q=q, k=k, v=v, summary=summary, ws={}, dws={}))
    log(f"[bench] {a.layers} layers ready, summary build {t_sum / a.layers * 1e6:.1f} us/layer "
        "(wall, first calls: includes setup)")
    summary_us = summary_event_us(layers[0]["k"][:, :a.context], layers[0]["v"][:, :a.context],
                                  cfg)
    log(f"[bench] summary kernel: {summary_us:.1f} us/layer (HIP events, 5 back-to-back calls "
        "after a warm one)")
    suffix_len = torch.zeros((), dtype=torch.int32, device=dev)

    def step(config, key):
        suffix_len.add_(1)
        for L in layers:
            if a.flip_query:
                L["q"].neg_()
            sparse_attention(L["q"], L["summary"], L["k"][:, a.context:], L["v"][:, a.context:],
                             config, workspace=L[key], suffix_length=suffix_len)

    def timed_graph(config, key, warmup, steps):
        suffix_len.fill_(0)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(warmup):
                step(config, key)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(config, key)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end), graph

    # ---- headline: graph replays over the timed window ------------------
    torch.cuda.synchronize()
    ms, graph = timed_graph(cfg, "ws", a.warmup, a.steps)
    us_layer = ms * 1e3 / (a.steps * a.layers)
    log(f"[bench] refinekv graph: {ms / a.steps:.3f} ms/step, {us_layer:.2f} us/layer-step")
    del graph
    if a.graph_only:
        print(json.dumps(dict(metric=METRIC, value=round(us_layer, 3), unit="us/step/layer")))
        return

    # Masks of the last step (suffix = warmup + steps) for f and bytes.
    masks = []
    for L in layers:
        res = sparse_attention(L["q"], L["summary"], L["k"][:, a.context:], L["v"][:, a.context:],
                               cfg, workspace=L["ws"], return_selected=True,
                               suffix_length=suffix_len)
        masks.append(res.selected.clone())
    masks = torch.stack(masks)
    frac = masks.float().mean().item()
    counts = layers[0]["summary"].counts
    suffix_now = int(suffix_len.item())
    nbytes = algorithmic_bytes(a, masks, counts, suffix_now)
    total_bytes = nbytes["decode"]

    # ---- per-kernel durations with HIP events on the kernels' own stream --
    # The one-launch step runs one kernel per layer-step, so the timed
    # region's own events (on the stream the graphs replay on) give its
    # average duration directly.  The three-kernel path has the library
    # record events around each kernel of eager calls, which also bracket
    # part of the host's launch latency.
    if kernels == ("step",):
        kernel_us = {"step": us_layer}
        timing = (f"graph replays bracketed by HIP events on the kernels' stream, "
                  f"{a.steps} x {a.layers} launches")
    else:
        n_ev = len(kernels) + 1
        ev = HipEvents(n_ev * a.layers)
        kernel_ms = {k: 0.0 for k in kernels}
        reps = 3
        for _ in range(reps):
            for i, L in enumerate(layers):
                lib.rkv_set_profile_events(ev.ptr(n_ev * i))
                sparse_attention(L["q"], L["summary"], L["k"][:, a.context:],
                                 L["v"][:, a.context:], cfg, workspace=L["ws"],
                                 suffix_length=suffix_len)
            lib.rkv_set_profile_events(None)
            torch.cuda.synchronize()
            for i in range(a.layers):
                for j, name in enumerate(kernels):
                    kernel_ms[name] += ev.elapsed_ms(n_ev * i + j, n_ev * i + j + 1)
        ev.close()
        kernel_us = {k: v * 1e3 / (reps * a.layers) for k, v in kernel_ms.items()}
        timing = f"library HIP events around each kernel of eager calls, {reps} x {a.layers}"
    dominant = max(kernel_us, key=kernel_us.get)
    achieved = nbytes[dominant] / (kernel_us[dominant] * 1e-6) / 1e9
    traffic = measured_traffic(dominant)
    log(f"[bench] kernels (us; {timing}): "
        + ", ".join(f"{k} {v:.2f}" for k, v in kernel_us.items())
        + f"; expanded {frac:.4f}")

    # ---- dense baselines on the same GPU ----------------------------------
    # (1) the dense decode kernel (rkv_dense_decode: every visible token, no
    # summary reads; the reference's "Full" is SDPA decode over the cache),
    # (2) RefineKV's own step at eps 0 (every block expanded).  The speedup
    # is quoted against the faster of the two.
    dense_us = eps0_us = None
    if not a.no_dense:
        d_steps = min(a.steps, 20)
        visible = torch.zeros((), dtype=torch.int32, device=dev)

        def dense_step():
            visible.add_(1)
            for L in layers:
                _hip.dense_decode(L["q"][:, :, 0], L["k"], L["v"], length=visible,
                                  workspace=L["dws"])

        visible.fill_(a.context)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            dense_step()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            dense_step()
        visible.fill_(a.context + a.warmup)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(d_steps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        dense_us = start.elapsed_time(end) * 1e3 / (d_steps * a.layers)
        del graph
        log(f"[bench] dense decode kernel graph: {dense_us:.2f} us/layer-step")
        for L in layers:
            L["dws"].clear()
        ms_d, graph = timed_graph(dense_cfg, "dws", 1, d_steps)
        eps0_us = ms_d * 1e3 / (d_steps * a.layers)
        del graph
        log(f"[bench] refinekv eps=0 graph: {eps0_us:.2f} us/layer-step")
        for L in layers:
            L["dws"].clear()
    dense_best = None if dense_us is None else min(dense_us, eps0_us)

    # ---- blocks within 1e-6 relative of eps ------------------------------
    near, blocks = near_eps_blocks(a, layers, suffix_now)
    log(f"[bench] near-eps blocks: {near} of {blocks}")

    # ---- CPU baseline: the reference's torch CPU backend -------------------
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(a, layers[0], suffix_now)
        log(f"[bench] cpu torch backend: {cpu['value']:.0f} us/layer-step on {cpu['cores']} "
            f"cores, {cpu['one_thread_value']:.0f} on one")

    result = {
        "metric": METRIC,
        "value": round(us_layer, 3),
        "unit": "us/step/layer",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms / a.steps, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (refinekv.testing recipe on GPU: N(0,1) K/V, block key offsets, "
                f"{a.spikes:.0%} query-aligned spike blocks)",
        "config": {
            "workload": f"RefineKV decode attention, Llama-3.1-8B attention shape: {a.layers} "
                        f"layers x {a.heads * a.group}q/{a.heads}kv heads, d{a.dim}, "
                        f"{a.context} prompt tokens, block {a.block}, eps {a.eps}, "
                        f"GQA {a.reduction}, suffix {a.warmup + 1}..{suffix_now}, HIP graph "
                        "per decode step",
            "context": a.context, "layers": a.layers, "kv_heads": a.heads,
            "q_heads": a.heads * a.group, "head_dim": a.dim, "block_size": a.block,
            "eps": a.eps, "gqa_reduction": a.reduction, "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": None if traffic is None else traffic["traffic_bytes"],
            "traffic_source": None if traffic is None else traffic["source"],
        },
        "cpu_baseline": cpu,
        "expanded_fraction": round(frac, 5),
        "near_eps_blocks": near,
        "near_eps_of_blocks": blocks,
        "kernel_us": {k: round(v, 3) for k, v in kernel_us.items()},
        "kernel_timing": timing,
        "algorithmic_bytes": {k: int(v) for k, v in nbytes.items()},
        "step_GBps": round(total_bytes / (us_layer * 1e-6) / 1e9, 1),
        "step_frac_of_peak": round(total_bytes / (us_layer * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
        "dense_us_per_layer_step": None if dense_us is None else round(dense_us, 3),
        "dense_eps0_us_per_layer_step": None if eps0_us is None else round(eps0_us, 3),
        "dense_GBps": None if dense_us is None else round(
            dense_bytes(a, suffix_now) / (dense_us * 1e-6) / 1e9, 1),
        "speedup_vs_dense": None if dense_best is None else round(dense_best / us_layer, 3),
        "summary_us_per_layer": round(summary_us, 1),
        "summary_timing": "HIP events around 5 back-to-back build_summary calls of one layer's "
                          "prompt after a warm call (the queue stays ahead of the host)",
        "attention_tokens_per_s": round(1e6 / (us_layer * a.layers), 1),
    }
    print(json.dumps(result), flush=True)


# Stamp slots of the phase-stamps build (enum Stamp in csrc/rkv_decode.hip).
STAMPS = ("entry", "dots", "stats", "gather", "decided", "ring", "pages_wave0", "combine",
          "published", "merge_start", "merged", "spec", "end", "merge_loaded", "merge_folded",
          "merge_stored", "merge_counted", "chunk0", "chunk1", "chunk2", "issued2", "fold0_start",
          "ring_start", "issue2_addr") + tuple(f"fold_start{j}" for j in range(6)) + tuple(
              f"fold_end{j}" for j in range(6)) + tuple(f"issue_start{j}" for j in range(2, 8))
STAMP_ROWS_PER_HEAD = 256
STAMP_HEADS = 64


def phase_timeline(a):
    """Phase timeline of the one-launch step on the headline workload: the
    step kernel of librefinekv_hip_phases.so (the same source built with
    RKV_PHASE_STAMPS) notes a 100 MHz clock in LDS at each phase boundary of
    every workgroup; after graph replays of one decode step over the layers
    the last layer's stamps are read back.  Times are microseconds from the
    launch's first workgroup start."""
    import numpy as np
    from refinekv import RefineKVConfig, build_summary, sparse_attention, _hip

    assert torch.cuda.is_available(), "bench.py --phases needs a GPU"
    _hip.LIB_PATH = os.path.join(os.path.dirname(_hip.LIB_PATH), "librefinekv_hip_phases.so")
    lib = _hip.lib()
    lib.rkv_phase_stamps_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    _hip.set_speculation(a.speculation)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layers = min(a.layers, 8)
    gen = torch.Generator(device=dev).manual_seed(a.seed)
    cfg = RefineKVConfig(backend="hip", block_size=a.block, eps=a.eps, gqa_reduction=a.reduction)
    stack = []
    for _ in range(layers):
        q, k, v = make_layer(gen, a, 128, dev)
        stack.append((q, k, v, build_summary(k[:, :a.context], v[:, :a.context], cfg), {}))
    suffix = torch.tensor(a.warmup + a.steps, dtype=torch.int32, device=dev).clamp(max=127)

    def step():
        r = None
        for (q, k, v, summ, ws) in stack:
            r = sparse_attention(q, summ, k[:, a.context:], v[:, a.context:], cfg, workspace=ws,
                                 suffix_length=suffix, return_selected=True)
        return r

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = step()
    for _ in range(20):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 50
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / (reps * layers)
    frac = res.selected.float().mean().item()
    buf = np.zeros((STAMP_HEADS * STAMP_ROWS_PER_HEAD, len(STAMPS)), np.uint64)
    assert lib.rkv_phase_stamps_read(buf.ctypes.data, buf.nbytes) == 0
    lay = (ctypes.c_int64 * 13)()
    n_blocks = -(-a.context // a.block)
    _hip._check(lib.rkv_workspace_layout(a.heads, a.group, a.dim, n_blocks, lay),
                "rkv_workspace_layout")
    W = int(lay[12])
    rows = np.concatenate([np.arange(h * STAMP_ROWS_PER_HEAD, h * STAMP_ROWS_PER_HEAD + W)
                           for h in range(a.heads)])
    st = buf[rows].astype(np.int64)
    col = {n: i for i, n in enumerate(STAMPS)}
    t0 = st[:, col["entry"]].min()
    t = (st - t0) * 0.01  # 100 MHz clock -> us
    spec = st[:, col["spec"]] == 1
    print(f"# step phase timeline: {a.heads} kv heads x {W} workgroups, {a.context} tokens, "
          f"block {a.block}, eps {a.eps}, {a.spikes:.0%} spikes; graph {us:.2f} us/layer-step "
          f"(phases build), last layer f {frac:.4f}, speculating workgroups {int(spec.sum())}")
    print("| phase (thread 0 of each workgroup unless noted) | mean us | p10 | p50 | p90 | max "
          "| ends mean | ends max |")
    print("|---|---|---|---|---|---|---|---|")
    seq = [("entry", "dots", "score: q staging, summary loads, dot products"),
           ("dots", "stats", "statistics, LSE slots out, decision-independent loads issued"),
           ("stats", "gather", "wait for the head's LSE slots (wave 0, row 0)"),
           ("gather", "decided", "LSE merge, risk, GQA reduction, mask"),
           ("decided", "ring", "representative, suffix and page-row chunks (wave 0)"),
           ("ring", "pages_wave0", "mask and speculation flag stores"),
           ("pages_wave0", "combine", "waiting for the other waves' page rows"),
           ("combine", "published", "combine, partial slots out")]
    for a0, a1, name in seq:
        d = t[:, col[a1]] - t[:, col[a0]]
        e = t[:, col[a1]]
        qs = np.quantile(d, [0.1, 0.5, 0.9])
        print(f"| {name} | {d.mean():.2f} | {qs[0]:.2f} | {qs[1]:.2f} | {qs[2]:.2f} | "
              f"{d.max():.2f} | {e.mean():.2f} | {e.max():.2f} |")
    for a0, a1, name in (("merge_start", "merge_loaded", "mergers: poll until the head's partials are in, fold own lanes' partials"),
                         ("merge_loaded", "merge_folded", "mergers: folds across lanes"),
                         ("merge_folded", "merge_stored", "mergers: give-up check, normalize, bf16 store"),
                         ("merge_stored", "merge_counted", "mergers: access count (slice 0)"),
                         ("decided", "ring_start", "ring: set-up after the decision"),
                         ("ring_start", "issue2_addr", "ring: chunk 2's rows found"),
                         ("issue2_addr", "issued2", "ring: chunk 2's loads issued"),
                         ("issued2", "fold0_start", "ring: wait for chunk 0"),
                         ("fold0_start", "chunk0", "ring: chunk 0 fold"),
                         ("decided", "chunk0", "ring: wave 0's first chunk folded"),
                         ("chunk0", "chunk1", "ring: wave 0's second chunk"),
                         ("chunk1", "chunk2", "ring: wave 0's third chunk")):
        mm = (st[:, col[a1]] > 0) & (st[:, col[a0]] > 0)
        d = t[mm][:, col[a1]] - t[mm][:, col[a0]]
        e = t[mm][:, col[a1]]
        if len(d):
            print(f"| {name} ({int(mm.sum())}) | {d.mean():.2f} | | | | {d.max():.2f} | "
                  f"{e.mean():.2f} | {e.max():.2f} |")
    ends = t[:, col["end"]]
    print(f"\nworkgroup starts {t[:, 0].min():.2f}..{t[:, 0].max():.2f} us, ends "
          f"{ends.min():.2f}..{ends.max():.2f} us")
    by_head = ends.reshape(a.heads, W).max(1)
    print("last end per head (us): " + ", ".join(f"{x:.2f}" for x in by_head))
    dots_by_head = t[:, col["dots"]].reshape(a.heads, W).mean(1)
    print("score end per head, mean (us): " + ", ".join(f"{x:.2f}" for x in dots_by_head))
    print(json.dumps(dict(phases_us_per_layer_step=round(us, 3), workgroups=int(len(rows)),
                          last_end_us=round(float(ends.max()), 2),
                          expanded_fraction=round(frac, 5))))


def sweep(a):
    """The isolated decode-op sweep of BASELINE.json configs[4]: 8 KV / 32
    query heads, d 128, bf16, GQA "any"; context x block x eps x spike
    fraction.  Each (context, block, spikes) gets its own layers (own caches
    and summaries, enough of them that one graph step touches >= ~1.5 GB of
    summaries where that fits 256 layers, so the Infinity Cache does not hold
    a step); each eps is timed as graph replays of decode steps over those
    layers.  Prints one JSON line per point: us per layer-step, the expanded
    fraction f, algorithmic bytes and HBM GB/s."""
    from refinekv import RefineKVConfig, build_summary, sparse_attention, _hip

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _hip.lib()
    # the three kernels past 256 tiles per head or a grid larger than the
    # device holds at once (two step workgroups per CU)
    _hip.set_decode_path("step")
    warmup, steps = 2, 10
    capacity = warmup + steps + 1
    contexts = [int(x) for x in a.sweep_contexts.split(",")]
    blocks = [int(x) for x in a.sweep_blocks.split(",")]
    for context in contexts:
        for block in blocks:
            n = -(-context // block)
            per_layer = a.heads * n * a.dim * 2 * 3  # key/value means and ellipsoid
            n_layers = max(4, min(256, -(-1_500_000_000 // per_layer)))
            for spikes in (0.01, 0.05, 0.2):
                pa = argparse.Namespace(**{**vars(a), "context": context, "block": block,
                                          "spikes": spikes})
                gen = torch.Generator(device=dev).manual_seed(a.seed)
                layers = []
                for _ in range(n_layers):
                    q, k, v = make_layer(gen, pa, capacity, dev)
                    cfg0 = RefineKVConfig(backend="hip", block_size=block)
                    layers.append(dict(q=q, k=k, v=v, ws={},
                                       summary=build_summary(k[:, :context], v[:, :context], cfg0)))
                torch.cuda.synchronize()
                suffix_len = torch.zeros((), dtype=torch.int32, device=dev)
                for eps in (0.001, 0.01, 0.1):
                    cfg = RefineKVConfig(backend="hip", block_size=block, eps=eps,
                                         gqa_reduction=a.reduction)
                    for L in layers:
                        L["ws"] = {}

                    def step():
                        suffix_len.add_(1)
                        for L in layers:
                            sparse_attention(L["q"], L["summary"], L["k"][:, context:],
                                             L["v"][:, context:], cfg, workspace=L["ws"],
                                             suffix_length=suffix_len)

                    suffix_len.fill_(0)
                    for _ in range(warmup):
                        step()
                    torch.cuda.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph):
                        step()
                    torch.cuda.synchronize()
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    for _ in range(steps):
                        graph.replay()
                    e1.record()
                    torch.cuda.synchronize()
                    us = e0.elapsed_time(e1) * 1e3 / (steps * n_layers)
                    del graph
                    masks = torch.stack([
                        sparse_attention(L["q"], L["summary"], L["k"][:, context:],
                                         L["v"][:, context:], cfg, workspace=L["ws"],
                                         return_selected=True,
                                         suffix_length=suffix_len).selected.clone()
                        for L in layers])
                    f = masks.float().mean().item()
                    nbytes = algorithmic_bytes(pa, masks, layers[0]["summary"].counts,
                                               int(suffix_len.item()))["decode"]
                    gbps = nbytes / (us * 1e-6) / 1e9
                    point = dict(context=context, block=block, eps=eps, spikes=spikes,
                                 layers=n_layers,
                                 path=_hip.decode_plan(a.heads, a.group, a.dim, n, block),
                                 us_per_layer_step=round(us, 2), expanded_fraction=round(f, 5),
                                 algorithmic_bytes=int(nbytes), GBps=round(gbps, 1),
                                 frac_of_peak=round(gbps / PEAK_HBM_GBPS, 4))
                    print(json.dumps(point), flush=True)
                del layers
                torch.cuda.empty_cache()


def _model(family, max_positions, seed):
    """Random-init Llama-3.1-8B / Qwen2.5-7B-shaped causal LM, bf16, built on
    the GPU."""
    import transformers

    if family == "llama":
        config = transformers.LlamaConfig(
            vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
            num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=max_positions,
            rms_norm_eps=1e-5, rope_parameters={"rope_type": "default", "rope_theta": 500000.0},
            bos_token_id=None, eos_token_id=None, pad_token_id=None)
        cls = transformers.LlamaForCausalLM
    else:
        config = transformers.Qwen2Config(
            vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
            num_attention_heads=28, num_key_value_heads=4, max_position_embeddings=4 * 32768,
            rms_norm_eps=1e-6, rope_parameters={"rope_type": "yarn", "factor": 4.0,
                                                "original_max_position_embeddings": 32768,
                                                "rope_theta": 1000000.0},
            use_sliding_window=False, bos_token_id=None, eos_token_id=None, pad_token_id=None)
        cls = transformers.Qwen2ForCausalLM
    torch.manual_seed(seed)
    saved = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = cls(config)
    finally:
        torch.set_default_dtype(saved)
    return model.eval(), config


class _GraphTap:
    """Wraps the RefineKV hook's sparse_attention.  Every decode call adds
    its mask to a per-layer count of how often each block expanded (made on
    the layer's first, eager, call); under graph capture the add and a copy
    of the layer's query become part of the captured step, so every replay
    refreshes them.  It keeps the layer's call arguments for the isolated
    replay afterwards."""

    def __init__(self, real):
        self.real = real
        self.layers = []
        self.expanded = {}  # id(workspace) -> (int32 counts, calls)

    def __call__(self, query, summary, key_suffix, value_suffix, config, *, anchor_mask=None,
                 workspace=None, return_selected=False, suffix_length=None,
                 access_counter=None):
        from refinekv.attention import AttentionResult

        result = self.real(query, summary, key_suffix, value_suffix, config,
                           anchor_mask=anchor_mask, workspace=workspace, return_selected=True,
                           suffix_length=suffix_length, access_counter=access_counter)
        capturing = torch.cuda.is_current_stream_capturing()
        key = id(workspace)
        if key not in self.expanded:
            assert not capturing, "the first decode call of a layer runs eagerly"
            self.expanded[key] = [torch.zeros(result.selected.shape, dtype=torch.int32,
                                              device=query.device), 0]
        counts = self.expanded[key]
        counts[0].add_(result.selected)
        counts[1] += 1
        if capturing:
            self.layers.append(dict(query=query.clone(), summary=summary, key_suffix=key_suffix,
                                    value_suffix=value_suffix, config=config,
                                    anchor=anchor_mask, suffix_length=suffix_length,
                                    expanded=counts))
        return AttentionResult(result.output, result.selected if return_selected else None)


def model_bench(a):
    """BASELINE.json configs[1..3] as random-init model stacks: prefill with
    RefineKV (dense SDPA prefill, summaries, prompt anchors), then
    --new-tokens greedy tokens as replays of one captured HIP graph per
    token.  Reports per layer the fraction of blocks expanded over the
    replays, and the attention op's us per layer-step: its kernels timed in
    isolation by replaying all layers' decode calls (the last step's query,
    summary, suffix and anchors) as one graph, 125 times."""
    import statistics

    from refinekv import RefineKV, RefineKVConfig, _hip, sparse_attention
    from refinekv.integrations import transformers as hook

    spec = MODEL_CONFIGS[a.model]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    new = a.new_tokens
    t0 = time.perf_counter()
    model, mconfig = _model(spec["family"], spec["prompt"] + new + 8, a.seed)
    torch.cuda.synchronize()
    log(f"[model] {a.model}: {sum(p.numel() for p in model.parameters()) / 1e9:.2f}B parameters "
        f"initialised in {time.perf_counter() - t0:.1f} s")
    gen = torch.Generator().manual_seed(a.seed + 1)
    ids = torch.randint(0, mconfig.vocab_size, (1, spec["prompt"]), generator=gen).to(dev)
    cfg = RefineKVConfig(backend="hip", block_size=spec["block"], eps=spec["eps"],
                         gqa_reduction=spec["reduction"], anchor_tokens=spec["anchors"])
    tap = _GraphTap(hook.sparse_attention)
    hook.sparse_attention = tap
    try:
        with RefineKV(model, cfg, cuda_graph=True) as session:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = model.generate(input_ids=ids, attention_mask=torch.ones_like(ids),
                                 max_new_tokens=new, min_new_tokens=new, eos_token_id=None,
                                 forced_eos_token_id=None, do_sample=False)
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            assert out.shape[1] == spec["prompt"] + new
            replays = new - 1 - min(2, new - 2)
            layers = tap.layers
            # eager warm-up calls, the capture (recorded, not run) and the replays
            calls = [L["expanded"][1] - 1 + replays for L in layers]
            fractions = [float(L["expanded"][0].float().mean().item()) / n
                         for L, n in zip(layers, calls)]
            # the attention op alone: every layer's decode call of the last step
            suffix_now = int(layers[0]["suffix_length"].item())
            steps = 125
            for L in layers:
                L["ws"] = {}
                L["args"] = (L["query"], L["summary"], L["key_suffix"], L["value_suffix"],
                             L["config"])

            def op_step(config=None):
                for L in layers:
                    sparse_attention(*L["args"][:4], config or L["config"],
                                     anchor_mask=L["anchor"], workspace=L["ws"],
                                     suffix_length=L["suffix_length"])

            def time_graph(config=None, step=None):
                step = step or (lambda: op_step(config))
                step()
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    step()
                graph.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(steps):
                    graph.replay()
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) * 1e3 / (steps * len(layers))

            us = time_graph()
            for L in layers:
                L["ws"] = {}
            dense_us = time_graph(RefineKVConfig(backend="hip", block_size=spec["block"],
                                                 eps=0.0, gqa_reduction=spec["reduction"]))

            # the dense decode kernel over each layer's whole visible cache
            # (prompt + suffix): the static cache's (H, capacity, D) view
            # that the suffix views start inside
            def whole(t, prompt):
                return t.as_strided((t.shape[0], prompt + t.shape[1], t.shape[2]), t.stride(),
                                    t.storage_offset() - prompt * t.stride(1))

            for L in layers:
                P = L["summary"].prompt_length
                L["dense"] = (L["query"][:, :, 0], whole(L["key_suffix"], P),
                              whole(L["value_suffix"], P),
                              (L["suffix_length"] + P).to(torch.int32), {})

            def dense_step():
                for L in layers:
                    q, k, v, n, ws = L["dense"]
                    _hip.dense_decode(q, k, v, length=n, workspace=ws)

            dense_kernel_us = time_graph(step=dense_step)
            check = session.check_handoffs
            check()
    finally:
        hook.sparse_attention = tap.real
    heads, group, dim = layers[0]["query"].shape[0], layers[0]["query"].shape[1], 128
    result = {
        "metric": f"RefineKV decode attention on a random-init model stack, {a.model}",
        "config_index": spec["config_index"],
        "model": {"family": spec["family"], "layers": len(layers), "kv_heads": heads,
                  "q_heads": heads * group, "head_dim": dim, "weights": "random init (seeded)",
                  "prompt": "uniform random token ids"},
        "prompt_tokens": spec["prompt"], "new_tokens": new,
        "refinekv": {"block_size": spec["block"], "eps": spec["eps"],
                     "gqa_reduction": spec["reduction"], "anchor_tokens": spec["anchors"]},
        "expanded_fraction_mean": round(statistics.fmean(fractions), 5),
        "decode_calls_per_layer": calls[0],
        "expanded_fraction_per_layer": [round(f, 4) for f in fractions],
        "attention_us_per_layer_step": round(us, 3),
        "attention_timing": f"the {len(layers)} layers' decode calls at suffix {suffix_now} "
                            f"(last step's queries), one HIP graph, {steps} replays",
        "dense_eps0_us_per_layer_step": round(dense_us, 3),
        "dense_kernel_us_per_layer_step": round(dense_kernel_us, 3),
        "speedup_vs_dense": round(min(dense_us, dense_kernel_us) / us, 3),
        "generate_wall_s": round(wall, 2),
    }
    print(json.dumps(result), flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` as profiled, not measured in this run:
    the committed rocprofv3 PMC summary profiles/traffic.json (FETCH_SIZE and
    WRITE_SIZE runs scaled by a plain copy's readings) with the commit and
    date of the kernel it was taken on, or None when it has none."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            doc = json.load(f)
        entry = doc["kernels"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None
    if entry is None:
        return None
    return {"traffic_bytes": entry["traffic_bytes"],
            "source": f"profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE, "
                      f"kernel of commit {doc.get('kernel_commit', 'unrecorded')}, "
                      f"{doc.get('measured', 'undated')}), not measured in this run"}


def summary_event_us(k, v, cfg):
    """build_summary of one layer's prompt: a warm call, then HIP events around
    5 back-to-back calls (each call's host work overlaps the previous call's
    kernels), per call."""
    from refinekv import build_summary

    build_summary(k, v, cfg)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        build_summary(k, v, cfg)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / 5


def copy_calibration():
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE counter
    readings per byte convert the decode kernels' readings to bytes."""
    n = 64 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "copies": 5}))


def summary_only(a):
    """build_summary of one layer's prompt, three calls, HIP events around
    each: the prefill kernels alone, for kernel traces and counters."""
    from refinekv import RefineKVConfig, build_summary

    gen = torch.Generator(device="cuda").manual_seed(a.seed)
    shape = (a.heads, a.context, a.dim)
    k = torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16)
    cfg = RefineKVConfig(backend="hip", block_size=a.block)
    times = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        build_summary(k, v, cfg)
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3)
    print(json.dumps({"summary_us_per_call": [round(t, 1) for t in times],
                      "bytes_read": 2 * k.numel() * k.element_size(),
                      "shape": {"heads": a.heads, "tokens": a.context, "dim": a.dim,
                                "block": a.block}}))


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_us(fn, reps, warmup=3, budget_s=None):
    """Median wall time of fn() in us over `reps` runs after `warmup` runs
    (fewer runs, at least 5, if `budget_s` runs out first)."""
    for _ in range(warmup):
        fn()
    times, t_start = [], time.perf_counter()
    while len(times) < reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if budget_s is not None and len(times) >= 5 and time.perf_counter() - t_start > budget_s:
            break
    times.sort()
    return times[len(times) // 2] * 1e6, len(times)


def cpu_baseline(a, layer, suffix):
    """The reference's PyTorch CPU backend (this package's torch restatement
    of it, bit-identical to the reference on the golden fixtures) timed on
    this host: sparse_attention (selection + mixed attention) on one layer of
    the headline workload, with every usable core and with one thread, median
    of >= 30 runs after 3 warm-ups; and BASELINE.json configs[0] (fp32, 4096
    prompt + 16 suffix tokens, 32 anchors): sparse_attention and
    build_summary, with every usable core and one thread."""
    from refinekv import RefineKVConfig, build_summary, sparse_attention, testing
    from refinekv.summary import BlockSummary

    cores = len(os.sched_getaffinity(0))
    saved = torch.get_num_threads()
    s = layer["summary"]
    # the GPU summary equals the torch path's bit for bit (pinned by the tests)
    cpu_summary = BlockSummary(**{f: (getattr(s, f).cpu() if torch.is_tensor(getattr(s, f))
                                      else getattr(s, f))
                                  for f in ("keys", "values", "counts", "key_mean", "value_mean",
                                            "ellipsoid", "value_norm", "max_value_norm",
                                            "prompt_length", "block_size")})
    q = layer["q"].cpu()
    ks = layer["k"][:, a.context:a.context + suffix].cpu()
    vs = layer["v"][:, a.context:a.context + suffix].cpu()
    cfg = RefineKVConfig(backend="torch", block_size=a.block, eps=a.eps,
                         gqa_reduction=a.reduction)
    head = lambda: sparse_attention(q, cpu_summary, ks, vs, cfg)

    inp = testing.decode_inputs(heads=8, group=4, dim=128, prompt=4096, suffix=16, block=32,
                                spike_fraction=0.02, anchors=32, seed=0)
    cfg1 = RefineKVConfig(backend="torch", block_size=32, eps=0.01, gqa_reduction="any",
                          anchor_tokens=32)
    s1 = build_summary(inp["prompt_keys"], inp["prompt_values"], cfg1)
    from refinekv.attention import select_blocks_union
    anchor1 = select_blocks_union(inp["anchor_queries"], s1, cfg1)
    c1_attn = lambda: sparse_attention(inp["query"], s1, inp["suffix_keys"],
                                       inp["suffix_values"], cfg1, anchor_mask=anchor1)
    c1_summ = lambda: build_summary(inp["prompt_keys"], inp["prompt_values"], cfg1)
    out = {}
    try:
        for threads in (cores, 1):
            torch.set_num_threads(threads)
            key = "all" if threads == cores else "one"
            out[f"head_{key}"] = _median_us(head, 30, budget_s=20.0)
            out[f"c1_attn_{key}"] = _median_us(c1_attn, 30)
            out[f"c1_summ_{key}"] = _median_us(c1_summ, 30)
    finally:
        torch.set_num_threads(saved)
    (v_all, n_all), (v_one, n_one) = out["head_all"], out["head_one"]
    return {
        "value": round(v_all, 1), "unit": "us/step/layer", "cores": cores, "kind": "port",
        "sample": f"reference torch CPU backend (refinekv backend='torch', bit-identical to the "
                  f"reference's torch path on the golden fixtures): sparse_attention on one "
                  f"layer of the headline workload ({a.context} tokens, suffix {suffix}, bf16), "
                  f"median of {n_all} runs after 3 warm-ups with torch.set_num_threads({cores}) "
                  f"(len(os.sched_getaffinity(0))); CPU {_cpu_model()}, torch {torch.__version__}",
        "one_thread_value": round(v_one, 1),
        "one_thread_runs": n_one,
        "config1_fp32": {
            "workload": "BASELINE configs[0]: 8 KV / 32 q heads, d128, fp32, 4096 prompt + 16 "
                        "suffix tokens, block 32, eps 0.01, any, 32 anchors",
            "sparse_attention_us": {"all_cores": round(out["c1_attn_all"][0], 1),
                                    "one_thread": round(out["c1_attn_one"][0], 1)},
            "build_summary_us": {"all_cores": round(out["c1_summ_all"][0], 1),
                                 "one_thread": round(out["c1_summ_one"][0], 1)},
            "runs": 30, "warmup": 3,
        },
    }


def near_eps_blocks(a, layers, suffix_len):
    """Blocks whose GQA-reduced risk lies within 1e-6 relative of eps (where
    the north star allows a mask to differ from the reference's fp32 order),
    over every layer at the current step: (count, blocks)."""
    from refinekv import _hip

    count = total = 0
    cfg = _hip_cfg(a)
    for L in layers:
        s = L["summary"]
        risk = torch.empty(a.heads, a.group, s.num_blocks, device=L["q"].device)
        _hip.select(L["q"], s, cfg, {}, risk_out=risk)
        reduced = risk.mean(1) if a.reduction == "mean" else risk.amax(1)
        count += int(((reduced - a.eps).abs() <= 1e-6 * a.eps).sum().item())
        total += reduced.numel()
    return count, total


def _hip_cfg(a):
    from refinekv import RefineKVConfig

    return RefineKVConfig(backend="hip", block_size=a.block, eps=a.eps,
                          gqa_reduction=a.reduction)


if __name__ == "__main__":
    main()
