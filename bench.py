"""Benchmark of the quantized MoE layer on one MI355X (BASELINE.json metric: MoE-layer tokens/s + HBM GB/s at decode,
MXFP4 TFLOPS at prefill).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one MoE layer forward over one batch of synthetic tokens: routing (softmax top-8 + align tables, and at
T <= 64 the per-token fp8 quant of x in the same launch) -> grouped gate_up GEMM -> SiLU*up + fp8 quant -> grouped
down GEMM (router weight folded) -> top-k sum. At the headline point the middle three run as one launch
(r9k_moe_stream_layer: each 16-row routing block's gate_up, SiLU + quant and down in one workgroup), so the T=64
step is three launches: routing, the layer, the sum. The headline `value`
is BASELINE config 2 (E=288 experts, hidden 2048, expert intermediate 512, top-8) at T=64 tokens, the
bandwidth-bound decode point; T = 1, 8, 16, the config 3 prefill (T=8192) and the router gate GEMM that produces
the layer's logits (r9k_router_gemm against stock's F.linear) are reported beside it, with config 4 (NVFP4 -> MXFP4
conversion of a [17408, 5120] weight, then the dense GEMM at M = 1, 4, 16, 4096) and config 5 (E=384, hidden 4096,
Zipf-skewed routing, T = 1, 32, 256, 4096).

Method: weights and inputs are resident in HBM before timing. Steps run as HIP-graph replays that cycle through
COPIES independent weight copies (> 2x the 256 MB Infinity Cache per cycle), so weight bytes come from HBM, not from
a cache warmed by the previous step. The dominant kernel (r9k_moe_stream_layer at T=64) is also launched on its own,
bracketed by HIP events on the stream it runs on, for the roofline figure. The CPU baselines are the oracle's
dequant-then-matmul layer and converter (oracle/, the reference's torch CPU path restated) timed on this host on
bounded samples: config 2 T=64 (`cpu_baseline`), config 1, the config 3 prefill, the config 4 conversion and GEMM,
config 5 T=4096.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "r9700-stack_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP8_PEAK_TFLOPS = 5000.0       # dense fp8 MFMA
FP4_PEAK_TFLOPS = 10100.0      # dense fp4 / fp6 MFMA
COPIES = 4
HIT_LAYERS = COPIES           # cached layers in the expert cache's all-hit graph
SEED = 20261201


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the T=8192 prefill line")
    ap.add_argument("--no-router", action="store_true", help="skip the router gate GEMM timings")
    ap.add_argument("--no-cfg4", action="store_true", help="skip the config 4 converter + dense GEMM lines")
    ap.add_argument("--no-cfg5", action="store_true", help="skip the config 5 (E=384, Zipf) layer lines")
    ap.add_argument("--no-cache", action="store_true", help="skip the host-offloaded expert cache lines")
    return ap.parse_args()


class Layer:
    """One MoE layer's MXFP4 weights in COPIES independent HBM copies (kernel layout), plus copy 0 in checkpoint
    layout for the CPU baseline."""

    def __init__(self, E, H, I, dev, lo=118, hi=126, copies=COPIES, seed=SEED):
        from r9700_vllm.kernels import moe as K
        g = torch.Generator(device=dev).manual_seed(seed)
        rnd = lambda shape, a, b: torch.randint(a, b + 1, shape, generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
        self.p13, self.e13 = rnd((E, 2 * I, H // 2), 0, 255), rnd((E, 2 * I, H // 32), lo, hi)
        self.p2, self.e2 = rnd((E, H, I // 2), 0, 255), rnd((E, H, I // 32), lo, hi)
        W13 = K.prepare_mxfp4_weights(self.p13, self.e13)
        W2 = K.prepare_mxfp4_weights(self.p2, self.e2)
        self.W13 = [W13] + [K.Mxfp4Experts(W13.wq.clone(), W13.wsr.clone(), W13.N, W13.K) for _ in range(copies - 1)]
        self.W2 = [W2] + [K.Mxfp4Experts(W2.wq.clone(), W2.wsr.clone(), W2.N, W2.K) for _ in range(copies - 1)]
        self.E, self.H, self.I = E, H, I

    def bytes_per_expert(self) -> int:
        H, I = self.H, self.I
        return 2 * I * H // 2 + 2 * I * H // 32 + H * I // 2 + H * I // 32


class Step:
    """The layer forward for T tokens, graph-capturable: fused routing when the decode router path applies
    (T * topk <= 4096 rows, as R9kTopKRouter), otherwise top-k + activation quant in one launch (as R9kTopKRouter
    above its row limit) and the in-apply align."""

    def __init__(self, layer: Layer, T: int, topk: int, dev, seed: int, zipf: bool = False):
        from r9700_vllm.kernels import moe as K
        from r9700_vllm.moe import route
        from r9700_vllm.moe.experts import R9700Mxfp4Experts
        self.K, self.route = K, route
        self.layer, self.T, self.topk, self.dev = layer, T, topk, dev
        g = torch.Generator().manual_seed(seed)
        self.x_cpu = torch.randn(T, layer.H, generator=g).to(torch.bfloat16)
        logits = torch.randn(T, layer.E, generator=g)
        if zipf:
            # config 5's skew: expert popularity ~ Zipf(1.1) over a seeded ranking of the experts
            rank = torch.randperm(layer.E, generator=g).float() + 1
            logits = logits - 1.1 * torch.log(rank)[None, :]
        self.logits_cpu = logits.to(torch.bfloat16)
        self.x = self.x_cpu.to(dev)
        self.logits = self.logits_cpu.to(dev)
        self.out = torch.empty(T, layer.H, dtype=torch.bfloat16, device=dev)
        self.numel = T * topk
        self.fused = self.numel <= 4096 and T <= route.MAX_ROWS
        E = layer.E
        self.blk = K.MOE_BLOCK * K.pick_mt(self.numel, E)
        cap = route.capacity(self.numel, E, self.blk)
        self.sid = torch.empty(cap, dtype=torch.int32, device=dev)
        self.eid = torch.empty(cap // self.blk, dtype=torch.int32, device=dev)
        self.ntpp = torch.zeros(1, dtype=torch.int32, device=dev)
        self.scratch = torch.zeros(route.scratch_ints(E), dtype=torch.int32, device=dev)
        # the router's second (256-row) layout for steps the device may route to big blocks (route.dual_wanted)
        capb = route.capacity(self.numel, E, 256)
        self.big = (torch.empty(capb, dtype=torch.int32, device=dev),
                    torch.empty(capb // 256, dtype=torch.int32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev))
        self.experts = [R9700Mxfp4Experts.standalone(w13.wsr, w2.wsr) for w13, w2 in zip(layer.W13, layer.W2)]

        class _Routed:
            _r9k_tables = None
        self.routed = _Routed()
        for ex in self.experts:
            ex.r9k_layer = self.routed

    def __call__(self, c: int):
        K, route, L = self.K, self.route, self.layer
        fused = self.fused and not route.split_planned(self.routed, self.numel, L.E)
        bb = route.dual_wanted(self.routed, self.numel, L.E) if fused else 0
        if bb == 256:
            # as R9kTopKRouter for a wide decode step of a layer that runs the device-picked pair: both layouts
            w, ids, xq, xs = route.moe_route_dual(self.logits, self.topk, True, self.blk, self.sid, self.eid,
                                                  self.ntpp, self.scratch, self.x, bb, *self.big, K.DEVICE_MIN_ROWS)
            self.routed._r9k_tables = route.Tables(ids, self.sid, self.eid, self.ntpp, self.blk, self.numel,
                                                   self.x, self.x._version, xq, xs, big=(*self.big, bb))
        elif fused:
            w, ids, xq, xs = route.moe_route_quant(self.logits, self.topk, True, self.blk, self.sid, self.eid,
                                                   self.ntpp, self.scratch, self.x)
            self.routed._r9k_tables = route.Tables(ids, self.sid, self.eid, self.ntpp, self.blk, self.numel,
                                                   self.x, self.x._version, xq, xs)
        else:
            # prefill widths, as R9kTopKRouter: top-k and the activation quant in one launch, tables in apply
            r = K.moe_topk_quant(self.logits, self.topk, True, self.x)
            if r is None:
                w, ids = K.moe_topk(self.logits, self.topk, True)
                self.routed._r9k_tables = None
            else:
                w, ids, xq, xs = r
                self.routed._r9k_tables = route.Tables(ids, None, None, None, -1, self.numel, self.x,
                                                       self.x._version, xq, xs)
        self.experts[c].apply(self.out, self.x, L.W13[c].wq, L.W2[c].wq, w, ids, "silu", L.E, None, None, None,
                              None, None, None, False)
        self.w, self.ids = w, ids
        return self.out


def graph_time(step: Step, steps: int, warmup: int, windows: int = 1, min_warm_ms: float = 40.0):
    """ms per step from a HIP graph that cycles the weight copies (one replay = `copies` steps).

    Warm-up: `warmup` eager steps, then graph replays until at least max(warmup steps, min_warm_ms of replays) have
    run, so every point starts from steady state (clocks, caches, allocator) whatever --warmup says. windows == 1 (the
    headline): exactly `steps` steps (a multiple of the copy count) in one timed window. windows > 1 (side lines):
    the median of `windows` windows of `steps` steps each. Returns (ms per step, steps in one window)."""
    copies = len(step.layer.W13)
    for i in range(max(2, warmup)):
        step(i % copies)
    torch.cuda.synchronize()
    ref = step(copies - 1).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in range(copies):
            step(c)
    g.replay()
    torch.cuda.synchronize()
    if not torch.equal(step.out, ref):
        raise RuntimeError("graph replay output differs from the eager step")
    t_w = time.perf_counter()
    n_w = 1
    while n_w * copies < warmup or (time.perf_counter() - t_w) * 1e3 < min_warm_ms:
        g.replay()
        n_w += 1
        if n_w % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    reps = max(1, steps // copies)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(windows):
        torch.cuda.synchronize()
        t0.record()
        for _ in range(reps):
            g.replay()
        t1.record()
        torch.cuda.synchronize()
        times.append(t0.elapsed_time(t1) / (reps * copies))
    if not torch.equal(step.out, ref):
        raise RuntimeError("graph replay output differs from the eager step")
    return float(np.median(times)), reps * copies


def layer_kernel_time(step: Step, reps: int = 40):
    """Average duration (ms) of the T=64 step's dominant launch alone: r9k_moe_stream_layer (gate_up, SiLU + quant
    and down of each 16-row routing block in one workgroup), HIP events on its stream, rotating weight copies. Returns
    (ms, algorithmic bytes per launch, flops per launch, experts touched): bytes = the touched experts' gate_up and
    down codes + e8m0 exponents, the fp8 input rows and their scales, the router weights and the bf16 down rows."""
    K, L = step.K, step.layer
    step(0)
    torch.cuda.synchronize()
    ids = step.ids
    E = L.E
    tabs = K.moe_align(ids, K.MOE_BLOCK, E)
    xq, xs = K.quant_rows_fp8(step.x)
    tw = step.w.reshape(-1).to(torch.float32).contiguous()
    down = torch.empty(step.numel, L.H, dtype=torch.bfloat16, device=step.dev)
    copies = len(L.W13)

    def launch(c):
        if not K.moe_stream_layer(xq, xs, L.W13[c], L.W2[c], down, *tabs, step.numel, step.topk, tw, E):
            raise RuntimeError("r9k_moe_stream_layer does not serve the T=64 step")

    for i in range(8):
        launch(i % copies)
    torch.cuda.synchronize()
    # `reps` back-to-back launches in one HIP graph, HIP events around its replay on this stream: the average is the
    # kernel's own duration (separate event pairs per launch would add the launch gap to every sample)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(reps):
            launch(i % copies)
    g.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(s)
    g.replay()
    b.record(s)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    touched = int(torch.unique(ids).numel())
    H, I = L.H, L.I
    nbytes = touched * L.bytes_per_expert() + step.T * H + step.T * 4 + step.numel * 4 + step.numel * H * 2
    flops = 2 * step.numel * (2 * I * H + H * I)
    return ms, nbytes, flops, touched


def events_ms(fn, reps: int) -> float:
    """Average ms of fn() over `reps` calls, HIP events on the current stream around them (after one warm call)."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(s)
    for _ in range(reps):
        fn()
    b.record(s)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def cfg4_lines(dev, cpu: bool = False) -> dict:
    """the load-time NVFP4 -> MXFP4 conversion of a [17408, 5120] dense weight (uniform codes,
    s16 = e4m3(|N(0,1)| * 0.05), global 1), one launch over all rows, then the fp8-act x MXFP4 GEMM on the converted
    weight at M = 1, 4, 16, 4096 (ops.mxfp4_linear: per-row quant + GEMM), and the native NVFP4 GEMM
    (ops.nvfp4_linear, exact checkpoint bits) at M = 1, 4, 16, 4096. GEMM timing: one HIP graph cycling through 12 weight
    copies (570-600 MB, > 2x the Infinity Cache), HIP events around its replays."""
    from r9700_vllm import ops
    from r9700_vllm.kernels import moe as K
    from r9700_vllm.quant import nvfp4 as NV
    N, Kd = 17408, 5120
    g = torch.Generator(device=dev).manual_seed(SEED + 4000)
    packed = torch.randint(0, 256, (N, Kd // 2), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    s16 = (torch.randn(N, Kd // 16, generator=g, device=dev).abs() * 0.05).to(torch.float8_e4m3fn)
    row_div = torch.ones(N, device=dev)
    res = {}
    conv = lambda: NV.nvfp4_to_mxfp4(packed, s16, row_div, rows_per_chunk=N)
    ms = events_ms(conv, 5)
    cin, cout = N * Kd // 2 + N * Kd // 16, N * Kd // 2 + N * Kd // 32
    res["convert"] = {"ms": round(ms, 4), "GBps": round((cin + cout) / (ms * 1e-3) / 1e9, 1),
                      "bytes_in": cin, "bytes_out": cout}
    print(f"# cfg4 convert [17408, 5120]: {ms * 1e3:.1f} us, {res['convert']['GBps']} GB/s", file=sys.stderr,
          flush=True)
    mp, me = conv()
    if cpu:
        res["cpu"] = cpu_cfg4(packed, s16, mp, me, g, dev)
    W0 = K.prepare_mxfp4_weights(mp.unsqueeze(0), me.unsqueeze(0))
    del packed, s16, mp, me
    Ws = [W0] + [K.Mxfp4Experts(W0.wq.clone(), W0.wsr.clone(), N, Kd) for _ in range(11)]
    wbytes = N * Kd // 2 + N * Kd // 32
    gemm = {}
    for M in (1, 4, 16, 4096):
        x = torch.randn(M, Kd, generator=g, device=dev).to(torch.bfloat16)
        calls = Ws if M <= 16 else Ws[:2]
        for W in calls[:2]:
            ops.mxfp4_linear(x, W.wq, W.wsr, N, Kd)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for W in calls:
                ops.mxfp4_linear(x, W.wq, W.wsr, N, Kd)
        reps = 20 if M <= 16 else 5
        ms = events_ms(gr.replay, reps) / len(calls)
        del gr
        nbytes = wbytes + M * Kd * 2 + M * N * 2
        flops = 2 * M * N * Kd
        gemm[str(M)] = {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "TFLOPS": round(flops / (ms * 1e-3) / 1e12, 1)}
        print(f"# cfg4 GEMM M={M}: {ms * 1e3:.1f} us, {gemm[str(M)]['GBps']} GB/s, {gemm[str(M)]['TFLOPS']} TFLOPS",
              file=sys.stderr, flush=True)
    res["gemm"] = gemm
    del Ws, W0
    # native NVFP4 (the checkpoint's codes and e4m3 scales kept; the reference's default for dense NVFP4 linears) on
    # the same codes, decode widths, the same copy rotation
    pk = torch.randint(0, 256, (1, N, Kd // 2), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    s16b = (torch.randn(1, N, Kd // 16, generator=g, device=dev).abs() * 0.05).to(torch.float8_e4m3fn)
    WN0 = K.prepare_nvfp4_weights(pk, s16b, torch.ones(1, N, device=dev))
    del pk, s16b
    WNs = [WN0] + [K.Nvfp4Experts(WN0.wq.clone(), WN0.ws.clone(), WN0.wg.clone(), N, Kd) for _ in range(11)]
    nbytes_w = N * Kd // 2 + N * Kd // 16 + N * 4
    native = {}
    for M in (1, 4, 16, 4096):
        x = torch.randn(M, Kd, generator=g, device=dev).to(torch.bfloat16)
        calls = WNs if M <= 16 else WNs[:2]
        for W in calls[:2]:
            ops.nvfp4_linear(x, W.wq, W.ws, W.wg, N, Kd)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for W in calls:
                ops.nvfp4_linear(x, W.wq, W.ws, W.wg, N, Kd)
        ms = events_ms(gr.replay, 20 if M <= 16 else 5) / len(calls)
        del gr
        nbytes = nbytes_w + M * Kd * 2 + M * N * 2
        native[str(M)] = {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                          "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                          "TFLOPS": round(2 * M * N * Kd / (ms * 1e-3) / 1e12, 1)}
        print(f"# cfg4 native NVFP4 GEMM M={M}: {ms * 1e3:.1f} us, {native[str(M)]['GBps']} GB/s, "
              f"{native[str(M)]['TFLOPS']} TFLOPS", file=sys.stderr, flush=True)
    res["gemm_nvfp4_native"] = native
    del WNs, WN0
    torch.cuda.empty_cache()
    return {"workload": "cfg4 dense [17408, 5120]: NVFP4 -> MXFP4 conversion, then fp8-act x MXFP4 GEMM", **res}


def cfg5_lines(dev, steps: int, warmup: int, cpu: bool = False) -> dict:
    """hidden 4096, intermediate 2048, 384 experts (e8m0 in [116, 126]), top-8 over Zipf(1.1)-biased
    logits, T = 1, 32, 256, 4096; the same Step and graph timing as config 2 (4 weight copies, 19 GB)."""
    layer = Layer(384, 4096, 2048, dev, lo=116, hi=126, seed=SEED + 5000)
    out = {}
    for T in (1, 32, 256, 4096):
        st = Step(layer, T, 8, dev, SEED + 5000 + T, zipf=True)
        ms, n = graph_time(st, max(40, steps) if T < 4096 else 8, warmup, windows=5)
        nbytes, touched = layer_bytes(st)
        counts = torch.bincount(st.ids.reshape(-1).long(), minlength=layer.E).float()
        flops = 6 * T * 8 * layer.H * layer.I
        out[str(T)] = {"ms_per_step": round(ms, 5), "tokens_per_s": round(T / (ms * 1e-3), 1),
                       "experts_touched": touched, "layer_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                       "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                       "TFLOPS": round(flops / (ms * 1e-3) / 1e12, 1),
                       "top_expert_share": round(float(counts.max() / counts.sum()), 4)}
        print(f"# cfg5 T={T}: {ms * 1e3:.1f} us/layer, {out[str(T)]['layer_GBps']} GB/s, "
              f"{out[str(T)]['TFLOPS']} TFLOPS over {touched} experts", file=sys.stderr, flush=True)
        if cpu and T == 4096:
            out[str(T)]["cpu"] = cpu_layer_sample(st, 64)
        del st
    del layer
    torch.cuda.empty_cache()
    return {"workload": "cfg5 layer: E=384, hidden 4096, intermediate 2048, top-8, Zipf(1.1) routing",
            "sweep": out}


def cache_lines(dev, steps: int) -> dict:
    """Host-offloaded experts (moe/cache.py) on config 2's layer (E=288, hidden 2048, intermediate 512, top-8) with a
    64-slot VRAM cache over the mapped host store, each from a HIP graph of the whole apply (LRU manage, gather,
    align tables, GEMMs over the slots and, when needed, over host memory):
      hit:   T = 1 routed to 8 resident experts every step (the cold pass is provably empty, no inserts), four
             layers in one graph, each with its own cache over one shared host store (as the resident decode lines
             replay four steps a graph: one apply a replay measures the host's graph launch rate, ~22 us, not the
             GPU);
      wide:  T = 64 (~240 distinct experts > the 63-expert threshold): every non-resident expert is read through
             from host memory inside the GEMMs (PCIe);
      wide staged: the wide step with R9K_STAGE_COLD=1 (the cold experts gathered into VRAM first, then read there);
      gather: r4d_lru_gather of 64 experts host -> slots alone (1.67 MB each)."""
    from r9700_vllm.kernels import moe as K
    from r9700_vllm.moe import cache as C
    from r9700_vllm.moe.experts import R9700Mxfp4Experts
    E, H, I, topk, S = 288, 2048, 512, 8, 64
    layer = Layer(E, H, I, dev, copies=1, seed=SEED + 9000)
    W13, W2 = layer.W13[0], layer.W2[0]
    cache = C.LayerCache(0, C.to_host(W13.wq), C.to_host(W2.wq), W13.wsr, W2.wsr, 2 * I, H, H, I, S)
    ex = R9700Mxfp4Experts.standalone(cache.h_s13, cache.h_s2)
    ex.r9k_cache = cache
    g = torch.Generator(device=dev).manual_seed(SEED + 9001)
    out = {"slots": S, "bytes_per_expert": layer.bytes_per_expert()}

    def timed(fns, n):
        """ms per apply over a graph of the applies in `fns`, replayed n times."""
        for _ in range(2):
            for fn in fns:
                fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for fn in fns:
                fn()
        gr.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            gr.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (n * len(fns))

    # the hit step's other three layers: caches of their own (arena, LRU state) over the same host store
    hit_layers = [(ex, cache)]
    for i in range(1, HIT_LAYERS):
        c = C.LayerCache(i, cache.h_w13, cache.h_w2, W13.wsr, W2.wsr, 2 * I, H, H, I, S)
        e = R9700Mxfp4Experts.standalone(c.h_s13, c.h_s2)
        e.r9k_cache = c
        hit_layers.append((e, c))

    for name, T, ids_fn in (("hit_T1", 1, lambda: torch.arange(8, dtype=torch.int32, device=dev).view(1, 8)),
                            ("wide_T64", 64, None)):
        x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
        logits = torch.randn(T, E, generator=g, device=dev).to(torch.bfloat16)
        w, ids = K.moe_topk(logits, topk, True)
        if ids_fn is not None:
            ids = ids_fn()
        o = torch.empty(T, H, dtype=torch.bfloat16, device=dev)

        def apply(e, c):
            return lambda: e.apply(o, x, c.h_w13, c.h_w2, w, ids, "silu", E, None, None, None, None, None, None, False)
        fns = [apply(e, c) for e, c in hit_layers] if T == 1 else [apply(ex, cache)]
        ms = timed(fns, steps if T == 1 else max(4, steps // 10))
        distinct = int(torch.unique(ids).numel())
        resident = int((cache.table[ids.reshape(-1).long()] >= 0).sum())
        cold = distinct - int((cache.table[torch.unique(ids).long()] >= 0).sum())
        row = {"T": T, "ms_per_step": round(ms, 5), "distinct": distinct, "read_through": cold,
               "layers_a_graph": len(fns)}
        if cold:
            row["host_GBps"] = round(cold * layer.bytes_per_expert() / (ms * 1e-3) / 1e9, 1)
        out[name] = row
        print(f"# cache {name}: {ms * 1e3:.1f} us/layer, {distinct} experts, {cold} read through from host, "
              f"{resident} of {ids.numel()} rows resident", file=sys.stderr, flush=True)
    # the same wide step with cold staging (R9K_STAGE_COLD=1): the cold experts gathered into a VRAM staging area in
    # one bulk copy, then the cold pass over that copy instead of reading host memory inside the GEMMs
    os.environ["R9K_STAGE_COLD"] = "1"
    try:
        sc = C.LayerCache(0, cache.h_w13, cache.h_w2, W13.wsr, W2.wsr, 2 * I, H, H, I, S)
    finally:
        del os.environ["R9K_STAGE_COLD"]
    exs = R9700Mxfp4Experts.standalone(sc.h_s13, sc.h_s2)
    exs.r9k_cache = sc
    ms = timed([lambda: exs.apply(o, x, sc.h_w13, sc.h_w2, w, ids, "silu", E, None, None, None, None, None, None,
                                  False)], max(4, steps // 10))
    out["wide_T64_staged"] = {"T": 64, "ms_per_step": round(ms, 5), "staged": int(sc.stage_n.item())}
    print(f"# cache wide_T64 staged: {ms * 1e3:.1f} us/layer, {out['wide_T64_staged']['staged']} experts staged "
          f"into VRAM first", file=sys.stderr, flush=True)
    del exs, sc
    miss = torch.stack([torch.arange(100, 164, dtype=torch.int32), torch.arange(0, 64, dtype=torch.int32)], 1)
    cache.miss[:64].copy_(miss.to(dev))
    cache.n_miss.fill_(64)
    ms = timed([cache._gather], 10)
    cache.n_miss.zero_()
    nbytes = 64 * sum(cache.bytes)
    out["gather_64"] = {"ms": round(ms, 4), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes}
    print(f"# cache gather of 64 experts: {ms * 1e3:.0f} us, {out['gather_64']['GBps']} GB/s host -> HBM",
          file=sys.stderr, flush=True)
    del ex, cache, layer, hit_layers
    torch.cuda.empty_cache()
    return out


def router_times(dev, reps_bytes: int = 512 << 20):
    """The router gate GEMM (r9k_router_gemm via router.router_gemm, bf16 out) beside stock's F.linear, kernel time
    alone: back-to-back launches in one HIP graph cycling through enough weight copies (>= 512 MB, twice the Infinity
    Cache) that every launch reads its weight from HBM, HIP events on the stream around the replay. Shapes: config 2's
    gate (E=288, hidden 2048) and the reference's Flash-Next gate (E=512, hidden 2560) at decode widths."""
    from r9700_vllm import router as R
    g = torch.Generator(device=dev).manual_seed(SEED + 77)
    out = []
    for E, H in ((288, 2048), (512, 2560)):
        wbytes = E * H * 2
        copies = -(-reps_bytes // wbytes)
        ws = [(torch.randn(E, H, generator=g, device=dev) * 0.05).to(torch.bfloat16) for _ in range(copies)]
        for M in (1, 8, 32):
            x = torch.randn(M, H, generator=g, device=dev).to(torch.bfloat16)
            row = {"E": E, "hidden": H, "M": M}
            for name, fn in (("r9k", lambda w: R.router_gemm(x, w, True)),
                             ("stock", lambda w: torch.nn.functional.linear(x, w))):
                for w in ws[:4]:
                    fn(w)
                torch.cuda.synchronize()
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    for w in ws:
                        fn(w)
                gr.replay()
                torch.cuda.synchronize()
                s = torch.cuda.current_stream()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(s)
                gr.replay()
                b.record(s)
                torch.cuda.synchronize()
                row[f"{name}_us"] = round(a.elapsed_time(b) * 1e3 / copies, 3)
                del gr
            nbytes = wbytes + M * H * 2 + M * E * 2
            row["r9k_GBps"] = round(nbytes / (row["r9k_us"] * 1e-6) / 1e9, 1)
            row["speedup_vs_stock"] = round(row["stock_us"] / row["r9k_us"], 3)
            out.append(row)
            print(f"# router E={E} H={H} M={M}: {row['r9k_us']} us (stock F.linear {row['stock_us']} us)",
                  file=sys.stderr, flush=True)
        del ws
    return {"kernel": "r9k_router_gemm (bf16 out)", "shapes": out}


CALIB_BYTES = 256 << 20
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "moe_decode_t64_pmc_traffic.md")


def calib_copy(dev) -> None:
    """One plain elementwise copy of known size (CALIB_BYTES read, CALIB_BYTES written; torch's neg kernel on fp32),
    outside every timed region: the reference the PMC byte counters (FETCH_SIZE, WRITE_SIZE) are scaled by when the
    traffic profile is made from this script."""
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()


def copy_rate_gbs(dev, nbytes: int = 512 << 20, reps: int = 10) -> float:
    """Bytes moved per second (read + write) by a plain device-to-device copy of `nbytes`, over 4 rotating buffer
    pairs (2 GiB in all, past the 256 MB Infinity Cache): the practical ceiling of a kernel whose traffic is half reads
    and half writes, the mix of the prefill layer's intermediates."""
    src = [torch.ones(nbytes // 4, dtype=torch.float32, device=dev) for _ in range(4)]
    dst = [torch.empty_like(t) for t in src]
    k = [0]

    def one():
        i = k[0] % 4
        dst[i].copy_(src[i])
        k[0] += 1
    ms = events_ms(one, reps)
    del src, dst
    torch.cuda.empty_cache()
    return 2 * nbytes / (ms * 1e-3) / 1e9


def prefill_dataflow_bytes(T: int, topk: int, H: int, I: int, E: int) -> int:
    """HBM bytes of the routed prefill layer's dataflow, each launch reading its inputs once and writing its outputs
    once (gathered activation rows counted per routed row, as the GEMMs fetch them): routing + quant (logits, x in,
    fp8 codes out), gate_up (weights of every expert, codes, bf16 out), SiLU + quant (bf16 in, codes out), down
    (weights, codes, bf16 rows out) and the weighted top-k sum (rows in, bf16 out)."""
    R = T * topk
    w13 = E * (2 * I * H // 2 + 2 * I * H // 32)
    w2 = E * (H * I // 2 + H * I // 32)
    route = T * E * 2 + T * H * 2 + T * H
    gate_up = w13 + R * H + R * 2 * I * 2
    silu = R * 2 * I * 2 + R * I
    down = w2 + R * I + R * H * 2
    msum = R * H * 2 + T * H * 2
    return route + gate_up + silu + down + msum


def measured_traffic():
    """HBM bytes per r9k_moe_stream_layer launch at T=64 from the committed PMC summary (its line
    'traffic_bytes_per_launch: N'), or None when there is none."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def layer_bytes(step: Step) -> tuple[int, int]:
    """Algorithmic bytes of one layer step (touched-expert weights + x + logits + out) and experts touched."""
    touched = int(torch.unique(step.ids).numel())
    L, T = step.layer, step.T
    return touched * L.bytes_per_expert() + T * L.H * 2 + T * L.E * 2 + T * L.H * 2, touched


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(step: Step, budget_s: float = 10.0) -> dict:
    """The oracle's CPU layer (route, quant, per-expert dequant + fp32 matmul, SiLU quant, down, sum) on this host's
    cores, on the first tokens of the same workload; tokens/s."""
    from oracle import oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    L = step.layer
    T = step.T
    x, logits = step.x_cpu, step.logits_cpu
    ids = O.route(logits, step.topk, True)[1]
    need = np.unique(ids)
    p13 = {int(e): L.p13[int(e)].cpu() for e in need}
    e13 = {int(e): L.e13[int(e)].cpu() for e in need}
    p2 = {int(e): L.p2[int(e)].cpu() for e in need}
    e2 = {int(e): L.e2[int(e)].cpu() for e in need}
    n, t0 = 0, time.perf_counter()
    while True:
        O.moe_layer(x, logits, (p13, e13), (p2, e2), step.topk, True)
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s or n >= 30:
            break
    return {"value": round(n * T / el, 3), "unit": "tokens/s", "cores": threads, "cpu_model": cpu_model(),
            "kind": "port",
            "sample": f"{n} full layer forward(s) of the T={T} workload (E={L.E}, H={L.H}, I={L.I}, top-{step.topk}),"
                      f" oracle dequant-then-matmul in fp32 on {threads} host threads, {el:.1f} s"}


def _budget_loop(fn, budget_s: float, max_n: int = 30):
    """Calls fn() until budget_s seconds have passed (at least once); (calls, seconds)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s or n >= max_n:
            return n, el


def cpu_layer_sample(step: Step, ntok: int, budget_s: float = 6.0) -> dict:
    """The oracle's CPU layer on the first `ntok` tokens of a step's workload (the reference's CPU path: per-token
    quant, per-expert dequant + fp32 matmul, SiLU quant, down, sum); tokens/s of that batch."""
    from oracle import oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    L = step.layer
    x, logits = step.x_cpu[:ntok], step.logits_cpu[:ntok]
    ids = O.route(logits, step.topk, True)[1]
    need = np.unique(ids)
    w = [{int(e): t[int(e)].cpu() for e in need} for t in (L.p13, L.e13, L.p2, L.e2)]
    n, el = _budget_loop(lambda: O.moe_layer(x, logits, (w[0], w[1]), (w[2], w[3]), step.topk, True), budget_s)
    return {"value": round(n * ntok / el, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the first {ntok} of the step's {step.T} tokens as one batch ({len(need)} experts touched), "
                      f"{n} forward(s) in {el:.1f} s, oracle dequant-then-matmul in fp32"}


def cpu_cfg1(dev, budget_s: float = 3.0) -> dict:
    """BASELINE config 1 on the GPU (ops.mxfp4_linear, [16, 2048] x [1024, 2048]) and on the reference's CPU torch
    path (the oracle's per-token fp8 quant, MXFP4 dequant, fp32 matmul)."""
    from oracle import oracle as O
    from r9700_vllm import ops
    from r9700_vllm.kernels import moe as K
    M, N, Kd = 16, 1024, 2048
    g = torch.Generator().manual_seed(SEED + 1000)
    packed = torch.randint(0, 256, (N, Kd // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    e8 = torch.randint(118, 127, (N, Kd // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    x = torch.randn(M, Kd, generator=g).to(torch.bfloat16)
    W = K.prepare_mxfp4_weights(packed.unsqueeze(0).to(dev), e8.unsqueeze(0).to(dev))
    xd = x.to(dev)
    for _ in range(2):
        ops.mxfp4_linear(xd, W.wq, W.wsr, N, Kd)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()                               # 20 calls a replay: the launches' own time
    with torch.cuda.graph(gr):
        for _ in range(20):
            ops.mxfp4_linear(xd, W.wq, W.wsr, N, Kd)
    gpu_ms = events_ms(gr.replay, 10) / 20
    del gr
    threads = os.cpu_count() or 1

    def cpu_call():
        q, sc = O.quant_rows_fp8(x)
        O.grouped_gemm(q, sc, {0: O.mxfp4_dequant(packed, e8, torch.float32)}, np.zeros(M, dtype=np.int32), 1,
                       acc_dtype=torch.float32)
    n, el = _budget_loop(cpu_call, budget_s)
    return {"workload": "cfg1 dense MXFP4 linear [16, 2048] x [1024, 2048]", "gpu_us": round(gpu_ms * 1e3, 2),
            "cpu": {"value": round(el / n * 1e6, 1), "unit": "us per call", "cores": threads, "kind": "port",
                    "sample": f"{n} whole calls (quant, dequant, fp32 matmul) in {el:.1f} s"}}


def cpu_cfg4(packed, s16, mp, me, g, dev, budget_s: float = 4.0) -> dict:
    """BASELINE config 4 on the reference's CPU path: the NVFP4 -> MXFP4 conversion (oracle restatement of the
    reference's torch converter) on a 512-row sample, scaled to the [17408, 5120] matrix; the GEMM as the CPU path
    runs it per call (quant, dequant of the whole weight, fp32 matmul) at M = 1, 4, 16 and, on 256 of its rows, 4096."""
    from oracle import oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    N, Kd = packed.shape[0], packed.shape[1] * 2
    rows = 512
    p_s, s_s = packed[:rows].cpu().numpy(), s16[:rows].view(torch.uint8).cpu().numpy()
    div = np.ones(rows, dtype=np.float32)
    n, el = _budget_loop(lambda: O.nvfp4_to_mxfp4(p_s, s_s, div), budget_s)
    conv_ms = el / n * 1e3 * N / rows
    wp, we = mp.cpu(), me.cpu()
    t0 = time.perf_counter()
    Wd = O.mxfp4_dequant(wp, we, torch.float32)
    deq_ms = (time.perf_counter() - t0) * 1e3
    gemm = {}
    for M in (1, 4, 16, 4096):
        m = min(M, 256)
        x = torch.randn(m, Kd, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16)

        def mm():
            q, sc = O.quant_rows_fp8(x)
            return (O.e4m3_dequant(q, torch.float32) @ Wd.T) * torch.from_numpy(sc)[:, None]
        n, el = _budget_loop(mm, budget_s / 4)
        gemm[str(M)] = round(deq_ms + el / n * 1e3 * M / m, 1)
    return {"convert_ms": round(conv_ms, 1), "gemm_ms_per_call": gemm, "dequant_ms": round(deq_ms, 1),
            "cores": threads, "kind": "port",
            "sample": f"conversion on {rows} of {N} rows scaled by {N / rows:.1f}; GEMM = one whole-weight dequant "
                      f"({deq_ms:.0f} ms) + quant and fp32 matmul, M = 4096 timed on 256 rows and scaled by 16"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    from r9700_vllm.kernels import moe as K
    K.lib()
    topk = 8
    t_build = time.perf_counter()
    layer = Layer(288, 2048, 512, dev)
    print(f"# weights ready ({COPIES} copies, {time.perf_counter() - t_build:.1f} s)", file=sys.stderr, flush=True)

    sweep = {}
    main_step = None
    for T in (1, 8, 16, 64):
        st = Step(layer, T, topk, dev, SEED + 2000 + T)
        # the headline point (T = 64) is exactly --steps steps in one window; the others a median of 5 windows
        ms, n = (graph_time(st, args.steps, args.warmup) if T == 64
                 else graph_time(st, max(40, args.steps), args.warmup, windows=5))
        nbytes, touched = layer_bytes(st)
        sweep[str(T)] = {"ms_per_step": round(ms, 5), "tokens_per_s": round(T / (ms * 1e-3), 1),
                         "experts_touched": touched, "layer_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        print(f"# T={T}: {ms * 1e3:.1f} us/layer, {sweep[str(T)]['layer_GBps']} GB/s over {touched} experts",
              file=sys.stderr, flush=True)
        if T == 64:
            main_step, main_ms, main_n = st, ms, n

    calib_copy(dev)
    k_ms, k_bytes, k_flops, k_touched = layer_kernel_time(main_step)
    k_gbs = k_bytes / (k_ms * 1e-3) / 1e9
    print(f"# stream layer launch alone: {k_ms * 1e3:.1f} us, {k_gbs:.0f} GB/s", file=sys.stderr, flush=True)

    prefill = None
    if not args.no_prefill:
        pl = Step(layer, 8192, topk, dev, SEED + 3000 + 8192)
        ms, n = graph_time(pl, 8, max(4, args.warmup // 4), windows=5)
        flops = 6 * 8192 * topk * layer.H * layer.I
        tf = flops / (ms * 1e-3) / 1e12
        pl_cpu = None if args.no_cpu else cpu_layer_sample(pl, 256)
        del pl
        torch.cuda.empty_cache()
        db = prefill_dataflow_bytes(8192, topk, layer.H, layer.I, layer.E)
        cgbs = copy_rate_gbs(dev)
        prefill = {"workload": "cfg3 prefill T=8192", "ms_per_step": round(ms, 4), "tokens_per_s": round(8192 / (ms * 1e-3)),
                   "TFLOPS": round(tf, 1), "frac_fp4_peak": round(tf / FP4_PEAK_TFLOPS, 4),
                   "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4), "steps": n,
                   "dataflow": {"what": "HBM bytes of the layer's launches (each input read once, each output written "
                                        "once) / ms_per_step, against a measured device copy (read + write)",
                                "bytes": db, "achieved_GBps": round(db / (ms * 1e-3) / 1e9, 1),
                                "copy_GBps": round(cgbs, 1), "frac_copy": round(db / (ms * 1e-3) / 1e9 / cgbs, 4)},
                   "cpu": pl_cpu}
        print(f"# prefill T=8192: {ms:.3f} ms/layer, {tf:.1f} TFLOPS; dataflow {db / 1e9:.3f} GB at "
              f"{db / (ms * 1e-3) / 1e12:.2f} TB/s (device copy {cgbs / 1e3:.2f} TB/s)", file=sys.stderr, flush=True)

    router = None if args.no_router else router_times(dev)
    cfg4 = None if args.no_cfg4 else cfg4_lines(dev, cpu=not args.no_cpu)
    cfg5 = None if args.no_cfg5 else cfg5_lines(dev, args.steps, args.warmup, cpu=not args.no_cpu)
    cfg1 = None if args.no_cpu else cpu_cfg1(dev)
    cache = None if args.no_cache else cache_lines(dev, args.steps)
    cpu = None if args.no_cpu else cpu_baseline(main_step)
    line = {
        "metric": "MoE-layer tokens/s + HBM GB/s (decode) / MXFP4 TFLOPS (prefill), 1 GPU",
        "value": sweep["64"]["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": main_n,
        "warmup": args.warmup,
        "ms_per_step": sweep["64"]["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 x mxfp4 (fp32 accumulate)",
        "data": "synthetic (seeded random e2m1 codes, e8m0 in [118,126], N(0,1) tokens and router logits)",
        "config": {"workload": "cfg2 decode MoE layer: E=288, hidden 2048, intermediate 512, top-8, T=64 tokens",
                   "tokens": 64, "experts": 288, "hidden": 2048, "intermediate": 512, "topk": 8,
                   "weight_copies_rotated": COPIES},
        "roofline": {"bound": "hbm", "kernel": "r9k_moe_stream_layer (gate_up + SiLU + quant + down, T=64)",
                     "achieved": round(k_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(k_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "traffic_source": "not measured in this run: the committed PMC summary "
                                       "profiles/moe_decode_t64_pmc_traffic.md (rocprofv3 --pmc FETCH_SIZE, then "
                                       "WRITE_SIZE, scaled by this script's 256 MiB calibration copy)",
                     "kernel_us": round(k_ms * 1e3, 2), "bytes_per_launch": k_bytes,
                     "layer": {"what": "whole T=64 layer (all launches), algorithmic bytes / ms_per_step",
                               "achieved": sweep["64"]["layer_GBps"], "frac": sweep["64"]["hbm_frac"]}},
        "cpu_baseline": cpu,
        "cfg1": cfg1,
        "decode_sweep": sweep,
        "prefill": prefill,
        "router": router,
        "cfg4": cfg4,
        "cfg5": cfg5,
        "expert_cache": cache,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
