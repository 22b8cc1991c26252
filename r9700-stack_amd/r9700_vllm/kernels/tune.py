"""Sweep of the decode GEMM's launch shapes on this GPU, writing the launch table kernels/tuned.py reads.

    python -m r9700_vllm.kernels.tune [--out PATH] [--reps 20]

For each dense product (N, K) in SHAPES and each row count M in MS (the rows between the dense weight stream's 16 and
the prefill kernel's 128, where ops.mxfp4_gemm_q runs r9k_moe_mxfp4a8 over identity tables), every built launch
shape (WV, SK, NPW in {1, 2, 4}, those legal_cfg accepts) and the kernel's own choice (0, 0, 0) are timed: a HIP
graph of `reps` launches cycling through enough weight copies to exceed the 256 MB Infinity Cache, HIP events around
its replay. The fastest shape is written with its time and the kernel's own choice's, so the table records how much
each entry gains.
"""
from __future__ import annotations

import argparse
import datetime
import itertools
import json
import sys

import torch

SHAPES = ((1024, 2048), (17408, 5120), (2048, 2048), (4096, 4096))
MS = (17, 24, 32, 48, 64, 96, 127)


def time_shape(N: int, K: int, M: int, cfgs, reps: int) -> dict:
    from .. import ops
    from . import moe as KM
    dev = torch.device("cuda", torch.cuda.current_device())
    g = torch.Generator(device=dev).manual_seed(N * 7 + K)
    packed = torch.randint(0, 256, (1, N, K // 2), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    e8 = torch.randint(118, 127, (1, N, K // 32), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    W0 = KM.prepare_mxfp4_weights(packed, e8)
    wbytes = N * K // 2 + N * K // 32
    copies = max(2, min(64, -(-(512 << 20) // wbytes)))
    Ws = [W0] + [KM.Mxfp4Experts(W0.wq.clone(), W0.wsr.clone(), N, K) for _ in range(copies - 1)]
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    q, s = KM.quant_rows_fp8(x)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    MT = ops._decode_mt(M)
    tabs = ops.IdentityTables.get(dev, M, KM.MOE_BLOCK * MT)
    res = {}
    for cfg in cfgs:
        def launch(i):
            KM.moe_gemm(q, s, Ws[i % copies], out, *tabs, M, 1, None, *cfg, num_experts=1, MT=MT)
        for i in range(2):
            launch(i)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(reps):
                launch(i)
        gr.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = float("inf")
        for _ in range(3):
            a.record()
            gr.replay()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3 / reps)
        res[cfg] = best
        del gr
    del Ws, W0
    torch.cuda.empty_cache()
    return res


def main(argv=None) -> int:
    from . import moe as KM
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default="tuned.json")
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("tune: needs a GPU", file=sys.stderr)
        return 1
    entries = []
    for N, K in SHAPES:
        for M in MS:
            cands = [(0, 0, 0)] + [c for c in itertools.product(KM.BUILT_KNOBS, repeat=3)
                                   if KM.legal_cfg(c, N, K, MT=KM.decode_mt(M)) == c]
            res = time_shape(N, K, M, cands, args.reps)
            cfg, us = min(res.items(), key=lambda kv: kv[1])
            entries.append({"kind": "mxfp4", "N": N, "K": K, "M": M, "cfg": list(cfg), "us": round(us, 2),
                            "auto_us": round(res[(0, 0, 0)], 2)})
            print(f"N={N} K={K} M={M}: best {cfg} {us:.2f} us (kernel's own choice {res[(0, 0, 0)]:.2f} us)",
                  flush=True)
    doc = {"device": torch.cuda.get_device_properties(0).name,
           "arch": getattr(torch.cuda.get_device_properties(0), "gcnArchName", ""),
           "source": "python -m r9700_vllm.kernels.tune (r9k_moe_mxfp4a8 over identity tables; graph of "
                     f"{args.reps} launches over rotating weight copies; best of 3 replays)",
           "date": datetime.date.today().isoformat(), "torch": torch.__version__, "entries": entries}
    with open(args.out, "w") as f:
        json.dump(doc, f, indent=1)
    print(f"wrote {len(entries)} entries to {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
