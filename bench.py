"""DSA decode layer-step benchmark on one MI355X (gfx950).

A step is one layer of the DSA decode path over the batch: lightning indexer over every cached token -> exact
top-2048 per row -> sparse MLA attention over the selected FP8 rows, all three as HIP kernels of libdsa_gfx950.so on
one stream, with every input resident in HBM before the timed region. The workload is BASELINE.json's main decode
shape (config 2: B=8 sequences x 32,768 tokens, 64 query heads of 512 latent + 64 rope, 64 indexer heads x 128, FP8
e4m3 paged caches with per-token fp32 scales, pages of 64, top-2048), synthetic seeded data.

Prints ONE JSON line: the layer-step rate (value), the roofline of the dominant kernel (the indexer: its algorithmic
bytes per launch over its HIP-event-timed average duration) and the CPU baseline (the oracle's torch restatement of
the reference arithmetic, timed on this host's cores on a bounded sample of the same workload).

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--config 2] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s


def _indexer_bytes(lengths, Hi, page_size=64):
    """Algorithmic bytes of one indexer launch: its inputs once (FP8 key 128 B + fp32 scale 4 B per token, the page
    table, the bf16 indexer queries and fp32 head weights); the scores it writes are an intermediate of the layer and
    are not counted."""
    return sum(132 * L + 4 * -(-L // page_size) + 256 * Hi + 4 * Hi for L in lengths)


def cpu_baseline(inp, budget_s: float = 15.0) -> dict:
    """The oracle (oracle/dsa_oracle.py, torch fp32 on the host) run on whole layer-steps of the same inputs, as many
    as fit in about budget_s seconds (at least one)."""
    import torch

    from oracle import dsa_oracle as O

    cores = min(len(os.sched_getaffinity(0)), 16)  # the box's CPU share for one GPU
    torch.set_num_threads(cores)
    cpu = inp.to("cpu")
    O.decode_layer_ref(cpu)  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        O.decode_layer_ref(cpu)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or n >= 50:
            break
    model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": n / dt, "unit": "layer-steps/s", "cores": cores, "kind": "port",
            "sample": f"{n} full layer-steps of the same workload (indexer + top-k + attention, torch fp32, "
                      f"{dt:.1f} s, {cores} threads on {model or 'the host CPU'})"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} is not supported (each sequence's decode is "
              f"independent, so N GPUs would run N independent batches)", file=sys.stderr)
        return 2

    import torch

    from trnrt_amd import _lib
    from trnrt_amd import workloads as W
    from trnrt_amd.kernels import _common as C
    from trnrt_amd.kernels.dsa_layer import DecodeLayer

    cfg = W.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = W.make_inputs(cfg, seed=0, device=dev)
    layer = DecodeLayer(cfg.B, cfg.Hi, cfg.H, inp.max_pages, cfg.page_size, inp.num_pages, cfg.keep, cfg.scale,
                        max_len=max(inp.lengths), splits=args.splits, device=dev)
    g = inp
    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream

    def step():
        layer.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len,
                   check=False)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # the timed region: exactly `steps` layer-steps
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps

    # per-kernel HIP events on the launch stream over the same number of steps, the three operators called one by
    # one (the same kernels dsa_decode_layer enqueues)
    stride = layer.stride
    ws = layer.workspace
    from trnrt_amd._lib import workspace_bytes

    t_need = workspace_bytes(_lib.DSA_WS_TOPK, cfg.B, cfg.H, cfg.keep, layer.max_len)
    t_need = (t_need + 255) // 256 * 256
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    for i in range(args.steps):
        e = evs[i]
        e[0].record(stream)
        st = lib.dsa_indexer_decode(g.q_idx.data_ptr(), g.w_k.data_ptr(), g.k_cache.data_ptr(), g.k_scale.data_ptr(),
                                    g.table.data_ptr(), g.ctx_len.data_ptr(), None, layer.scores.data_ptr(), cfg.B,
                                    cfg.Hi, 128, inp.max_pages, cfg.page_size, inp.num_pages, stride, sp)
        e[1].record(stream)
        st |= lib.dsa_topk(layer.scores.data_ptr(), g.ctx_len.data_ptr(), layer.idx.data_ptr(), layer.cnt.data_ptr(),
                           ws.data_ptr(), t_need, cfg.B, stride, layer.max_len, cfg.keep, 1, sp)
        e[2].record(stream)
        st |= lib.dsa_sparse_mla_decode(g.q.data_ptr(), g.kv_cache.data_ptr(), g.kv_scale.data_ptr(),
                                        layer.idx.data_ptr(), layer.cnt.data_ptr(), g.table.data_ptr(), None, None,
                                        layer.out.data_ptr(), None, layer.lse.data_ptr(), ws.data_ptr() + t_need,
                                        ws.numel() - t_need, cfg.B, cfg.H, 576, 512, cfg.keep, inp.max_pages,
                                        cfg.page_size, inp.num_pages, cfg.scale, args.splits, sp)
        e[3].record(stream)
        if st:
            raise RuntimeError(f"launch status {st}")
    torch.cuda.synchronize()
    k_ms = [sum(e[j].elapsed_time(e[j + 1]) for e in evs) / args.steps for j in range(3)]

    lengths = inp.lengths
    idx_bytes = _indexer_bytes(lengths, cfg.Hi, cfg.page_size)
    achieved = idx_bytes / (k_ms[0] * 1e-3) / 1e9
    layer_bytes = W.algorithmic_bytes(lengths, cfg.H, cfg.Hi, cfg.keep, cfg.page_size)
    layer_gbs = layer_bytes / (ms * 1e-3) / 1e9

    out = {
        "metric": "DSA decode layer-steps/sec at B=8, 32K ctx; achieved HBM GB/s (% of 8 TB/s)",
        "value": round(1e3 / ms, 1),
        "unit": "layer-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"config {args.config}: {cfg.name}", "batch": cfg.B, "context": max(lengths),
                   "q_heads": cfg.H, "indexer_heads": cfg.Hi, "keep": cfg.keep, "page_size": cfg.page_size,
                   "kv": "fp8 e4m3 [576] + fp32 scale per token", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "indexer_decode_kernel", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "algorithmic_bytes": idx_bytes, "avg_ms": round(k_ms[0], 5)},
        "layer": {"algorithmic_bytes": layer_bytes, "achieved_GBs": round(layer_gbs, 1),
                  "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                  "kernel_ms": {"indexer": round(k_ms[0], 5), "topk": round(k_ms[1], 5),
                                "attention": round(k_ms[2], 5)}},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(inp)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
