"""DSA decode layer-step benchmark on one MI355X (gfx950).

A step is one layer of the DSA decode path over the batch: lightning indexer over every cached token -> exact
top-2048 per row -> sparse MLA attention over the selected FP8 rows, as HIP kernels of libdsa_gfx950.so on one
stream, with every input resident in HBM before the timed region. The workload is BASELINE.json's main decode
shape (config 2: B=8 sequences x 32,768 tokens, 64 query heads of 512 latent + 64 rope, 64 indexer heads x 128, FP8
e4m3 paged caches with per-token fp32 scales, pages of 64, top-2048), synthetic seeded data.

Prints ONE JSON line: the layer-step rate (value), the roofline of the dominant kernel and the CPU baseline (the
oracle's torch restatement of the reference arithmetic, timed on this host's cores on a bounded sample of the same
workload, each operator's median reported beside the step's). Rows of up to 32,768 tokens run as one launch per
8 rows (decode_fused_kernel: the whole layer), so its roofline is the layer's algorithmic bytes over that kernel's
HIP-event-timed duration; longer rows run the separate kernels, whose roofline is the indexer's. layer.step_us gives
the median, p10 and p90 of single steps, each timed by a pair of events around it.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--config 2] [--no-cpu-baseline]
    python bench.py --chain             # config 2 through the separate kernels (dsa_decode_layer_chain)
    python bench.py --config 5          # the chunked-prefill step (65,536 cached + 2,048 new queries): its own line
    python bench.py --config 6          # the pooled (GLM-5.3-Flash, kpool 4) decode step at B=8 x 32K: its own line
    python bench.py --config 7          # the pooled (GLM) chunked-prefill step (65,536 cached + 2,048 new queries)
    python bench.py --copy-probe 512    # plain device copies of 512 MiB: the calibration run for HBM counters

roofline.traffic (HBM bytes per launch of the roofline's kernel) comes from rocprofv3 FETCH_SIZE / WRITE_SIZE counter runs of this
script, each scaled by the same counter's reading for the --copy-probe kernels; the measured figures are kept in
profiles/traffic.json and reported when they were taken on the same workload.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense fp8 MFMA
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def copy_probe(mib: int) -> int:
    """Device-to-device copies of known size for calibrating the HBM byte counters: torch's copy_ of mib MiB and an
    elementwise kernel of the same size (neg, fp32), 5 launches each; each reads and writes mib MiB."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n * 4, "copy_probe_bytes_written": n * 4, "launches": 5}), flush=True)
    return 0


def measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload` from profiles/traffic.json (counter runs), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    ent = rec.get(kernel)
    if not ent or ent.get("workload") != workload:
        return None
    return ent.get("bytes_per_launch")


def _indexer_bytes(lengths, Hi, page_size=64):
    """Algorithmic bytes of one indexer launch: its inputs once (FP8 key 128 B + fp32 scale 4 B per token, the page
    table, the bf16 indexer queries and fp32 head weights); the scores it writes are an intermediate of the layer and
    are not counted."""
    return sum(132 * L + 4 * -(-L // page_size) + 256 * Hi + 4 * Hi for L in lengths)


def _host_model() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "the host CPU"


def _cpu_threads() -> int:
    """The host threads a CPU baseline uses: every core of this process's affinity set, capped at 16 (a one-GPU box's
    CPU share; its affinity set may list the whole machine's cores)."""
    return min(len(os.sched_getaffinity(0)), 16)


def cpu_baseline(inp, budget_s: float = 15.0) -> dict:
    """The oracle (oracle/dsa_oracle.py, torch fp32 on the host) run on whole layer-steps of the same inputs, as many
    as fit in about budget_s seconds (at least three), each operator timed on its own: value = 1 / the median step;
    ops_median_s = each operator's median."""
    import torch

    from oracle import dsa_oracle as O

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    cpu = inp.to("cpu")
    cfg = cpu.cfg
    stride = cpu.max_pages * cfg.page_size

    def one():
        t = [time.perf_counter()]
        sc = O.indexer_ref(cpu.q_idx, cpu.w_k, cpu.k_cache, cpu.k_scale, cpu.table, cpu.ctx_len, cfg.page_size, stride)
        t.append(time.perf_counter())
        idx, cnt = O.topk_ref(sc, cfg.keep, cpu.ctx_len)
        t.append(time.perf_counter())
        O.sparse_mla_ref(cpu.q, cpu.kv_cache, cpu.kv_scale, idx, cnt, cpu.table, cfg.page_size, cfg.scale)
        t.append(time.perf_counter())
        return [t[i + 1] - t[i] for i in range(3)]

    one()  # warm-up
    rows, t0 = [], time.perf_counter()
    while True:
        rows.append(one())
        dt = time.perf_counter() - t0
        if (dt >= budget_s and len(rows) >= 3) or len(rows) >= 5000:
            break

    def med(v):
        v = sorted(v)
        return v[len(v) // 2]

    step = med([sum(r) for r in rows])
    ops = {name: round(med([r[i] for r in rows]), 6) for i, name in enumerate(("indexer", "topk", "sparse_mla"))}
    return {"value": round(1.0 / step, 3), "unit": "layer-steps/s", "cores": cores, "kind": "port",
            "ops_median_s": ops,
            "sample": f"{len(rows)} full layer-steps of the same workload (indexer + top-k + attention, torch fp32, "
                      f"{dt:.1f} s, {cores} threads = this process's affinity set capped at 16 on {_host_model()}); "
                      f"value = 1 / the median step"}


def kernel_times(lib, step, steps: int, pairs: int = 32) -> dict:
    """{kernel name: average device duration in us} of the kernels one call of step() launches (summed over the
    launches of one name, e.g. a tiled selection's per-tile kernels), each timed by a pair of HIP events that the
    runtime records at the kernel's own start and end (dsa_timing_begin; at most 32 launches per step)."""
    import ctypes

    import torch

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    evs = []
    for _ in range(2 * pairs * steps):
        e = ctypes.c_void_p()
        if hip.hipEventCreate(ctypes.byref(e)) != 0:
            raise RuntimeError("hipEventCreate failed")
        evs.append(e)
    arrs = [(ctypes.c_void_p * (2 * pairs))(*[e.value for e in evs[2 * pairs * i: 2 * pairs * (i + 1)]])
            for i in range(steps)]
    names, n = [], 0
    for i in range(steps):
        lib.dsa_timing_begin(arrs[i], pairs)
        try:
            step()
        finally:
            n = lib.dsa_timing_end()
        if i == 0:
            names = [lib.dsa_timing_kernel_name(k).decode() for k in range(min(n, pairs))]
    torch.cuda.synchronize()
    tot: dict = {}
    ms = ctypes.c_float()
    for i in range(steps):
        for k, name in enumerate(names):
            if hip.hipEventElapsedTime(ctypes.byref(ms), arrs[i][2 * k], arrs[i][2 * k + 1]) != 0:
                raise RuntimeError("hipEventElapsedTime failed")
            tot[name] = tot.get(name, 0.0) + ms.value * 1e3
    for e in evs:
        hip.hipEventDestroy(e.value)
    return {k: v / steps for k, v in tot.items()}


def step_times(step, steps: int) -> list:
    """Each of `steps` calls of step() timed on its own by a pair of torch CUDA events on the current stream (the
    stream the library launches on), in us."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record()
        step()
        b.record()
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e3 for a, b in evs]


def graph_step_us(step, steps: int, per_graph: int = 8) -> float:
    """The same step replayed from a HIP graph (torch.cuda.CUDAGraph) that captures `per_graph` steps: us per step
    over `steps` steps of replays, between a pair of events. The step allocates nothing and issues no memset, so its
    capture replays the eager launches (tests/test_gpu_graph.py checks replays against eager steps)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            step()
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * per_graph)


def percentiles(v) -> dict:
    """median, p10 and p90 (nearest rank) of a list of durations."""
    v = sorted(v)
    at = lambda f: v[min(len(v) - 1, int(f * len(v)))]
    return {"median": round(at(0.5), 3), "p10": round(at(0.1), 3), "p90": round(at(0.9), 3)}


def prefill_cpu_baseline(inp, cfg, budget_s: float = 15.0) -> dict:
    """The oracle's chunk step (prefill_scores_ref + topk_ref + sparse_mla_ref, torch fp32 on the host) over whole
    query rows of the same chunk, as many rows as fit in about budget_s seconds; reported as chunks per second
    (rows / 2,048)."""
    import torch

    from oracle import dsa_oracle as O

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    cpu = inp.to("cpu")
    qv = cpu.q_values()  # the queries' values (dequantised when FP8)
    rows, t0, n = 4, time.perf_counter(), 0
    table = cpu.table.view(1, -1).expand(rows, -1)
    while True:
        r0 = (n * rows) % cfg.chunk
        sl = slice(r0, r0 + rows)
        sc = O.prefill_scores_ref(qv[sl], cpu.w[sl], cpu.k8, cpu.k_scale, cpu.npool[sl], cfg.scale)
        idx, cnt = O.topk_ref(sc, cfg.keep)
        O.sparse_mla_ref(cpu.q[sl], cpu.kv_cache, cpu.kv_scale, idx, cnt, table, cfg.page_size, cfg.softmax_scale)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or n * rows >= cfg.chunk:
            break
    done = n * rows
    return {"value": done / cfg.chunk / dt, "unit": "chunks/s", "cores": cores, "kind": "port",
            "sample": f"{done} of the chunk's {cfg.chunk} query rows (scores over {cfg.P} keys + top-{cfg.keep} + "
                      f"sparse MLA over the selection, torch fp32, {dt:.1f} s, {cores} threads)"}


WHOLE_CHUNK_NOTE = ("one launch of the kernel over the whole chunk, timed alone (the step runs the same kernel per "
                    "query tile, tiles alternating between two streams, so per-tile durations overlap)")


def whole_chunk_indexer_us(lib, kname: str, run, steps: int) -> float:
    """Average device duration (us) of kname launched once over the whole chunk by run(), HIP-event timed."""
    import torch

    run()
    torch.cuda.synchronize()
    return kernel_times(lib, run, steps)[kname]


def prefill_main(args) -> int:
    """The chunked-prefill DSA step (config 5): the dense indexer scores of the chunk's queries over the cached + new
    keys, the exact top-2048 of every query row (dsa_long_select.select), and sparse MLA of every query over its
    selected tokens (the token form through the context's page table). roofline: the indexer kernel's algorithmic
    MFMA work (2 Hi D per causal (query, key) pair) over its HIP-event-timed duration; `attention` gives the same for
    the attention kernel (2 H (576 + 512) per selected token; the many-row form, sparse_mla_wide_kernel, at this
    size)."""
    import torch

    from trnrt_amd import _lib
    from trnrt_amd import workloads as W
    from trnrt_amd.kernels import dsa_decode
    from trnrt_amd.kernels import dsa_long_select as LS

    cfg = W.PREFILL_CONFIGS[args.config]
    if args.bf16_queries:
        # the reference's own query precision: bf16 indexer queries (the bf16-query indexer kernel)
        cfg = dataclasses.replace(cfg, q_fp8=False)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = W.make_prefill_inputs(cfg, seed=0, device=dev, attention=True)
    C = cfg.chunk
    wsb = LS.workspace_bytes(C, cfg.P, cfg.keep)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=dev)  # the top-k histograms start (and end) at zero
    wsa_b = _lib.workspace_bytes(_lib.DSA_WS_ATTENTION, C, cfg.H, cfg.keep, 0, 0)
    wsa = torch.zeros(max(wsa_b, 256), dtype=torch.uint8, device=dev)
    table = inp.table.view(1, -1).expand(C, -1).contiguous()  # every query row reads the context's pages
    o = torch.empty(C, cfg.H, cfg.dv, dtype=torch.bfloat16, device=dev)
    lib = _lib.lib()

    def step():
        pools, cnt, _ = LS.select(inp.qI, inp.w, inp.k8, inp.npool, cfg.keep, cfg.scale, pk_scale=inp.k_scale,
                                  qI_scale=inp.qI_scale, workspace=ws)
        dsa_decode.attend_tokens(inp.q, inp.kv_cache, inp.kv_scale, pools, cnt, table, cfg.page_size,
                                 cfg.softmax_scale, out=o, workspace=wsa)

    steps = min(args.steps, 20)
    for _ in range(min(args.warmup, 5)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    k_us = kernel_times(lib, step, steps)
    flops = W.prefill_flops(cfg)
    kname = "indexer_prefill_fp8_kernel" if cfg.q_fp8 else "indexer_prefill_kernel"
    sc_buf = torch.empty(C, cfg.P, dtype=torch.float32, device=dev)
    idx_us = whole_chunk_indexer_us(lib, kname, lambda: LS.scores(
        inp.qI, inp.w, inp.k8, inp.npool, cfg.scale, pk_scale=inp.k_scale, qI_scale=inp.qI_scale, out=sc_buf), steps)
    del sc_buf
    tflops = flops / (idx_us * 1e-6) / 1e12
    att_flops = W.prefill_attention_flops(cfg)
    att_kernel = "sparse_mla_wide_kernel" if "sparse_mla_wide_kernel" in k_us else "sparse_mla_kernel"
    att_us = k_us[att_kernel] + k_us.get("combine_splits_kernel", 0.0)
    att_tflops = att_flops / (att_us * 1e-6) / 1e12
    out = {
        "metric": "DSA chunked-prefill step (indexer + top-2048 + sparse MLA) chunks/sec; indexer MFMA TFLOP/s",
        "value": round(1e3 / ms, 2),
        "unit": "chunks/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": min(args.warmup, 5),
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8" if cfg.q_fp8 else "bf16",
        "data": "synthetic",
        "config": {"workload": f"config {args.config}: {cfg.name}" + (" (bf16 queries)" if args.bf16_queries else ""),
                   "cached": cfg.cached, "chunk": C,
                   "queries": "fp8 e4m3 + fp32 scale per (query, head)" if cfg.q_fp8 else "bf16",
                   "indexer_heads": cfg.Hi, "q_heads": cfg.H, "keep": cfg.keep, "page_size": cfg.page_size,
                   "keys": "fp8 e4m3 [128] + fp32 scale per token", "kv": "fp8 e4m3 [576] + fp32 scale per token",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": kname, "achieved": round(tflops, 1),
                     "peak": FP8_PEAK_TFLOPS if cfg.q_fp8 else BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / (FP8_PEAK_TFLOPS if cfg.q_fp8 else BF16_PEAK_TFLOPS), 4),
                     "bf16_peak_frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "algorithmic_flops": flops, "avg_us": round(idx_us, 3), "measured": WHOLE_CHUNK_NOTE},
        "attention": {"kernel": att_kernel, "avg_us": round(att_us, 3), "achieved": round(att_tflops, 1),
                      "unit": "TFLOP/s", "peak": BF16_PEAK_TFLOPS, "frac": round(att_tflops / BF16_PEAK_TFLOPS, 4),
                      "algorithmic_flops": att_flops},
        "kernel_us": {k: round(v, 3) for k, v in k_us.items()},
        "kernel_us_note": "per step, summed over the launches of one name (the tiles' launches overlap on two streams)",
        "selection_memory": {"workspace_bytes": wsb, "scores": "two query tiles' scores held in the workspace"},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = prefill_cpu_baseline(inp, cfg)
    print(json.dumps(out), flush=True)
    return 0


def pooled_cpu_baseline(inp, cfg, npool, positions, budget_s: float = 15.0) -> dict:
    """The oracle's pooled decode step (indexer_ref over the pool keys + topk_ref + pool_slots_ref +
    sparse_mla_slots_ref, torch fp32 on the host) on rows of the same batch, as many as fit in about budget_s seconds;
    reported as steps per second (rows / B)."""
    import torch

    from oracle import dsa_oracle as O

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    cpu = inp.to("cpu")
    keys = cpu.pool_key.view(-1, cfg.D)
    ones = torch.ones(keys.shape[0])
    ppp = cfg.page_size // cfg.kp
    n, t0 = 0, time.perf_counter()
    while True:
        b = n % cfg.B
        sl = slice(b, b + 1)
        sc = O.indexer_ref(cpu.q_idx[sl], cpu.w[sl], keys, ones, cpu.table[sl], npool[sl], ppp)
        pools, cnt = O.topk_ref(sc, cfg.keep)
        rows, bias = O.pool_slots_ref(pools, cnt, npool[sl], positions[sl], cpu.table[sl], cfg.page_size, cfg.kp,
                                      cfg.keep + 1)
        tok = (rows.unsqueeze(-1) * cfg.kp + torch.arange(cfg.kp)).reshape(1, -1)
        O.sparse_mla_slots_ref(cpu.q[sl], cpu.kv_cache, cpu.kv_scale, tok, bias.reshape(1, -1), cfg.scale)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or n >= 4 * cfg.B:
            break
    return {"value": n / cfg.B / dt, "unit": "layer-steps/s", "cores": cores, "kind": "port",
            "sample": f"{n} query rows of the batch's {cfg.B} (pool scores + top-{cfg.keep} pools + slots + sparse "
                      f"MLA over {cfg.kp * (cfg.keep + 1)} token slots, torch fp32, {dt:.1f} s, {cores} threads)"}


def pooled_main(args) -> int:
    """The pooled (GLM-5.3-Flash) decode step (config 6): the current tokens' pool-key write, then the pooled layer
    (the indexer over the bf16 pool-key cache, the exact top-512 pools, sparse MLA over the selected pools' tokens and
    the tail, over the 512-wide NoPE latent): dsa_pooled_decode_step, one launch; with --chain dsa_pool_keys_write and
    the separate kernels. roofline: the one launch's algorithmic bytes (W.pooled_step_bytes) over its
    HIP-event-timed duration, or with --chain the indexer kernel's."""
    import torch

    from trnrt_amd import _lib
    from trnrt_amd import workloads as W
    from trnrt_amd.kernels import dsa_cache
    from trnrt_amd.kernels.dsa_layer import PooledDecodeLayer

    cfg = W.POOLED_CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = W.make_pooled_inputs(cfg, seed=0, device=dev)
    lib = _lib.lib()
    ps, kp = cfg.page_size, cfg.kp
    pos = inp.positions
    slot_mapping = dsa_cache.slots_of(pos, inp.table, ps)
    npool_d = torch.div(pos + 1, kp, rounding_mode="floor").to(torch.int32)
    layer = PooledDecodeLayer(cfg.B, cfg.Hi, cfg.H, cfg.dqk, inp.table.shape[1], ps, inp.pool_key.shape[0] // ps, kp,
                              cfg.keep, cfg.scale, splits=args.splits, device=dev, chain=args.chain)

    write = (inp.rows, inp.ape, slot_mapping, inp.rows_scale)

    def step():
        # the pool-key write of the rows' current tokens, then the layer (dsa_pooled_decode_step: one launch, or
        # with --chain the write's kernel and the separate kernels)
        layer.step(inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale, inp.table, npool_d, pos,
                   check=False, write=write)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    k_us = kernel_times(lib, step, args.steps)
    spans = step_times(step, args.steps)
    if layer.status()["gave_up"]:
        raise RuntimeError("bench.py: a barrier wait of the pooled attention launch gave up")
    positions = pos.cpu().long()
    npool = torch.div(positions + 1, kp, rounding_mode="floor")
    tail = [int(p) + 1 - kp * int(n) for p, n in zip(positions, npool)]
    tokens = [kp * min(int(n), cfg.keep) + t for n, t in zip(npool, tail)]
    if "decode_pooled_fused_kernel" in k_us:
        # the one-launch step (the pool-key write, the indexer, the selection, the attention): the step's bytes
        kname, kbytes = "decode_pooled_fused_kernel", W.pooled_step_bytes(cfg, npool.tolist(), tokens)
    else:
        # the separate kernels: the indexer, the kernel that streams the whole pool-key cache
        kname, kbytes = "indexer_decode_bf16_kernel", W.pooled_indexer_bytes(cfg, npool.tolist())
    k_time = k_us[kname]
    achieved = kbytes / (k_time * 1e-6) / 1e9
    step_bytes = W.pooled_step_bytes(cfg, npool.tolist(), tokens)
    step_gbs = step_bytes / (ms * 1e-3) / 1e9
    out = {
        "metric": "DSA pooled decode layer-steps/sec (GLM kpool 4) at B=8, 32K ctx; achieved HBM GB/s (% of 8 TB/s)",
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
        "config": {"workload": f"config {args.config}: {cfg.name}" + (" (separate kernels)" if args.chain else ""),
                   "batch": cfg.B, "context": cfg.L,
                   "q_heads": cfg.H, "indexer_heads": cfg.Hi, "kpool": kp, "keep_pools": cfg.keep,
                   "page_size": ps, "pool_keys": "bf16 [128] per pool (kpool pieces)",
                   "kv": f"fp8 e4m3 [{cfg.dqk}] + fp32 scale per token", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(f"config {args.config}: {cfg.name}", kname),
                     "algorithmic_bytes": kbytes, "avg_us": round(k_time, 3),
                     "launches_per_step": -(-cfg.B // 8) if kname == "decode_pooled_fused_kernel" else 1},
        "layer": {"algorithmic_bytes": step_bytes, "achieved_GBs": round(step_gbs, 1),
                  "frac": round(step_gbs / HBM_PEAK_GBS, 4), "kernel_us": {k: round(v, 3) for k, v in k_us.items()},
                  "step_us": percentiles(spans)},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = pooled_cpu_baseline(inp, cfg, npool, positions)
    print(json.dumps(out), flush=True)
    return 0


def pooled_prefill_main(args) -> int:
    """The GLM pooled chunked-prefill step (config 7): the prefill indexer over the context's bf16 pool keys with the
    exact top-512 pools (dsa_long_select.select -> dsa_prefill_select), then absorbed MLA of every query over its
    pools' tokens and its tail (dsa_long.attend_pooled -> dsa_sparse_mla_pooled). roofline: the indexer kernel's
    algorithmic MFMA work (2 Hi D per causal (query, pool) pair) against the bf16 peak; `attention` the same for the
    attention kernel (2 H (512 + 512) per attended token)."""
    import torch

    from trnrt_amd import _lib
    from trnrt_amd import workloads as W
    from trnrt_amd.kernels import dsa_long_select as LS
    from trnrt_amd.models import dsa_long

    cfg = W.POOLED_PREFILL_CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = W.make_pooled_prefill_inputs(cfg, seed=0, device=dev)
    C = cfg.chunk
    lib = _lib.lib()
    ws = torch.zeros(LS.workspace_bytes(C, cfg.P, cfg.keep), dtype=torch.uint8, device=dev)
    wsa = torch.zeros(max(int(lib.dsa_sparse_mla_pooled_workspace_bytes(C, cfg.H, cfg.keep, cfg.kp, 0)), 256),
                      dtype=torch.uint8, device=dev)
    table = inp.table.view(1, -1).expand(C, -1).contiguous()  # every query row reads the context's pages

    def step():
        pools, cnt, _ = LS.select(inp.qI, inp.w, inp.pk, inp.npool, cfg.keep, cfg.scale, workspace=ws)
        dsa_long.attend_pooled(inp.q, inp.kv_cache, inp.kv_scale, pools, cnt, inp.npool, inp.positions, table,
                               cfg.page_size, cfg.kp, cfg.softmax_scale, workspace=wsa)

    steps = min(args.steps, 20)
    for _ in range(min(args.warmup, 5)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    k_us = kernel_times(lib, step, steps)
    npool = inp.npool.long().cpu()
    pairs = int(npool.clamp(max=cfg.P).sum())
    flops = 2 * cfg.Hi * cfg.D * pairs
    sc_buf = torch.empty(C, cfg.P, dtype=torch.float32, device=dev)
    idx_us = whole_chunk_indexer_us(lib, "indexer_prefill_kernel", lambda: LS.scores(
        inp.qI, inp.w, inp.pk, inp.npool, cfg.scale, out=sc_buf), steps)
    del sc_buf
    tflops = flops / (idx_us * 1e-6) / 1e12
    tail = (inp.positions.long().cpu() + 1 - cfg.kp * npool)
    tokens = int((cfg.kp * npool.clamp(max=cfg.keep) + tail).sum())
    att_flops = 2 * cfg.H * (cfg.dqk + 512) * tokens
    att_kernel = "sparse_mla_wide_kernel" if "sparse_mla_wide_kernel" in k_us else "sparse_mla_kernel"
    att_us = k_us[att_kernel] + k_us.get("combine_splits_kernel", 0.0)
    att_tflops = att_flops / (att_us * 1e-6) / 1e12
    out = {
        "metric": "GLM pooled chunked-prefill step (indexer + top-512 pools + sparse MLA) chunks/sec",
        "value": round(1e3 / ms, 2),
        "unit": "chunks/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": min(args.warmup, 5),
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"config {args.config}: {cfg.name}", "cached": cfg.cached, "chunk": C,
                   "indexer_heads": cfg.Hi, "q_heads": cfg.H, "kpool": cfg.kp, "keep_pools": cfg.keep,
                   "pool_keys": "bf16 [128] per pool", "kv": f"fp8 e4m3 [{cfg.dqk}] + fp32 scale per token",
                   "page_size": cfg.page_size, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "indexer_prefill_kernel", "achieved": round(tflops, 1),
                     "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": None, "algorithmic_flops": flops, "avg_us": round(idx_us, 3),
                     "measured": WHOLE_CHUNK_NOTE},
        "attention": {"kernel": att_kernel, "avg_us": round(att_us, 3), "achieved": round(att_tflops, 1),
                      "unit": "TFLOP/s", "peak": BF16_PEAK_TFLOPS, "frac": round(att_tflops / BF16_PEAK_TFLOPS, 4),
                      "algorithmic_flops": att_flops},
        "kernel_us": {k: round(v, 3) for k, v in k_us.items()},
        "kernel_us_note": "per step, summed over the launches of one name (the tiles' launches overlap on two streams)",
        "selection_memory": {"workspace_bytes": ws.numel(), "scores": "two query tiles' scores held in the workspace"},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = pooled_prefill_cpu_baseline(inp, cfg)
    print(json.dumps(out), flush=True)
    return 0


def pooled_prefill_cpu_baseline(inp, cfg, budget_s: float = 15.0) -> dict:
    """The oracle's pooled chunk step (prefill_scores_ref over the pool keys + topk_ref + pool_slots_ref +
    sparse_mla_slots_ref, torch fp32 on the host) over whole query rows, as many as fit in about budget_s seconds;
    reported as chunks per second."""
    import torch

    from oracle import dsa_oracle as O

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    c = inp.to("cpu")
    ones = torch.ones(cfg.P)
    rows, t0, n = 4, time.perf_counter(), 0
    while True:
        r0 = (n * rows) % cfg.chunk
        sl = slice(r0, r0 + rows)
        sc = O.prefill_scores_ref(c.qI[sl], c.w[sl], c.pk, ones, c.npool[sl], cfg.scale)
        pools, cnt = O.topk_ref(sc, cfg.keep, c.npool[sl])
        rw, bias = O.pool_slots_ref(pools, cnt, c.npool[sl], c.positions[sl].long(), c.table, cfg.page_size, cfg.kp,
                                    cfg.keep + 1)
        tok = (rw.unsqueeze(-1) * cfg.kp + torch.arange(cfg.kp)).reshape(rows, -1)
        O.sparse_mla_slots_ref(c.q[sl], c.kv_cache, c.kv_scale, tok, bias.reshape(rows, -1), cfg.softmax_scale)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or n * rows >= cfg.chunk:
            break
    done = n * rows
    return {"value": done / cfg.chunk / dt, "unit": "chunks/s", "cores": cores, "kind": "port",
            "sample": f"{done} of the chunk's {cfg.chunk} query rows (scores over {cfg.P} pools + top-{cfg.keep} + "
                      f"slots + sparse MLA over {cfg.kp * (cfg.keep + 1)} token slots, torch fp32, {dt:.1f} s, "
                      f"{cores} threads)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--chain", action="store_true",
                    help="run the separate kernels (dsa_decode_layer_chain) even where the one-launch layer applies")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--bf16-queries", action="store_true",
                    help="config 5: bf16 indexer queries (the reference's precision) instead of e4m3 with scales")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this path runs on one GPU; --gpus {args.gpus} is not supported (each sequence's decode is "
              f"independent, so N GPUs would run N independent batches)", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe(args.copy_probe)
    if args.config == 5:
        return prefill_main(args)
    if args.config == 6:
        return pooled_main(args)
    if args.config == 7:
        return pooled_prefill_main(args)

    import torch

    from trnrt_amd import _lib
    from trnrt_amd import workloads as W
    from trnrt_amd.kernels.dsa_layer import DecodeLayer

    cfg = W.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = W.make_inputs(cfg, seed=0, device=dev)
    layer = DecodeLayer(cfg.B, cfg.Hi, cfg.H, inp.max_pages, cfg.page_size, inp.num_pages, cfg.keep, cfg.scale,
                        max_len=max(inp.lengths), splits=args.splits, device=dev, chain=args.chain)
    g = inp
    lib = _lib.lib()

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

    # per-kernel device durations inside the same layer-step: HIP events recorded by the runtime at each kernel's own
    # start and end (hipExtLaunchKernel on the launch stream), over another `steps` steps; then each step's own device
    # time (a pair of events around it) over another `steps`, for the median / p10 / p90
    k_us = kernel_times(lib, step, args.steps)
    spans = step_times(step, args.steps)
    g_us = graph_step_us(step, args.steps)
    # no barrier wait of any step above gave up (the one-launch kernel's workgroups were all resident): the outputs
    # the timed steps produced are the layer's
    st = layer.status()
    if st["gave_up"]:
        raise RuntimeError(f"bench.py: {st['gave_up']} barrier wait(s) gave up during the benchmark")

    lengths = inp.lengths
    layer_bytes = W.algorithmic_bytes(lengths, cfg.H, cfg.Hi, cfg.keep, cfg.page_size)
    layer_gbs = layer_bytes / (ms * 1e-3) / 1e9
    if "decode_fused_kernel" in k_us:
        # the one-launch layer (rows of up to 32K tokens): its launches together move the layer's algorithmic bytes
        kname, kbytes = "decode_fused_kernel", layer_bytes
    else:
        # the separate-kernel layer: the indexer, the kernel that streams the whole key cache (its streaming form
        # past 32K tokens)
        kname = "indexer_decode_long_kernel" if "indexer_decode_long_kernel" in k_us else "indexer_decode_kernel"
        kbytes = _indexer_bytes(lengths, cfg.Hi, cfg.page_size)
    k_time = k_us[kname]
    achieved = kbytes / (k_time * 1e-6) / 1e9

    workload = f"config {args.config}: {cfg.name}" + (" (separate kernels)" if args.chain else "")
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
        "config": {"workload": workload, "batch": cfg.B, "context": max(lengths),
                   "q_heads": cfg.H, "indexer_heads": cfg.Hi, "keep": cfg.keep, "page_size": cfg.page_size,
                   "kv": "fp8 e4m3 [576] + fp32 scale per token", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(workload, kname), "algorithmic_bytes": kbytes,
                     "avg_us": round(k_time, 3), "launches_per_step": -(-cfg.B // 8) if kname == "decode_fused_kernel"
                     else 1},
        "layer": {"algorithmic_bytes": layer_bytes, "achieved_GBs": round(layer_gbs, 1),
                  "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                  "kernel_us": {k: round(v, 3) for k, v in k_us.items()},
                  "step_us": percentiles(spans), "graph_step_us": round(g_us, 3)},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(inp)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
