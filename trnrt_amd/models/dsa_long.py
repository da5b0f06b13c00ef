"""The DSA path's scores, selection, slots and attention (the functions of trnrt/models/dsa_long.py that the decode
and chunked-prefill paths call; a candidate is one token at kpool 1, a pool of kpool tokens above).

- scores: the index scores of a prefill chunk (2-D keys, csrc/dsa_prefill.hip) or a decode batch (one context per
  row, csrc/dsa_indexer.hip) (trnrt/models/dsa_long.py:74-84);
- select_device / select: the exact top-keep of scores [N, P] as (indices [N, keep] int64 ascending, 0 past the
  count; count [N] int64) (trnrt/models/dsa_long.py:135-186), by the gfx950 top-k kernel;
- compact: a 0 / 1 mask's ones as ascending indices and a count (trnrt/models/dsa_long.py:140-166), by a HIP
  compaction kernel;
- slots: selected pools -> cache pool rows and the 0 / NEG_INF bias with the query's tail pool
  (trnrt/models/dsa_long.py:189-215, any kpool);
- attend: absorbed MLA over the slots (trnrt/models/dsa_long.py:218-223);
- attend_pooled: slots + attend of a pooled selection in one kernel (no slot rows materialised);
- decode_pooled: a pooled (GLM) decode batch through all four over the bf16 pool-key cache
  (trnrt/models/mla.py:505-526 `attention_long`).
"""

from __future__ import annotations

import torch

from .. import _lib
from ..kernels import _common as C
from ..kernels import dsa_decode, dsa_index, dsa_long_select, dsa_topk

NEG_INF = -1e30  # trnrt/models/decoder.py NEG_INF
VISIBLE = -5e29  # trnrt/kernels/dsa_topk.VISIBLE


def npools(positions: torch.Tensor, kp: int) -> torch.Tensor:
    """[N] int64: the complete pools a query at each position may select, floor((pos + 1) / kp)
    (trnrt/models/dsa_long.py:65-71; pos + 1 at kp = 1)."""
    if kp < 1 or kp & (kp - 1):
        raise ValueError(f"kpool {kp} is not a power of two")
    return torch.div(positions.to(torch.int64) + 1, kp, rounding_mode="floor")


def scores(qI: torch.Tensor, w: torch.Tensor, pk: torch.Tensor, npool: torch.Tensor, scale: float, *,
           pk_scale: torch.Tensor | None = None) -> torch.Tensor:
    """[N, P] fp32: every key's index score, NEG_INF for the non-candidates (p >= npool) (trnrt/models/dsa_long.py:
    74-84). qI [N, Hi, 128] bf16, w [N, Hi] fp32, pk the FP8 e4m3 keys with pk_scale their per-token fp32 scales, or
    a chunk's bf16 pool keys [P, 128] (GLM's context_pool_keys, trnrt/models/mla.py:491-503) with no scale:
    [P, 128] (one sequence: a prefill chunk) or [N, P, 128] (one context per row: a decode batch, FP8), pk_scale [P]
    or [N, P], npool [N]. The decode form needs P a multiple of 32 (each row's keys are one page of the decode
    indexer)."""
    if pk.dim() == 2:
        return dsa_long_select.scores(qI, w, pk, npool, scale, pk_scale=pk_scale)
    if pk.dim() != 3 or pk.shape[0] != qI.shape[0]:
        raise ValueError(f"dsa_long.scores: pk {tuple(pk.shape)} for {qI.shape[0]} queries")
    N, P, _ = pk.shape
    if P % 32:
        raise NotImplementedError(f"dsa_long.scores: {P} keys per row; the decode indexer takes multiples of 32")
    dev = C.on_gpu(qI, w, pk, pk_scale, npool)
    table = torch.arange(N, dtype=torch.int32, device=dev).view(N, 1)
    lens = npool.reshape(-1).clamp(0, P).to(torch.int32)
    ks = None if pk_scale is None else pk_scale.reshape(-1)
    return dsa_index.decode_scores(qI, w.float() * float(scale), pk.reshape(N * P, -1), ks, table, lens, P, P)


def select_device(sc: torch.Tensor, keep: int, lengths: torch.Tensor | None = None, *,
                  workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The exact selection of scores [N, P] (non-candidates at or below VISIBLE) as (indices [N, keep] int64
    ascending, 0 past the count; count [N] int64). lengths [N] int32 optionally bounds each row's candidates.
    workspace: the caller's top-k workspace (dsa_topk.select_indices), or None for one kept per stream."""
    idx, cnt = dsa_topk.select_indices(sc, keep, lengths=lengths, vis_only=True, workspace=workspace)
    return idx.to(torch.int64), cnt.to(torch.int64)


def select(sc: torch.Tensor, keep: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The selection (trnrt/models/dsa_long.py:135-137): select_device."""
    return select_device(sc, keep)


def compact(sel: torch.Tensor, keep: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(indices [N, keep] int64 ascending, count [N] int64) of a 0 / 1 float mask sel [N, M]: the positions of each
    row's ones, the first keep of them in a row with more, 0 past the count, count = min(ones, keep)
    (trnrt/models/dsa_long.py:140-166). An entry counts as a one when above 0.5. One HIP kernel
    (csrc/dsa_compact.hip): a workgroup per row, its walk stopping once keep ones are placed."""
    dev = C.on_gpu(sel)
    if sel.dim() != 2 or sel.shape[1] < 1:
        raise ValueError(f"dsa_long.compact: mask {tuple(sel.shape)}, expected [N, M]")
    if keep < 1:
        raise ValueError(f"dsa_long.compact: keep {keep}")
    N, M = sel.shape
    s = C.as_f32(sel).contiguous()
    idx = torch.empty(N, keep, dtype=torch.int64, device=dev)
    cnt = torch.empty(N, dtype=torch.int64, device=dev)
    st = _lib.lib().dsa_compact_mask(C.ptr(s), N, M, int(keep), C.ptr(idx), C.ptr(cnt), C.stream_ptr(dev))
    _lib.check(st, "dsa_long.compact")
    return idx, cnt


def slots(pools: torch.Tensor, cnt: torch.Tensor, npool: torch.Tensor, positions: torch.Tensor, table: torch.Tensor,
          page_size: int, kp: int, n_slots: int) -> tuple[torch.Tensor, torch.Tensor]:
    """rows [N, n_slots] int64 (each slot's pool row, the latent cache viewed as [slots / kp, kp R]) and bias
    [N, n_slots, kp] fp32 (0 for a token to attend, NEG_INF otherwise) for N queries
    (trnrt/models/dsa_long.py:189-215): slots 0 .. keep - 1 the selected pools (pools [N, keep], cnt [N] valid),
    slot keep the query's tail pool npool (its tokens kp npool .. pos; none when pos + 1 is a multiple of kp), the rest
    padding. table: [Pp] one sequence's pages (a prefill chunk) or [N, Pp] one per row (a decode batch). At kp 1 a
    pool is a token and the tail is always empty."""
    N, keep = pools.shape
    ppp = page_size // kp if kp >= 1 else 0
    if kp < 1 or page_size % kp or ppp & (ppp - 1) or n_slots < keep + 1:
        raise ValueError(f"slots: page_size {page_size}, kpool {kp}, {n_slots} slots for {keep} + 1 pools")
    dev = C.on_gpu(pools, cnt, npool, positions, table)
    tb = C.as_i32(table)
    if tb.dim() not in (1, 2) or (tb.dim() == 2 and tb.shape[0] != N):
        raise ValueError(f"slots: table {tuple(table.shape)} for {N} queries")
    # the converted inputs stay referenced until the launch: a temporary freed before it could be reused (and
    # overwritten) by the next conversion on the same stream
    pl = C.need(C.as_i32(pools), "pools", torch.int32, (N, keep))
    cn = C.need(C.as_i32(cnt.reshape(-1)), "cnt", torch.int32, (N,))
    npl = C.need(C.as_i32(npool.reshape(-1)), "npool", torch.int32, (N,))
    pos = C.need(C.as_i32(positions.reshape(-1)), "positions", torch.int32, (N,))
    rows = torch.empty(N, n_slots, dtype=torch.int32, device=dev)
    bias = torch.empty(N, n_slots, kp, dtype=torch.float32, device=dev)
    st = _lib.lib().dsa_pool_slots(C.ptr(pl), C.ptr(cn), C.ptr(npl), C.ptr(pos), C.ptr(tb), int(tb.dim() == 1),
                                   C.ptr(rows), C.ptr(bias), N, keep, n_slots, tb.shape[-1], page_size, kp,
                                   C.stream_ptr(dev))
    _lib.check(st, "dsa_long.slots")
    return rows.to(torch.int64), bias


def attend(q_lat: torch.Tensor, kc: torch.Tensor, rows: torch.Tensor, bias: torch.Tensor, scale: float, *,
           kc_scale: torch.Tensor | None = None) -> torch.Tensor:
    """o [N, H, 512] fp32: absorbed MLA of N queries over their slots (trnrt/models/dsa_long.py:218-223); kc_scale
    None: the reference's unscaled cache."""
    return dsa_decode.attend(q_lat, kc, rows, bias, scale, kc_scale=kc_scale)


def attend_pooled(q_lat: torch.Tensor, kc: torch.Tensor, kc_scale: torch.Tensor | None, pools: torch.Tensor,
                  cnt: torch.Tensor, npool: torch.Tensor, positions: torch.Tensor, table: torch.Tensor,
                  page_size: int, kp: int, scale: float, *, lse: bool = False,
                  workspace: torch.Tensor | None = None, splits: int = 0):
    """attend(slots(...)) in one kernel (trnrt/models/dsa_long.py:189-223): absorbed MLA of N queries over the kp
    tokens of each of their selected pools (pools [N, keep] ascending, cnt [N] valid) and the tail tokens
    kp npool .. positions[n] of their incomplete pool, read through the page table ([Pp] shared, or [N, Pp]); the
    slot rows and biases are never materialised. q_lat [N, H, R] bf16 (R 512 or 576), kc [slots, R] e4m3fn with
    kc_scale [slots]. Returns o [N, H, 512] fp32 (and lse [N, H] with lse). workspace: the split partials
    (dsa_sparse_mla_pooled_workspace_bytes), allocated here when not given; splits: the attention's split-K (0: chosen
    for the GPU)."""
    N, keep = pools.shape
    if kp < 2 or kp & (kp - 1) or page_size % kp:
        raise ValueError(f"attend_pooled: kpool {kp} with pages of {page_size}")
    dev = C.on_gpu(q_lat, kc, kc_scale, pools, cnt, npool, positions, table)
    if q_lat.dim() != 3 or q_lat.shape[0] != N or q_lat.shape[2] not in dsa_decode.DQK_WIDTHS:
        raise ValueError(f"attend_pooled: q_lat {tuple(q_lat.shape)} for {N} queries")
    H, dqk = q_lat.shape[1], q_lat.shape[2]
    q = C.as_bf16(q_lat)
    kv = C.fp8_bytes(kc, "kc").reshape(-1, dqk)
    slots_n = kv.shape[0]
    ks = None if kc_scale is None else C.need(C.as_f32(kc_scale).reshape(-1), "kc_scale", torch.float32, (slots_n,))
    pl = C.need(C.as_i32(pools), "pools", torch.int32, (N, keep))
    cn = C.need(C.as_i32(cnt.reshape(-1)), "cnt", torch.int32, (N,))
    npl = C.need(C.as_i32(npool.reshape(-1)), "npool", torch.int32, (N,))
    pos = C.need(C.as_i32(positions.reshape(-1)), "positions", torch.int32, (N,))
    tb = C.as_i32(table)
    tb = tb.view(1, -1).expand(N, -1).contiguous() if tb.dim() == 1 else tb
    if tb.shape[0] != N:
        raise ValueError(f"attend_pooled: table {tuple(table.shape)} for {N} queries")
    if slots_n % page_size:
        raise ValueError(f"attend_pooled: {slots_n} cache slots are not whole pages of {page_size}")
    out = torch.empty(N, H, dsa_decode.DV, dtype=torch.float32, device=dev)
    ls = torch.empty(N, H, dtype=torch.float32, device=dev) if lse else None
    lib = _lib.lib()
    wsb = int(lib.dsa_sparse_mla_pooled_workspace_bytes(N, H, keep, kp, int(splits)))
    ws = workspace if workspace is not None else C.cached_workspace(dev, wsb, "attention")
    st = lib.dsa_sparse_mla_pooled(C.ptr(q), C.ptr(kv), C.ptr(ks), C.ptr(pl), C.ptr(cn), C.ptr(npl), C.ptr(pos),
                                   C.ptr(tb), None, C.ptr(out), C.ptr(ls), C.ptr(ws), ws.numel(), N, H, dqk, keep, kp,
                                   tb.shape[1], page_size, slots_n // page_size, float(scale), int(splits),
                                   C.stream_ptr(dev))
    _lib.check(st, "dsa_long.attend_pooled")
    return (out, ls) if lse else out


def decode_pooled(q_idx: torch.Tensor, w: torch.Tensor, pool_key: torch.Tensor, q_lat: torch.Tensor,
                  kc: torch.Tensor, kc_scale: torch.Tensor | None, positions: torch.Tensor, table: torch.Tensor,
                  page_size: int, kp: int, topk: int, index_scale: float, softmax_scale: float, *,
                  parts: bool = False):
    """One pooled decode batch's attention core after its rows and pool keys were written (trnrt/models/mla.py:505-526
    `attention_long` for a decode batch, scoring the pool-key cache's page rows in place as trnrt/models/mla.py:
    615-630 does): the scores of the complete pools (bf16 pool keys pool_key [slots, 128 / kp], page rows of
    page_size / kp pools), their exact top topk / kp, the slots with the tail pool, absorbed MLA over those pools'
    tokens. q_idx [B, Hi, 128] bf16, w [B, Hi] fp32 (the head weights, index_scale applied here), q_lat [B, H, R]
    bf16, kc [slots, R] e4m3fn with kc_scale [slots], positions [B], table [B, pages] int32. Returns o [B, H, 512]
    fp32, and with parts also (scores, pools, cnt, rows, bias)."""
    B = q_idx.shape[0]
    keep = topk // kp
    ppp = page_size // kp
    if kp < 2 or page_size % kp or topk % kp:
        raise ValueError(f"decode_pooled: kpool {kp}, page_size {page_size}, topk {topk}")
    if pool_key.dtype != torch.bfloat16 or pool_key.shape[-1] * kp != dsa_index.D:
        raise ValueError(f"decode_pooled: pool_key {tuple(pool_key.shape)} {pool_key.dtype}, expected bf16 pieces of "
                         f"{dsa_index.D} / {kp}")
    npool = npools(positions, kp).to(torch.int32)
    sc = dsa_index.scores(q_idx, w.float() * float(index_scale), pool_key.view(-1, ppp * dsa_index.D), table, None,
                          ctx_len=npool)
    pools, cnt = select_device(sc, keep, lengths=npool)
    rows, bias = slots(pools, cnt, npool, positions, table, page_size, kp, keep + 1)
    o = attend(q_lat, kc, rows, bias, softmax_scale, kc_scale=kc_scale)
    return (o, (sc, pools, cnt, rows, bias)) if parts else o
