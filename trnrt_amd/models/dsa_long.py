"""The per-token DSA decode path's selection, slots and attention (the functions of trnrt/models/dsa_long.py that
the decode path calls, at kpool 1: each candidate is one token).

- scores: the index scores of a prefill chunk (2-D keys, csrc/dsa_prefill.hip) or a decode batch (one context per
  row, csrc/dsa_indexer.hip) (trnrt/models/dsa_long.py:74-84);
- select_device / select: the exact top-keep of scores [N, P] as (indices [N, keep] int64 ascending, 0 past the
  count; count [N] int64) (trnrt/models/dsa_long.py:135-186), by the gfx950 top-k kernel;
- slots: token indices -> cache rows and the 0 / NEG_INF bias (trnrt/models/dsa_long.py:189-215 at kp 1, where a
  query's tail pool is always empty);
- attend: absorbed MLA over the slots (trnrt/models/dsa_long.py:218-223).
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
           pk_scale: torch.Tensor) -> torch.Tensor:
    """[N, P] fp32: every key's index score, NEG_INF for the non-candidates (p >= npool) (trnrt/models/dsa_long.py:
    74-84). qI [N, Hi, 128] bf16, w [N, Hi] fp32, pk the FP8 e4m3 keys: [P, 128] (one sequence: a prefill chunk) or
    [N, P, 128] (one context per row: a decode batch), pk_scale their per-token fp32 scales ([P] or [N, P]), npool
    [N]. The decode form needs P a multiple of 32 (each row's keys are one page of the decode indexer)."""
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
    return dsa_index.decode_scores(qI, w.float() * float(scale), pk.reshape(N * P, -1), pk_scale.reshape(-1), table,
                                   lens, P, P)


def select_device(sc: torch.Tensor, keep: int, lengths: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The exact selection of scores [N, P] (non-candidates at or below VISIBLE) as (indices [N, keep] int64
    ascending, 0 past the count; count [N] int64). lengths [N] int32 optionally bounds each row's candidates."""
    idx, cnt = dsa_topk.select_indices(sc, keep, lengths=lengths, vis_only=True)
    return idx.to(torch.int64), cnt.to(torch.int64)


def select(sc: torch.Tensor, keep: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The selection (trnrt/models/dsa_long.py:135-137): select_device."""
    return select_device(sc, keep)


def slots(pools: torch.Tensor, cnt: torch.Tensor, npool: torch.Tensor, positions: torch.Tensor, table: torch.Tensor,
          page_size: int, kp: int, n_slots: int) -> tuple[torch.Tensor, torch.Tensor]:
    """rows [N, n_slots] int64 (each slot's cache row) and bias [N, n_slots, 1] fp32 (0 to attend, NEG_INF not) for
    the selected tokens pools [N, keep] (cnt [N] valid) of N decode rows with their own tables [N, Pp]: slot k < keep
    is the k-th selected token, slot keep the query's tail (empty at kp 1), the rest padding
    (trnrt/models/dsa_long.py:189-215 at kp = 1)."""
    if kp != 1:
        raise NotImplementedError("dsa_long.slots: the pooled form (kp > 1) is not implemented on gfx950")
    N, keep = pools.shape
    if n_slots < keep + 1:
        raise ValueError(f"slots: {n_slots} slots for {keep} + 1 pools")
    dev = C.on_gpu(pools, cnt, table)
    tb = C.as_i32(table if table.dim() == 2 else table.view(1, -1).expand(N, -1))
    Pp = tb.shape[1]
    idx = C.as_i32(pools)
    cn = C.as_i32(cnt)
    rows = torch.zeros(N, n_slots, dtype=torch.int32, device=dev)
    bias = torch.full((N, n_slots), NEG_INF, dtype=torch.float32, device=dev)
    sel_rows = torch.empty(N, keep, dtype=torch.int32, device=dev)
    sel_bias = torch.empty(N, keep, dtype=torch.float32, device=dev)
    num_pages = (2**31 - 1) // page_size  # rows are computed, not read: no page clamp is needed here
    st = _lib.lib().dsa_token_rows(C.ptr(idx), C.ptr(cn), C.ptr(tb), C.ptr(sel_rows), C.ptr(sel_bias), N, keep, Pp,
                                   page_size, num_pages, C.stream_ptr(dev))
    _lib.check(st, "dsa_long.slots")
    rows[:, :keep] = sel_rows
    bias[:, :keep] = sel_bias
    # the tail slot reads position min(npool, last) (its tokens are none at kp 1), the padding slots position 0
    tail = npool.to(torch.int64).clamp(max=Pp * page_size - 1).view(N, 1)
    tpage = tb.to(torch.int64).gather(1, torch.div(tail, page_size, rounding_mode="floor"))
    rows[:, keep:keep + 1] = (tpage * page_size + tail % page_size).to(torch.int32)
    pad_row = tb[:, :1].to(torch.int64) * page_size
    if n_slots > keep + 1:
        rows[:, keep + 1:] = pad_row.to(torch.int32)
    del positions
    return rows.to(torch.int64), bias.view(N, n_slots, 1)


def attend(q_lat: torch.Tensor, kc: torch.Tensor, rows: torch.Tensor, bias: torch.Tensor, scale: float, *,
           kc_scale: torch.Tensor) -> torch.Tensor:
    """o [N, H, 512] fp32: absorbed MLA of N queries over their slots (trnrt/models/dsa_long.py:218-223)."""
    return dsa_decode.attend(q_lat, kc, rows, bias, scale, kc_scale=kc_scale)
