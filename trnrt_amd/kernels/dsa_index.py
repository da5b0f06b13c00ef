"""The DSA lightning indexer's decode scores on gfx950 (the operator surface of trnrt/kernels/dsa_index.py).

What it computes, per decode row b and cached token t (trnrt/kernels/dsa_index.py:44-50, trnrt/models/dsa_long.py:
74-84, with D ** -0.5 folded into w as at trnrt/models/mla.py:629, and the FP8 key's per-token scale):

    score[b, t] = k_scale[t] * sum_h w[b, h] relu(q[b, h] . k_fp8[t]) + cand[b, t]

over the keys read in place from the paged FP8 indexer-key cache through the page table. relu(s x) = s relu(x) for
the positive scale s, so scaling after the dot product is the reference's dequantised key up to rounding. The HIP
kernel (libdsa_gfx950.so, csrc/dsa_indexer.hip) runs the q . k contraction on bf16 MFMA with the e4m3 keys converted
exactly to bf16 in registers, and the weighted relu head sum in fp32 registers; only the [B, P] fp32 scores are
written.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _common as C

NEG_INF = -1e30  # trnrt/models/decoder.py NEG_INF
D = 128  # index_head_dim


def page_groups(table: torch.Tensor) -> torch.Tensor:
    """ppg [128, B, NG] int32 from the rows' page table [B, NPg] (NPg = 128 NG), the page of group g on partition p
    being page p NG + g of the row: the reference's layout (trnrt/kernels/dsa_index.py:234-240), accepted by
    scores() for drop-in callers. ValueError unless NPg is a multiple of 128."""
    B, NPg = table.shape
    if NPg % 128:
        raise ValueError(f"dsa_index: {NPg} pages per row, the kernel needs a multiple of 128")
    return table.reshape(B, 128, NPg // 128).permute(1, 0, 2).contiguous().to(torch.int32)


def _table(ppg: torch.Tensor, B: int) -> torch.Tensor:
    """[B, NPg] page table from page_groups' layout (its inverse, trnrt/kernels/dsa_index.py:251) or from a plain
    table."""
    if ppg.dim() == 3:
        if ppg.shape[1] != B:
            raise ValueError(f"dsa_index: page groups {tuple(ppg.shape)} for {B} rows")
        return ppg.permute(1, 0, 2).reshape(B, -1)
    if ppg.dim() != 2 or ppg.shape[0] != B:
        raise ValueError(f"dsa_index: page table {tuple(ppg.shape)} for {B} rows")
    return ppg


def decode_scores(q: torch.Tensor, w: torch.Tensor, k_cache: torch.Tensor, k_scale: torch.Tensor | None,
                  table: torch.Tensor, ctx_len: torch.Tensor | None, page_size: int, score_stride: int | None = None,
                  cand: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """[B, score_stride] fp32 scores in the cache's native layout: q [B, Hi, 128] bf16, w [B, Hi] fp32 (head weights
    times D ** -0.5), k_cache [slots, 128] e4m3fn with k_scale [slots] fp32 (pages of a multiple of 32 keys), or
    bf16 with k_scale None (GLM's pool keys: pages of any number of keys), slots = pages x page_size, table
    [B, max_pages] int32, ctx_len [B] int32 (None: every row's length is score_stride), cand [B, score_stride]
    additive fp32 or None. Positions at or past a row's length score NEG_INF."""
    dev = C.on_gpu(q, w, k_cache, k_scale, table, ctx_len, cand, out)
    B, Hi, Dq = q.shape
    if Dq != D:
        raise ValueError(f"dsa_index: head dim {Dq}, the kernel implements {D}")
    q = C.as_bf16(q)
    w = C.need(C.as_f32(w), "w", torch.float32, (B, Hi))
    bf16_keys = k_cache.dtype == torch.bfloat16
    if bf16_keys != (k_scale is None):
        raise ValueError("dsa_index: FP8 keys need their k_scale, bf16 keys take none")
    if not bf16_keys:
        k_cache = C.fp8_bytes(k_cache, "k_cache")
    elif not k_cache.is_contiguous():
        raise ValueError("k_cache: must be contiguous")
    if k_cache.dim() != 2 or k_cache.shape[1] != D:
        k_cache = k_cache.reshape(-1, D)
    slots = k_cache.shape[0]
    if slots % page_size:
        raise ValueError(f"dsa_index: {slots} cache slots are not whole pages of {page_size}")
    if not bf16_keys:
        k_scale = C.need(C.as_f32(k_scale).reshape(-1), "k_scale", torch.float32, (slots,))
    table = C.as_i32(table)
    if table.dim() != 2 or table.shape[0] != B:
        raise ValueError(f"dsa_index: page table {tuple(table.shape)} for {B} rows")
    max_pages = table.shape[1]
    if score_stride is None:
        score_stride = max_pages * page_size
    if ctx_len is not None:
        ctx_len = C.need(C.as_i32(ctx_len), "ctx_len", torch.int32, (B,))
    if cand is not None:
        cand = C.need(C.as_f32(cand), "cand", torch.float32, (B, score_stride))
    if out is None:
        out = torch.empty(B, score_stride, dtype=torch.float32, device=dev)
    else:
        C.need(out, "out", torch.float32, (B, score_stride))
    if bf16_keys:
        st = _lib.lib().dsa_indexer_decode_bf16(C.ptr(q), C.ptr(w), C.ptr(k_cache), C.ptr(table), C.ptr(ctx_len),
                                                C.ptr(cand), C.ptr(out), B, Hi, D, max_pages, page_size,
                                                slots // page_size, score_stride, C.stream_ptr(dev))
    else:
        st = _lib.lib().dsa_indexer_decode(C.ptr(q), C.ptr(w), C.ptr(k_cache), C.ptr(k_scale), C.ptr(table),
                                           C.ptr(ctx_len), C.ptr(cand), C.ptr(out), B, Hi, D, max_pages, page_size,
                                           slots // page_size, score_stride, C.stream_ptr(dev))
    _lib.check(st, "dsa_index.decode_scores")
    return out


def scores(q: torch.Tensor, w: torch.Tensor, pkc: torch.Tensor, ppg: torch.Tensor, cand: torch.Tensor | None,
           dge: int | None = None, *, pkc_scale: torch.Tensor | None = None,
           ctx_len: torch.Tensor | None = None) -> torch.Tensor:
    """[B, P] fp32 scores (trnrt/kernels/dsa_index.py:243-268 `scores`): q [B, Hi, D], w [B, Hi] fp32 (head weights
    times D ** -0.5), pkc [Npages, page_size D] the key cache as page rows: FP8 e4m3 with pkc_scale [Npages,
    page_size] fp32 the keys' scales (one key per token, kpool 1), or bf16 with no scale (GLM's pool-key cache,
    trnrt/models/mla.py:628-629: page_size pools per page); ppg page_groups(table) [128, B, NG] or a table [B, NPg]
    int32, cand [B, P] fp32 (0 / NEG_INF) or None, ctx_len [B] int32 or None. P = NPg page_size. dge is the
    reference's Trainium DMA knob and is ignored."""
    del dge
    B = q.shape[0]
    table = _table(ppg, B)
    page_size = pkc.shape[1] // D if pkc.dim() == 2 else None
    if page_size is None or pkc.shape[1] != page_size * D:
        raise ValueError(f"dsa_index: pkc {tuple(pkc.shape)} is not [pages, page_size x {D}]")
    P = table.shape[1] * page_size
    ks = None if pkc_scale is None else pkc_scale.reshape(-1)
    return decode_scores(q, w, pkc.reshape(-1, D), ks, table, ctx_len, page_size, P, cand)
