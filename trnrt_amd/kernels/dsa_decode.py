"""Sparse MLA decode attention over the selected tokens on gfx950 (the operator surface of
trnrt/kernels/dsa_decode.py, with trnrt/kernels/dsa_slots.py's log-sum-exp).

What it computes, per row b and head h (trnrt/kernels/dsa_decode.py:26-37, absorbed MLA), over the row's slots k:
    s[k] = scale q[b, h] . K[k] + bias[b, k],  p = softmax(s),  o[b, h] = sum_k p[k] V[k]
    lse[b, h] = max_k s + log sum_k exp(s - max)                              (trnrt/kernels/dsa_slots.py:8-11)
with K[k] the slot's FP8 cache row times its per-token scale, 576 wide (512 latent + 64 rope columns) or 512 wide
(GLM's NoPE latent), and V[k] its first 512 columns (the reference's NoPE latent is both; with rope the value is the
latent part). A row whose slots are
all masked at NEG_INF averages them uniformly and has lse NEG_INF, as in the reference.

The HIP kernel (csrc/dsa_attention.hip) gathers the rows into LDS per 64-slot chunk, runs both products on bf16 MFMA
with exact e4m3 -> bf16 conversion, keeps an fp32 online softmax, and splits the slots over workgroups when the
batch x heads under-fill the GPU, merging the splits by log-sum-exp (trnrt/models/mla.py:853-856).
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _common as C

NEG_INF = -1e30  # trnrt/models/decoder.py NEG_INF
DQK = 576  # kv_lora_rank 512 + qk_rope_head_dim 64 (this build's cache format)
DQK_WIDTHS = (576, 512)  # the row widths the kernel takes: with rope, and GLM's NoPE latent
DV = 512  # kv_lora_rank


def _run(q: torch.Tensor, kv: torch.Tensor, kv_scale: torch.Tensor | None, scale: float, *, idx=None, cnt=None,
         table=None, page_size: int = 1, rows=None, bias=None, lse: bool = False, out_dtype=torch.float32,
         splits: int = 0, out: torch.Tensor | None = None, workspace: torch.Tensor | None = None, n_live=None):
    dev = C.on_gpu(q, kv, kv_scale, idx, cnt, table, rows, bias, out, workspace, n_live)
    if q.dim() != 3 or q.shape[2] not in DQK_WIDTHS:
        raise ValueError(f"dsa_decode: q {tuple(q.shape)}, expected [B, H, 576 or 512]")
    B, H, dqk = q.shape
    if H % 16:
        raise NotImplementedError(f"dsa_decode: {H} heads (the kernel takes multiples of 16)")
    q = C.as_bf16(q)
    kv = C.fp8_bytes(kv, "kv cache").reshape(-1, dqk)
    slots = kv.shape[0]
    if kv_scale is not None:  # None: the reference's unscaled cache (every scale 1, trnrt/models/decoder.py:481-486)
        kv_scale = C.need(C.as_f32(kv_scale).reshape(-1), "kv_scale", torch.float32, (slots,))
    if idx is not None:
        keep = idx.shape[1]
        idx = C.need(C.as_i32(idx), "idx", torch.int32, (B, keep))
        cnt = C.need(C.as_i32(cnt), "cnt", torch.int32, (B,))
        table = C.as_i32(table)
        if table.dim() != 2 or table.shape[0] != B:
            raise ValueError(f"dsa_decode: page table {tuple(table.shape)} for {B} rows")
        max_pages = table.shape[1]
        if slots % page_size:
            raise ValueError(f"dsa_decode: {slots} cache slots are not whole pages of {page_size}")
        num_pages = slots // page_size
    else:
        keep = rows.shape[1]
        rows = C.need(C.as_i32(rows), "rows", torch.int32, (B, keep))
        bias = C.as_f32(bias).reshape(B, -1)
        if bias.shape[1] != keep:
            raise ValueError(f"dsa_decode: bias {tuple(bias.shape)} for {keep} slots (kp = 1)")
        bias = bias.contiguous()
        max_pages, page_size, num_pages = 1, 1, slots
    if out is None:
        out = torch.empty(B, H, DV, dtype=out_dtype, device=dev)
    if out.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"dsa_decode: output dtype {out.dtype}")
    C.need(out, "out", out.dtype, (B, H, DV))
    ls = (torch.zeros if n_live is not None else torch.empty)(B, H, dtype=torch.float32, device=dev) if lse else None
    wsb = _lib.workspace_bytes(_lib.DSA_WS_ATTENTION, B, H, keep, 0, splits)
    if workspace is None and wsb:
        # the split partials (written before they are read: no zero fill), kept per stream
        workspace = C.cached_workspace(dev, wsb, "attention")
    ws_len = 0 if workspace is None else workspace.numel() * workspace.element_size()
    o_bf = out if out.dtype == torch.bfloat16 else None
    o_32 = out if out.dtype == torch.float32 else None
    if n_live is not None:
        # the rows + bias form over the first n_live[0] rows (the rest left unwritten)
        if rows is None:
            raise ValueError("dsa_decode: a live-row count takes the rows + bias form")
        st = _lib.lib().dsa_sparse_mla_slots_n(
            C.ptr(q), C.ptr(kv), C.ptr(kv_scale), C.ptr(rows), C.ptr(bias), C.ptr(n_live), C.ptr(o_bf), C.ptr(o_32),
            C.ptr(ls), C.ptr(workspace), ws_len, B, H, dqk, keep, slots, float(scale), int(splits), C.stream_ptr(dev))
        _lib.check(st, "dsa_slots_n.attend")
        return (out, ls) if lse else out
    st = _lib.lib().dsa_sparse_mla_decode(
        C.ptr(q), C.ptr(kv), C.ptr(kv_scale), C.ptr(idx), C.ptr(cnt), C.ptr(table), C.ptr(rows), C.ptr(bias),
        C.ptr(o_bf), C.ptr(o_32), C.ptr(ls), C.ptr(workspace), ws_len, B, H, dqk, DV, keep, max_pages, page_size,
        num_pages, float(scale), int(splits), C.stream_ptr(dev))
    _lib.check(st, "dsa_decode.attend")
    return (out, ls) if lse else out


def pool_token_rows(rows: torch.Tensor, bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Slots of kp tokens each (rows [B, NS] pool rows of the cache viewed as [slots / kp, kp R], bias [B, NS, kp])
    as token slots: rows [B, NS kp] = pool row kp + t, bias [B, NS kp] (trnrt/kernels/dsa_decode.py:26-37 reads a
    pool row as its kp tokens)."""
    B, NS = rows.shape
    kp = bias.shape[-1] if bias.dim() == 3 else 1
    if kp == 1:
        return rows, bias.reshape(B, NS)
    t = torch.arange(kp, device=rows.device, dtype=torch.int64)
    tok = (rows.to(torch.int64).unsqueeze(-1) * kp + t).reshape(B, NS * kp)
    return tok, bias.reshape(B, NS * kp)


def attend(q_lat: torch.Tensor, kc: torch.Tensor, rows: torch.Tensor, bias: torch.Tensor, scale: float, *,
           kc_scale: torch.Tensor | None = None, lse: bool = False, splits: int = 0,
           workspace: torch.Tensor | None = None):
    """o [B, H, 512] fp32 (trnrt/kernels/dsa_decode.py:40-43 `attend`, called as the reference calls it:
    attend(q_lat, kc, rows, bias, scale)): q_lat [B, H, 576 or 512], kc the FP8 cache [N, 1, D] or [N, D] (e4m3fn;
    for kp > 1 it may be the reference's pool view [N / kp, kp D]), kc_scale [N] fp32 its per-token scales or None
    for the reference's unscaled cache (scale 1), rows [B, NS] int each slot's row, bias [B, NS] or [B, NS, kp] fp32
    (0 / NEG_INF): with kp > 1 a slot is a pool of kp consecutive tokens. With lse also lse [B, H] fp32. workspace:
    the split partials (dsa_workspace_bytes(DSA_WS_ATTENTION, ...)), or None for one kept per stream."""
    rows, bias = pool_token_rows(rows, bias)
    return _run(q_lat, kc, kc_scale, scale, rows=rows, bias=bias, lse=lse, splits=splits, workspace=workspace)


def attend_tokens(q: torch.Tensor, kv_cache: torch.Tensor, kv_scale: torch.Tensor | None, idx: torch.Tensor,
                  cnt: torch.Tensor, table: torch.Tensor, page_size: int, scale: float, *, lse: bool = True,
                  out_dtype=torch.bfloat16, splits: int = 0, out: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None):
    """The decode path's form: the selected token positions idx [B, keep] (ascending, cnt [B] valid) read through the
    page table [B, max_pages] (trnrt/models/dsa_long.py:189-215 `slots` folded into the gather). Returns o
    [B, H, 512] in out_dtype (bf16 by default) and lse [B, H] fp32. kv_scale None: the unscaled cache."""
    return _run(q, kv_cache, kv_scale, scale, idx=idx, cnt=cnt, table=table, page_size=page_size, lse=lse,
                out_dtype=out_dtype, splits=splits, out=out, workspace=workspace)
