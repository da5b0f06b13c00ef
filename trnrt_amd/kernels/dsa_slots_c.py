"""Slot attention over each row's visible tokens only (the operator surface of trnrt/kernels/dsa_slots_c.py
`attend`, trnrt/kernels/dsa_slots_c.py:416-447): the arithmetic of dsa_decode.attend's row form, with the row's
slots compacted on the GPU first, so a row whose slot list is mostly padding (a context-parallel rank's share of the
selection) costs only its visible tokens.

A compaction kernel (csrc/dsa_compact.hip) lists each row's visible tokens (bias above NEG_INF / 2), pool row kp + t
in slot order, with their count; the attention kernel (csrc/dsa_attention.hip) then runs its rows + count form over
that list. The same tokens with the same scores as the uncompacted form, so the two agree to fp32 summation order.
A row with no visible token attends pool row 0's kp tokens, all masked (their uniform mean, lse NEG_INF): the
reference's compacted form fills its empty entries with pool row 0 (trnrt/kernels/dsa_slots_c.py:92-103). The
reference caps a row at 128 live slots and then falls back to its uncompacted kernel for every row of the call; this
build compacts any number of slots, so it never needs that fallback.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _common as C
from .dsa_decode import DQK_WIDTHS, DV

NEG_INF = -1e30  # trnrt/models/decoder.py NEG_INF
C_SLOTS = 128  # the reference's compacted slots per row (its device layout; no limit here)


def live_tokens(bias: torch.Tensor) -> torch.Tensor:
    """[N, NS] fp32: the visible tokens of every slot (bias above NEG_INF / 2), 0 .. kp
    (trnrt/kernels/dsa_slots_c.py:56-59)."""
    return (bias > NEG_INF / 2).to(torch.float32).sum(-1)


def attend(q_lat: torch.Tensor, kc: torch.Tensor, rows: torch.Tensor, bias: torch.Tensor, scale: float,
           lse: bool = False, *, kc_scale: torch.Tensor | None = None, splits: int = 0,
           workspace: torch.Tensor | None = None):
    """o [N, H, 512] fp32 (and lse [N, H] fp32) of q_lat [N, H, 576 or 512] bf16 over the visible tokens of rows
    [N, NS] (pool rows of the FP8 cache kc viewed as [slots / kp, kp rows]; kc [slots, 1, D] or [slots, D] e4m3fn
    with kc_scale [slots] fp32 its per-token scales, or None for the reference's unscaled cache) with bias
    [N, NS, kp] or [N, NS] fp32 (0 / NEG_INF). workspace: dsa_slots_compact_workspace_bytes(N, H, NS, kp, splits)
    bytes (no zero fill needed), or None for one kept per stream."""
    dev = C.on_gpu(q_lat, kc, rows, bias, kc_scale, workspace)
    if q_lat.dim() != 3 or q_lat.shape[2] not in DQK_WIDTHS:
        raise ValueError(f"dsa_slots_c: q_lat {tuple(q_lat.shape)}, expected [N, H, 576 or 512]")
    N, H, dqk = q_lat.shape
    if H % 16:
        raise NotImplementedError(f"dsa_slots_c: {H} heads (the kernel takes multiples of 16)")
    if rows.dim() != 2 or rows.shape[0] != N:
        raise ValueError(f"dsa_slots_c: rows {tuple(rows.shape)} for {N} queries")
    NS = rows.shape[1]
    kp = bias.shape[-1] if bias.dim() == 3 else 1
    b = C.as_f32(bias).reshape(N, -1).contiguous()
    if b.shape[1] != NS * kp:
        raise ValueError(f"dsa_slots_c: bias {tuple(bias.shape)} for {NS} slots")
    q = C.as_bf16(q_lat)
    kv = C.fp8_bytes(kc, "kv cache").reshape(-1, dqk)
    num_slots = kv.shape[0]
    if num_slots % kp or num_slots < kp:
        raise ValueError(f"dsa_slots_c: {num_slots} cache rows are not whole pools of {kp}")
    ks = None if kc_scale is None else C.need(C.as_f32(kc_scale).reshape(-1), "kc_scale", torch.float32,
                                              (num_slots,))
    r = C.need(C.as_i32(rows), "rows", torch.int32, (N, NS))
    out = torch.empty(N, H, DV, dtype=torch.float32, device=dev)
    ls = torch.empty(N, H, dtype=torch.float32, device=dev) if lse else None
    wsb = _lib.lib().dsa_slots_compact_workspace_bytes(N, H, NS, kp, int(splits))
    ws = workspace if workspace is not None else C.cached_workspace(dev, wsb, "slots_compact")
    if ws.numel() * ws.element_size() < wsb:
        raise ValueError(f"dsa_slots_c.attend: workspace of {ws.numel() * ws.element_size()} bytes, needs {wsb}")
    st = _lib.lib().dsa_sparse_mla_slots_compact(
        C.ptr(q), C.ptr(kv), C.ptr(ks), C.ptr(r), C.ptr(b), None, C.ptr(out), C.ptr(ls), C.ptr(ws), wsb, N, H, dqk,
        NS, kp, num_slots, float(scale), int(splits), C.stream_ptr(dev))
    _lib.check(st, "dsa_slots_c.attend")
    return (out, ls) if lse else out
