"""Exact top-k selection of DSA index scores on gfx950 (the operator surface of trnrt/kernels/dsa_topk.py).

The rule (trnrt/models/dsa_select.py:10-38, trnrt/kernels/dsa_topk.py:10-22): per row the `keep` largest scores;
every selected score >= every unselected one; among the scores equal to the keep-th largest, the lowest indices; with
vis_only only scores above VISIBLE are selectable, so a row with fewer than keep of them selects exactly those.
Comparisons are IEEE fp32 (-0.0 == +0.0, subnormals compared exactly); scores must not be NaN.

The HIP kernel (csrc/dsa_topk.hip) holds a row as order-preserving integer keys in one workgroup's registers,
narrows the threshold by LDS histograms, and takes the lowest-index ties with a block-wide prefix count; rows longer
than 32,768 scores go through the reference's two-level exact selection (trnrt/models/dsa_long.py:26-42).
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _common as C

NEG_INF = -1e30  # trnrt/models/decoder.py NEG_INF
VISIBLE = -5e29  # trnrt/kernels/dsa_topk.py:58


def supported(rows: int, n: int, keep: int = 2048, vis_only: bool = True) -> bool:
    """Whether the kernel selects `keep` of rows of n scores (trnrt/kernels/dsa_topk.py:489-490; rows is accepted
    for the reference's signature: every row count is supported)."""
    del rows
    return bool(_lib.lib().dsa_topk_supported(int(n), int(keep), int(vis_only)))


def select_indices(scores: torch.Tensor, keep: int, lengths: torch.Tensor | None = None, vis_only: bool = True,
                   max_len: int | None = None, idx: torch.Tensor | None = None, cnt: torch.Tensor | None = None,
                   workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(idx int32 [R, keep] ascending selected positions, 0 past the count; cnt int32 [R]) of scores [R, P] fp32.
    lengths [R] int32: positions at or past a row's length are not selectable (None: all P); max_len an upper bound
    of the lengths (default P). workspace: the caller's (dsa_workspace_bytes(DSA_WS_TOPK, R, 0, keep, max_len),
    zero-filled before its first use; calls leave it so), or None for one kept per stream."""
    dev = C.on_gpu(scores, lengths, idx, cnt, workspace)
    if scores.dim() != 2:
        raise ValueError(f"dsa_topk: scores {tuple(scores.shape)}, expected [rows, P]")
    scores = C.need(C.as_f32(scores), "scores", torch.float32)
    R, P = scores.shape
    if keep < 1:
        raise ValueError(f"dsa_topk: keep {keep}")
    if lengths is not None:
        lengths = C.need(C.as_i32(lengths), "lengths", torch.int32, (R,))
    n = P if (lengths is None or max_len is None) else int(max_len)
    if not 0 <= n <= P:
        raise ValueError(f"dsa_topk: max_len {n} outside [0, {P}]")
    if not supported(R, max(n, 1), keep, vis_only):
        raise NotImplementedError(f"DSA top-k kernel: keep {keep} of {n} scores per row (vis_only={vis_only})")
    if idx is None:
        idx = torch.empty(R, keep, dtype=torch.int32, device=dev)
    if cnt is None:
        cnt = torch.empty(R, dtype=torch.int32, device=dev)
    C.need(idx, "idx", torch.int32, (R, keep))
    C.need(cnt, "cnt", torch.int32, (R,))
    wsb = _lib.workspace_bytes(_lib.DSA_WS_TOPK, R, 0, keep, max(n, 1))
    if workspace is None:
        # the histogram region starts (and ends) at zero: one zero-filled buffer per stream serves every call
        workspace = C.cached_workspace(dev, wsb, "topk")
    ws_len = workspace.numel() * workspace.element_size()
    st = _lib.lib().dsa_topk(C.ptr(scores), C.ptr(lengths), C.ptr(idx), C.ptr(cnt), C.ptr(workspace), ws_len, R, P,
                             n, keep, int(vis_only), C.stream_ptr(dev))
    _lib.check(st, "dsa_topk.select_indices")
    return idx, cnt


def select(scores: torch.Tensor, keep: int, vis_only: bool = True, group: bool = True, kp: int = 1,
           tail: bool = False) -> torch.Tensor:
    """Additive float32 [..., P kp] (0 = selected, NEG_INF = not) of the selection over the last axis
    (trnrt/kernels/dsa_topk.py:495-514 `select`): kp > 1 gives each score's kp tokens its value, tail also takes the
    non-candidate scores' tokens (<= VISIBLE; the caller's causal mask limits them to its own incomplete pool),
    dsa_topk.py:89-93. group is the reference's Trainium layout knob and is ignored."""
    del group
    if tail and not vis_only:
        raise ValueError("tail needs vis_only")
    if kp < 1:
        raise ValueError(f"dsa_topk.select: kp {kp}")
    *lead, P = scores.shape
    R = 1
    for d in lead:
        R *= d
    s = C.as_f32(scores).reshape(R, P)
    dev = C.on_gpu(s)
    mask = torch.empty(R, P * kp, dtype=torch.float32, device=dev)
    if keep >= P:
        # every selectable score, no selection run (the reference's short-cut, dsa_topk.py:510-511 and 103-105):
        # the visible scores with vis_only, else every score
        st = _lib.lib().dsa_topk_mask(None, None, C.ptr(s) if vis_only else None, C.ptr(mask), R, P, P, kp,
                                      int(tail), C.stream_ptr(dev))
        _lib.check(st, "dsa_topk.select")
        return mask.reshape(*lead, P * kp)
    idx, cnt = select_indices(s, keep, vis_only=vis_only)
    st = _lib.lib().dsa_topk_mask(C.ptr(idx), C.ptr(cnt), C.ptr(s) if tail else None, C.ptr(mask), R, keep, P, kp,
                                  int(tail), C.stream_ptr(dev))
    _lib.check(st, "dsa_topk.select")
    return mask.reshape(*lead, P * kp)
