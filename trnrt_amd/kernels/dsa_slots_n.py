"""Slot attention over a run-time number of query rows (the operator surface of trnrt/kernels/dsa_slots_n.py
`attend`, trnrt/kernels/dsa_slots_n.py:154-203): the arithmetic of dsa_decode.attend's row form
(trnrt/kernels/dsa_slots.py:48-65), o and optionally lse, over the first n rows only.

n is a one-element int tensor on the device (the reference's padded prefill calls pass their live row count that
way, trnrt/models/mla.py:1208,1215), read by the kernels themselves: every workgroup of a row at or past n returns at
once, so those rows cost nothing and their outputs are not written. The reference leaves them unwritten on its
device and zero on the host; the outputs allocated here start at zero, so they read as the host's, and an `out`
passed in keeps whatever it held there.
"""

from __future__ import annotations

import torch

from . import _common as C
from . import dsa_decode

NEG_INF = -1e30


def attend(q_lat: torch.Tensor, kc: torch.Tensor, rows: torch.Tensor, bias: torch.Tensor, scale: float,
           n: torch.Tensor | int | None = None, lse: bool = False, fallback=False, *,
           kc_scale: torch.Tensor | None = None, out: torch.Tensor | None = None, splits: int = 0,
           workspace: torch.Tensor | None = None):
    """o [N, H, 512] fp32 (and lse [N, H]) of q_lat [N, H, 576 or 512] over rows [N, NS] with bias [N, NS] or
    [N, NS, kp] (kp tokens per slot, as dsa_decode.attend), for rows r < n: n a one-element int tensor (on the device:
    no host synchronisation) or an int, 0 .. N (None: every row). kc_scale: the cache's per-token scales, or None for
    the reference's unscaled cache. fallback (the reference's choice among its Trainium kernels) is accepted for its
    signature. out: fp32 [N, H, 512] to write the live rows into (the others untouched)."""
    del fallback
    N = q_lat.shape[0]
    dev = C.on_gpu(q_lat, kc, rows, bias, kc_scale, out)
    if n is None:
        n_live = torch.full((1,), N, dtype=torch.int32, device=dev)
    elif isinstance(n, torch.Tensor):
        if n.numel() != 1:
            raise ValueError(f"dsa_slots_n.attend: n has {n.numel()} elements, expected one")
        n_live = n.reshape(1).to(device=dev, dtype=torch.int32)
    else:
        n_live = torch.full((1,), int(n), dtype=torch.int32, device=dev)
    rows, bias = dsa_decode.pool_token_rows(rows, bias)
    if out is None:
        out = torch.zeros(N, q_lat.shape[1], dsa_decode.DV, dtype=torch.float32, device=dev)
    return dsa_decode._run(q_lat, kc, kc_scale, scale, rows=rows, bias=bias, lse=lse, splits=splits, out=out,
                           workspace=workspace, n_live=n_live)
