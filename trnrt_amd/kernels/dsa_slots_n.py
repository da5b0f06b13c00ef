"""Slot attention over a run-time number of query rows (the operator surface of trnrt/kernels/dsa_slots_n.py
`attend`): the same arithmetic as dsa_decode.attend (trnrt/kernels/dsa_slots.py:48-65), o and optionally lse.

On gfx950 one launch covers every row (there is no device loop to bound), so the rows past n are computed as well;
the reference leaves them unwritten on its device and callers read only the first n.
"""

from __future__ import annotations

import torch

from . import dsa_decode

NEG_INF = -1e30


def attend(q_lat: torch.Tensor, kc: torch.Tensor, rows: torch.Tensor, bias: torch.Tensor, scale: float,
           n: torch.Tensor | int | None = None, lse: bool = False, fallback=False, *, kc_scale: torch.Tensor):
    """o [N, H, 512] fp32 (and lse [N, H]) of q_lat [N, H, 576] over rows [N, NS] with bias [N, NS] or [N, NS, kp]
    (kp tokens per slot, as dsa_decode.attend); n (a 1-element int tensor or int) is the reference's live-row count
    and fallback its Trainium kernel choice, both accepted for its signature."""
    del n, fallback
    return dsa_decode.attend(q_lat, kc, rows, bias, scale, kc_scale=kc_scale, lse=lse)
