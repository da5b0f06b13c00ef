"""Exact indexer selection of a prefill chunk on gfx950 (the operator surface of trnrt/kernels/dsa_long_select.py).

What it computes, for N queries that share ONE context's keys (trnrt/kernels/dsa_long_select.py:5-11, 119-133):

    index[n, p] = sum_h w[n, h] relu(scale (qI[n, h] . pk[p]))     for p < npool[n]  (NEG_INF otherwise)

with pk the FP8 e4m3 keys times their per-token fp32 scales, then the keep largest candidates of each query, ties to
the lowest key index, all of them when fewer, returned as key indices [N, keep] in ascending order with 0 past the
count min(npool, keep).

How: two launches. csrc/dsa_prefill.hip scores the chunk as a batched GEMM on MFMA, writing the [N, P] fp32 scores
once: with bf16 queries (the reference's form) on bf16 MFMA, the e4m3 keys converted exactly to bf16 once per
workgroup in LDS and shared by four queries; with FP8 e4m3 queries and per-(query, head) scales (qI_scale=) on the
FP8 f8f6f4 MFMA, the keys staying FP8, and each query scale folded into its head weight (relu(a x) = a relu(x),
a > 0), which is the reference's arithmetic on the dequantised queries. Either way relu, the head weights and the
per-token key scale are applied to the fp32 accumulators in registers. csrc/dsa_topk.hip then selects each row
exactly (rows above 32,768 keys by the two-level exact selection of trnrt/models/dsa_long.py:26-42).
The reference's `sub` (its sub-block size) is accepted and ignored: the selection is exact for every shape.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _common as C
from . import dsa_topk

NEG_INF = -1e30  # trnrt/models/decoder.py NEG_INF
VISIBLE = -5e29  # trnrt/kernels/dsa_topk.VISIBLE
D = 128  # index_head_dim
HI_MAX = 64  # heads per query the kernel holds (the reference's NKI kernel takes 32)


def supported(Hi: int, D_: int, P: int, keep: int, sub: int = 0) -> bool:
    """Shapes the kernels take (trnrt/kernels/dsa_long_select.py:136-145): 128-dim keys, 1..64 heads, and a top-k
    of keep out of P that the selection kernel supports. sub is the reference's knob and does not restrict."""
    del sub
    return D_ == D and 1 <= Hi <= HI_MAX and P >= 1 and keep >= 1 and dsa_topk.supported(1, P, keep, True)


def pick_sub(P: int, keep: int) -> int:
    """The reference's sub-block choice (trnrt/kernels/dsa_long_select.py:475-491) has no meaning here: 0."""
    del P, keep
    return 0


def _keys(pk: torch.Tensor, pk_scale: torch.Tensor | None, fp8_q: bool):
    """(key tensor for the C ABI, its scales or None): e4m3fn keys (or their uint8 bits) with pk_scale [P] fp32, or
    bf16 keys without scales (GLM's pool keys, bf16 queries only)."""
    if pk.dtype == torch.bfloat16:
        if pk_scale is not None:
            raise ValueError("dsa_long_select: bf16 keys take no pk_scale")
        if fp8_q:
            raise NotImplementedError("dsa_long_select: FP8 queries take FP8 keys")
        return pk.contiguous(), None
    if pk_scale is None:
        raise ValueError("dsa_long_select: FP8 keys need pk_scale")
    return C.fp8_bytes(pk, "pk"), pk_scale


def scores(qI: torch.Tensor, w: torch.Tensor, pk: torch.Tensor, npool: torch.Tensor, scale: float, *,
           pk_scale: torch.Tensor | None = None, qI_scale: torch.Tensor | None = None, stride: int | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """[N, stride] fp32 index scores (NEG_INF at p >= npool[n] and past P): qI [N, Hi, 128] bf16, or e4m3fn (its
    uint8 bits) with qI_scale [N, Hi] fp32 > 0 (the queries are qI * qI_scale), w [N, Hi] fp32, pk [P, 128] e4m3fn
    keys (or their uint8 bits) with pk_scale [P] fp32, or bf16 keys with no scale (GLM's pool keys; bf16 queries,
    Hi <= 32), npool [N] int (clamped to [0, P]), scale > 0 (trnrt/kernels/dsa_long_select.py:119-133
    `emulate_scores`)."""
    dev = C.on_gpu(qI, w, pk, pk_scale, npool, qI_scale, out)
    fp8_q = qI.dtype in (C.FP8, torch.uint8)
    if fp8_q != (qI_scale is not None):
        raise ValueError("dsa_long_select: FP8 queries need qI_scale, bf16 queries take none")
    if qI.dim() != 3:
        raise ValueError(f"dsa_long_select: qI {tuple(qI.shape)}, expected [N, Hi, {D}]")
    N, Hi, Dq = qI.shape
    pk, pk_scale = _keys(pk, pk_scale, fp8_q)
    if pk.dim() != 2:
        raise ValueError(f"dsa_long_select: pk {tuple(pk.shape)}, expected [P, {D}]")
    P = pk.shape[0]
    if Dq != D or pk.shape[1] != D or not 1 <= Hi <= HI_MAX:
        raise NotImplementedError(f"dsa_long_select: Hi {Hi}, D {Dq}/{pk.shape[1]} (the kernel takes D {D}, "
                                  f"Hi <= {HI_MAX})")
    if not scale > 0:
        raise ValueError(f"dsa_long_select: scale {scale} must be positive")
    stride = P if stride is None else int(stride)
    if stride < P:
        raise ValueError(f"dsa_long_select: stride {stride} < {P} keys")
    if pk_scale is None and Hi > 32:
        raise NotImplementedError(f"dsa_long_select: {Hi} heads over bf16 keys (the kernel takes up to 32)")
    w = C.need(C.as_f32(w), "w", torch.float32, (N, Hi))
    if pk_scale is not None:
        pk_scale = C.need(C.as_f32(pk_scale).reshape(-1), "pk_scale", torch.float32, (P,))
    npool = C.need(C.as_i32(npool.reshape(-1).clamp(0, P)), "npool", torch.int32, (N,))
    if out is None:
        out = torch.empty(N, stride, dtype=torch.float32, device=dev)
    else:
        C.need(out, "out", torch.float32, (N, stride))
    if fp8_q:
        qI = C.fp8_bytes(qI, "qI")
        qI_scale = C.need(C.as_f32(qI_scale), "qI_scale", torch.float32, (N, Hi))
        st = _lib.lib().dsa_indexer_prefill_fp8(C.ptr(qI), C.ptr(qI_scale), C.ptr(w), C.ptr(pk), C.ptr(pk_scale),
                                                C.ptr(npool), C.ptr(out), N, Hi, D, P, stride, float(scale),
                                                C.stream_ptr(dev))
    else:
        qI = C.as_bf16(qI)
        st = _lib.lib().dsa_indexer_prefill(C.ptr(qI), C.ptr(w), C.ptr(pk), C.ptr(pk_scale), C.ptr(npool),
                                            C.ptr(out), N, Hi, D, P, stride, float(scale), C.stream_ptr(dev))
    _lib.check(st, "dsa_long_select.scores")
    return out


def value_order(pools: torch.Tensor, cnt: torch.Tensor, vals: torch.Tensor):
    """A selection (pools [N, keep] ascending, count [N], scores [N, keep]; 0 / NEG_INF past the count) in the
    reference's vorder form (trnrt/kernels/dsa_long_select.py:74-84): the selected pools by score descending, equal
    scores by pool ascending, then 0 / NEG_INF. One HIP kernel (csrc/dsa_compact.hip: a bitonic sort of each row's
    (score key, entry index) pairs in LDS); keep <= 8192."""
    dev = C.on_gpu(pools, cnt, vals)
    N, keep = pools.shape
    p = C.need(pools.to(torch.int64).contiguous(), "pools", torch.int64, (N, keep))
    c = C.need(cnt.to(torch.int64).reshape(N).contiguous(), "cnt", torch.int64, (N,))
    v = C.need(C.as_f32(vals).contiguous(), "vals", torch.float32, (N, keep))
    op = torch.empty(N, keep, dtype=torch.int64, device=dev)
    ov = torch.empty(N, keep, dtype=torch.float32, device=dev)
    st = _lib.lib().dsa_value_order(C.ptr(p), C.ptr(c), C.ptr(v), N, keep, C.ptr(op), C.ptr(ov), C.stream_ptr(dev))
    _lib.check(st, "dsa_long_select.value_order")
    return op, cnt, ov


def workspace_bytes(N: int, P: int, keep: int, tile_rows: int = 0) -> int:
    """Workspace bytes of select() over N queries and P keys (its score tiles included)."""
    return int(_lib.lib().dsa_prefill_select_workspace_bytes(N, P, P, keep, tile_rows, 1))


def select(qI: torch.Tensor, w: torch.Tensor, pk: torch.Tensor, npool: torch.Tensor, keep: int, scale: float,
           sub: int | None = None, vorder: bool = False, *, pk_scale: torch.Tensor | None = None,
           qI_scale: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
           tile_rows: int = 0) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(pools [N, keep] int64 ascending, 0 past the count; count [N] int64; scores [N, keep] fp32, NEG_INF past the
    count) (trnrt/kernels/dsa_long_select.py:494-528 `select`): the scores above (FP8 queries with qI_scale as there),
    then the exact top-keep per query, in one call of dsa_prefill_select (the indexer writes the two-level
    selection's sub-block maxima, and the selection writes the reference's outputs directly). The queries go in
    tiles of tile_rows (0: score tiles of at most 64 MiB), only two tiles' scores held at once (the reference's
    per-tile form, trnrt/kernels/dsa_long_pipe.py:15-25), tiles alternating between the current stream and the
    library's second stream so that one tile's selection overlaps the next tile's scores.
    vorder: the pools in (score descending, pool ascending) order instead. sub is accepted and ignored. workspace:
    workspace_bytes(N, P, keep, tile_rows) bytes, zero-filled before its first use (calls leave it so)."""
    del sub
    dev = C.on_gpu(qI, w, pk, pk_scale, npool, qI_scale, workspace)
    fp8_q = qI.dtype in (C.FP8, torch.uint8)
    if fp8_q != (qI_scale is not None):
        raise ValueError("dsa_long_select: FP8 queries need qI_scale, bf16 queries take none")
    if qI.dim() != 3 or pk.dim() != 2:
        raise ValueError(f"dsa_long_select: qI {tuple(qI.shape)}, pk {tuple(pk.shape)}")
    N, Hi, Dq = qI.shape
    P = pk.shape[0]
    pk, pk_scale = _keys(pk, pk_scale, fp8_q)
    if not supported(Hi, Dq, P, keep) or pk.shape[1] != D or (pk_scale is None and Hi > 32):
        raise NotImplementedError(f"dsa_long_select: Hi {Hi}, D {Dq}, P {P}, keep {keep}")
    if not scale > 0:
        raise ValueError(f"dsa_long_select: scale {scale} must be positive")
    w = C.need(C.as_f32(w), "w", torch.float32, (N, Hi))
    if pk_scale is not None:
        pk_scale = C.need(C.as_f32(pk_scale).reshape(-1), "pk_scale", torch.float32, (P,))
    npool = C.need(C.as_i32(npool.reshape(-1)), "npool", torch.int32, (N,))  # clamped to [0, P] by the kernels
    if fp8_q:
        qI = C.fp8_bytes(qI, "qI")
        qI_scale = C.need(C.as_f32(qI_scale), "qI_scale", torch.float32, (N, Hi))
    else:
        qI = C.as_bf16(qI)
    if tile_rows < 0:
        raise ValueError(f"dsa_long_select: tile_rows {tile_rows}")
    lib = _lib.lib()
    if workspace is None:
        # zero-filled before its first use, left so by every call: one per stream serves every call
        workspace = C.cached_workspace(dev, workspace_bytes(N, P, keep, tile_rows), "prefill_select")
    ws_len = workspace.numel() * workspace.element_size()
    pools = torch.empty(N, keep, dtype=torch.int64, device=dev)
    cnt = torch.empty(N, dtype=torch.int64, device=dev)
    vals = torch.empty(N, keep, dtype=torch.float32, device=dev)
    st = lib.dsa_prefill_select(C.ptr(qI), C.ptr(qI_scale), C.ptr(w), C.ptr(pk), C.ptr(pk_scale), C.ptr(npool),
                                None, C.ptr(pools), C.ptr(cnt), C.ptr(vals), C.ptr(workspace), ws_len, N, Hi, D,
                                P, P, keep, float(scale), int(tile_rows), C.stream_ptr(dev))
    _lib.check(st, "dsa_long_select.select")
    if vorder:
        return value_order(pools, cnt, vals)
    return pools, cnt, vals
