"""CPU oracle of the DSA decode path — TEST INFRASTRUCTURE, never the product.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the checker
(or the timed CPU baseline). The product path (trnrt_amd) never calls it and has no CPU fallback.

A restatement, in torch on the CPU in fp32, of the reference's arithmetic for the DSA path: the per-token (kpool 1)
decode and chunked-prefill forms with per-token FP8 scales and 576-wide KV rows (512 latent + 64 rope columns, value =
the latent part), and GLM's pooled (kpool > 1) forms (pool keys, the bucketed selection with the tail, pool slots,
attention over 512-wide NoPE rows). Each function cites the reference lines it follows. How each one is pinned
(tests/test_oracle_*.py):
- indexer_ref: brute-force per-token loops, exact rational arithmetic on a tiny case, the scale-folding and
  dequantisation invariants, planted mistakes (no relu, a transposed table) that must fail;
- prefill_scores_ref: exact rational arithmetic on a tiny case, a brute-force float64 loop, indexer_ref through an
  identity page table, planted mistakes (an off-by-one candidate mask, no relu, one accumulator dropped) that must
  fail;
- topk_ref: the tie rule as a stable sort; pinned against a second independent form (topk_radix_ref, the
  reference's radix + tie search), a brute-force Python loop, the reference's literal known answer, its adversarial
  score kinds, and a planted wrong tie rule that must fail;
- two_level_ref: equal to topk_ref on the reference's own adversarial cases (trnrt/models/dsa_long.py:26-42 proves
  it exact);
- topk_mask_ref: selection_mask's pins, plus a literal known answer of the pooled form (kp 4 with the tail: each
  score's value over its pool's tokens, every non-candidate kept);
- pool_slots_ref: the tokens its slots attend are exactly the bucketed selection with the tail intersected with the
  causal visibility (the reference's own check, tests/test_dsa_long.py:140-177), for one shared table and per-query
  tables, pages of 4, 8 and 64, kpool 4 and 1; planted mistakes (the tail's last token dropped, no tail) must fail;
- pool_keys_ref / write_pool_keys_ref: a float64 loop over the softmax-gated mean, the known answer of equal gates
  (the plain mean of the keys), the slot layout (pieces of a pool contiguous per page) and a planted mistake (the
  pool-position bias dropped) that must fail;
- cache_write_ref: torch's float -> e4m3fn cast checked against a round-to-nearest-even encoder written from the
  OCP e4m3fn definition over every representable value, every midpoint and its neighbours; known-answer rows; the
  per-token round trip within half an e4m3 step; planted mistakes (no clamp, truncation instead of rounding) that
  must fail;
- sparse_mla_ref: brute-force float64 loops, one selected token -> that row, all masked -> the uniform mean,
  lse == log-sum-exp, split-K combine == unsplit, slot-order invariance;
- splitk_combine_ref: any partition of the slots combines to the unsplit result;
- compact_ref: a brute-force Python loop over every position, the literal known answer of a small mask, equal to
  ascending() when a row has at most keep ones, and a planted mistake (the count not clamped to keep) that must fail;
- slots_compact_ref: equal to sparse_mla_slots_ref (the uncompacted form) on rows with a visible token (masked
  tokens weigh exactly 0), the uniform mean of pool row 0's tokens on an empty row (closed form), invariant under a
  permutation of the slots.
Nothing here is "parity unpinned".
"""

from __future__ import annotations

import math

import torch

NEG_INF = -1e30  # trnrt/models/decoder.py NEG_INF
VISIBLE = -5e29  # trnrt/kernels/dsa_topk.py:58
BIG = float(2**20)  # trnrt/kernels/dsa_topk.py:59


# -- the paged FP8 cache (trnrt/models/decoder.py:481-490, 658-667) ------------------------------------------------


def dequant(q8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 rows of an e4m3fn cache with per-row scales (the reference's `kv.to(dtype)` load, decoder.py:488-490,
    times the BASELINE per-token scale)."""
    return q8.float() * scale.float().reshape(-1, 1)


def token_slots(table_row: torch.Tensor, positions: torch.Tensor, page_size: int) -> torch.Tensor:
    """Cache slots of token positions through one row's page table (trnrt/models/decoder.py:658-667 `_slots`)."""
    pos = positions.long()
    return table_row.long()[pos // page_size] * page_size + pos % page_size


def row_tokens(cache: torch.Tensor, scale: torch.Tensor, table_row: torch.Tensor, L: int, page_size: int):
    """The fp32 dequantised cache rows of positions 0 .. L - 1 of one sequence, in position order."""
    slots = token_slots(table_row, torch.arange(L), page_size)
    return dequant(cache[slots], scale[slots])


# -- indexer (trnrt/kernels/dsa_index.py:44-50; trnrt/models/dsa_long.py:74-84) ------------------------------------


def indexer_ref(q_idx: torch.Tensor, w_k: torch.Tensor, k_cache: torch.Tensor, k_scale: torch.Tensor,
                table: torch.Tensor, ctx_len, page_size: int, stride: int | None = None) -> torch.Tensor:
    """[B, stride] fp32: score[b, t] = sum_h w_k[b, h] relu(q[b, h] . K[t]) for t < ctx_len[b], NEG_INF after
    (the candidate mask, dsa_long.py:82-84). K = the dequantised keys; w_k carries D ** -0.5 (mla.py:629), so this is
    dsa_long.scores' `w relu(s scale)` with the scale folded into w (relu(a x) = a relu(x), a > 0)."""
    B = q_idx.shape[0]
    lens = [int(x) for x in ctx_len]
    stride = max(lens) if stride is None else stride
    out = torch.full((B, stride), NEG_INF, dtype=torch.float32)
    for b in range(B):
        L = lens[b]
        if L == 0:
            continue
        K = row_tokens(k_cache, k_scale, table[b], L, page_size)  # [L, D]
        s = torch.einsum("hd,td->ht", q_idx[b].float(), K)  # dsa_long.py:79-80 (the 3-D branch, one row)
        out[b, :L] = torch.einsum("h,ht->t", w_k[b].float(), torch.relu(s))  # dsa_long.py:81
    return out


def prefill_scores_ref(qI: torch.Tensor, w: torch.Tensor, k8: torch.Tensor, k_scale: torch.Tensor,
                       npool: torch.Tensor, scale: float, stride: int | None = None) -> torch.Tensor:
    """[N, stride] fp32 index scores of N queries over one context's P keys (a prefill chunk), the arithmetic of
    trnrt/kernels/dsa_long_select.py:119-133 `emulate_scores` with pk the dequantised FP8 keys: r_h = relu(scale
    (qI_h . pk)) in fp32, the even heads summed in head order into A0 (which starts at the candidate term: 0 for
    p < npool[n], NEG_INF otherwise, dsa_long_select.py:59-61), the odd heads into A1, the score A0 + A1; positions
    P .. stride - 1 are NEG_INF."""
    N, Hi, _ = qI.shape
    P = k8.shape[0]
    stride = P if stride is None else stride
    pk = dequant(k8, k_scale)  # [P, D]
    s = torch.einsum("nhd,pd->nhp", qI.float(), pk)
    r = torch.relu(s * scale)
    npool = npool.long().clamp(0, P).view(N, 1)
    a0 = torch.where(torch.arange(P).view(1, P) < npool, 0.0, NEG_INF).float()
    a1 = torch.zeros_like(a0)
    for h in range(Hi):
        if h % 2:
            a1 = r[:, h] * w[:, h:h + 1].float() + a1
        else:
            a0 = r[:, h] * w[:, h:h + 1].float() + a0
    out = torch.full((N, stride), NEG_INF, dtype=torch.float32)
    out[:, :P] = a0 + a1
    return out


# -- the cache-store step (trnrt/models/decoder.py:481-486) ----------------------------------------------------------


def cache_write_ref(cache: torch.Tensor, scale: torch.Tensor | None, slots: torch.Tensor, x: torch.Tensor,
                    fp8_max: float = 448.0, per_token: bool = True):
    """(cache', scale') after writing rows x [T, W] at slots [T] (trnrt/models/decoder.py:481-486 `_store`: the row
    clamped to +-fp8_max, then cast to float8_e4m3fn, written with index_put_). per_token: the row is first divided
    by its scale s = max(absmax, 1e-30) / 448, and s is written to scale[slot]; otherwise the scale is 1. Rows whose
    slot is outside the cache are skipped."""
    W = cache.shape[-1]
    c = cache.clone().view(torch.uint8).reshape(-1, W)
    sc = None if scale is None else scale.clone().reshape(-1)
    xf = x.float().reshape(-1, W)
    if per_token:
        s = xf.abs().amax(-1).clamp(min=1e-30) / 448.0
        q = (xf / s.unsqueeze(-1)).clamp(-fp8_max, fp8_max).to(torch.float8_e4m3fn)
    else:
        s = torch.ones(xf.shape[0])
        q = xf.clamp(-fp8_max, fp8_max).to(torch.float8_e4m3fn)
    sl = slots.reshape(-1).long()
    ok = (sl >= 0) & (sl < c.shape[0])
    c[sl[ok]] = q.view(torch.uint8)[ok]
    if sc is not None:
        sc[sl[ok]] = s[ok]
    return c.view(cache.dtype).reshape(cache.shape), sc


def pool_keys_ref(rows: torch.Tensor, ape: torch.Tensor) -> torch.Tensor:
    """Each pool's key [..., Di] from its kpool tokens' indexer rows [..., kpool, 2 Di] (bf16 values: key, then gate
    logits): the per-channel softmax over the pool of gate + ape weighting the keys, in bf16 as
    trnrt/models/glm5_next.py:151-160 `pool_keys` computes it (softmax in fp32, weights and products rounded to
    bf16, the sum over the pool in fp32 rounded to bf16)."""
    Di = ape.shape[-1]
    k = rows[..., :Di].to(torch.bfloat16)
    logits = rows[..., Di:2 * Di].float() + ape.float()
    return (torch.softmax(logits, dim=-2).to(torch.bfloat16) * k).sum(dim=-2)


def write_pool_keys_ref(pool_key: torch.Tensor, rows: torch.Tensor, rows_scale: torch.Tensor | None,
                        positions: torch.Tensor, table: torch.Tensor, slot_mapping: torch.Tensor, ape: torch.Tensor,
                        page_size: int, kp: int) -> torch.Tensor:
    """pool_key' after trnrt/models/mla.py:1277-1296 `write_pool_keys`: the slots of each written token's pool
    (mla.py:1262-1274 `_pool_key_slots`: through the table, or the row's own slot kp times for a padded row), the
    rows there read as bf16 (an FP8 cache through its per-token scale when given), their pool key (pool_keys_ref),
    written as kp pieces. A padded row's kp pieces all land in its own slot; the last one is kept."""
    T = positions.shape[0]
    Di = ape.shape[-1]
    first = positions.long() - positions.long() % kp
    pos = first.view(T, 1) + torch.arange(kp).view(1, kp)
    tb = table.long()
    pages = tb[pos // page_size] if tb.dim() == 1 else tb.gather(1, pos // page_size)
    slots = pages * page_size + pos % page_size
    real = (slot_mapping.long() >= page_size).view(T, 1)
    slots = torch.where(real, slots, slot_mapping.long().view(T, 1).expand(T, kp))
    W = rows.shape[-1]
    r = rows.reshape(-1, W)[slots.reshape(-1)]
    if r.dtype in (torch.float8_e4m3fn, torch.uint8):
        r = r.view(torch.float8_e4m3fn).float()
        if rows_scale is not None:
            r = r * rows_scale.reshape(-1)[slots.reshape(-1)].view(-1, 1)
    keys = pool_keys_ref(r.to(torch.bfloat16).reshape(T, kp, W)[..., :2 * Di], ape)  # [T, Di]
    out = pool_key.clone().reshape(-1, Di // kp)
    pieces = keys.reshape(T, kp, Di // kp)
    for n in range(T):
        for i in range(kp):
            out[int(slots[n, i])] = pieces[n, i]
    return out.reshape(pool_key.shape)


def e4m3fn_encode(v: float) -> int:
    """The OCP e4m3fn byte of a finite |v| <= 448 by its definition (1 sign bit, 4 exponent bits with bias 7, 3
    mantissa bits; exponent 0 is subnormal with step 2^-9; no infinities; 0x7F is NaN), rounded to nearest with ties
    to the even code, in exact rational arithmetic: the independent form that torch's cast is checked against."""
    from fractions import Fraction

    a = abs(Fraction(v))
    sign = 0x80 if math.copysign(1.0, v) < 0 else 0
    vals = []  # (value, code) of every non-negative finite code, ascending
    for code in range(0x7F):
        e, m = code >> 3, code & 7
        vals.append((Fraction(m, 8) * Fraction(2) ** -6 if e == 0 else (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7),
                     code))
    lo = max((c for c in vals if c[0] <= a), key=lambda c: c[0])
    hi = min((c for c in vals if c[0] >= a), key=lambda c: c[0])
    if a - lo[0] < hi[0] - a or lo[0] == a:
        code = lo[1]
    elif a - lo[0] > hi[0] - a:
        code = hi[1]
    else:  # a tie: the even code
        code = lo[1] if lo[1] % 2 == 0 else hi[1]
    return sign | code


# -- selection (trnrt/models/dsa_select.py:33-38; trnrt/models/dsa_long.py:94-137) ----------------------------------


def selection_mask(scores: torch.Tensor, keep: int, vis_only: bool = True) -> torch.Tensor:
    """bool [R, P]: the tie rule as a stable sort (dsa_select.reference_mask: descending score, then ascending
    index, the first keep), restricted to scores > VISIBLE under vis_only (tests/test_dsa_topk.py:56-60)."""
    s = scores.float()
    if keep >= s.shape[-1]:
        sel = torch.ones_like(s, dtype=torch.bool)
    else:
        order = torch.sort(s, dim=-1, descending=True, stable=True).indices[..., :keep]
        sel = torch.zeros_like(s, dtype=torch.bool).scatter(-1, order, True)
    if vis_only:
        sel &= s > VISIBLE
    return sel


def ascending(sel: torch.Tensor, keep: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(indices [R, keep] int64 ascending, 0 past the count; count [R]) of a mask with <= keep True per row
    (dsa_long.py:94-112 `_ascending`)."""
    R, P = sel.shape
    idx = torch.zeros(R, keep, dtype=torch.int64)
    cnt = sel.sum(-1).to(torch.int64)
    for r in range(R):
        nz = sel[r].nonzero().flatten()
        idx[r, : nz.numel()] = nz
    return idx, cnt


def compact_ref(sel: torch.Tensor, keep: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(indices [N, keep] int64 ascending, count [N] int64) of a 0 / 1 float mask [N, M] (an entry counts as a one
    when above 0.5): the positions of each row's first keep ones, 0 past the count, count = min(ones, keep)
    (trnrt/models/dsa_long.py:140-166 `compact`: the k-th one for k < count, the count clamped to [0, keep])."""
    N, M = sel.shape
    idx = torch.zeros(N, keep, dtype=torch.int64)
    cnt = torch.zeros(N, dtype=torch.int64)
    for n in range(N):
        nz = (sel[n].float() > 0.5).nonzero().flatten()[:keep]
        idx[n, : nz.numel()] = nz
        cnt[n] = nz.numel()
    return idx, cnt


def topk_ref(scores: torch.Tensor, keep: int, lengths=None, vis_only: bool = True):
    """(idx [R, keep] int64 ascending, cnt [R]) of the exact selection (dsa_long.select_reference, dsa_long.py:
    114-118); positions at or past lengths[r] are not candidates (the NEG_INF of dsa_long.scores, :82-84)."""
    s = scores.float().clone()
    if lengths is not None:
        P = s.shape[1]
        L = torch.as_tensor([int(x) for x in lengths]).view(-1, 1)
        dead = torch.arange(P).view(1, P) >= L
        if vis_only:
            s[dead] = NEG_INF
        else:
            s[dead] = float("-inf")
    sel = selection_mask(s, keep, vis_only)
    if lengths is not None and not vis_only:
        sel &= ~dead
    return ascending(sel, keep)


def topk_mask_ref(scores: torch.Tensor, keep: int, vis_only: bool = True, kp: int = 1,
                  tail: bool = False) -> torch.Tensor:
    """The additive mask [R, P kp] of dsa_topk.select (trnrt/kernels/dsa_topk.py:89-93 `_out`): the selection
    (selection_mask), with tail also every non-candidate score (<= VISIBLE), each score's value repeated for its kp
    tokens."""
    sel = selection_mask(scores, keep, vis_only)
    if tail:
        sel = sel | ~(scores.float() > VISIBLE)
    out = torch.where(sel, 0.0, NEG_INF)
    return out.repeat_interleave(kp, dim=-1) if kp > 1 else out


def topk_radix_ref(scores: torch.Tensor, keep: int, vis_only: bool = True) -> torch.Tensor:
    """bool [R, P]: the reference kernel's algorithm (trnrt/kernels/dsa_topk.py:96-127 `emulate`), a second form
    independent of the sort: the sign step, a radix search over the threshold's bit pattern (31 rounds), and the
    lowest-index tie search over positions by binary lifting."""
    s = scores.float()
    R, P = s.shape
    vis = s > VISIBLE
    if keep >= P:
        return vis.clone() if vis_only else torch.ones_like(vis)
    f = (s >= 0).float().sum(-1, keepdim=True) < keep
    sg = torch.where(f, -1.0, 1.0)
    s2 = s * sg
    k2 = torch.where(f, float(P + 1 - keep), float(keep))
    pre = torch.zeros(R, 1, dtype=torch.int32)
    for b in range(30, -1, -1):
        cand = pre | (1 << b)
        ok = (s2 >= cand.view(torch.float32)).float().sum(-1, keepdim=True) >= k2
        pre = pre | (ok.to(torch.int32) << b)
    th = pre.view(torch.float32) * sg
    above = s > th
    room = keep - above.float().sum(-1, keepdim=True)
    j = torch.arange(P, dtype=torch.float32)
    tj = torch.where(s == th, j, BIG)
    lim = torch.zeros(R, 1)
    for b in range(P.bit_length() - 1, -1, -1):
        ok = (tj < lim + 2.0**b).float().sum(-1, keepdim=True) < room
        lim = lim + ok.float() * 2.0**b
    sel = above | (tj <= lim)
    if vis_only:
        sel &= vis
    return sel


def two_level_ref(scores: torch.Tensor, keep: int, sub: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The two-level exact selection by sub-block maxima (trnrt/models/dsa_long.py:26-42 proof, 120-132 algorithm):
    the top-keep sub-blocks by maximum (ties to the lowest block), then the top-keep of their elements in position
    order."""
    R, P = scores.shape
    NB = -(-P // sub)
    if NB <= keep:
        return ascending(selection_mask(scores, keep), keep)
    pad = NB * sub - P
    s = torch.cat([scores.float(), torch.full((R, pad + sub), NEG_INF)], dim=1)
    blocks = s.view(R, NB + 1, sub)
    bm = blocks[:, :NB].amax(-1)
    bidx, bcnt = ascending(selection_mask(bm, keep), keep)
    bidx = torch.where(torch.arange(keep).view(1, keep) < bcnt.view(R, 1), bidx, NB)
    cand = torch.gather(blocks, 1, bidx.unsqueeze(-1).expand(R, keep, sub)).reshape(R, keep * sub)
    cidx, cnt = ascending(selection_mask(cand, keep), keep)
    pools = torch.gather(bidx, 1, cidx // sub) * sub + cidx % sub
    pools = torch.where(torch.arange(keep).view(1, keep) < cnt.view(R, 1), pools, 0)
    return pools, cnt


# -- sparse MLA attention (trnrt/kernels/dsa_decode.py:26-37; trnrt/kernels/dsa_slots.py:48-65) ---------------------


def pool_slots_ref(pools: torch.Tensor, cnt: torch.Tensor, npool: torch.Tensor, positions: torch.Tensor,
                   table: torch.Tensor, page_size: int, kp: int, n_slots: int):
    """(rows [N, n_slots] int64, bias [N, n_slots, kp]) of trnrt/models/dsa_long.py:189-215 `slots`: slot s < keep the
    selected pool pools[n, s] (live below cnt[n]), slot keep the tail pool npool[n] (min(npool, last pool); its tokens
    kp npool + t <= positions[n] live), the rest pool 0 (dead); rows = table[pool // ppp] ppp + pool % ppp (the latent
    cache viewed as [slots / kp, kp R], ppp = page_size / kp); table [Pp] shared or [N, Pp] per query."""
    N, keep = pools.shape
    ppp = page_size // kp
    Pp = table.shape[-1]
    tb = table.long().view(1, Pp).expand(N, Pp) if table.dim() == 1 else table.long()
    rows = torch.zeros(N, n_slots, dtype=torch.int64)
    bias = torch.full((N, n_slots, kp), NEG_INF)
    for n in range(N):
        for s in range(n_slots):
            if s < keep:
                pl = int(pools[n, s])
            elif s == keep:
                pl = min(int(npool[n]), Pp * ppp - 1)
            else:
                pl = 0
            rows[n, s] = int(tb[n, pl // ppp]) * ppp + pl % ppp
            for t in range(kp):
                live = (s < keep and s < int(cnt[n])) or (s == keep and int(npool[n]) * kp + t <= int(positions[n]))
                if live:
                    bias[n, s, t] = 0.0
    return rows, bias


def sparse_mla_rows_ref(q: torch.Tensor, K: torch.Tensor, bias: torch.Tensor, scale: float, dv: int = 512):
    """(o [H, dv], lse [H]) of one query row over its gathered fp32 key rows K [NS, dqk] with additive bias [NS]:
    s = scale q . K + bias, p = softmax(s), o = p K[:, :dv] (dsa_decode.emulate with the value = the first dv
    columns), lse = max + log sum exp(s - max) (dsa_slots.emulate)."""
    s = torch.einsum("hr,tr->ht", q.float(), K) * scale + bias.view(1, -1)
    p = torch.softmax(s, dim=-1)
    o = p @ K[:, :dv]
    m = s.amax(-1)
    return o, m + torch.log(torch.exp(s - m.unsqueeze(-1)).sum(-1))


def sparse_mla_ref(q: torch.Tensor, kv_cache: torch.Tensor, kv_scale: torch.Tensor, idx: torch.Tensor,
                   cnt: torch.Tensor, table: torch.Tensor, page_size: int, scale: float, dv: int = 512):
    """(o [B, H, dv] fp32, lse [B, H]) over the selected tokens: slot k of row b is token idx[b, k] (its cache row
    through the page table, dsa_long.slots at kp 1, dsa_long.py:189-215), bias 0 for k < cnt[b] and NEG_INF after
    (the slots past the count read token idx[b, k], 0 in the selection's output)."""
    B, H, _ = q.shape
    keep = idx.shape[1]
    o = torch.empty(B, H, dv)
    lse = torch.empty(B, H)
    for b in range(B):
        slots = token_slots(table[b], idx[b].long().clamp(min=0), page_size)
        K = dequant(kv_cache[slots], kv_scale[slots])
        bias = torch.where(torch.arange(keep) < int(cnt[b]), 0.0, NEG_INF)
        o[b], lse[b] = sparse_mla_rows_ref(q[b], K, bias, scale, dv)
    return o, lse


def sparse_mla_slots_ref(q: torch.Tensor, kv_cache: torch.Tensor, kv_scale: torch.Tensor, rows: torch.Tensor,
                         bias: torch.Tensor, scale: float, dv: int = 512):
    """The row form (dsa_decode.attend's `rows` + `bias`): slot k of row b is cache row rows[b, k]."""
    B, H, _ = q.shape
    o = torch.empty(B, H, dv)
    lse = torch.empty(B, H)
    for b in range(B):
        r = rows[b].long()
        K = dequant(kv_cache[r], kv_scale[r])
        o[b], lse[b] = sparse_mla_rows_ref(q[b], K, bias[b].float().reshape(-1), scale, dv)
    return o, lse


def slots_compact_ref(q: torch.Tensor, kv_cache: torch.Tensor, kv_scale: torch.Tensor, rows: torch.Tensor,
                      bias: torch.Tensor, scale: float, dv: int = 512):
    """The compacted slot attention (trnrt/kernels/dsa_slots_c.py:92-103 `emulate`): rows [B, NS] pool rows of the
    cache viewed as [slots / kp, kp rows], bias [B, NS, kp]. A row attends its visible tokens (bias above
    NEG_INF / 2; pool row kp + t) with bias 0; a row with none attends pool row 0's kp tokens all at NEG_INF (the
    compacted form's empty entries), i.e. their uniform mean."""
    B, H, _ = q.shape
    kp = bias.shape[-1] if bias.dim() == 3 else 1
    o = torch.empty(B, H, dv)
    lse = torch.empty(B, H)
    for b in range(B):
        bb = bias[b].float().reshape(-1)
        vis = (bb > NEG_INF / 2).nonzero().flatten()
        if vis.numel():
            tok = rows[b].long()[vis // kp] * kp + vis % kp
            bz = torch.zeros(vis.numel())
        else:
            tok = torch.arange(kp)
            bz = torch.full((kp,), NEG_INF)
        K = dequant(kv_cache[tok], kv_scale[tok])
        o[b], lse[b] = sparse_mla_rows_ref(q[b], K, bz, scale, dv)
    return o, lse


def splitk_combine_ref(o_parts: torch.Tensor, lse_parts: torch.Tensor):
    """(o, lse) of partial attentions over disjoint slot sets (trnrt/models/mla.py:853-856, 1152-1160):
    LSE = logsumexp_r lse_r, o = sum_r exp(lse_r - LSE) o_r. o_parts [R, ..., dv], lse_parts [R, ...]."""
    LSE = torch.logsumexp(lse_parts, dim=0)
    return (o_parts * torch.exp(lse_parts - LSE).unsqueeze(-1)).sum(0), LSE


# -- the layer (trnrt/models/mla.py:506-528 `attention_long`, kp 1) -------------------------------------------------


def decode_layer_ref(inp, keep: int | None = None):
    """(scores, idx, cnt, o, lse) of one decode layer step on an Inputs bundle (trnrt_amd.workloads): indexer ->
    exact top-keep -> sparse MLA over the selected tokens."""
    cfg = inp.cfg
    keep = cfg.keep if keep is None else keep
    stride = inp.max_pages * cfg.page_size
    sc = indexer_ref(inp.q_idx, inp.w_k, inp.k_cache, inp.k_scale, inp.table, inp.ctx_len, cfg.page_size, stride)
    idx, cnt = topk_ref(sc, keep, inp.ctx_len)
    o, lse = sparse_mla_ref(inp.q, inp.kv_cache, inp.kv_scale, idx, cnt, inp.table, cfg.page_size, cfg.scale)
    return sc, idx, cnt, o, lse
