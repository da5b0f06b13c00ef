"""Quantise-on-write into the paged FP8 caches on gfx950: the cache-store step before the DSA path (the operator of
trnrt/models/decoder.py:481-486 `_store`, which trnrt/models/mla.py:445-446 calls for the latent rows and the
indexer-key rows at the step's slot_mapping).

    store(cache, slots, x, fp8_max)             the reference's form: cache[slot] = e4m3fn(clamp(x, +-fp8_max))
    store(cache, slots, x, fp8_max, scale=s)    this build's format: per-token s = max(absmax(row), 1e-30) / 448,
                                                cache[slot] = e4m3fn(clamp(x / s, +-fp8_max)), s[slot] = s

The HIP kernel (csrc/dsa_cache.hip) converts each row in one wave: fp32 arithmetic with a correctly rounded
division and round-to-nearest-even into e4m3fn, which is torch's float -> float8_e4m3fn cast.

write_pool_keys is the pooled (GLM) indexer's key write of the same step (trnrt/models/mla.py:1277-1296): each written
token's pool key, a softmax-gated mean of the pool's cached indexer keys, into the pool-key cache.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _common as C

FP8_MAX = 448.0  # the e4m3fn maximum (trnrt/engine/model_runner.py:62-70 off Neuron)


def slots_of(positions: torch.Tensor, table: torch.Tensor, page_size: int) -> torch.Tensor:
    """Cache slots of token positions [T] through one sequence's table [P] or per-row tables [T, P]
    (trnrt/models/decoder.py:658-667 `_slots` for one position per row): table[pos // ps] * ps + pos % ps, int64."""
    pos = positions.to(torch.int64)
    tb = table.to(torch.int64)
    pages = tb[pos // page_size] if tb.dim() == 1 else tb.gather(1, (pos // page_size).view(-1, 1)).view(-1)
    return pages * page_size + pos % page_size


def store(cache: torch.Tensor, slots: torch.Tensor, x: torch.Tensor, fp8_max: float = FP8_MAX, *,
          scale: torch.Tensor | None = None) -> None:
    """Writes the rows x [T, W] (or [T, 1, W]; bf16 or fp32) into cache [slots, W] (or [slots, 1, W]; e4m3fn or its
    uint8 bits) at slots [T] int64, in place, on the current stream. With scale [slots] fp32 (this build's format)
    each row gets its own scale; without, the rows are clamped and cast as the reference does (KV scale 1.0). Rows
    whose slot is outside the cache are not written."""
    dev = C.on_gpu(cache, slots, x, scale)
    if cache.dtype not in (C.FP8, torch.uint8):
        raise NotImplementedError(f"dsa_cache.store: a {cache.dtype} cache; the kernel writes float8_e4m3fn caches")
    if not cache.is_contiguous():
        raise ValueError("dsa_cache.store: the cache must be contiguous")
    W = cache.shape[-1]
    num_slots = cache.numel() // W
    if x.shape[-1] != W or x.numel() % W:
        raise ValueError(f"dsa_cache.store: rows {tuple(x.shape)} for a cache of width {W}")
    T = x.numel() // W
    if x.dtype == torch.bfloat16:
        x_fp32 = 0
    elif x.dtype == torch.float32:
        x_fp32 = 1
    else:
        raise ValueError(f"dsa_cache.store: rows of dtype {x.dtype}, expected bfloat16 or float32")
    x = x.contiguous()
    slots = C.need(slots.reshape(-1).to(torch.int64).contiguous(), "slots", torch.int64, (T,))
    if scale is not None:
        scale = C.need(scale.reshape(-1), "scale", torch.float32, (num_slots,))
    if not 0.0 < fp8_max <= FP8_MAX:
        raise ValueError(f"dsa_cache.store: fp8_max {fp8_max} outside (0, {FP8_MAX}]")
    st = _lib.lib().dsa_cache_write(C.ptr(x), x_fp32, C.ptr(slots), C.ptr(cache), C.ptr(scale), T, W, num_slots,
                                    int(scale is not None), float(fp8_max), C.stream_ptr(dev))
    _lib.check(st, "dsa_cache.store")


def write_pool_keys(pool_key: torch.Tensor, rows: torch.Tensor, positions: torch.Tensor, table: torch.Tensor,
                    slot_mapping: torch.Tensor, ape: torch.Tensor, page_size: int, kp: int, *,
                    rows_scale: torch.Tensor | None = None) -> None:
    """Recomputes the pool key of every written token's pool and writes it to pool_key [slots, 128 / kp] bf16 as kp
    pieces, one per slot of the pool (trnrt/models/mla.py:1277-1296 `write_pool_keys`, glm5_next.py:151-160
    `pool_keys`): rows the cached indexer rows [slots, W >= 256] ([key 128 | gate logits 128], e4m3fn with optional
    per-token rows_scale, or bf16), positions [T], table [T, Pp] or one [Pp], slot_mapping [T] (a padded row, in the
    null page, writes only its own slot), ape [kp, 128] (the pool-position bias, idx_pool_ape)."""
    dev = C.on_gpu(pool_key, rows, positions, table, slot_mapping, ape, rows_scale)
    if pool_key.dtype != torch.bfloat16 or not pool_key.is_contiguous():
        raise ValueError("dsa_cache.write_pool_keys: pool_key must be a contiguous bf16 cache")
    W = rows.shape[-1]
    num_slots = rows.numel() // W
    if pool_key.numel() != num_slots * (128 // kp):
        raise ValueError(f"dsa_cache.write_pool_keys: pool_key {tuple(pool_key.shape)} for {num_slots} slots, kp {kp}")
    fp8 = rows.dtype in (C.FP8, torch.uint8)
    if not fp8 and rows.dtype != torch.bfloat16:
        raise ValueError(f"dsa_cache.write_pool_keys: rows of dtype {rows.dtype}")
    if not rows.is_contiguous():
        raise ValueError("dsa_cache.write_pool_keys: rows must be contiguous")
    T = positions.numel()
    pos = C.need(C.as_i32(positions.reshape(-1)), "positions", torch.int32, (T,))
    sm = C.need(slot_mapping.reshape(-1).to(torch.int64).contiguous(), "slot_mapping", torch.int64, (T,))
    tb = C.as_i32(table)
    if tb.dim() not in (1, 2) or (tb.dim() == 2 and tb.shape[0] != T):
        raise ValueError(f"dsa_cache.write_pool_keys: table {tuple(table.shape)} for {T} rows")
    ap = C.need(C.as_f32(ape), "ape", torch.float32, (kp, 128))
    rs = None if rows_scale is None else C.need(C.as_f32(rows_scale).reshape(-1), "rows_scale", torch.float32,
                                                 (num_slots,))
    st = _lib.lib().dsa_pool_keys_write(C.ptr(rows), int(fp8), C.ptr(rs), W, C.ptr(ap), C.ptr(pos), C.ptr(tb),
                                        int(tb.dim() == 1), tb.shape[-1], C.ptr(sm), C.ptr(pool_key), T, kp,
                                        page_size, num_slots, C.stream_ptr(dev))
    _lib.check(st, "dsa_cache.write_pool_keys")
