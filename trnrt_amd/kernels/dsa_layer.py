"""One DSA decode layer step on gfx950 in one call: indexer -> top-k -> sparse MLA, the order of
trnrt/models/mla.py:506-528 `attention_long` (at kpool 1, with the q_lat / W_UV projections outside, as there). For
rows of up to 32,768 tokens the step is one kernel launch (csrc/dsa_fused.hip); otherwise, or with chain=True, the
separate kernels enqueued back to back.

DecodeLayer preallocates the intermediates (scores, indices, counts) and the workspace once for a batch shape, so a
step allocates nothing and can be captured in a HIP graph; step() enqueues the three operators on the current stream
through the C ABI's dsa_decode_layer. PooledDecodeLayer is the same for GLM's pooled indexer (kpool > 1): scores of
the bf16 pool keys, the top pools, attention over their tokens and the query's tail pool (dsa_pooled_decode_layer).
"""

from __future__ import annotations

import torch

from .. import _lib
from . import _common as C

NEG_INF = -1e30


def _status(workspace: torch.Tensor | None, device: torch.device, clear: bool) -> dict:
    ptr = workspace.data_ptr() if workspace is not None else None
    gave_up, two = _lib.layer_status(ptr, torch.cuda.current_stream(device).cuda_stream, clear)
    return {"gave_up": gave_up, "two_exchange": two}


def _verify(workspace: torch.Tensor | None, device: torch.device, what: str) -> None:
    """RuntimeError if a barrier wait on this workspace gave up since the last check (the count is then cleared):
    the reference raises on the host, never in a kernel (trnrt/kernels/dsa_index.py:258-259)."""
    st = _status(workspace, device, clear=False)
    if st["gave_up"]:
        _status(workspace, device, clear=True)
        raise RuntimeError(f"{what}: {st['gave_up']} barrier wait(s) gave up; the outputs of the steps since the last "
                           "check may be wrong (another kernel held CUs the one-launch layer needs)")


class DecodeLayer:
    """Buffers and launch parameters of a decode step over B rows with up to max_pages pages each.

    B, Hi (indexer heads), H (query heads), max_pages, page_size, num_pages (cache pages incl. the null page 0),
    keep (top-k), scale (softmax scale), max_len (the longest context a step may see; default max_pages page_size),
    splits (attention split-K; 0 = chosen for the GPU)."""

    def __init__(self, B: int, Hi: int, H: int, max_pages: int, page_size: int, num_pages: int, keep: int = 2048,
                 scale: float = 192 ** -0.5, max_len: int | None = None, splits: int = 0,
                 device: torch.device | str = "cuda", chain: bool = False):
        self.chain = chain  # True: the separate-kernel form (dsa_decode_layer_chain) even where one launch applies
        self.B, self.Hi, self.H = B, Hi, H
        self.max_pages, self.page_size, self.num_pages = max_pages, page_size, num_pages
        self.keep, self.scale, self.splits = keep, float(scale), splits
        self.stride = max_pages * page_size
        self.max_len = self.stride if max_len is None else int(max_len)
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("trnrt_amd DSA kernels run on the GPU only (libdsa_gfx950.so)")
        self.device = dev
        self.scores = torch.empty(B, self.stride, dtype=torch.float32, device=dev)
        self.idx = torch.empty(B, keep, dtype=torch.int32, device=dev)
        self.cnt = torch.empty(B, dtype=torch.int32, device=dev)
        self.out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty(B, H, dtype=torch.float32, device=dev)
        wsb = _lib.workspace_bytes(_lib.DSA_WS_LAYER, B, H, keep, self.max_len, splits)
        # zero once: the calls keep the regions that must start at zero (the top-k histograms) at zero
        self.workspace = C.zeroed_workspace(max(wsb, 256), dev)

    def status(self, clear: bool = False) -> dict:
        """The workspace's status words since the last clear (synchronises the current stream): `gave_up`, barrier
        waits that gave up (non-zero: some step's outputs may be wrong; the one-launch kernel needs all its
        workgroups resident at once), and `two_exchange`, rows selected in the two-exchange form."""
        return _status(self.workspace, self.device, clear)

    def step(self, q_idx: torch.Tensor, w: torch.Tensor, k_cache: torch.Tensor, k_scale: torch.Tensor,
             q: torch.Tensor, kv_cache: torch.Tensor, kv_scale: torch.Tensor | None, table: torch.Tensor,
             ctx_len: torch.Tensor, check: bool = True, verify: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """(out bf16 [B, H, 512], lse fp32 [B, H]) of one layer step; self.scores / idx / cnt hold the intermediates.
        q_idx [B, Hi, 128] bf16, w [B, Hi] fp32 (D ** -0.5 folded in), k_cache [slots, 128] e4m3fn + k_scale [slots],
        q [B, H, 576] bf16, kv_cache [slots, 576] e4m3fn + kv_scale [slots] (None: the reference's unscaled cache),
        table [B, max_pages] int32, ctx_len [B] int32 (each <= max_len). check=False skips the Python-side argument
        checks (the C ABI still checks sizes).
        verify=True synchronises after the step and raises RuntimeError if a barrier wait of this or an earlier
        unverified step gave up (clearing the count)."""
        B, Hi, H = self.B, self.Hi, self.H
        if check:
            C.on_gpu(q_idx, w, k_cache, k_scale, q, kv_cache, kv_scale, table, ctx_len)
            C.need(q_idx, "q_idx", torch.bfloat16, (B, Hi, 128))
            C.need(w, "w", torch.float32, (B, Hi))
            C.need(q, "q", torch.bfloat16, (B, H, 576))
            C.need(table, "table", torch.int32, (B, self.max_pages))
            C.need(ctx_len, "ctx_len", torch.int32, (B,))
            C.fp8_bytes(k_cache, "k_cache")
            C.fp8_bytes(kv_cache, "kv_cache")
            slots = self.num_pages * self.page_size
            if k_cache.numel() != slots * 128 or kv_cache.numel() != slots * 576:
                raise ValueError(f"caches of {k_cache.numel()} / {kv_cache.numel()} bytes for {slots} slots")
            C.need(k_scale, "k_scale", torch.float32, (slots,))
            if kv_scale is not None:
                C.need(kv_scale, "kv_scale", torch.float32, (slots,))
        fn = _lib.lib().dsa_decode_layer_chain if self.chain else _lib.lib().dsa_decode_layer
        st = fn(
            q_idx.data_ptr(), w.data_ptr(), k_cache.data_ptr(), k_scale.data_ptr(), q.data_ptr(),
            kv_cache.data_ptr(), C.ptr(kv_scale), table.data_ptr(), ctx_len.data_ptr(), self.scores.data_ptr(),
            self.idx.data_ptr(), self.cnt.data_ptr(), self.out.data_ptr(), self.lse.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), B, Hi, H, self.max_pages, self.page_size,
            self.num_pages, self.stride, self.max_len, self.keep, self.scale, self.splits,
            torch.cuda.current_stream(self.device).cuda_stream)
        _lib.check(st, "dsa_layer.step")
        if verify:
            _verify(self.workspace, self.device, "dsa_layer.step")
        return self.out, self.lse


class PooledDecodeLayer:
    """Buffers and launch parameters of a pooled (GLM, kpool kp > 1) decode step over B rows with up to max_pages
    pages each: the pooled indexer over the bf16 pool-key cache, the exact top-keep pools, sparse MLA over their
    tokens and the tail (trnrt/models/mla.py:505-526 `attention_long` for a decode batch), enqueued by one call of the
    C ABI's dsa_pooled_decode_layer: one kernel launch per 8 rows where the shapes allow (512-wide rows, at most 32
    indexer heads, rows of at most 8,192 pools), the separate kernels otherwise or with chain=True. Nothing is
    allocated per step.

    B, Hi (indexer heads), H (query heads), dqk (512: GLM's NoPE latent, or 576), max_pages, page_size, num_pages
    (cache pages incl. the null page 0), kp, keep (pools: topk / kp), scale (softmax scale), splits (attention
    split-K; 0 = chosen for the GPU; any other count takes the separate kernels)."""

    def __init__(self, B: int, Hi: int, H: int, dqk: int, max_pages: int, page_size: int, num_pages: int, kp: int,
                 keep: int, scale: float, splits: int = 0, device: torch.device | str = "cuda", chain: bool = False):
        self.chain = chain  # True: the separate kernels (dsa_pooled_decode_layer_chain) even where one launch applies
        self.B, self.Hi, self.H, self.dqk = B, Hi, H, dqk
        self.max_pages, self.page_size, self.num_pages = max_pages, page_size, num_pages
        self.kp, self.keep, self.scale, self.splits = kp, keep, float(scale), splits
        if kp < 2 or kp & (kp - 1) or page_size % kp:
            raise ValueError(f"PooledDecodeLayer: kpool {kp} with pages of {page_size}")
        self.stride = max_pages * (page_size // kp)
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("trnrt_amd DSA kernels run on the GPU only (libdsa_gfx950.so)")
        self.device = dev
        self.scores = torch.empty(B, self.stride, dtype=torch.float32, device=dev)
        self.pools = torch.empty(B, keep, dtype=torch.int32, device=dev)
        self.cnt = torch.empty(B, dtype=torch.int32, device=dev)
        self.out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty(B, H, dtype=torch.float32, device=dev)
        wsb = int(_lib.lib().dsa_pooled_workspace_bytes(B, H, keep, self.stride, kp, splits))
        if wsb == 0:
            raise ValueError(f"PooledDecodeLayer: no workspace size for B={B} H={H} keep={keep}")
        # zero once: the calls keep the regions that must start at zero (the top-k histograms) at zero
        self.workspace = C.zeroed_workspace(wsb, dev)

    def step(self, q_idx: torch.Tensor, w: torch.Tensor, pool_key: torch.Tensor, q: torch.Tensor,
             kv_cache: torch.Tensor, kv_scale: torch.Tensor | None, table: torch.Tensor, npool: torch.Tensor,
             positions: torch.Tensor, check: bool = True, verify: bool = False,
             write: tuple | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """(out bf16 [B, H, 512], lse fp32 [B, H]); self.scores / pools / cnt hold the intermediates. q_idx
        [B, Hi, 128] bf16, w [B, Hi] fp32 (128 ** -0.5 folded in), pool_key bf16 [slots, 128 / kp], q [B, H, dqk]
        bf16, kv_cache [slots, dqk] e4m3fn + kv_scale [slots] (None: unscaled), table [B, max_pages] int32, npool
        [B] int32 ((positions + 1) // kp), positions [B] int32. check=False skips the Python-side checks (the C ABI still
        checks sizes); verify as DecodeLayer.step.

        write = (rows, ape, slot_mapping, rows_scale): the step's pool-key write first (dsa_cache.write_pool_keys of
        each row's written token at positions[b], slot slot_mapping[b] int64 [B]; rows the indexer rows cache [slots,
        W >= 256] e4m3fn or bf16, ape [kp, 128] fp32, rows_scale [slots] fp32 or None), as the reference's decode step
        writes before it attends (trnrt/models/mla.py:448-452): the C ABI's dsa_pooled_decode_step, in the same
        launch as the layer where the layer is one launch."""
        B, Hi, H = self.B, self.Hi, self.H
        if write is not None:
            rows, ape, slot_mapping, rows_scale = write
            if check:
                C.on_gpu(rows, ape, slot_mapping, rows_scale)
                slots = self.num_pages * self.page_size
                if not rows.is_contiguous() or rows.dim() != 2 or rows.shape[0] != slots or rows.shape[1] < 256:
                    raise ValueError(f"PooledDecodeLayer.step: rows {tuple(rows.shape)} for {slots} slots")
                if rows.dtype not in (C.FP8, torch.uint8, torch.bfloat16):
                    raise ValueError(f"PooledDecodeLayer.step: rows of dtype {rows.dtype}")
                C.need(ape, "ape", torch.float32, (self.kp, 128))
                C.need(slot_mapping, "slot_mapping", torch.int64, (B,))
                if rows_scale is not None:
                    C.need(rows_scale, "rows_scale", torch.float32, (slots,))
            if self.chain:
                from . import dsa_cache
                dsa_cache.write_pool_keys(pool_key, rows, positions, table, slot_mapping, ape, self.page_size,
                                          self.kp, rows_scale=rows_scale)
                write = None
        if check:
            C.on_gpu(q_idx, w, pool_key, q, kv_cache, kv_scale, table, npool, positions)
            C.need(q_idx, "q_idx", torch.bfloat16, (B, Hi, 128))
            C.need(w, "w", torch.float32, (B, Hi))
            C.need(q, "q", torch.bfloat16, (B, H, self.dqk))
            C.need(table, "table", torch.int32, (B, self.max_pages))
            C.need(npool, "npool", torch.int32, (B,))
            C.need(positions, "positions", torch.int32, (B,))
            C.fp8_bytes(kv_cache, "kv_cache")
            slots = self.num_pages * self.page_size
            C.need(pool_key, "pool_key", torch.bfloat16, (slots, 128 // self.kp))
            if kv_cache.numel() != slots * self.dqk:
                raise ValueError(f"kv cache of {kv_cache.numel()} bytes for {slots} slots of {self.dqk}")
            if kv_scale is not None:
                C.need(kv_scale, "kv_scale", torch.float32, (slots,))
        if write is not None:
            rows, ape, slot_mapping, rows_scale = write
            pre = (rows.data_ptr(), int(rows.dtype != torch.bfloat16), C.ptr(rows_scale), rows.shape[1],
                   ape.data_ptr(), slot_mapping.data_ptr())
            fn = lambda *args: _lib.lib().dsa_pooled_decode_step(*pre, *args)  # noqa: E731
        else:
            fn = _lib.lib().dsa_pooled_decode_layer_chain if self.chain else _lib.lib().dsa_pooled_decode_layer
        st = fn(
            q_idx.data_ptr(), w.data_ptr(), pool_key.data_ptr(), q.data_ptr(), kv_cache.data_ptr(),
            C.ptr(kv_scale), table.data_ptr(), npool.data_ptr(), positions.data_ptr(), self.scores.data_ptr(),
            self.pools.data_ptr(), self.cnt.data_ptr(), self.out.data_ptr(), self.lse.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), B, Hi, H, self.dqk, self.max_pages, self.page_size,
            self.num_pages, self.kp, self.keep, self.scale, self.splits,
            torch.cuda.current_stream(self.device).cuda_stream)
        _lib.check(st, "dsa_layer.PooledDecodeLayer.step")
        if verify:
            _verify(self.workspace, self.device, "dsa_layer.PooledDecodeLayer.step")
        return self.out, self.lse

    def status(self, clear: bool = False) -> dict:
        """The workspace's status words since the last clear (as DecodeLayer.status; the attention launch's
        barrier waits)."""
        return _status(self.workspace, self.device, clear)
