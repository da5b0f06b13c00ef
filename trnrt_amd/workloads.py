"""The decode workloads of the DSA path and their seeded synthetic inputs (shared by the tests, the smoke check and
the benchmark; the same seed gives the same tensors on the same device type).

Cache format (trnrt/models/decoder.py:459-490, 658-667; trnrt/engine/kv_pool.py:1-15), extended with per-token
scales: pages of `page_size` token slots, page 0 the null page, token t of row b in slot
table[b, t // page_size] * page_size + t % page_size; the page table is a seeded random permutation of pages 1..N.
Keys and latent rows are ~N(0, 1), quantised per token to OCP e4m3fn with scale absmax / 448 (448 = the e4m3fn
maximum, trnrt/engine/model_runner.py:62-70; the per-token scale replaces the reference's unscaled clamp,
trnrt/models/decoder.py:481-486).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


@dataclass(frozen=True)
class Config:
    name: str
    B: int
    L: int  # context per sequence (the longest one when ragged)
    H: int  # query heads
    Hi: int  # indexer heads
    keep: int = 2048
    page_size: int = 64
    D: int = 128  # indexer head dim
    dqk: int = 576  # 512 latent + 64 rope
    dv: int = 512
    ragged: tuple[int, int] | None = None  # lengths ~ U[lo, hi] (seeded) instead of L each

    @property
    def scale(self) -> float:
        return 192 ** -0.5  # 1 / sqrt(128 + 64)


CONFIGS = {
    1: Config("b1-ctx4k-h16", B=1, L=4096, H=16, Hi=16),
    2: Config("b8-ctx32k-h64", B=8, L=32768, H=64, Hi=64),
    3: Config("b12-ragged8k-128k-h64", B=12, L=131072, H=64, Hi=64, ragged=(8192, 131072)),
    4: Config("b4-ctx1m-h64", B=4, L=1048576, H=64, Hi=64),
}


def lengths_of(cfg: Config, seed: int = 0) -> list[int]:
    if cfg.ragged is None:
        return [cfg.L] * cfg.B
    g = torch.Generator().manual_seed(1000 + seed)
    lo, hi = cfg.ragged
    return [int(x) for x in torch.randint(lo, hi + 1, (cfg.B,), generator=g)]


def algorithmic_bytes(lengths: list[int], H: int, Hi: int, keep: int = 2048, page_size: int = 64) -> int:
    """Bytes one layer-step must move at least: every input once, every output once, no intermediates
    (FP8 key + fp32 scale per token, page table, indexer q (bf16) and weights (fp32), attention q (576 bf16), the
    selected KV rows (576 B + fp32 scale), and the bf16 output)."""
    tot = 0
    for L in lengths:
        tot += 132 * L + 4 * math.ceil(L / page_size) + 256 * Hi + 4 * Hi + 1152 * H + 580 * min(keep, L) + 1024 * H
    return tot


@dataclass
class Inputs:
    cfg: Config
    lengths: list[int]
    q_idx: torch.Tensor  # [B, Hi, 128] bf16
    w: torch.Tensor  # [B, Hi] fp32 head weights (before D ** -0.5)
    w_k: torch.Tensor  # [B, Hi] fp32 the kernel's weights: w * D ** -0.5 (trnrt/models/mla.py:629)
    q: torch.Tensor  # [B, H, 576] bf16
    k_cache: torch.Tensor  # [slots, 128] e4m3fn
    k_scale: torch.Tensor  # [slots] fp32
    kv_cache: torch.Tensor  # [slots, 576] e4m3fn
    kv_scale: torch.Tensor  # [slots] fp32
    table: torch.Tensor  # [B, max_pages] int32
    ctx_len: torch.Tensor  # [B] int32
    num_pages: int
    max_pages: int

    @property
    def page_size(self) -> int:
        return self.cfg.page_size

    def to(self, device) -> "Inputs":
        kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return Inputs(**kw)


def quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row e4m3fn quantisation: scale = absmax / 448, q = (x / scale) clamped to +-448 (the clamp before the cast
    of trnrt/models/decoder.py:481-486)."""
    s = x.abs().amax(dim=-1).clamp(min=1e-30) / FP8_MAX
    q = (x / s.unsqueeze(-1)).clamp(-FP8_MAX, FP8_MAX).to(FP8)
    return q, s.float()


def _gen(device) -> torch.Generator:
    return torch.Generator(device=device)


def make_inputs(cfg: Config, seed: int = 0, device: str | torch.device = "cpu", lengths: list[int] | None = None,
                chunk: int = 65536) -> Inputs:
    """Seeded inputs of one decode layer step for cfg, generated on `device` (cache rows in chunks of `chunk`
    slots, so a 1M-token cache never needs its fp32 form at once)."""
    device = torch.device(device)
    lengths = lengths_of(cfg, seed) if lengths is None else list(lengths)
    B, ps = cfg.B, cfg.page_size
    g = _gen(device)
    g.manual_seed(seed)
    npg = [math.ceil(L / ps) for L in lengths]
    max_pages = max(max(npg), 1)
    num_pages = 1 + sum(npg)
    q_idx = torch.randn(B, cfg.Hi, cfg.D, generator=g, device=device).to(torch.bfloat16)
    w = torch.randn(B, cfg.Hi, generator=g, device=device) * 0.25  # N(0, 1/16)
    q = torch.randn(B, cfg.H, cfg.dqk, generator=g, device=device).to(torch.bfloat16)
    perm = torch.randperm(num_pages - 1, generator=g, device=device) + 1
    table = torch.zeros(B, max_pages, dtype=torch.int32, device=device)
    o = 0
    for b in range(B):
        table[b, : npg[b]] = perm[o : o + npg[b]].to(torch.int32)
        o += npg[b]
    slots = num_pages * ps
    k_cache = torch.empty(slots, cfg.D, dtype=FP8, device=device)
    kv_cache = torch.empty(slots, cfg.dqk, dtype=FP8, device=device)
    k_scale = torch.empty(slots, dtype=torch.float32, device=device)
    kv_scale = torch.empty(slots, dtype=torch.float32, device=device)
    for s0 in range(0, slots, chunk):
        n = min(chunk, slots - s0)
        kq, ks = quantize_rows(torch.randn(n, cfg.D, generator=g, device=device))
        vq, vs = quantize_rows(torch.randn(n, cfg.dqk, generator=g, device=device))
        k_cache[s0 : s0 + n] = kq
        k_scale[s0 : s0 + n] = ks
        kv_cache[s0 : s0 + n] = vq
        kv_scale[s0 : s0 + n] = vs
    # the null page holds zeros (what a padded row's write leaves; never a live token)
    k_cache[:ps].view(torch.uint8).zero_()
    kv_cache[:ps].view(torch.uint8).zero_()
    k_scale[:ps] = 1.0
    kv_scale[:ps] = 1.0
    ctx_len = torch.tensor(lengths, dtype=torch.int32, device=device)
    return Inputs(cfg, lengths, q_idx, w, w * cfg.D ** -0.5, q, k_cache, k_scale, kv_cache, kv_scale, table, ctx_len,
                  num_pages, max_pages)


# -- the chunked-prefill indexer (one sequence: cached tokens plus a chunk of new queries, causal) -----------------


@dataclass(frozen=True)
class PrefillConfig:
    name: str
    cached: int  # tokens already in the cache
    chunk: int  # new query tokens (their keys are in the cache too)
    Hi: int = 64
    keep: int = 2048
    D: int = 128
    q_fp8: bool = False  # indexer queries as e4m3 with per-(query, head) scales (the FP8-MFMA form)
    H: int = 64  # attention query heads
    dqk: int = 576  # 512 latent + 64 rope
    dv: int = 512
    page_size: int = 64

    @property
    def P(self) -> int:
        return self.cached + self.chunk

    @property
    def scale(self) -> float:
        return self.D ** -0.5  # the indexer's softmax-free scale (trnrt/models/mla.py:629)

    @property
    def softmax_scale(self) -> float:
        return 192 ** -0.5  # 1 / sqrt(128 + 64)


PREFILL_CONFIGS = {
    5: PrefillConfig("prefill-65536+2048-h64", cached=65536, chunk=2048, q_fp8=True),
}


def prefill_attention_flops(cfg: PrefillConfig) -> int:
    """Algorithmic MFMA work of the chunk's sparse attention: per query, head and selected token, a 576-dim score
    and a 512-dim value product (2 FLOP per multiply-add)."""
    return 2 * cfg.chunk * cfg.H * min(cfg.keep, cfg.cached + 1) * (cfg.dqk + cfg.dv)


def prefill_flops(cfg: PrefillConfig) -> int:
    """Algorithmic MFMA work of the chunk's scores: 2 Hi D per (query, candidate key), query i of the chunk seeing
    cached + i + 1 keys (causal)."""
    n = cfg.chunk * (cfg.cached + 1) + cfg.chunk * (cfg.chunk - 1) // 2
    return 2 * cfg.Hi * cfg.D * n


@dataclass
class PrefillInputs:
    cfg: PrefillConfig
    qI: torch.Tensor  # [C, Hi, 128] bf16, or e4m3fn when cfg.q_fp8
    qI_scale: torch.Tensor | None  # [C, Hi] fp32 per-(query, head) scales of e4m3fn queries (absmax / 448), or None
    w: torch.Tensor  # [C, Hi] fp32 ~ N(0, 1/16)
    k8: torch.Tensor  # [P, 128] e4m3fn
    k_scale: torch.Tensor  # [P] fp32
    npool: torch.Tensor  # [C] int32: position + 1 (causal: key t <= the query's position)
    # the attention's inputs (make_prefill_inputs(attention=True)), else None:
    q: torch.Tensor | None = None  # [C, H, 576] bf16 absorbed queries
    kv_cache: torch.Tensor | None = None  # [slots, 576] e4m3fn latent rows of the context, paged
    kv_scale: torch.Tensor | None = None  # [slots] fp32
    table: torch.Tensor | None = None  # [P / page_size] int32: the context's pages (a seeded permutation of 1..)

    def to(self, device) -> "PrefillInputs":
        kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return PrefillInputs(**kw)

    def q_values(self) -> torch.Tensor:
        """The queries' values in fp32 (dequantised when FP8): what the reference's arithmetic sees."""
        if self.qI_scale is None:
            return self.qI.float()
        return self.qI.float() * self.qI_scale.unsqueeze(-1)


def make_prefill_inputs(cfg: PrefillConfig, seed: int = 0, device: str | torch.device = "cpu",
                        chunk: int = 65536, attention: bool = False) -> PrefillInputs:
    """Seeded inputs of one chunk's indexer: queries ~N(0, 1) in bf16 (with cfg.q_fp8 quantised per (query, head)
    to e4m3fn, scale absmax / 448), weights ~N(0, 1/16), keys ~N(0, 1) quantised per token to e4m3fn (scale
    absmax / 448); query i sits at position cached + i."""
    device = torch.device(device)
    g = _gen(device)
    g.manual_seed(seed)
    C, P = cfg.chunk, cfg.P
    qI = torch.randn(C, cfg.Hi, cfg.D, generator=g, device=device).to(torch.bfloat16)
    qI_scale = None
    if cfg.q_fp8:
        qI, qI_scale = quantize_rows(qI.float())
    w = torch.randn(C, cfg.Hi, generator=g, device=device) * 0.25
    k8 = torch.empty(P, cfg.D, dtype=FP8, device=device)
    ks = torch.empty(P, dtype=torch.float32, device=device)
    for s0 in range(0, P, chunk):
        n = min(chunk, P - s0)
        k8[s0:s0 + n], ks[s0:s0 + n] = quantize_rows(torch.randn(n, cfg.D, generator=g, device=device))
    npool = (cfg.cached + 1 + torch.arange(C, device=device)).to(torch.int32)
    inp = PrefillInputs(cfg, qI, qI_scale, w, k8, ks, npool)
    if attention:
        ps = cfg.page_size
        npg = math.ceil(P / ps)
        inp.q = torch.randn(C, cfg.H, cfg.dqk, generator=g, device=device).to(torch.bfloat16)
        inp.table = (torch.randperm(npg, generator=g, device=device) + 1).to(torch.int32)
        slots = (npg + 1) * ps
        inp.kv_cache = torch.zeros(slots, cfg.dqk, dtype=FP8, device=device)
        inp.kv_scale = torch.ones(slots, dtype=torch.float32, device=device)
        for s0 in range(ps, slots, chunk):
            n = min(chunk, slots - s0)
            inp.kv_cache[s0:s0 + n], inp.kv_scale[s0:s0 + n] = quantize_rows(
                torch.randn(n, cfg.dqk, generator=g, device=device))
    return inp


# -- GLM-5.3-Flash's pooled decode (the reference's own model semantics: trnrt/models/glm5_next.py) ------------------


@dataclass(frozen=True)
class PooledConfig:
    """GLM-5.3-Flash's DSA decode shapes (tests/fixtures/GLM-5.3-Flash-config.json in the reference): 64 heads over a
    512-wide NoPE latent (softmax scale qk_nope_head_dim ** -0.5 = 1/16), a 32-head indexer of dim 128 over pool keys
    of kpool 4 tokens, top 2048 tokens = 512 pools plus the query's own incomplete pool."""
    name: str
    B: int
    L: int
    H: int = 64
    Hi: int = 32
    kp: int = 4
    topk: int = 2048
    D: int = 128
    dqk: int = 512
    page_size: int = 64

    @property
    def keep(self) -> int:
        return self.topk // self.kp

    @property
    def scale(self) -> float:
        return 256 ** -0.5  # qk_nope_head_dim ** -0.5 (GLM-5.3-Flash)


POOLED_CONFIGS = {
    6: PooledConfig("glm-pooled-b8-ctx32k", B=8, L=32768),
}


def pooled_indexer_bytes(cfg: PooledConfig, npool: list[int]) -> int:
    """Algorithmic bytes of one pooled indexer launch: every scored pool key once (bf16, 128 x 2 B), the page-table
    entries they span, the bf16 queries and fp32 head weights; the scores are an intermediate and are not counted."""
    ppp = cfg.page_size // cfg.kp
    return sum(2 * cfg.D * n + 4 * math.ceil(n / ppp) + 2 * cfg.D * cfg.Hi + 4 * cfg.Hi for n in npool)


def pooled_step_bytes(cfg: PooledConfig, npool: list[int], tokens: list[int]) -> int:
    """Bytes one pooled decode step must move at least: the pool-key write (the current pool's kp indexer rows of
    256 B + scale, the kp pieces of 2 D / kp B), the indexer's inputs (pooled_indexer_bytes), the attention's bf16
    queries, the attended tokens' latent rows (dqk B + fp32 scale) and the bf16 output."""
    tot = pooled_indexer_bytes(cfg, npool)
    for t in tokens:
        tot += cfg.kp * (2 * cfg.D + 4) + 2 * cfg.D + 2 * cfg.H * cfg.dqk + (cfg.dqk + 4) * t + 2 * cfg.H * 512
    return tot


def pooled_layer_bytes(cfg: PooledConfig, npool: list[int], tokens: list[int]) -> int:
    """Algorithmic bytes of the pooled layer itself (dsa_pooled_decode_layer: every input and output once, as
    algorithmic_bytes counts the kpool-1 layer): the indexer's inputs (pooled_indexer_bytes), then per row the bf16
    attention queries, the attended tokens' latent rows (dqk B + fp32 scale) and the bf16 output."""
    tot = pooled_indexer_bytes(cfg, npool)
    for t in tokens:
        tot += 2 * cfg.H * cfg.dqk + (cfg.dqk + 4) * t + 2 * cfg.H * 512
    return tot


@dataclass
class PooledInputs:
    cfg: PooledConfig
    rows: torch.Tensor  # [slots, 256] e4m3fn indexer rows: key 128 | pool gate logits 128
    rows_scale: torch.Tensor  # [slots] fp32
    ape: torch.Tensor  # [kp, 128] fp32 pool-position bias (idx_pool_ape)
    pool_key: torch.Tensor  # [slots, 128 / kp] bf16: every pool's key, written from the rows
    kv_cache: torch.Tensor  # [slots, 512] e4m3fn latent rows
    kv_scale: torch.Tensor  # [slots] fp32
    table: torch.Tensor  # [B, pages] int32
    positions: torch.Tensor  # [B] int32: each row's current position (L - 1)
    q_idx: torch.Tensor  # [B, Hi, 128] bf16
    w: torch.Tensor  # [B, Hi] fp32 head weights times 128 ** -0.5
    q: torch.Tensor  # [B, H, 512] bf16 absorbed queries

    def to(self, device) -> "PooledInputs":
        kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return PooledInputs(**kw)


def make_pooled_inputs(cfg: PooledConfig, seed: int = 0, device: str | torch.device = "cpu",
                       chunk: int = 65536) -> PooledInputs:
    """Seeded inputs of one pooled decode step: indexer rows ~N(0, 1) and latent rows ~N(0, 1), both quantised per
    token to e4m3fn; the pool keys are written by the library's kernel from those rows (the cache-store step), so
    this needs the GPU library when device is a GPU."""
    device = torch.device(device)
    g = _gen(device)
    g.manual_seed(seed)
    B, ps = cfg.B, cfg.page_size
    npg = math.ceil(cfg.L / ps)
    num_pages = 1 + B * npg
    slots = num_pages * ps
    rows = torch.empty(slots, 2 * cfg.D, dtype=FP8, device=device)
    rs = torch.empty(slots, dtype=torch.float32, device=device)
    kv = torch.empty(slots, cfg.dqk, dtype=FP8, device=device)
    ks = torch.empty(slots, dtype=torch.float32, device=device)
    for s0 in range(0, slots, chunk):
        n = min(chunk, slots - s0)
        rows[s0:s0 + n], rs[s0:s0 + n] = quantize_rows(torch.randn(n, 2 * cfg.D, generator=g, device=device))
        kv[s0:s0 + n], ks[s0:s0 + n] = quantize_rows(torch.randn(n, cfg.dqk, generator=g, device=device))
    table = (torch.randperm(num_pages - 1, generator=g, device=device)[: B * npg] + 1).view(B, npg).to(torch.int32)
    ape = torch.randn(cfg.kp, cfg.D, generator=g, device=device) * 0.5
    q_idx = torch.randn(B, cfg.Hi, cfg.D, generator=g, device=device).to(torch.bfloat16)
    w = torch.randn(B, cfg.Hi, generator=g, device=device) * 0.25 * cfg.D ** -0.5
    q = torch.randn(B, cfg.H, cfg.dqk, generator=g, device=device).to(torch.bfloat16)
    positions = torch.full((B,), cfg.L - 1, dtype=torch.int32, device=device)
    pool_key = torch.zeros(slots, cfg.D // cfg.kp, dtype=torch.bfloat16, device=device)
    inp = PooledInputs(cfg, rows, rs, ape, pool_key, kv, ks, table, positions, q_idx, w, q)
    if device.type != "cpu":
        from .kernels import dsa_cache

        pos = torch.arange(cfg.L, device=device).repeat(B)
        tb = table.repeat_interleave(cfg.L, dim=0)
        sm = tb.long().gather(1, (pos // ps).view(-1, 1)).view(-1) * ps + pos % ps
        dsa_cache.write_pool_keys(pool_key, rows, pos, tb, sm, ape, ps, cfg.kp, rows_scale=rs)
    return inp


# -- GLM-5.3-Flash's pooled chunked prefill (trnrt/models/mla.py:505-526 `attention_long` for a chunk) --------------


@dataclass(frozen=True)
class PooledPrefillConfig:
    """A GLM-5.3-Flash prefill chunk over a long context: `chunk` new queries after `cached` tokens, a 32-head indexer
    over the context's bf16 pool keys (kpool 4), the top 512 pools per query plus its tail, 64 heads of absorbed MLA
    over the 512-wide NoPE latent."""
    name: str
    cached: int
    chunk: int
    Hi: int = 32
    H: int = 64
    kp: int = 4
    topk: int = 2048
    D: int = 128
    dqk: int = 512
    page_size: int = 64

    @property
    def keep(self) -> int:
        return self.topk // self.kp

    @property
    def L(self) -> int:
        return self.cached + self.chunk

    @property
    def P(self) -> int:  # pools of the context
        return math.ceil(self.L / self.kp)

    @property
    def scale(self) -> float:  # index_head_dim ** -0.5
        return self.D ** -0.5

    @property
    def softmax_scale(self) -> float:  # qk_nope_head_dim ** -0.5
        return 256 ** -0.5


POOLED_PREFILL_CONFIGS = {
    7: PooledPrefillConfig("glm-prefill-65536+2048", cached=65536, chunk=2048),
}


@dataclass
class PooledPrefillInputs:
    cfg: PooledPrefillConfig
    qI: torch.Tensor  # [C, Hi, 128] bf16
    w: torch.Tensor  # [C, Hi] fp32 head weights
    pk: torch.Tensor  # [P, 128] bf16: the context's pool keys in pool order (context_pool_keys)
    positions: torch.Tensor  # [C] int32
    npool: torch.Tensor  # [C] int32 complete pools per query
    q: torch.Tensor  # [C, H, 512] bf16 absorbed queries
    kv_cache: torch.Tensor  # [slots, 512] e4m3fn latent rows
    kv_scale: torch.Tensor  # [slots] fp32
    table: torch.Tensor  # [pages] int32 the sequence's block table

    def to(self, device) -> "PooledPrefillInputs":
        kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return PooledPrefillInputs(**kw)


def make_pooled_prefill_inputs(cfg: PooledPrefillConfig, seed: int = 0, device: str | torch.device = "cpu",
                               chunk: int = 65536) -> PooledPrefillInputs:
    """Seeded inputs of one pooled chunk: pool keys ~N(0, 1) in bf16, queries ~N(0, 1) in bf16, weights ~N(0, 1/16),
    latent rows ~N(0, 1) quantised per token to e4m3fn, the sequence's pages in a random order; query i at position
    cached + i."""
    device = torch.device(device)
    g = _gen(device)
    g.manual_seed(seed)
    C, P, ps = cfg.chunk, cfg.P, cfg.page_size
    qI = torch.randn(C, cfg.Hi, cfg.D, generator=g, device=device).to(torch.bfloat16)
    w = torch.randn(C, cfg.Hi, generator=g, device=device) * 0.25
    pk = torch.randn(P, cfg.D, generator=g, device=device).to(torch.bfloat16)
    positions = (cfg.cached + torch.arange(C, device=device)).to(torch.int32)
    npool = torch.div(positions + 1, cfg.kp, rounding_mode="floor").to(torch.int32)
    q = torch.randn(C, cfg.H, cfg.dqk, generator=g, device=device).to(torch.bfloat16)
    npg = math.ceil(cfg.L / ps)
    table = (torch.randperm(npg, generator=g, device=device) + 1).to(torch.int32)
    slots = (npg + 1) * ps
    kv = torch.zeros(slots, cfg.dqk, dtype=FP8, device=device)
    ks = torch.ones(slots, dtype=torch.float32, device=device)
    for s0 in range(ps, slots, chunk):
        n = min(chunk, slots - s0)
        kv[s0:s0 + n], ks[s0:s0 + n] = quantize_rows(torch.randn(n, cfg.dqk, generator=g, device=device))
    return PooledPrefillInputs(cfg, qI, w, pk, positions, npool, q, kv, ks, table)
