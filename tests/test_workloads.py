"""The synthetic workloads (trnrt_amd/workloads.py): the per-token e4m3fn quantiser, the paged layout (page 0 the null
page, a permutation of pages 1..N across rows), the ragged lengths, and the algorithmic-byte formula against the
value the baseline quotes for config 2."""

import torch

from trnrt_amd import workloads as W


def test_quantiser():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1000, 128, generator=g) * 3
    q, s = W.quantize_rows(x)
    assert q.dtype == torch.float8_e4m3fn
    deq = q.float() * s[:, None]
    assert (q.float().abs().amax(-1) == 448).all()  # each row's absmax lands on the e4m3fn maximum
    err = (deq - x).abs() / x.abs().amax(-1, keepdim=True)
    assert float(err.max()) <= 2 ** -4  # 3 mantissa bits: half an ulp of the largest binade


def test_paged_layout():
    cfg = W.Config("t", B=3, L=200, H=16, Hi=16)
    inp = W.make_inputs(cfg, seed=1, lengths=[200, 64, 1])
    assert inp.num_pages == 1 + 4 + 1 + 1 and inp.max_pages == 4
    pages = []
    for b, L in enumerate(inp.lengths):
        n = -(-L // 64)
        row = inp.table[b, :n].tolist()
        assert all(1 <= p < inp.num_pages for p in row)
        assert (inp.table[b, n:] == 0).all()
        pages += row
    assert sorted(pages) == list(range(1, inp.num_pages))
    assert (inp.k_cache[:64].view(torch.uint8) == 0).all()


def test_ragged_lengths_are_seeded():
    a = W.lengths_of(W.CONFIGS[3], 0)
    assert a == W.lengths_of(W.CONFIGS[3], 0) and len(a) == 12
    assert all(8192 <= x <= 131072 for x in a)


def test_algorithmic_bytes_of_config2():
    assert W.algorithmic_bytes([32768] * 8, 64, 64) == 45_369_344
    assert W.algorithmic_bytes([4096], 16, 16) == 1_767_744
    assert W.algorithmic_bytes([1 << 20] * 4, 64, 64) == 559_285_248


def test_pooled_config_is_glm53_flash():
    cfg = W.POOLED_CONFIGS[6]
    assert (cfg.B, cfg.L, cfg.H, cfg.Hi, cfg.kp, cfg.topk, cfg.dqk) == (8, 32768, 64, 32, 4, 2048, 512)
    assert cfg.keep == 512 and cfg.scale == 1 / 16
    small = W.PooledConfig("t", B=2, L=256)
    inp = W.make_pooled_inputs(small, seed=3)
    assert inp.rows.shape == (576, 256) and inp.kv_cache.shape == (576, 512) and inp.pool_key.shape == (576, 32)
    assert inp.table.shape == (2, 4) and sorted(inp.table.view(-1).tolist()) == list(range(1, 9))
    assert inp.positions.tolist() == [255, 255]


def test_pooled_bytes_of_config6():
    cfg = W.POOLED_CONFIGS[6]
    # per row: 8,192 pool keys x 256 B + 512 table entries + 32 bf16 queries of 128 + 32 fp32 weights
    assert W.pooled_indexer_bytes(cfg, [8192] * 8) == 8 * 2_107_520
    # + the pool-key write (4 rows x 260 B + 256 B), the 64 x 512 bf16 queries, 2,048 tokens x 516 B, the bf16 output
    assert W.pooled_step_bytes(cfg, [8192] * 8, [2048] * 8) == 8 * (2_107_520 + 1_040 + 256 + 65_536 + 1_056_768
                                                                    + 65_536)
