"""The pooled (GLM kpool 4) decode layer in one launch (dsa_pooled_decode_layer on 512-wide rows of at most 8,192
pools: csrc/dsa_fused.hip decode_pooled_fused_kernel) against the oracle and against the separate kernels
(dsa_pooled_decode_layer_chain) on the same seeded inputs.

Bounds (the north star's): pool scores within 1e-2 row-relative of oracle indexer_ref over the bf16 pool keys (and
bit-equal to the separate kernels' bf16 indexer, the same arithmetic in the same order); the selected pools and
their count bit-exact against topk_ref over the kernel's own scores (trnrt/models/dsa_select.py:33-38: ties to the
lowest pool); the bf16 output within 2e-2 and lse within 1e-3 of the oracle attention over the selected pools'
tokens and the row's tail (pool_slots_ref, after trnrt/models/dsa_long.py:189-223). Cases: config 6's shape (8
rows of 8,192 pools, 64 heads), every tail length 0-3, rows with no complete pool (only a tail), fewer complete
pools than keep, 32 query heads, pool keys taking 1, 2 and 100 distinct values (the keep-th largest tied), two
launches (12 rows), and the workspace left clean (no barrier wait given up)."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, launched_kernels, row_rel_err, say
from tests.test_gpu_fused import sync_block
from trnrt_amd import workloads as W
from trnrt_amd.kernels.dsa_layer import PooledDecodeLayer

pytestmark = pytest.mark.gpu


def _layer(cfg, inp, chain=False):
    ps, kp = cfg.page_size, cfg.kp
    return PooledDecodeLayer(cfg.B, cfg.Hi, cfg.H, cfg.dqk, inp.table.shape[1], ps, inp.pool_key.shape[0] // ps, kp,
                             cfg.keep, cfg.scale, chain=chain)


def _step(layer, inp, npool, positions):
    return layer.step(inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale, inp.table, npool, positions)


def _check(cfg, inp, layer, positions, npool, scores=True):
    """Every stage of one step of `layer` against the oracle."""
    c = inp.to("cpu")
    kp, ps = cfg.kp, cfg.page_size
    ppp = ps // kp
    sc = layer.scores.cpu()
    if scores:
        keys = c.pool_key.view(-1, 128)
        ref = O.indexer_ref(c.q_idx, c.w, keys, torch.ones(keys.shape[0]), c.table, npool, ppp, stride=sc.shape[1])
        live = ref > -1e29
        err = row_rel_err(sc, ref, live)
        say(f"  pool scores rel err {err:.3e}")
        assert err <= 1e-2
        assert torch.all(sc[~live] == O.NEG_INF)
    want_p, want_c = O.topk_ref(sc, cfg.keep, npool)
    assert torch.equal(layer.cnt.cpu().long(), want_c)
    assert torch.equal(layer.pools.cpu().long(), want_p)
    rows, bias = O.pool_slots_ref(want_p, want_c, npool.long(), positions.long(), c.table, ps, kp, cfg.keep + 1)
    tok = (rows.unsqueeze(-1) * kp + torch.arange(kp)).reshape(cfg.B, -1)
    want_o, want_lse = O.sparse_mla_slots_ref(c.q, c.kv_cache, c.kv_scale, tok, bias.reshape(cfg.B, -1), cfg.scale)
    assert_attention_close(layer.out.float(), want_o)
    live = want_lse > -1e29
    torch.testing.assert_close(layer.lse.cpu()[live], want_lse[live], atol=1e-3, rtol=1e-4)
    assert torch.all(layer.lse.cpu()[~live] < -1e29)
    assert layer.status()["gave_up"] == 0


def _inputs(B, L, positions, H=64, seed=0, kp=4):
    cfg = W.PooledConfig("glm-fused", B=B, L=L, H=H, kp=kp)
    inp = W.make_pooled_inputs(cfg, seed=seed, device="cuda")
    pos = torch.tensor(positions, dtype=torch.int32)
    npool = torch.div(pos + 1, cfg.kp, rounding_mode="floor").to(torch.int32)
    return cfg, inp, pos, npool


def test_pooled_fused_config6_one_launch():
    """Config 6's shape: 8 rows of 32,768 tokens (8,192 complete pools each at the last position), one launch."""
    cfg = W.POOLED_CONFIGS[6]
    say("pooled one-launch layer, config 6")
    inp = W.make_pooled_inputs(cfg, seed=61, device="cuda")
    pos = inp.positions.cpu()
    npool = torch.div(pos + 1, cfg.kp, rounding_mode="floor").to(torch.int32)
    layer = _layer(cfg, inp)
    names = launched_kernels(lambda: _step(layer, inp, npool.cuda(), pos.cuda()))
    assert names == ["decode_pooled_fused_kernel"], names
    torch.cuda.synchronize()
    _check(cfg, inp, layer, pos, npool)


@pytest.mark.parametrize("H", [64, 32])
def test_pooled_fused_tails_and_short_rows(H):
    """Positions giving every tail length (0-3 tokens of the incomplete pool), rows with no complete pool (a tail
    only: positions 0, 1, 2), exactly keep pools and fewer; the one launch equals the separate kernels (scores
    bit-equal, selection equal, outputs within the bound) and matches the oracle."""
    positions = [8191, 8190, 4097, 2050, 2048, 2047, 700, 0] if H == 64 else [1, 2, 3, 8189]
    cfg, inp, pos, npool = _inputs(len(positions), 8192, positions, H=H, seed=62 + H)
    say(f"pooled one-launch layer H={H} positions={positions}")
    f, ch = _layer(cfg, inp), _layer(cfg, inp, chain=True)
    names = launched_kernels(lambda: _step(f, inp, npool.cuda(), pos.cuda()))
    assert names == ["decode_pooled_fused_kernel"], names
    _step(ch, inp, npool.cuda(), pos.cuda())
    torch.cuda.synchronize()
    assert torch.equal(f.scores, ch.scores)
    assert torch.equal(f.pools, ch.pools) and torch.equal(f.cnt, ch.cnt)
    assert_attention_close(f.out, ch.out)
    _check(cfg, inp, f, pos, npool)


def test_pooled_fused_two_launches():
    """12 rows (two launches of 8 and 4 rows on one workspace), random positions in a 16,384-token context."""
    g = torch.Generator().manual_seed(63)
    positions = [int(x) for x in torch.randint(0, 16384, (12,), generator=g)]
    cfg, inp, pos, npool = _inputs(12, 16384, positions, seed=63)
    say(f"pooled one-launch layer, 12 rows {positions}")
    layer = _layer(cfg, inp)
    names = launched_kernels(lambda: _step(layer, inp, npool.cuda(), pos.cuda()))
    assert names == ["decode_pooled_fused_kernel"] * 2, names
    torch.cuda.synchronize()
    _check(cfg, inp, layer, pos, npool)


@pytest.mark.parametrize("values", [1, 2, 100])
def test_pooled_fused_ties(values):
    """Pool keys taking `values` distinct rows (pool row r of the cache: pattern r % values), so a row's scores take at
    most that many values and the keep-th largest is tied with pools that are not taken (the lowest pools are)."""
    positions = [8191, 5000, 3000, 1999]
    cfg, inp, pos, npool = _inputs(len(positions), 8192, positions, seed=64 + values)
    keys = inp.pool_key.view(-1, 128)
    base = keys[16:16 + values].clone()
    rep = (keys.shape[0] + values - 1) // values
    keys.copy_(base.repeat(rep, 1)[:keys.shape[0]])
    say(f"pooled one-launch layer ties values={values}")
    layer = _layer(cfg, inp)
    _step(layer, inp, npool.cuda(), pos.cuda())
    torch.cuda.synchronize()
    sc = layer.scores.cpu()
    for b, n in enumerate(npool.tolist()):
        assert len(torch.unique(sc[b, :n])) <= values
    _check(cfg, inp, layer, pos, npool, scores=False)


def test_pooled_fused_repeated_steps():
    """Five steps on one workspace with the inputs changed in place between them: each equals a fresh layer's."""
    positions = [8191, 6000, 4093, 17]
    cfg, inp, pos, npool = _inputs(len(positions), 8192, positions, seed=65)
    say("pooled one-launch layer, repeated steps")
    layer = _layer(cfg, inp)
    for i in range(5):
        inp.q.mul_(-1.0) if i % 2 else inp.q_idx.mul_(-1.0)
        _step(layer, inp, npool.cuda(), pos.cuda())
    fresh = _layer(cfg, inp)
    _step(fresh, inp, npool.cuda(), pos.cuda())
    torch.cuda.synchronize()
    assert torch.equal(layer.pools, fresh.pools) and torch.equal(layer.cnt, fresh.cnt)
    assert torch.equal(layer.out, fresh.out) and torch.equal(layer.lse, fresh.lse)
    ws = layer.workspace.view(torch.int32).cpu()
    ctr, sync = sync_block(ws)
    assert torch.all(ctr % 256 == 0) and torch.all(sync[:, 1] == 0), "barrier words not at a launch boundary"
    assert layer.status()["gave_up"] == 0


def _order_bins(sc: torch.Tensor) -> torch.Tensor:
    """The 12-bit first-level bins (order key >> 20) of fp32 scores: the key maps floats to unsigned integers in
    value order (negative values complemented, non-negative with the sign bit set; -0 as +0)."""
    u = sc.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    u = torch.where(u == 0x80000000, torch.zeros_like(u), u)
    key = torch.where(u >= 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)
    return key >> 20


def test_pooled_fused_header_fallback():
    """Rows of 8,192 pools whose first block (256 pools) holds keys spread over 32 octaves, far above the rest of the
    row: that list's header (its 64 highest nonzero bins) stops above the bin of the keep-th largest key, so the
    first level also counts the keys below each list's header one by one. The test first shows that the row meets
    that condition, then checks selection and outputs against the oracle."""
    positions = [32767, 32767]
    cfg, inp, pos, npool = _inputs(len(positions), 32768, positions, seed=66)
    ppp = cfg.page_size // cfg.kp
    keys = inp.pool_key.view(-1, 128)
    keys.mul_(2.0 ** -8)
    scale = 2.0 ** (torch.arange(256, device="cuda").float() / 8 + 8)
    for b in range(len(positions)):
        pages = inp.table[b, : 256 // ppp].long()
        rows = (pages.unsqueeze(1) * ppp + torch.arange(ppp, device="cuda")).reshape(-1)
        keys[rows] = (keys[rows].float() * scale.unsqueeze(1)).to(keys.dtype)
    say("pooled one-launch layer, header fallback")
    layer = _layer(cfg, inp)
    _step(layer, inp, npool.cuda(), pos.cuda())
    torch.cuda.synchronize()
    sc = layer.scores.cpu()
    for b in range(len(positions)):
        n = int(npool[b])
        bins = _order_bins(sc[b, :n])
        c0 = int(torch.sort(bins, descending=True).values[cfg.keep - 1])
        lows = []
        for blk in bins.view(32, -1):
            nzb = torch.unique(blk).flip(0)
            lows.append(int(nzb[63]) if len(nzb) > 64 else 0)
        assert c0 < max(lows), (c0, max(lows))
    _check(cfg, inp, layer, pos, npool)


@pytest.mark.parametrize("H,kp", [(64, 4), (32, 4), (64, 2)])
def test_pooled_step_writes_then_attends_in_one_launch(H, kp):
    """dsa_pooled_decode_step (the pool-key write of each row's written token, then the layer) against the write
    (dsa_cache.write_pool_keys) followed by the separate kernels, on the same inputs: one launch at kpool 4 (the
    write's kernel, then the layer's one launch, at kpool 2), the written pools' keys bit-equal in the cache, scores
    bit-equal (the completed pool scored from its new key), selection equal, outputs within the bound, and the oracle
    on the written cache. The written tokens' indexer rows are redrawn first, so that each written pool's new key
    differs from the one in the cache; rows: complete and incomplete written pools, a pool 0 (position kp - 1), a row
    with no complete pool (position 0), and a padded row (null-page slot)."""
    from trnrt_amd.kernels import dsa_cache

    positions = [8191, 8190, 4095, 2050, kp - 1, 0, 6001, 0]
    cfg, inp, pos, npool = _inputs(len(positions), 8192, positions, H=H, seed=70 + H + kp, kp=kp)
    ps, kp = cfg.page_size, cfg.kp
    sm = dsa_cache.slots_of(pos.cuda(), inp.table, ps)
    sm[-1] = 7  # a padded row: its slot in the null page
    g = torch.Generator(device="cuda").manual_seed(71)
    new_rows, new_scale = W.quantize_rows(torch.randn(len(positions), inp.rows.shape[1], generator=g, device="cuda")
                                          * 3.0)
    inp.rows[sm] = new_rows
    inp.rows_scale[sm] = new_scale
    write = (inp.rows, inp.ape, sm, inp.rows_scale)
    say(f"pooled one-launch step H={H} kp={kp} positions={positions}")
    # the stale scores (the cache before the write), to show that the write changes the completed pools' scores
    stale = _layer(cfg, inp)
    _step(stale, inp, npool.cuda(), pos.cuda())
    pk_ref = inp.pool_key.clone()
    f, ch = _layer(cfg, inp), _layer(cfg, inp, chain=True)
    names = launched_kernels(lambda: f.step(inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale,
                                            inp.table, npool.cuda(), pos.cuda(), write=write))
    want = ["decode_pooled_fused_kernel"] if kp == 4 else ["pool_keys_kernel", "decode_pooled_fused_kernel"]
    assert names == want, names
    dsa_cache.write_pool_keys(pk_ref, inp.rows, pos.cuda(), inp.table, sm, inp.ape, ps, kp,
                              rows_scale=inp.rows_scale)
    ch.step(inp.q_idx, inp.w, pk_ref, inp.q, inp.kv_cache, inp.kv_scale, inp.table, npool.cuda(), pos.cuda())
    torch.cuda.synchronize()
    assert torch.equal(inp.pool_key, pk_ref), "the written pool keys differ"
    assert torch.equal(f.scores, ch.scores)
    assert torch.equal(f.pools, ch.pools) and torch.equal(f.cnt, ch.cnt)
    assert_attention_close(f.out, ch.out)
    changed = 0
    for b, p in enumerate(positions):
        if (p + 1) % kp == 0 and b < len(positions) - 1:  # a completed pool, scored this step
            P = p // kp
            changed += int(f.scores[b, P] != stale.scores[b, P])
    assert changed >= 3, "the written pools' scores did not change: the test does not exercise the write"
    _check(cfg, inp, f, pos, npool)
    assert f.status()["gave_up"] == 0
