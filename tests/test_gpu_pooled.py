"""GPU parity of the pooled (kpool > 1) forms of the path against the oracle: the slots of selected pools with the
query's tail pool (trnrt_amd.models.dsa_long.slots -> dsa_pool_slots, after trnrt/models/dsa_long.py:189-215,
bit-exact), and sparse MLA over pool slots of kp tokens each (dsa_long.attend, after trnrt/kernels/dsa_decode.py:
26-37 with bias [N, S, kp]; 2e-2 abs/rel in bf16)."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, say
from trnrt_amd import workloads as W
from trnrt_amd.models import dsa_long

pytestmark = pytest.mark.gpu


def _selection(N, L, kp, keep, positions, seed):
    g = torch.Generator().manual_seed(seed)
    P = L // kp
    npool = torch.div(positions + 1, kp, rounding_mode="floor")
    sc = torch.randn(N, P, generator=g)
    sc = sc + torch.where(torch.arange(P).view(1, P) < npool.view(N, 1), 0.0, O.NEG_INF)
    pools, cnt = O.topk_ref(sc, keep)
    return pools, cnt, npool


@pytest.mark.parametrize("kp,ps", [(4, 64), (4, 8), (4, 4), (1, 64)])
@pytest.mark.parametrize("shared", [True, False])
def test_slots_bit_exact(kp, ps, shared):
    say(f"pool slots kp={kp} ps={ps} shared={shared}")
    L = 2048
    positions = torch.tensor([0, 3, 4, 5, 100, 1023, 2046, 2047, 777])
    N = positions.shape[0]
    keep = 64 if kp == 4 else 256
    pools, cnt, npool = _selection(N, L, kp, keep, positions, seed=kp * 10 + ps)
    pages = L // ps
    g = torch.Generator().manual_seed(ps)
    table = torch.randperm(4 * pages, generator=g)[:pages].to(torch.int32) + 1
    tb = table if shared else torch.stack([table.roll(i) for i in range(N)])
    rows, bias = dsa_long.slots(pools.cuda(), cnt.cuda(), npool.cuda(), positions.cuda(), tb.cuda(), ps, kp, keep + 5)
    torch.cuda.synchronize()
    want_r, want_b = O.pool_slots_ref(pools, cnt, npool, positions, tb, ps, kp, keep + 5)
    assert torch.equal(rows.cpu(), want_r)
    assert torch.equal(bias.cpu(), want_b)


def test_pooled_attention_vs_oracle():
    """Absorbed MLA over 64 selected pools of 4 tokens plus the tail pool, through a paged FP8 cache."""
    say("pooled attention kp=4")
    cfg = W.Config("pooled", B=6, L=1024, H=32, Hi=16)
    inp = W.make_inputs(cfg, seed=4, lengths=[1024] * 6)
    kp, keep, ps = 4, 64, cfg.page_size
    positions = torch.tensor([1023, 1000, 514, 13, 4, 3])
    pools, cnt, npool = _selection(cfg.B, 1024, kp, keep, positions, seed=5)
    rows, bias = dsa_long.slots(pools.cuda(), cnt.cuda(), npool.cuda(), positions.cuda(), inp.table.cuda(), ps, kp,
                                keep + 1)
    o = dsa_long.attend(inp.q.cuda(), inp.kv_cache.cuda(), rows, bias, cfg.scale, kc_scale=inp.kv_scale.cuda())
    torch.cuda.synchronize()
    tok = (rows.cpu().unsqueeze(-1) * kp + torch.arange(kp)).reshape(cfg.B, -1)
    ref, _ = O.sparse_mla_slots_ref(inp.q, inp.kv_cache, inp.kv_scale, tok, bias.cpu().reshape(cfg.B, -1), cfg.scale)
    assert_attention_close(o, ref)


@pytest.mark.parametrize("kp,dqk,splits", [(2, 576, 0), (4, 512, 0), (8, 512, 0), (8, 576, 0), (4, 512, 1),
                                           (4, 576, 3), (8, 512, 1)])
def test_attend_pooled_tails_vs_oracle(kp, dqk, splits):
    """dsa_long.attend_pooled (selected pools and the tail read through the page table) over rows with every tail
    length 0 .. kp - 1, fewer selected pools than keep, and no complete pool, against the oracle over the slots of
    the reference's own arithmetic (pool_slots_ref). The split form adds the tail in the workgroup that holds a
    row's last slot; at kp 8 with 576-wide rows it keeps the tail among the slots instead: both are covered, with
    several splits per row (splits 0: chosen for the GPU, 16 here), one split (the tail added by the only workgroup,
    the output written directly) or 3 uneven ones, and with lse."""
    say(f"attend_pooled tails kp={kp} dqk={dqk} splits={splits}")
    g = torch.Generator().manual_seed(kp * 1000 + dqk)
    L, ps, H = 2048, 64, 32
    keep = 512 // kp
    pos = [L - 1, L - 2, 1000, kp * keep + 3, 77, kp - 2, 2 * kp - 1, 1500 + kp // 2]
    B = len(pos)
    positions = torch.tensor(pos)
    npg = L // ps
    num_pages = 1 + B * npg
    kv, ks = W.quantize_rows(torch.randn(num_pages * ps, dqk, generator=g))
    table = (torch.randperm(num_pages - 1, generator=g)[: B * npg] + 1).view(B, npg).to(torch.int32)
    q = torch.randn(B, H, dqk, generator=g).to(torch.bfloat16)
    pools, cnt, npool = _selection(B, L, kp, keep, positions, seed=kp + dqk)
    tails = (positions + 1 - npool * kp).tolist()
    assert set(tails) == (set(range(kp)) if kp < 8 else {0, 1, 4, 6, 7})
    o, lse = dsa_long.attend_pooled(q.cuda(), kv.cuda(), ks.cuda(), pools.cuda(), cnt.cuda(), npool.cuda(),
                                    positions.cuda(), table.cuda(), ps, kp, 192 ** -0.5, lse=True, splits=splits)
    torch.cuda.synchronize()
    want_r, want_b = O.pool_slots_ref(pools, cnt, npool, positions, table, ps, kp, keep + 1)
    tok = (want_r.unsqueeze(-1) * kp + torch.arange(kp)).reshape(B, -1)
    want_o, want_lse = O.sparse_mla_slots_ref(q, kv, ks, tok, want_b.reshape(B, -1), 192 ** -0.5)
    assert_attention_close(o, want_o)
    assert torch.allclose(lse.cpu(), want_lse, atol=1e-3, rtol=1e-4)


def _pool_setup(seed, fp8_rows, B=3, L=1024, ps=64, kp=4):
    """A GLM-like pooled cache: per token an indexer row [key 128 | gate logits 128] (bf16, or e4m3 with per-token
    scales), B sequences of L tokens through random page tables, and an empty pool-key cache."""
    g = torch.Generator().manual_seed(seed)
    npg = L // ps
    num_pages = 1 + B * npg
    slots = num_pages * ps
    x = torch.randn(slots, 256, generator=g) * 2
    if fp8_rows:
        rows, rs = W.quantize_rows(x)
    else:
        rows, rs = x.to(torch.bfloat16), None
    table = (torch.randperm(num_pages - 1, generator=g)[: B * npg] + 1).view(B, npg).to(torch.int32)
    ape = torch.randn(kp, 128, generator=g)
    return rows, rs, table, ape, slots


@pytest.mark.parametrize("fp8_rows", [False, True])
def test_pool_keys_write_vs_oracle(fp8_rows):
    say(f"pool keys write fp8_rows={fp8_rows}")
    kp, ps, L, B = 4, 64, 1024, 3
    rows, rs, table, ape, slots = _pool_setup(7, fp8_rows, B, L, ps, kp)
    # every token of every sequence written (one row per token, its own table), plus two padded rows
    positions = torch.arange(L).repeat(B)
    tb = table.repeat_interleave(L, dim=0)
    slot_mapping = tb.long().gather(1, (positions // ps).view(-1, 1)).view(-1) * ps + positions % ps
    positions = torch.cat([positions, torch.zeros(2, dtype=torch.int64)])
    tb = torch.cat([tb, table[:1].expand(2, -1)])
    slot_mapping = torch.cat([slot_mapping, torch.tensor([3, 5])])  # padded rows: slots in the null page
    pk0 = torch.zeros(slots, 128 // kp, dtype=torch.bfloat16)
    want = O.write_pool_keys_ref(pk0, rows, rs, positions, tb, slot_mapping, ape, ps, kp)
    pk = pk0.cuda()
    from trnrt_amd.kernels import dsa_cache
    dsa_cache.write_pool_keys(pk, rows.cuda(), positions.cuda(), tb.cuda(), slot_mapping.cuda(), ape.cuda(), ps, kp,
                              rows_scale=None if rs is None else rs.cuda())
    torch.cuda.synchronize()
    got = pk.cpu()[ps:].float()  # the null page's slots take the padded rows' pieces in an unspecified order
    ref = want[ps:].float()
    exact = (got == ref).float().mean().item()
    rel = ((got - ref).abs() / ref.abs().clamp(min=1e-20)).max().item()
    say(f"  exact fraction {exact:.5f}, max rel {rel:.3e}")
    assert exact >= 0.99 and rel <= 2 ** -6  # expf vs the host's exp may move a weight by one bf16 step


def test_pooled_indexer_over_written_pool_keys():
    """The pooled decode indexer (dsa_index.scores over the bf16 pool-key cache, 16 pools per 64-token page) on pool
    keys written by the kernel, against the oracle's indexer over the same keys; candidates: complete pools."""
    say("pooled indexer")
    from trnrt_amd.kernels import dsa_cache, dsa_index
    kp, ps, L, B, Hi = 4, 64, 1024, 3, 64
    rows, rs, table, ape, slots = _pool_setup(9, False, B, L, ps, kp)
    positions = torch.arange(L).repeat(B)
    tb = table.repeat_interleave(L, dim=0)
    slot_mapping = tb.long().gather(1, (positions // ps).view(-1, 1)).view(-1) * ps + positions % ps
    pk = torch.zeros(slots, 128 // kp, dtype=torch.bfloat16, device="cuda")
    dsa_cache.write_pool_keys(pk, rows.cuda(), positions.cuda(), tb.cuda(), slot_mapping.cuda(), ape.cuda(), ps, kp)
    g = torch.Generator().manual_seed(10)
    q = torch.randn(B, Hi, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(B, Hi, generator=g) * 0.25 * 128 ** -0.5
    pos_now = torch.tensor([1023, 514, 6])
    npool = torch.div(pos_now + 1, kp, rounding_mode="floor").to(torch.int32)
    ppp = ps // kp
    pkc = pk.view(-1, ppp * 128)  # the reference's page rows (trnrt/models/mla.py:629)
    got = dsa_index.scores(q.cuda(), w.cuda(), pkc, table.cuda(), None, ctx_len=npool.cuda())
    torch.cuda.synchronize()
    keys = pk.cpu().view(-1, 128)  # [pool slots, 128]: pool j of page p at p * ppp + j
    ref = O.indexer_ref(q, w, keys, torch.ones(keys.shape[0]), table, npool, ppp, stride=L // kp)
    live = ref > -1e29
    from tests._helpers import row_rel_err
    err = row_rel_err(got.cpu(), ref, live)
    say(f"  pooled indexer rel err {err:.3e}")
    assert err <= 1e-2
    assert torch.equal(got.cpu() < -1e29, ~live)


@pytest.mark.parametrize("dqk", [512, 576])
def test_pooled_attention_glm_latent_width(dqk):
    """GLM's NoPE latent (512 wide; with rope 576) through pool slots of kpool 4: the attention kernel's two row
    widths against the oracle."""
    say(f"pooled attention dqk={dqk}")
    g = torch.Generator().manual_seed(dqk)
    B, H, L, ps, kp, keep = 4, 32, 1024, 64, 4, 48
    npg = L // ps
    num_pages = 1 + B * npg
    kv, ks = W.quantize_rows(torch.randn(num_pages * ps, dqk, generator=g))
    table = (torch.randperm(num_pages - 1, generator=g)[: B * npg] + 1).view(B, npg).to(torch.int32)
    q = torch.randn(B, H, dqk, generator=g).to(torch.bfloat16)
    positions = torch.tensor([1023, 700, 9, 2])
    pools, cnt, npool = _selection(B, L, kp, keep, positions, seed=dqk + 1)
    rows, bias = dsa_long.slots(pools.cuda(), cnt.cuda(), npool.cuda(), positions.cuda(), table.cuda(), ps, kp,
                                keep + 1)
    o = dsa_long.attend(q.cuda(), kv.cuda(), rows, bias, 192 ** -0.5, kc_scale=ks.cuda())
    torch.cuda.synchronize()
    tok = (rows.cpu().unsqueeze(-1) * kp + torch.arange(kp)).reshape(B, -1)
    ref, _ = O.sparse_mla_slots_ref(q, kv, ks, tok, bias.cpu().reshape(B, -1), 192 ** -0.5)
    assert_attention_close(o, ref)


def test_glm_pooled_decode_step_end_to_end():
    """One GLM-5.3-Flash pooled decode batch (64 heads over the 512-wide NoPE latent, a 32-head indexer over pool keys
    of kpool 4, top 2048 tokens = 512 pools plus the tail) through dsa_long.decode_pooled, every stage against the
    oracle on the stage's own GPU inputs: the written pool keys, the pool scores (<= 1e-2 per row), the selection
    (bit-exact), the slots with the tail pool (bit-exact), the attention (2e-2)."""
    cfg = W.PooledConfig("glm-e2e", B=5, L=4096)
    say(f"GLM pooled decode step B={cfg.B} L={cfg.L} keep={cfg.keep}")
    inp = W.make_pooled_inputs(cfg, seed=21, device="cuda")
    kp, ps, ppp = cfg.kp, cfg.page_size, cfg.page_size // cfg.kp
    # a full context, a tail of one token, one of three, fewer complete pools than keep, no complete pool at all
    positions = torch.tensor([4095, 3000, 2050, 1500, 2], dtype=torch.int32)
    o, (sc, pools, cnt, rows, bias) = dsa_long.decode_pooled(
        inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale, positions.cuda(), inp.table, ps, kp,
        cfg.topk, 1.0, cfg.scale, parts=True)
    torch.cuda.synchronize()
    c = inp.to("cpu")
    npool = torch.div(positions.long() + 1, kp, rounding_mode="floor")

    # pool keys: every token of every sequence written by the kernel
    pos = torch.arange(cfg.L).repeat(cfg.B)
    tb = c.table.repeat_interleave(cfg.L, dim=0)
    sm = tb.long().gather(1, (pos // ps).view(-1, 1)).view(-1) * ps + pos % ps
    want_pk = O.write_pool_keys_ref(torch.zeros_like(c.pool_key), c.rows, c.rows_scale, pos, tb, sm, c.ape, ps, kp)
    got_pk, ref_pk = c.pool_key[ps:].float(), want_pk[ps:].float()
    exact = (got_pk == ref_pk).float().mean().item()
    rel = ((got_pk - ref_pk).abs() / ref_pk.abs().clamp(min=1e-20)).max().item()
    say(f"  pool keys: exact fraction {exact:.5f}, max rel {rel:.3e}")
    assert exact >= 0.99 and rel <= 2 ** -6

    # scores of the complete pools over the written pool keys
    keys = c.pool_key.view(-1, 128)
    ref = O.indexer_ref(c.q_idx, c.w, keys, torch.ones(keys.shape[0]), c.table, npool, ppp, stride=sc.shape[1])
    live = ref > -1e29
    from tests._helpers import row_rel_err
    err = row_rel_err(sc.cpu(), ref, live)
    say(f"  pool scores rel err {err:.3e}")
    assert err <= 1e-2
    assert torch.equal(sc.cpu() < -1e29, ~live)

    # the exact top 512 of the GPU's scores
    want_p, want_c = O.topk_ref(sc.cpu(), cfg.keep)
    assert torch.equal(cnt.cpu(), want_c) and torch.equal(pools.cpu(), want_p)
    assert cnt.cpu().tolist() == [512, 512, 512, 375, 0]

    # slots: the selected pools, then the tail pool
    want_r, want_b = O.pool_slots_ref(pools.cpu(), cnt.cpu(), npool, positions.long(), c.table, ps, kp, cfg.keep + 1)
    assert torch.equal(rows.cpu(), want_r) and torch.equal(bias.cpu(), want_b)
    tail_live = (bias.cpu()[:, cfg.keep] == 0).sum(-1).tolist()
    assert tail_live == [0, 1, 3, 1, 3]

    # absorbed MLA over the slots' tokens
    tok = (rows.cpu().unsqueeze(-1) * kp + torch.arange(kp)).reshape(cfg.B, -1)
    want_o, _ = O.sparse_mla_slots_ref(c.q, c.kv_cache, c.kv_scale, tok, bias.cpu().reshape(cfg.B, -1), cfg.scale)
    assert_attention_close(o, want_o)


@pytest.mark.parametrize("dqk,L,pos,H", [(512, 4096, (4095, 4094, 3001, 2050, 700, 1), 64),
                                         (576, 4096, (4095, 4094, 3001, 2050, 700, 1), 64),
                                         (512, 32768, (32767, 30001, 9000), 64),
                                         (512, 4096, (4094, 2050, 700, 1), 32)])
def test_pooled_decode_layer_matches_composition_and_oracle(dqk, L, pos, H):
    """The one-call pooled layer (dsa_pooled_decode_layer: the indexer with the fused first-level histogram, the
    top-k, attention over the selected pools' tokens and the tail read straight from the pool indices) against the
    reference-flow composition (dsa_long.decode_pooled: scores, select, slots, attend) and the oracle; at 32,768
    tokens (8,192 pools a row) the selection is the one-workgroup-per-row kernel fed by the fused histogram. With
    512-wide rows the attention and combine are one XCD-local launch (64 heads: 16 splits of 128 token slots; 32
    heads: 32 splits of 64), a row's tail in the split of its last selected token: the last split with a full
    selection (up to 131 rows there), a middle one (175 pools), split 0 (no complete pool); 576-wide rows take the
    split attention and the combine kernel."""
    _pooled_layer_check(dqk, L, pos, H, 30 + dqk + L)


@pytest.mark.parametrize("seed", [7, 8, 9])
def test_pooled_decode_layer_random_positions(seed):
    """Seeded random batches of the one-call pooled layer: 1 to 8 rows at random positions of a 4,096-token context
    (random tails of 0 to 3 tokens, rows with fewer complete pools than keep), 32 or 64 query heads, 512-wide rows:
    the XCD-local attention launch against the oracle."""
    g = torch.Generator().manual_seed(seed)
    B = int(torch.randint(1, 9, (1,), generator=g))
    H = [32, 64][int(torch.randint(0, 2, (1,), generator=g))]
    pos = tuple(int(x) for x in torch.randint(0, 4096, (B,), generator=g))
    _pooled_layer_check(512, 4096, pos, H, 1000 + seed)


def _pooled_layer_check(dqk, L, pos, H, seed):
    from trnrt_amd.kernels.dsa_layer import PooledDecodeLayer
    cfg = W.PooledConfig("glm-layer", B=len(pos), L=L, dqk=dqk, H=H)
    say(f"pooled layer dqk={dqk} H={H} B={cfg.B} L={cfg.L}")
    inp = W.make_pooled_inputs(cfg, seed=seed, device="cuda")
    kp, ps = cfg.kp, cfg.page_size
    positions = torch.tensor(pos, dtype=torch.int32)
    npool = torch.div(positions + 1, kp, rounding_mode="floor").to(torch.int32)
    layer = PooledDecodeLayer(cfg.B, cfg.Hi, cfg.H, dqk, inp.table.shape[1], ps, inp.pool_key.shape[0] // ps, kp,
                              cfg.keep, cfg.scale)
    out, lse = layer.step(inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale, inp.table, npool.cuda(),
                          positions.cuda())
    o_ref, (sc, pools, cnt, rows, bias) = dsa_long.decode_pooled(
        inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale, positions.cuda(), inp.table, ps, kp,
        cfg.topk, 1.0, cfg.scale, parts=True)
    torch.cuda.synchronize()
    assert torch.equal(layer.scores, sc)
    assert torch.equal(layer.cnt.long(), cnt) and torch.equal(layer.pools.long(), pools)
    c = inp.to("cpu")
    tok = (rows.cpu().unsqueeze(-1) * kp + torch.arange(kp)).reshape(cfg.B, -1)
    want_o, want_lse = O.sparse_mla_slots_ref(c.q, c.kv_cache, c.kv_scale, tok, bias.cpu().reshape(cfg.B, -1),
                                              cfg.scale)
    assert_attention_close(out.float(), want_o)
    assert_attention_close(o_ref, want_o)
    assert torch.allclose(lse.cpu(), want_lse, atol=1e-3, rtol=1e-4)
    # a second step with the histogram region left at zero by the first
    out1 = out.clone()
    out2, _ = layer.step(inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale, inp.table, npool.cuda(),
                         positions.cuda())
    torch.cuda.synchronize()
    assert torch.equal(layer.pools.long(), pools) and torch.equal(out2, out1)


@pytest.mark.parametrize("cached,chunk", [(2048, 96), (3000, 70)])
def test_glm_pooled_chunk_end_to_end(cached, chunk):
    """A GLM chunk (trnrt/models/mla.py:505-526 with a shared table): the prefill indexer over the context's bf16 pool
    keys, the exact top-512 pools (dsa_long_select.select), then absorbed MLA over the pools' tokens and each query's
    tail (dsa_long.attend_pooled, and the reference flow slots + attend), every stage against the oracle."""
    from trnrt_amd.kernels import dsa_long_select as LS
    cfg = W.PooledPrefillConfig("glm-chunk", cached=cached, chunk=chunk)
    say(f"GLM pooled chunk {cached}+{chunk}")
    inp = W.make_pooled_prefill_inputs(cfg, seed=cached + chunk, device="cuda")
    pools, cnt, vals = LS.select(inp.qI, inp.w, inp.pk, inp.npool, cfg.keep, cfg.scale)
    sc = dsa_long.scores(inp.qI, inp.w, inp.pk, inp.npool, cfg.scale)
    o = dsa_long.attend_pooled(inp.q, inp.kv_cache, inp.kv_scale, pools, cnt, inp.npool, inp.positions, inp.table,
                               cfg.page_size, cfg.kp, cfg.softmax_scale)
    rows, bias = dsa_long.slots(pools, cnt, inp.npool, inp.positions, inp.table, cfg.page_size, cfg.kp, cfg.keep + 1)
    o_ref_flow = dsa_long.attend(inp.q, inp.kv_cache, rows, bias, cfg.softmax_scale, kc_scale=inp.kv_scale)
    torch.cuda.synchronize()
    c = inp.to("cpu")
    ref = O.prefill_scores_ref(c.qI, c.w, c.pk, torch.ones(cfg.P), c.npool, cfg.scale)
    live = ref > -1e29
    from tests._helpers import row_rel_err
    err = row_rel_err(sc.cpu(), ref, live)
    say(f"  pool scores rel err {err:.3e}")
    assert err <= 1e-2 and torch.equal(sc.cpu() < -1e29, ~live)
    want_p, want_c = O.topk_ref(sc.cpu(), cfg.keep, c.npool)
    assert torch.equal(pools.cpu(), want_p) and torch.equal(cnt.cpu(), want_c)
    lv = torch.arange(cfg.keep).view(1, -1) < want_c.view(-1, 1)
    assert torch.equal(vals.cpu(), torch.where(lv, sc.cpu().gather(1, want_p), O.NEG_INF))
    want_r, want_b = O.pool_slots_ref(want_p, want_c, c.npool, c.positions.long(), c.table, cfg.page_size, cfg.kp,
                                      cfg.keep + 1)
    assert torch.equal(rows.cpu(), want_r) and torch.equal(bias.cpu(), want_b)
    tok = (want_r.unsqueeze(-1) * cfg.kp + torch.arange(cfg.kp)).reshape(cfg.chunk, -1)
    want_o, _ = O.sparse_mla_slots_ref(c.q, c.kv_cache, c.kv_scale, tok, want_b.reshape(cfg.chunk, -1),
                                       cfg.softmax_scale)
    assert_attention_close(o, want_o)
    assert_attention_close(o_ref_flow, want_o)
