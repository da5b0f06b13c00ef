"""GPU parity of the sparse MLA decode attention (trnrt_amd.kernels.dsa_decode -> dsa_sparse_mla_decode) against
the oracle (oracle/dsa_oracle.py sparse_mla_ref, trnrt/kernels/dsa_decode.py:26-37 + trnrt/kernels/dsa_slots.py:
48-65) on the same seeded inputs and selections; bound: bf16 output within 2e-2 abs/rel (the north star), lse within
1e-3 abs."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, say
from trnrt_amd import workloads as W
from trnrt_amd.kernels import dsa_decode

pytestmark = pytest.mark.gpu


def _selection(inp, keep=None):
    cfg = inp.cfg
    keep = cfg.keep if keep is None else keep
    sc = O.indexer_ref(inp.q_idx, inp.w_k, inp.k_cache, inp.k_scale, inp.table, inp.ctx_len, cfg.page_size,
                       inp.max_pages * cfg.page_size)
    return O.topk_ref(sc, keep, inp.ctx_len)


def _run(inp, idx, cnt, splits=0, out_dtype=torch.bfloat16):
    g = inp.to("cuda")
    o, lse = dsa_decode.attend_tokens(g.q, g.kv_cache, g.kv_scale, idx.cuda(), cnt.cuda(), g.table,
                                      inp.cfg.page_size, inp.cfg.scale, out_dtype=out_dtype, splits=splits)
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu()


def _ref(inp, idx, cnt):
    return O.sparse_mla_ref(inp.q, inp.kv_cache, inp.kv_scale, idx, cnt, inp.table, inp.cfg.page_size, inp.cfg.scale)


@pytest.mark.parametrize("splits", [0, 1, 5])
def test_config1(splits):
    say(f"attention config 1 splits={splits}")
    inp = W.make_inputs(W.CONFIGS[1], seed=0)
    idx, cnt = _selection(inp)
    o, lse = _run(inp, idx, cnt, splits)
    ro, rl = _ref(inp, idx, cnt)
    assert_attention_close(o, ro)
    torch.testing.assert_close(lse, rl, atol=1e-3, rtol=1e-4)


def test_config2_full():
    say("attention config 2")
    inp = W.make_inputs(W.CONFIGS[2], seed=0)
    idx, cnt = _selection(inp)
    o, lse = _run(inp, idx, cnt)
    ro, rl = _ref(inp, idx, cnt)
    assert_attention_close(o, ro)
    torch.testing.assert_close(lse, rl, atol=1e-3, rtol=1e-4)


def test_counts_below_keep_and_zero():
    """cnt < keep masks the tail slots; cnt 0 attends position 0 alone with lse NEG_INF (the reference's fully
    masked row over slots that all read position 0)."""
    say("attention short counts")
    cfg = W.Config("short", B=4, L=3000, H=32, Hi=16, keep=2048)
    inp = W.make_inputs(cfg, seed=5, lengths=[3000, 100, 1, 2500])
    idx, cnt = _selection(inp)
    cnt[2] = 0
    idx[2] = 0
    for splits in (0, 1, 3):
        o, lse = _run(inp, idx, cnt, splits, out_dtype=torch.float32)
        ro, rl = _ref(inp, idx, cnt)
        assert_attention_close(o, ro)
        torch.testing.assert_close(lse[[0, 1, 3]], rl[[0, 1, 3]], atol=1e-3, rtol=1e-4)
        assert (lse[2] < -1e29).all()


def test_row_form_equals_token_form():
    say("attention row form vs token form")
    cfg = W.Config("rows", B=2, L=4096, H=16, Hi=16, keep=1000)
    inp = W.make_inputs(cfg, seed=6)
    idx, cnt = _selection(inp, keep=1000)
    cnt[1] = 333
    idx[1, 333:] = 0
    rows = torch.stack([O.token_slots(inp.table[b], idx[b], 64) for b in range(2)])
    bias = torch.where(torch.arange(1000).view(1, -1) < cnt.view(2, 1), 0.0, O.NEG_INF)
    g = inp.to("cuda")
    o_row, l_row = dsa_decode.attend(g.q, g.kv_cache.view(-1, 1, 576), rows.cuda(), bias.cuda().unsqueeze(-1),
                                     cfg.scale, kc_scale=g.kv_scale, lse=True)
    o_tok, l_tok = _run(inp, idx, cnt, out_dtype=torch.float32)
    ro, rl = _ref(inp, idx, cnt)
    assert_attention_close(o_row.cpu(), ro)
    torch.testing.assert_close(o_row.cpu(), o_tok, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(l_row.cpu(), l_tok, atol=1e-5, rtol=1e-5)


def test_fully_masked_row_form_is_uniform():
    say("attention fully masked row form")
    cfg = W.Config("mask", B=1, L=512, H=16, Hi=16, keep=100)
    inp = W.make_inputs(cfg, seed=8)
    rows = torch.randint(64, 64 * 9, (1, 100), generator=torch.Generator().manual_seed(1))
    bias = torch.full((1, 100), O.NEG_INF)
    g = inp.to("cuda")
    o, lse = dsa_decode.attend(g.q, g.kv_cache, rows.cuda(), bias.cuda(), cfg.scale, kc_scale=g.kv_scale, lse=True)
    ro, rl = O.sparse_mla_slots_ref(inp.q, inp.kv_cache, inp.kv_scale, rows, bias, cfg.scale)
    assert_attention_close(o.cpu(), ro)
    assert (lse.cpu() < -1e29).all()


def test_wrong_scale_is_caught():
    """Positive control: per-token value scales shuffled between tokens must break the tolerance."""
    say("attention positive control")
    inp = W.make_inputs(W.CONFIGS[1], seed=9)
    idx, cnt = _selection(inp)
    bad = W.Inputs(**{**inp.__dict__, "kv_scale": inp.kv_scale[torch.randperm(inp.kv_scale.numel())]})
    o, _ = _run(bad, idx, cnt, out_dtype=torch.float32)
    ro, _ = _ref(inp, idx, cnt)
    assert (o - ro).abs().max() > 2e-2 * (1 + ro.abs().max())


@pytest.mark.parametrize("dqk", [576, 512])
def test_many_row_form_vs_oracle(dqk):
    """The many-row form (64-head workgroups, one per query row, pipelined gather: sparse_mla_wide_kernel), taken
    when one split suffices and the rows fill the GPU: ragged counts (0, 1, one chunk, a chunk and one slot, every
    slot, random), 64 heads, both row widths, against the oracle."""
    from tests._helpers import launched_kernels
    g = torch.Generator().manual_seed(dqk + 7)
    B, H, L, ps, keep = 300, 64, 1024, 64, 320
    say(f"attention many-row form dqk={dqk} B={B} keep={keep}")
    npg = L // ps
    num_pages = 1 + B * npg
    kv, ks = W.quantize_rows(torch.randn(num_pages * ps, dqk, generator=g))
    table = (torch.randperm(num_pages - 1, generator=g)[: B * npg] + 1).view(B, npg).to(torch.int32)
    q = torch.randn(B, H, dqk, generator=g).to(torch.bfloat16)
    cnt = torch.randint(0, keep + 1, (B,), generator=g)
    cnt[:6] = torch.tensor([0, 1, 64, 65, keep, 63])
    idx = torch.zeros(B, keep, dtype=torch.int64)
    for b in range(B):
        n = int(cnt[b])
        idx[b, :n] = torch.randperm(L, generator=g)[:n].sort().values
    qg, kvg, ksg, tg = q.cuda(), kv.cuda(), ks.cuda(), table.cuda()
    res = {}

    def step():
        res["o"], res["lse"] = dsa_decode.attend_tokens(qg, kvg, ksg, idx.cuda(), cnt.cuda(), tg, ps, 192 ** -0.5,
                                                        out_dtype=torch.float32)

    names = launched_kernels(step)
    assert names == ["sparse_mla_wide_kernel"], names
    ro, rl = O.sparse_mla_ref(q, kv, ks, idx, cnt, table, ps, 192 ** -0.5)
    assert_attention_close(res["o"], ro)
    live = cnt > 0
    torch.testing.assert_close(res["lse"].cpu()[live], rl[live], atol=1e-3, rtol=1e-4)
    assert (res["lse"].cpu()[~live] < -1e29).all()
