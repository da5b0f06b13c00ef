"""GPU parity of the prefill-chunk indexer and selection (trnrt_amd.kernels.dsa_long_select -> dsa_indexer_prefill,
dsa_topk) against the oracle (oracle/dsa_oracle.py prefill_scores_ref, after trnrt/kernels/dsa_long_select.py:
119-133; topk_ref, after trnrt/models/dsa_long.py:114-118) on the same seeded inputs.

Bounds: scores within max|diff| / max|ref| <= 1e-2 per row (the north star; the products are exact in bf16 x bf16
-> fp32, and in e4m3 x e4m3 -> fp32 for FP8 queries, whose oracle input is their dequantised value, so the real
error is fp32 summation order); the selection bit-exact when fed the kernel's own scores; the non-candidates
exactly NEG_INF."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, row_rel_err, say
from trnrt_amd import workloads as W
from trnrt_amd.kernels import dsa_decode
from trnrt_amd.kernels import dsa_long_select as LS
from trnrt_amd.models import dsa_long

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _inputs(N, Hi, P, seed, npool=None):
    g = torch.Generator().manual_seed(seed)
    qI = torch.randn(N, Hi, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(N, Hi, generator=g) * 0.25
    k8, ks = W.quantize_rows(torch.randn(P, 128, generator=g))
    if npool is None:
        npool = torch.randint(0, P + 1, (N,), generator=g)
    return qI, w, k8, ks, torch.as_tensor(npool, dtype=torch.int32)


def _fp8(qI):
    """FP8 e4m3 queries with per-(query, head) scales, and the values the oracle sees (their dequantised form)."""
    q8, qs = W.quantize_rows(qI.float())
    return q8, qs, q8.float() * qs.unsqueeze(-1)


def _check_scores(qI, w, k8, ks, npool, scale, stride=None, qI_scale=None, q_values=None):
    got = LS.scores(qI.cuda(), w.cuda(), k8.cuda(), npool.cuda(), scale, pk_scale=ks.cuda(), stride=stride,
                    qI_scale=None if qI_scale is None else qI_scale.cuda())
    torch.cuda.synchronize()
    got = got.cpu()
    ref = O.prefill_scores_ref(qI if q_values is None else q_values, w, k8, ks, npool, scale, stride)
    live = ref > -1e29
    err = row_rel_err(got, ref, live)
    say(f"  prefill scores rel err {err:.3e}")
    assert err <= TOL
    assert torch.all(got[~live] == O.NEG_INF)
    return got


@pytest.mark.parametrize("N,Hi,P,stride", [(5, 16, 100, None), (7, 64, 1000, 1100), (4, 48, 2053, None),
                                           (9, 33, 64, 96), (1, 1, 1, None), (13, 64, 4096, None)])
def test_scores_vs_oracle(N, Hi, P, stride):
    say(f"prefill scores N={N} Hi={Hi} P={P} stride={stride}")
    qI, w, k8, ks, npool = _inputs(N, Hi, P, seed=N * 1000 + Hi)
    npool[0] = P + 5  # clamped to P
    if N > 1:
        npool[1] = 0  # no candidates: a row of NEG_INF
    _check_scores(qI, w, k8, ks, npool, 128 ** -0.5, stride)


@pytest.mark.parametrize("N,Hi,P,stride", [(5, 16, 100, None), (7, 64, 1000, 1100), (4, 48, 2053, None),
                                           (9, 33, 64, 96), (1, 1, 1, None), (13, 64, 4096, None)])
def test_scores_fp8_queries_vs_oracle(N, Hi, P, stride):
    say(f"prefill scores fp8 q N={N} Hi={Hi} P={P} stride={stride}")
    qI, w, k8, ks, npool = _inputs(N, Hi, P, seed=N * 1000 + Hi + 7)
    npool[0] = P + 5
    if N > 1:
        npool[1] = 0
    q8, qs, qv = _fp8(qI)
    _check_scores(q8, w, k8, ks, npool, 128 ** -0.5, stride, qI_scale=qs, q_values=qv)


def test_fp8_query_argument_checks():
    qI, w, k8, ks, npool = _inputs(2, 8, 64, seed=1)
    q8, qs, _ = _fp8(qI)
    with pytest.raises(ValueError):
        LS.scores(q8.cuda(), w.cuda(), k8.cuda(), npool.cuda(), 0.1, pk_scale=ks.cuda())  # no qI_scale
    with pytest.raises(ValueError):
        LS.scores(qI.cuda(), w.cuda(), k8.cuda(), npool.cuda(), 0.1, pk_scale=ks.cuda(), qI_scale=qs.cuda())


@pytest.mark.parametrize("q_fp8", [False, True])
def test_causal_chunk_small(q_fp8):
    """A small chunk of the config-5 form: 256 cached keys, 70 new queries at positions 256 .. 325."""
    say(f"prefill causal chunk 256+70 q_fp8={q_fp8}")
    cfg = W.PrefillConfig("small", cached=256, chunk=70, q_fp8=q_fp8)
    inp = W.make_prefill_inputs(cfg, seed=5)
    _check_scores(inp.qI, inp.w, inp.k8, inp.k_scale, inp.npool, cfg.scale, qI_scale=inp.qI_scale,
                  q_values=inp.q_values())


@pytest.mark.parametrize("P,keep", [(5000, 2048), (3000, 64), (40000, 2048), (40001, 2048), (300000, 16)])
def test_select_exact_on_the_kernels_scores(P, keep):
    """dsa_prefill_select against the exact selection of the kernel's own scores: flat rows (P <= 32,768), two levels
    with the sub-block maxima written by the indexer (sub 4; P a multiple of it or not), and two levels with sub-blocks
    too large for that (sub 128: block_max_kernel)."""
    say(f"prefill select P={P} keep={keep}")
    N = 6
    qI, w, k8, ks, npool = _inputs(N, 64, P, seed=P + keep)
    npool[2] = keep - 7  # fewer candidates than keep: all of them
    npool[3] = 0
    args = (qI.cuda(), w.cuda(), k8.cuda(), npool.cuda())
    sc = LS.scores(*args, 128 ** -0.5, pk_scale=ks.cuda()).cpu()
    pools, cnt, vals = LS.select(*args, keep, 128 ** -0.5, pk_scale=ks.cuda())
    torch.cuda.synchronize()
    ri, rc = O.topk_ref(sc, keep, npool)
    assert torch.equal(pools.cpu(), ri)
    assert torch.equal(cnt.cpu(), rc)
    assert torch.equal(cnt.cpu(), npool.long().clamp(0, P).clamp(max=keep))
    live = torch.arange(keep).view(1, -1) < rc.view(-1, 1)
    assert torch.equal(vals.cpu(), torch.where(live, sc.gather(1, ri), O.NEG_INF))
    vp, vc, vv = LS.select(*args, keep, 128 ** -0.5, vorder=True, pk_scale=ks.cuda())
    assert torch.equal(vc.cpu(), rc)
    for n in range(N):  # the same set, by score descending then pool ascending
        c = int(rc[n])
        assert torch.equal(torch.sort(vp[n, :c].cpu()).values, ri[n, :c])
        v = vv[n, :c].cpu()
        assert torch.all(v[:-1] >= v[1:])
        assert torch.all(vp[n, c:] == 0) and torch.all(vv[n, c:] == O.NEG_INF)


@pytest.mark.parametrize("q_fp8", [False, True])
def test_select_two_level_sub_blocks_of_two(q_fp8):
    """Two-level selection with sub-blocks of 2 (P 40,000, keep 6,000): the indexer writes the sub-block maxima
    score by score (a 16-byte read would take the next sub-block's scores into a maximum), and the selection is
    bit-exact against the exact selection of the kernel's own scores, for bf16 and FP8 queries."""
    P, keep, N = 40000, 6000, 6
    say(f"prefill select sub 2 P={P} keep={keep} q_fp8={q_fp8}")
    qI, w, k8, ks, npool = _inputs(N, 64, P, seed=77 + q_fp8)
    npool[0], npool[1], npool[2] = P, keep - 3, 0
    qs = None
    if q_fp8:
        qI, qs, _ = _fp8(qI)
        qs = qs.cuda()
    args = (qI.cuda(), w.cuda(), k8.cuda(), npool.cuda())
    sc = LS.scores(*args, 128 ** -0.5, pk_scale=ks.cuda(), qI_scale=qs).cpu()
    pools, cnt, vals = LS.select(*args, keep, 128 ** -0.5, pk_scale=ks.cuda(), qI_scale=qs)
    torch.cuda.synchronize()
    ri, rc = O.topk_ref(sc, keep, npool)
    assert torch.equal(cnt.cpu(), rc)
    assert torch.equal(pools.cpu(), ri)
    live = torch.arange(keep).view(1, -1) < rc.view(-1, 1)
    assert torch.equal(vals.cpu(), torch.where(live, sc.gather(1, ri), O.NEG_INF))


@pytest.mark.parametrize("P,keep,tile", [(5000, 2048, 8), (40000, 2048, 12), (40001, 2048, 7), (300000, 16, 10),
                                          (40000, 6000, 9)])
@pytest.mark.parametrize("q_fp8", [False, True])
def test_select_in_tiles(P, keep, tile, q_fp8):
    """dsa_prefill_select over several query tiles (tile_rows below N, the last tile shorter), through every
    selection plan: flat rows (P 5,000), two levels with the indexer's sub-block maxima (sub 4), the generic
    two-level form (sub 128: block maxima pass; sub 2 at keep 6,000: maxima score by score), each tile's selection
    on the second stream beside the next tile's scores where the plan allows. Bit-exact against the exact selection
    of the kernel's own scores, for the form that keeps two score tiles in the workspace and for the form that
    writes every score into the caller's buffer (whose scores must equal dsa_indexer_prefill's)."""
    N = 30
    say(f"prefill select in tiles P={P} keep={keep} tile={tile} q_fp8={q_fp8}")
    qI, w, k8, ks, npool = _inputs(N, 64, P, seed=P + keep + tile + q_fp8)
    npool[3], npool[4], npool[N - 1] = keep - 7, 0, P
    qs = None
    if q_fp8:
        qI, qs, _ = _fp8(qI)
        qs = qs.cuda()
    args = (qI.cuda(), w.cuda(), k8.cuda(), npool.cuda())
    sc = LS.scores(*args, 128 ** -0.5, pk_scale=ks.cuda(), qI_scale=qs).cpu()
    ri, rc = O.topk_ref(sc, keep, npool)
    live = torch.arange(keep).view(1, -1) < rc.view(-1, 1)
    want_vals = torch.where(live, sc.gather(1, ri), O.NEG_INF)
    ws = torch.zeros(LS.workspace_bytes(N, P, keep, tile), dtype=torch.uint8, device="cuda")
    for _ in range(2):  # the second call on the same workspace
        pools, cnt, vals = LS.select(*args, keep, 128 ** -0.5, pk_scale=ks.cuda(), qI_scale=qs, workspace=ws,
                                     tile_rows=tile)
        torch.cuda.synchronize()
        assert torch.equal(cnt.cpu(), rc)
        assert torch.equal(pools.cpu(), ri)
        assert torch.equal(vals.cpu(), want_vals)
    # the caller's-scores form through the C ABI: every score written, the same selection
    from trnrt_amd import _lib
    from trnrt_amd.kernels import _common as C
    lib = _lib.lib()
    stride = (P + 3) // 4 * 4 + 4
    wsb = int(lib.dsa_prefill_select_workspace_bytes(N, P, stride, keep, tile, 0))
    ws2 = torch.zeros(max(wsb, 256), dtype=torch.uint8, device="cuda")
    full = torch.full((N, stride), 7.0, device="cuda")
    pools2 = torch.empty(N, keep, dtype=torch.int64, device="cuda")
    cnt2 = torch.empty(N, dtype=torch.int64, device="cuda")
    vals2 = torch.empty(N, keep, dtype=torch.float32, device="cuda")
    q_arg = C.fp8_bytes(args[0], "qI") if q_fp8 else args[0]
    st = lib.dsa_prefill_select(C.ptr(q_arg), C.ptr(qs), C.ptr(args[1]), C.ptr(C.fp8_bytes(args[2], "pk")),
                                C.ptr(ks.cuda()), C.ptr(args[3]), C.ptr(full), C.ptr(pools2), C.ptr(cnt2),
                                C.ptr(vals2), C.ptr(ws2), wsb, N, 64, 128, P, stride, keep, 128 ** -0.5, tile,
                                C.stream_ptr(torch.device("cuda")))
    _lib.check(st, "dsa_prefill_select")
    torch.cuda.synchronize()
    assert torch.equal(full[:, :P].cpu(), sc)
    assert torch.all(full[:, P:].cpu() == O.NEG_INF)
    assert torch.equal(cnt2.cpu(), rc) and torch.equal(pools2.cpu(), ri) and torch.equal(vals2.cpu(), want_vals)


def test_decode_batch_form_of_dsa_long_scores():
    """dsa_long.scores with one context per row ([N, P, 128] keys) through the decode indexer."""
    say("dsa_long.scores 3-D keys")
    N, Hi, P = 3, 64, 320
    g = torch.Generator().manual_seed(9)
    qI = torch.randn(N, Hi, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(N, Hi, generator=g) * 0.25
    k8, ks = W.quantize_rows(torch.randn(N * P, 128, generator=g))
    npool = torch.tensor([320, 17, 0])
    got = dsa_long.scores(qI.cuda(), w.cuda(), k8.view(N, P, 128).cuda(), npool.cuda(), 128 ** -0.5,
                          pk_scale=ks.view(N, P).cuda())
    torch.cuda.synchronize()
    got = got.cpu()
    for n in range(N):
        ref = O.prefill_scores_ref(qI[n:n + 1], w[n:n + 1], k8[n * P:(n + 1) * P], ks[n * P:(n + 1) * P],
                                   npool[n:n + 1], 128 ** -0.5)
        live = ref > -1e29
        assert row_rel_err(got[n:n + 1], ref, live) <= TOL
        assert torch.all(got[n:n + 1][~live] < -1e29)


# 64 rows of a 2,048-query chunk: the first and last 16 and 32 spread between them
ROWS64 = list(range(16)) + [16 + 63 * i for i in range(32)] + list(range(2032, 2048))


def _prefill_ref_rows(c, rows, cfg, q_values):
    """prefill_scores_ref of the given rows in groups of 8 (the oracle's [rows, heads, keys] intermediate stays
    near 140 MB)."""
    out = []
    for i in range(0, len(rows), 8):
        r = rows[i:i + 8]
        out.append(O.prefill_scores_ref(q_values[r], c.w[r], c.k8, c.k_scale, c.npool[r], cfg.scale))
    return torch.cat(out)


def test_config5_full_size_sampled_rows():
    """Config 5 (65,536 cached + 2,048 new queries, 64 heads, FP8 queries): every row's candidate count and NEG_INF
    tail, and the oracle on 64 rows (the first and last 16); the selection of those rows bit-exact on the kernel's
    scores."""
    cfg = W.PREFILL_CONFIGS[5]
    say(f"prefill config 5 {cfg.name}")
    inp = W.make_prefill_inputs(cfg, seed=0, device="cuda")
    pools, cnt, vals = LS.select(inp.qI, inp.w, inp.k8, inp.npool, cfg.keep, cfg.scale, pk_scale=inp.k_scale,
                                 qI_scale=inp.qI_scale)
    sc = LS.scores(inp.qI, inp.w, inp.k8, inp.npool, cfg.scale, pk_scale=inp.k_scale, qI_scale=inp.qI_scale)
    torch.cuda.synchronize()
    assert torch.all(cnt == cfg.keep)
    P = cfg.P
    live = torch.arange(P, device="cuda").view(1, P) < inp.npool.view(-1, 1).long()
    assert torch.all((sc > -1e29) == live)
    rows = ROWS64
    c = inp.to("cpu")
    ref = _prefill_ref_rows(c, rows, cfg, c.q_values())
    got = sc[rows].cpu()
    err = row_rel_err(got, ref, ref > -1e29)
    say(f"  config 5 sampled rel err {err:.3e}")
    assert err <= TOL
    ri, rc = O.topk_ref(got, cfg.keep, c.npool[rows])
    assert torch.equal(pools[rows].cpu(), ri)
    assert torch.equal(vals[rows].cpu(), got.gather(1, ri))


def _chunk_attention(inp, cfg, pools, cnt, rows_form):
    """o [C, H, 512] of the chunk's queries over their selected tokens: the reference's flow (slots with the tail
    slot, then attend; trnrt/models/mla.py:524-526) or the token form through the shared page table."""
    C = cfg.chunk
    if rows_form:
        positions = torch.arange(cfg.cached, cfg.cached + C, device="cuda")
        rows, bias = dsa_long.slots(pools, cnt, inp.npool, positions, inp.table, cfg.page_size, 1, cfg.keep + 1)
        return dsa_long.attend(inp.q, inp.kv_cache, rows, bias, cfg.softmax_scale, kc_scale=inp.kv_scale), None
    table = inp.table.view(1, -1).expand(C, -1).contiguous()
    return dsa_decode.attend_tokens(inp.q, inp.kv_cache, inp.kv_scale, pools, cnt, table, cfg.page_size,
                                    cfg.softmax_scale)


@pytest.mark.parametrize("rows_form", [False, True])
def test_chunk_attention_vs_oracle(rows_form):
    """A small causal chunk end to end: FP8 indexer -> exact selection -> sparse MLA over the selected tokens, every
    row against the oracle's attention over the same selection."""
    cfg = W.PrefillConfig("small", cached=3000, chunk=24, keep=256, q_fp8=True)
    say(f"prefill chunk attention rows_form={rows_form}")
    inp = W.make_prefill_inputs(cfg, seed=8, device="cuda", attention=True)
    pools, cnt, _ = LS.select(inp.qI, inp.w, inp.k8, inp.npool, cfg.keep, cfg.scale, pk_scale=inp.k_scale,
                              qI_scale=inp.qI_scale)
    o, lse = _chunk_attention(inp, cfg, pools, cnt, rows_form)
    torch.cuda.synchronize()
    c = inp.to("cpu")
    table = c.table.view(1, -1).expand(cfg.chunk, -1)
    ref_o, ref_lse = O.sparse_mla_ref(c.q, c.kv_cache, c.kv_scale, pools.cpu(), cnt.cpu(), table, cfg.page_size,
                                      cfg.softmax_scale)
    assert_attention_close(o, ref_o)
    if lse is not None:
        torch.testing.assert_close(lse.cpu(), ref_lse, atol=1e-3, rtol=1e-3)


def test_config5_chunk_attention_sampled_rows():
    """Config 5 end to end at full size (2,048 queries over 67,584 keys, top-2048, 64 heads): the attention of 64
    rows (the first and last 16) against the oracle over the kernel's own selection."""
    cfg = W.PREFILL_CONFIGS[5]
    say("prefill config 5 chunk attention")
    inp = W.make_prefill_inputs(cfg, seed=1, device="cuda", attention=True)
    pools, cnt, _ = LS.select(inp.qI, inp.w, inp.k8, inp.npool, cfg.keep, cfg.scale, pk_scale=inp.k_scale,
                              qI_scale=inp.qI_scale)
    o, lse = _chunk_attention(inp, cfg, pools, cnt, rows_form=False)
    torch.cuda.synchronize()
    rows = ROWS64
    c = inp.to("cpu")
    table = c.table.view(1, -1).expand(len(rows), -1)
    ref_o, ref_lse = O.sparse_mla_ref(c.q[rows], c.kv_cache, c.kv_scale, pools[rows].cpu(), cnt[rows].cpu(), table,
                                      cfg.page_size, cfg.softmax_scale)
    assert_attention_close(o[rows], ref_o)
    torch.testing.assert_close(lse[rows].cpu(), ref_lse, atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("P", [40000, 65540])
def test_select_many_rows_every_row(P):
    """520 queries (the many-row forms: one workgroup per row for both levels, the second level reading the selected
    sub-blocks in place and writing the reference's outputs): every row bit-exact against the exact selection of the
    kernel's own scores, with sub-blocks of 4 and of 8 (65,540 keys: the last sub-block crosses the row's end)."""
    say(f"prefill select many rows P={P}")
    N, keep = 520, 2048
    qI, w, k8, ks, npool = _inputs(N, 16, P, seed=P + 1)
    npool[:4] = torch.tensor([0, 1, keep - 1, P])
    args = (qI.cuda(), w.cuda(), k8.cuda(), npool.cuda())
    sc = LS.scores(*args, 128 ** -0.5, pk_scale=ks.cuda()).cpu()
    pools, cnt, vals = LS.select(*args, keep, 128 ** -0.5, pk_scale=ks.cuda())
    torch.cuda.synchronize()
    ri, rc = O.topk_ref(sc, keep, npool)
    assert torch.equal(cnt.cpu(), rc)
    assert torch.equal(pools.cpu(), ri)
    live = torch.arange(keep).view(1, -1) < rc.view(-1, 1)
    assert torch.equal(vals.cpu(), torch.where(live, sc.gather(1, ri), O.NEG_INF))


def test_config5_size_bf16_query_indexer():
    """The bf16-query prefill indexer (the reference's own arithmetic, trnrt/kernels/dsa_long_select.py:119-133) at
    config 5's size (2,048 queries over 67,584 keys, 64 heads) against the oracle on 64 rows, and every row's NEG_INF
    tail; the selection of those rows bit-exact on the kernel's scores."""
    cfg = W.PrefillConfig("prefill-65536+2048-bf16q", cached=65536, chunk=2048, q_fp8=False)
    say(f"prefill {cfg.name}")
    inp = W.make_prefill_inputs(cfg, seed=3, device="cuda")
    sc = LS.scores(inp.qI, inp.w, inp.k8, inp.npool, cfg.scale, pk_scale=inp.k_scale)
    pools, cnt, vals = LS.select(inp.qI, inp.w, inp.k8, inp.npool, cfg.keep, cfg.scale, pk_scale=inp.k_scale)
    torch.cuda.synchronize()
    P = cfg.P
    live = torch.arange(P, device="cuda").view(1, P) < inp.npool.view(-1, 1).long()
    assert torch.all((sc > -1e29) == live)
    c = inp.to("cpu")
    ref = _prefill_ref_rows(c, ROWS64, cfg, c.qI)
    got = sc[ROWS64].cpu()
    err = row_rel_err(got, ref, ref > -1e29)
    say(f"  bf16-query rel err {err:.3e}")
    assert err <= TOL
    ri, rc = O.topk_ref(got, cfg.keep, c.npool[ROWS64])
    assert torch.equal(pools[ROWS64].cpu(), ri) and torch.equal(cnt[ROWS64].cpu(), rc)
