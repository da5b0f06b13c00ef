"""The one-launch decode layer (dsa_decode_layer on rows of up to 32,768 tokens: csrc/dsa_fused.hip) against the
oracle and against the separate-kernel form (dsa_decode_layer_chain) on the same seeded inputs.

Bounds (the north star's): indexer scores within 1e-2 row-relative of oracle/dsa_oracle.py indexer_ref (after
trnrt/kernels/dsa_index.py:44-50); the top-k indices and counts bit-exact against the oracle's selection of the
kernel's own scores (topk_ref, after trnrt/models/dsa_select.py:33-38); the bf16 output within 2e-2 and lse within
1e-3 of the oracle attention over the kernel's selection (after trnrt/kernels/dsa_decode.py:26-37). Cases: configs 1
and 2 in full, a ragged batch of 12 rows (two launches) with empty, one-token, shorter-than-keep and full rows, 16 and
32 query heads with 16 and 48 indexer heads, rows of equal scores (every key a tie: the candidates past the LDS
cache), of two and of a hundred score values, key scales over forty octaves, a row whose selection crowds into two
workgroups, and the workspace left as the next call needs it (histograms and barrier words zero, no barrier wait gave
up). Each case also checks which selection form its rows took (the one-exchange form from the key lists, or the
two-exchange form)."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, launched_kernels, row_rel_err, say
from tests.test_gpu_layer import _attention_check
from trnrt_amd import workloads as W
from trnrt_amd.kernels.dsa_layer import DecodeLayer

pytestmark = pytest.mark.gpu


def _run(g, chain=False):
    cfg = g.cfg
    L = DecodeLayer(cfg.B, cfg.Hi, cfg.H, g.max_pages, cfg.page_size, g.num_pages, cfg.keep, cfg.scale,
                    max_len=max(max(g.lengths), 1), chain=chain)
    L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len)
    torch.cuda.synchronize()
    return L


# The workspace's first 8 KiB: per XCD eight 128-byte lines, word 0 of each a copy of the barrier counter, the first
# line's words 2 and 3 the status words; the row histograms follow.
SYNC_LINES, LINE_WORDS = 8, 32
XCD_WORDS = SYNC_LINES * LINE_WORDS
SYNC_WORDS = 8 * XCD_WORDS


def sync_block(ws: torch.Tensor):
    """The barrier block of an int32 workspace: (the counter copies [8, 8], the first lines [8, 32]); asserts that
    every other word of it is zero and that every XCD's copies agree."""
    s = ws[:SYNC_WORDS].view(8, SYNC_LINES, LINE_WORDS)
    ctr = s[:, :, 0]
    assert torch.all(ctr == ctr[:, :1]), f"counter copies differ: {ctr.tolist()}"
    assert torch.all(s[:, 0, 4:] == 0) and torch.all(s[:, 1:, 1:] == 0), "words past the barrier and status words"
    return ctr, s[:, 0]


def _workspace_clean(L):
    """The per-XCD barrier counters hold a multiple of 256 (each launch adds 256 on the XCDs it uses), the word after
    each is zero, the histograms are zero again, and no barrier wait gave up (the status words, read through the C
    ABI's dsa_layer_status as well)."""
    ws = L.workspace.view(torch.int32).cpu()
    ctr, sync = sync_block(ws)
    assert torch.all(ctr % 256 == 0) and torch.all(sync[:, 1] == 0), f"barrier words: {sync[:, :3].tolist()}"
    assert torch.all(ws[SYNC_WORDS:SYNC_WORDS + L.B * 4096] == 0), "row histograms left non-zero"
    assert torch.all(sync[:, 2] == 0), "a barrier wait gave up"
    assert L.status()["gave_up"] == 0


def _two_exchange_per_xcd(L) -> list:
    """Per XCD, the rows that took the two-exchange selection (stages 2 and 3) since the workspace was made: the kernel
    counts them in the XCD's status words (row b of a launch runs on XCD b % 8); the others took the one-exchange
    selection from the key lists."""
    ws = L.workspace.view(torch.int32).cpu()
    per = sync_block(ws)[1][:, 3].tolist()
    assert L.status()["two_exchange"] == sum(per)
    return per


def _two_exchange_rows(L) -> int:
    return sum(_two_exchange_per_xcd(L))


def _check_full(inp, L, indexer=True):
    cfg = inp.cfg
    sc = L.scores.cpu()
    if indexer:
        ref = O.indexer_ref(inp.q_idx, inp.w_k, inp.k_cache, inp.k_scale, inp.table, inp.ctx_len, cfg.page_size,
                            sc.shape[1])
        err = row_rel_err(sc, ref, ref > -1e29)
        say(f"  indexer rel err {err:.3e}")
        assert err <= 1e-2
        assert torch.all(sc[ref <= -1e29] == O.NEG_INF)
    ri, rc = O.topk_ref(sc, cfg.keep, inp.ctx_len)
    assert torch.equal(L.cnt.cpu().long(), rc)
    assert torch.equal(L.idx.cpu().long(), ri)
    _attention_check(inp, L)


@pytest.mark.parametrize("c", [1, 2])
def test_fused_layer_configs(c):
    say(f"fused layer config {c}")
    inp = W.make_inputs(W.CONFIGS[c], seed=3)
    g = inp.to("cuda")
    L = _run(g)
    names = launched_kernels(lambda: L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale,
                                            g.table, g.ctx_len))
    assert names == ["decode_fused_kernel"], names
    _check_full(inp, L)
    _workspace_clean(L)
    # config 2's rows of 32,768 tokens select from the key lists, and so does config 1's row of 4,096 (blocks of 128
    # positions: every list holds all its workgroup's keys), in both steps
    assert _two_exchange_rows(L) == 0


def test_fused_layer_ragged_two_launches():
    lengths = [32768, 1, 0, 2047, 2048, 2049, 5000, 31999, 32000, 64, 100, 17000]
    say(f"fused layer ragged B=12 {lengths}")
    cfg = W.Config("fused-ragged", B=12, L=32768, H=64, Hi=64)
    inp = W.make_inputs(cfg, seed=4, lengths=lengths)
    g = inp.to("cuda")
    L = _run(g)
    names = launched_kernels(lambda: L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale,
                                            g.table, g.ctx_len))
    assert names == ["decode_fused_kernel"] * 2, names
    _check_full(inp, L)
    _workspace_clean(L)


def test_fused_layer_block_sizes():
    """Rows whose lengths sit at and just past multiples of 1,024 tokens: the workgroups' blocks of positions take
    sizes from 32 to 1,024 (32 ceil(L / 1024)), across the size past which a key list no longer holds a whole block
    (192 -> 224 positions) and with blocks ending inside pages; 16 rows, two launches, every position of every row
    against the oracle."""
    lengths = [1024, 1025, 2048, 3072, 3073, 6144, 6145, 7168, 12288, 16385, 20480, 25600, 26215, 30000, 31744,
               32767]
    say(f"fused layer block sizes B=16 {lengths}")
    cfg = W.Config("fused-blocks", B=16, L=32768, H=64, Hi=64)
    inp = W.make_inputs(cfg, seed=14, lengths=lengths)
    g = inp.to("cuda")
    L = _run(g)
    _check_full(inp, L)
    _workspace_clean(L)


@pytest.mark.parametrize("seed", [101, 202, 303, 404])
def test_fused_layer_random_batches(seed):
    """Seeded random batches: 1 to 12 rows of random lengths (1 .. 32,768, a third of them short), query heads 16, 32
    or 64 with 16 to 64 indexer heads; scores, selection and attention against the oracle on every position."""
    g = torch.Generator().manual_seed(seed)
    B = int(torch.randint(1, 13, (1,), generator=g))
    H = [16, 32, 64][int(torch.randint(0, 3, (1,), generator=g))]
    Hi = [16, 32, 48, 64][int(torch.randint(0, 4, (1,), generator=g))]
    lengths = [int(torch.randint(1, 32769, (1,), generator=g)) if torch.rand(1, generator=g) > 1 / 3
               else int(torch.randint(1, 4097, (1,), generator=g)) for _ in range(B)]
    say(f"fused layer random seed={seed} B={B} H={H} Hi={Hi} {lengths}")
    cfg = W.Config(f"fused-rand{seed}", B=B, L=32768, H=H, Hi=Hi)
    inp = W.make_inputs(cfg, seed=seed, lengths=lengths)
    gi = inp.to("cuda")
    L = _run(gi)
    _check_full(inp, L)
    _workspace_clean(L)


@pytest.mark.parametrize("H,Hi", [(16, 16), (32, 48), (128, 64)])
def test_fused_layer_head_counts(H, Hi):
    say(f"fused layer H={H} Hi={Hi}")
    keep = 1024 if H == 128 else 2048  # 128 heads: 4 splits of 256 slots
    cfg = W.Config(f"fused-h{H}", B=3, L=10000, H=H, Hi=Hi, keep=keep)
    inp = W.make_inputs(cfg, seed=5 + H, lengths=[4096, 3000, 10000])
    g = inp.to("cuda")
    L = _run(g)
    _check_full(inp, L)
    _workspace_clean(L)


def _tied_inputs(values: int):
    """A batch whose key rows take `values` patterns (row t of the cache: pattern t % values), so the scores of a row
    take at most that many values and the keep-th is tied with many others."""
    cfg = W.Config(f"fused-ties{values}", B=4, L=32768, H=64, Hi=64)
    inp = W.make_inputs(cfg, seed=6 + values, lengths=[32768, 20000, 2500, 7000])
    base_k, base_s = inp.k_cache[64:64 + values].clone(), inp.k_scale[64:64 + values].clone()
    n = inp.k_cache.shape[0]
    rep = (n + values - 1) // values
    inp.k_cache.copy_(base_k.repeat(rep, 1)[:n])
    inp.k_scale.copy_(base_s.repeat(rep)[:n])
    return inp


@pytest.mark.parametrize("values", [1, 2, 100])
def test_fused_layer_ties(values):
    """Rows of 32,768, 20,000, 2,500 and 7,000 tokens (blocks of 1024, 640, 96 and 224 positions; the last end inside
    pages). One score value: on the rows whose blocks hold more positions than a key list, every workgroup's keys fill
    one bin, its key list stays empty and the row takes the two-exchange selection. Two values: the same for the rows
    of 32,768 and 20,000 (a workgroup's larger value alone overfills a list); at 7,000 each list holds its block's
    keys of the larger value, which hold the whole selection, so the row selects from the lists, ties at T by
    position. The row of 2,500 (every list holds all its keys) always selects from the lists. A hundred values: the
    full row selects from the key lists, with the keep-th largest tied with keys that are not taken (the lowest
    positions of the tie are)."""
    say(f"fused layer ties values={values}")
    inp = _tied_inputs(values)
    L = _run(inp.to("cuda"))
    sc = L.scores.cpu()
    for b, n in enumerate(inp.lengths):  # ties by construction: one score value per pattern in each row
        assert len(torch.unique(sc[b, :n])) <= values
    _check_full(inp, L, indexer=False)
    _workspace_clean(L)
    per_row = _two_exchange_per_xcd(L)[:4]
    if values == 1:
        assert per_row == [1, 1, 0, 1], per_row
    elif values == 2:
        assert per_row == [1, 1, 0, 0], per_row
    else:
        assert per_row[0] == 0 and per_row[2] == 0, per_row
    if values == 100:
        keep = inp.cfg.keep
        t = sc[0][L.idx[0].cpu().long()].min()
        assert int((sc[0] == t).sum()) > int((sc[0][L.idx[0].cpu().long()] == t).sum()) > 0, "no partial tie at T"


def test_fused_layer_wide_scales():
    """Key scales spread over forty octaves: each workgroup's listed keys fall in more histogram bins than its list
    header carries, so the one-exchange selection counts those lists key by key; two full rows, both selecting from
    the lists."""
    say("fused layer wide scales")
    cfg = W.Config("fused-wide", B=2, L=32768, H=64, Hi=64)
    inp = W.make_inputs(cfg, seed=13)
    g = torch.Generator().manual_seed(13)
    inp.k_scale.copy_(torch.exp2(torch.randint(-20, 21, inp.k_scale.shape, generator=g).float()))
    L = _run(inp.to("cuda"))
    _check_full(inp, L)
    _workspace_clean(L)
    assert _two_exchange_rows(L) == 0


def test_fused_layer_concentrated_selection():
    """A full row whose largest scores crowd into its first 2,048 positions (their keys' scales raised a thousandfold):
    two workgroups hold most of the selection, more than their key lists can, so the row falls back to the
    two-exchange selection after reading the lists; a second full row selects from its lists in the same launch."""
    say("fused layer concentrated selection")
    cfg = W.Config("fused-crowded", B=2, L=32768, H=64, Hi=64)
    inp = W.make_inputs(cfg, seed=12)
    ps = cfg.page_size
    pos = torch.arange(2048)
    slots = inp.table[0, pos // ps].long() * ps + pos % ps
    inp.k_scale[slots] *= 1000.0
    L = _run(inp.to("cuda"))
    sel = L.idx[0].cpu().long()
    assert int((sel < 1024).sum()) > 192 and int(((sel >= 1024) & (sel < 2048)).sum()) > 192
    _check_full(inp, L)
    _workspace_clean(L)
    assert _two_exchange_rows(L) == 1


def test_fused_matches_chain():
    """The one-launch and the separate-kernel forms of the same step: the same scores and selection, outputs within
    the bound (the attention's split sizes differ, so fp32 summation order does too)."""
    say("fused vs chain")
    lengths = [32768, 9000, 30000, 2048, 12345, 32768, 700, 25000]
    cfg = W.Config("fused-vs-chain", B=8, L=32768, H=64, Hi=64)
    g = W.make_inputs(cfg, seed=9, lengths=lengths).to("cuda")
    Lf, Lc = _run(g), _run(g, chain=True)
    assert torch.equal(Lf.scores, Lc.scores)
    assert torch.equal(Lf.idx, Lc.idx) and torch.equal(Lf.cnt, Lc.cnt)
    assert_attention_close(Lf.out, Lc.out)
    torch.testing.assert_close(Lf.lse.cpu(), Lc.lse.cpu(), atol=1e-3, rtol=1e-4)


def test_fused_repeated_steps_same_workspace():
    """Ten steps on one workspace, the inputs changed in place between them: every step equals a fresh layer's."""
    say("fused repeated steps")
    cfg = W.CONFIGS[2]
    g = W.make_inputs(cfg, seed=10).to("cuda")
    L = _run(g)
    for i in range(10):
        g.q.mul_(-1.0) if i % 2 else g.q_idx.mul_(-1.0)
        L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len)
    torch.cuda.synchronize()
    F = _run(g)
    assert torch.equal(L.idx, F.idx) and torch.equal(L.cnt, F.cnt)
    assert torch.equal(L.out, F.out) and torch.equal(L.lse, F.lse)
    _workspace_clean(L)
