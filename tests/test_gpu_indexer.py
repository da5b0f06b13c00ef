"""GPU parity of the decode indexer (trnrt_amd.kernels.dsa_index -> dsa_indexer_decode) against the oracle
(oracle/dsa_oracle.py indexer_ref, trnrt/kernels/dsa_index.py:44-50) on the same seeded inputs; bound: max|diff| /
max|ref| <= 1e-2 per row (the north star; the products are exact, so the real error is fp32 summation order)."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import row_rel_err, say
from trnrt_amd import workloads as W
from trnrt_amd.kernels import dsa_index

pytestmark = pytest.mark.gpu
TOL = 1e-2
NEG32 = float(torch.tensor(O.NEG_INF, dtype=torch.float32))


def _check(inp, stride=None, cand=None, tol=TOL):
    cfg = inp.cfg
    stride = inp.max_pages * cfg.page_size if stride is None else stride
    g = inp.to("cuda")
    got = dsa_index.decode_scores(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.table, g.ctx_len, cfg.page_size, stride,
                                  cand=None if cand is None else cand.cuda())
    torch.cuda.synchronize()
    got = got.cpu()
    ref = O.indexer_ref(inp.q_idx, inp.w_k, inp.k_cache, inp.k_scale, inp.table, inp.ctx_len, cfg.page_size, stride)
    if cand is not None:
        ref = ref + cand
    live = ref > -1e29
    err = row_rel_err(got, ref, live)
    say(f"  indexer rel err {err:.3e}")
    assert err <= tol
    assert torch.equal(got < -1e29, ~live)
    return got, ref


@pytest.mark.parametrize("Hi", [16, 64])
def test_long_rows_ragged_batch(Hi):
    """Rows past 32,768 scores (the long-row streaming form): a ragged batch of empty, one-token, tile-edge and long
    rows, so that waves' tile ranges start and end inside and past contexts; every position against the oracle,
    NEG_INF past every context."""
    lengths = [70016, 0, 1, 31, 32, 33, 65, 5000, 32768, 32769, 1, 1, 1, 2, 3, 64, 12345, 70000, 69999, 100, 7,
               1024, 2048, 0]
    say(f"indexer long rows, ragged batch, Hi={Hi}")
    cfg = W.Config("long-ragged", B=len(lengths), L=70016, H=16, Hi=Hi)
    _check(W.make_inputs(cfg, seed=40 + Hi, lengths=lengths))


def test_config1():
    say("indexer config 1")
    _check(W.make_inputs(W.CONFIGS[1], seed=0))


@pytest.mark.parametrize("Hi", [16, 32, 48, 64])
def test_ragged_lengths_and_heads(Hi):
    say(f"indexer ragged Hi={Hi}")
    cfg = W.Config("ragged", B=4, L=300, H=16, Hi=Hi)
    _check(W.make_inputs(cfg, seed=Hi, lengths=[300, 64, 1, 129]))


def test_config2_full():
    say("indexer config 2")
    _check(W.make_inputs(W.CONFIGS[2], seed=0))


def test_cand_and_page_groups_surface():
    """The reference's call form: scores(q, w, pkc, page_groups(table), cand) with 128 pages per row and the last 3
    candidates NEG_INF (trnrt tests/test_dsa_index.py:33-42)."""
    say("indexer reference surface (page groups + cand)")
    cfg = W.Config("pg", B=2, L=128 * 64, H=16, Hi=32)
    inp = W.make_inputs(cfg, seed=3)
    P = 128 * 64
    cand = torch.zeros(2, P)
    cand[:, -3:] = O.NEG_INF
    g = inp.to("cuda")
    ps = cfg.page_size
    pkc = g.k_cache.view(-1, ps * 128)
    got = dsa_index.scores(g.q_idx, g.w_k, pkc, dsa_index.page_groups(g.table), cand.cuda(),
                           pkc_scale=g.k_scale.view(-1, ps)).cpu()
    ref = O.indexer_ref(inp.q_idx, inp.w_k, inp.k_cache, inp.k_scale, inp.table, inp.ctx_len, ps, P) + cand
    live = ref > -1e29
    assert row_rel_err(got, ref, live) <= TOL
    assert (got[:, -3:] < -1e29).all()


def test_wrong_table_is_caught():
    """Positive control: the kernel fed another row order of the page table must miss the oracle's scores."""
    say("indexer positive control")
    inp = W.make_inputs(W.Config("pc", B=2, L=512, H=16, Hi=16), seed=4)
    g = inp.to("cuda")
    got = dsa_index.decode_scores(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.table.flip(0).contiguous(), g.ctx_len,
                                  64).cpu()
    ref = O.indexer_ref(inp.q_idx, inp.w_k, inp.k_cache, inp.k_scale, inp.table, inp.ctx_len, 64)
    assert row_rel_err(got, ref, ref > -1e29) > TOL


def test_deterministic():
    say("indexer determinism")
    g = W.make_inputs(W.CONFIGS[1], seed=7).to("cuda")
    a = dsa_index.decode_scores(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.table, g.ctx_len, 64)
    b = dsa_index.decode_scores(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.table, g.ctx_len, 64)
    assert torch.equal(a, b)
