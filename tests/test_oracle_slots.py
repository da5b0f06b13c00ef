"""Pins the oracle's slots (oracle/dsa_oracle.py pool_slots_ref, after trnrt/models/dsa_long.py:189-215) the way the
reference pins its own (tests/test_dsa_long.py:140-177): the tokens a query's slots attend (rows expanded to their kp
tokens, bias 0) are exactly the bucketed selection with the tail (topk_mask_ref, trnrt/kernels/dsa_topk.py:89-93 as
used by trnrt/models/glm5_next.py:194-208) intersected with the causal visibility, for a chunk (one table) and a
decode batch (one table per query), pages of 4, 8 and 64 tokens, kpool 4 and 1; planted mistakes must fail."""

import pytest
import torch

from oracle import dsa_oracle as O


def _case(L, positions, kp, keep, seed):
    g = torch.Generator().manual_seed(seed)
    P = L // kp
    N = positions.shape[0]
    npool = torch.div(positions + 1, kp, rounding_mode="floor")
    index = torch.randn(N, P, generator=g)
    index[:, ::5] = 0.0  # ties
    sc = index + torch.where(torch.arange(P).view(1, P) < npool.view(N, 1), 0.0, O.NEG_INF)
    pools, cnt = O.topk_ref(sc, keep)
    vis = torch.arange(L).view(1, L) <= positions.view(N, 1)
    want = (O.topk_mask_ref(sc, keep, True, kp, True) == 0) & vis
    return pools, cnt, npool, want


def _attended(rows, bias, kp, table, ps, N):
    tok = (rows.unsqueeze(-1) * kp + torch.arange(kp)).reshape(N, -1)  # cache slots
    live = bias.reshape(N, -1) == 0
    slot_of = (table.view(-1, 1) * ps + torch.arange(ps)).reshape(-1)  # context position -> cache slot
    return tok, live, slot_of


@pytest.mark.parametrize("kp,ps", [(4, 4), (4, 8), (4, 64), (1, 64)])
def test_slots_attend_the_bucketed_selection(kp, ps):
    for L, positions in ((64 * 4, torch.tensor([0, 2, 3, 4, 11, 12, 13, 30, 47, 63, 255])),
                         (64 * 6, torch.tensor([383, 200, 17, 7]))):
        keep = 3 if kp == 4 else 12
        pools, cnt, npool, want = _case(L, positions, kp, keep, seed=L + kp + ps)
        N = positions.shape[0]
        pages = L // ps
        table = torch.randperm(500)[:pages] + 1
        rows, bias = O.pool_slots_ref(pools, cnt, npool, positions, table, ps, kp, keep + 3)
        tok, live, slot_of = _attended(rows, bias, kp, table, ps, N)
        for n in range(N):
            assert sorted(tok[n][live[n]].tolist()) == sorted(slot_of[want[n]].tolist()), (ps, L, n)
        rows2, bias2 = O.pool_slots_ref(pools, cnt, npool, positions, table.expand(N, pages), ps, kp, keep + 3)
        assert torch.equal(rows2, rows) and torch.equal(bias2, bias)


def test_planted_mistakes_fail():
    kp, ps, keep, L = 4, 8, 3, 64
    positions = torch.tensor([2, 13, 30, 47])
    pools, cnt, npool, want = _case(L, positions, kp, keep, seed=3)
    table = torch.randperm(100)[: L // ps] + 1
    rows, bias = O.pool_slots_ref(pools, cnt, npool, positions, table, ps, kp, keep + 1)
    for kind in ("tail_off_by_one", "no_tail"):
        bad = bias.clone()
        if kind == "tail_off_by_one":  # the tail's last visible token dropped
            for n in range(positions.shape[0]):
                t = int(positions[n]) - int(npool[n]) * kp
                if 0 <= t < kp:
                    bad[n, keep, t] = O.NEG_INF
        else:
            bad[:, keep, :] = O.NEG_INF
        tok, live, slot_of = _attended(rows, bad, kp, table, ps, positions.shape[0])
        ok = all(sorted(tok[n][live[n]].tolist()) == sorted(slot_of[want[n]].tolist())
                 for n in range(positions.shape[0]))
        assert not ok, kind
