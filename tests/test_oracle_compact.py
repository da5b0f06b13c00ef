"""Pins of oracle/dsa_oracle.py compact_ref (trnrt/models/dsa_long.py:140-166) and slots_compact_ref
(trnrt/kernels/dsa_slots_c.py:92-103) on the CPU: brute force, known answers, equivalences with the uncompacted
forms, and planted mistakes that must fail."""

import torch

from oracle import dsa_oracle as O


def _brute_compact(sel, keep):
    N, M = sel.shape
    idx = [[0] * keep for _ in range(N)]
    cnt = [0] * N
    for n in range(N):
        k = 0
        for p in range(M):
            if float(sel[n, p]) > 0.5 and k < keep:
                idx[n][k] = p
                k += 1
        cnt[n] = k
    return torch.tensor(idx, dtype=torch.int64), torch.tensor(cnt, dtype=torch.int64)


def test_compact_known_answer():
    sel = torch.tensor([[0, 1, 0, 1, 1, 0, 0, 1], [0] * 8, [1] * 8], dtype=torch.float32)
    idx, cnt = O.compact_ref(sel, 3)
    assert idx.tolist() == [[1, 3, 4], [0, 0, 0], [0, 1, 2]]
    assert cnt.tolist() == [3, 0, 3]


def test_compact_brute_force_and_ascending():
    g = torch.Generator().manual_seed(1)
    for M, keep, dens in ((1, 1, 0.5), (37, 5, 0.1), (100, 64, 0.9), (300, 8, 0.02), (64, 64, 1.0)):
        sel = (torch.rand(6, M, generator=g) < dens).float()
        idx, cnt = O.compact_ref(sel, keep)
        bi, bc = _brute_compact(sel, keep)
        assert torch.equal(idx, bi) and torch.equal(cnt, bc)
        few = sel.sum(-1) <= keep  # rows with at most keep ones: the reference's _ascending
        if few.any():
            ai, ac = O.ascending(sel[few] > 0.5, keep)
            assert torch.equal(idx[few], ai) and torch.equal(cnt[few], ac)


def test_compact_planted_unclamped_count_fails():
    sel = torch.ones(2, 10)
    _, cnt = O.compact_ref(sel, 4)
    wrong = sel.sum(-1).to(torch.int64)  # a count not clamped to keep
    assert not torch.equal(cnt, wrong)
    assert cnt.tolist() == [4, 4]


def _slots_case(B=3, H=16, NS=6, kp=4, seed=2):
    g = torch.Generator().manual_seed(seed)
    pools = 10
    kv = (torch.randn(pools * kp, 576, generator=g) * 0.5).to(torch.float8_e4m3fn)
    ks = torch.rand(pools * kp, generator=g) + 0.5
    q = torch.randn(B, H, 576, generator=g)
    rows = torch.randint(0, pools, (B, NS), generator=g)
    bias = torch.where(torch.rand(B, NS, kp, generator=g) < 0.5, 0.0, O.NEG_INF)
    return q, kv, ks, rows, bias


def test_slots_compact_equals_uncompacted_with_visible_tokens():
    q, kv, ks, rows, bias = _slots_case()
    bias[:, 0, 0] = 0.0  # every row has a visible token
    kp = bias.shape[-1]
    o, lse = O.slots_compact_ref(q, kv, ks, rows, bias, 0.07)
    tok = (rows.unsqueeze(-1) * kp + torch.arange(kp)).reshape(rows.shape[0], -1)
    ro, rl = O.sparse_mla_slots_ref(q, kv, ks, tok, bias.reshape(rows.shape[0], -1), 0.07)
    torch.testing.assert_close(o, ro, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(lse, rl, atol=1e-4, rtol=1e-6)
    # a permutation of the slots changes nothing
    perm = torch.randperm(rows.shape[1], generator=torch.Generator().manual_seed(5))
    po, pl = O.slots_compact_ref(q, kv, ks, rows[:, perm], bias[:, perm], 0.07)
    torch.testing.assert_close(po, o, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(pl, lse, atol=1e-4, rtol=1e-6)


def test_slots_compact_empty_row_is_pool_zero_mean():
    q, kv, ks, rows, bias = _slots_case(B=2)
    bias[1] = O.NEG_INF  # row 1: no visible token
    kp = bias.shape[-1]
    o, lse = O.slots_compact_ref(q, kv, ks, rows, bias, 0.07)
    mean = O.dequant(kv[:kp], ks[:kp])[:, :512].mean(0)
    torch.testing.assert_close(o[1], mean.expand(o.shape[1], -1), atol=1e-6, rtol=1e-6)
    assert torch.all(lse[1] < -1e29)
    # a planted mistake: the empty row over its own (masked) slots instead of pool row 0 differs
    tok = (rows[1].unsqueeze(-1) * kp + torch.arange(kp)).reshape(-1)
    wrong = O.dequant(kv[tok], ks[tok])[:, :512].mean(0)
    assert not torch.allclose(wrong, mean, atol=1e-3)
