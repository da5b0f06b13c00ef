"""Pins the oracle's sparse MLA attention (oracle/dsa_oracle.py) against a brute-force float64 loop and the
invariants the reference's tests hold (trnrt tests/test_dsa_slots.py:96-122): one live slot gives its row; a fully
masked row is the uniform mean with lse ~ NEG_INF; lse is the log-sum-exp; any split of the slots combines back
(trnrt/models/mla.py:853-856); slot order does not matter; the token form (positions + page table) equals the row
form. A planted mistake (the value over all 576 columns, or no softmax scale) must fail."""

import math

import torch

from oracle import dsa_oracle as O

FP8 = torch.float8_e4m3fn


def _rows(seed, H=4, NS=10, dqk=12, dv=8):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, dqk, generator=g).to(torch.bfloat16)
    K = torch.randn(NS, dqk, generator=g)
    return q, K, dv


def test_brute_force_float64():
    q, K, dv = _rows(0)
    bias = torch.zeros(K.shape[0])
    bias[3] = O.NEG_INF
    bias[7] = O.NEG_INF
    o, lse = O.sparse_mla_rows_ref(q, K, bias, 0.3, dv)
    for h in range(q.shape[0]):
        s = [0.3 * float((q[h].double() * K[t].double()).sum()) + float(bias[t]) for t in range(K.shape[0])]
        m = max(s)
        e = [math.exp(x - m) for x in s]
        Z = sum(e)
        for d in range(dv):
            ref = sum(e[t] * float(K[t, d]) for t in range(K.shape[0])) / Z
            assert abs(float(o[h, d]) - ref) < 1e-5
        assert abs(float(lse[h]) - (m + math.log(Z))) < 1e-4


def test_one_live_slot_is_its_row():
    q, K, dv = _rows(1)
    bias = torch.full((K.shape[0],), O.NEG_INF)
    bias[4] = 0.0
    o, lse = O.sparse_mla_rows_ref(q, K, bias, 0.5, dv)
    torch.testing.assert_close(o, K[4, :dv].expand_as(o), rtol=0, atol=0)
    torch.testing.assert_close(lse, 0.5 * (q.float() @ K[4]), rtol=1e-6, atol=1e-6)


def test_fully_masked_row_is_the_uniform_mean():
    q, K, dv = _rows(2)
    bias = torch.full((K.shape[0],), O.NEG_INF)
    o, lse = O.sparse_mla_rows_ref(q, K, bias, 0.5, dv)
    torch.testing.assert_close(o, K[:, :dv].mean(0).expand_as(o), rtol=1e-5, atol=1e-6)
    assert torch.isfinite(o).all() and (lse < -1e29).all()


def test_lse_is_logsumexp_and_split_combines():
    q, K, dv = _rows(3, NS=40)
    bias = torch.zeros(40)
    bias[::7] = O.NEG_INF
    o, lse = O.sparse_mla_rows_ref(q, K, bias, 0.2, dv)
    s = 0.2 * q.float() @ K.t() + bias
    torch.testing.assert_close(lse, torch.logsumexp(s, -1), rtol=1e-6, atol=1e-5)
    g = torch.Generator().manual_seed(9)
    for parts in (2, 3, 7):
        lab = torch.randint(0, parts, (40,), generator=g)
        lab[:parts] = torch.arange(parts)  # no empty part
        os, ls = [], []
        for r in range(parts):
            b = torch.where(lab == r, bias, torch.tensor(float("-inf")))
            o_r, l_r = O.sparse_mla_rows_ref(q, K, b, 0.2, dv)
            os.append(o_r)
            ls.append(l_r)
        oc, lc = O.splitk_combine_ref(torch.stack(os), torch.stack(ls))
        torch.testing.assert_close(oc, o, rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(lc, lse, rtol=1e-6, atol=1e-5)


def test_slot_order_does_not_matter():
    q, K, dv = _rows(4, NS=30)
    bias = torch.zeros(30)
    perm = torch.randperm(30, generator=torch.Generator().manual_seed(1))
    a = O.sparse_mla_rows_ref(q, K, bias, 0.3, dv)
    b = O.sparse_mla_rows_ref(q, K[perm], bias[perm], 0.3, dv)
    torch.testing.assert_close(a[0], b[0], rtol=1e-5, atol=1e-6)


def test_token_form_equals_row_form():
    g = torch.Generator().manual_seed(5)
    B, H, ps, npg, keep = 2, 16, 64, 9, 40
    q = torch.randn(B, H, 576, generator=g).to(torch.bfloat16)
    x = torch.randn(npg * ps, 576, generator=g)
    s = x.abs().amax(-1) / 448
    kv = (x / s[:, None]).clamp(-448, 448).to(FP8)
    table = (torch.randperm(npg - 1, generator=g)[:8].view(B, 4) + 1).to(torch.int32)
    idx = torch.sort(torch.randperm(256, generator=g)[:keep]).values.view(1, keep).repeat(B, 1)
    cnt = torch.tensor([keep, 17])
    idx[1, 17:] = 0
    o, lse = O.sparse_mla_ref(q, kv, s, idx, cnt, table, ps, 192 ** -0.5)
    rows = torch.stack([O.token_slots(table[b], idx[b], ps) for b in range(B)])
    bias = torch.where(torch.arange(keep).view(1, keep) < cnt.view(B, 1), 0.0, O.NEG_INF)
    o2, lse2 = O.sparse_mla_slots_ref(q, kv, s, rows, bias, 192 ** -0.5)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    # planted mistakes
    wrong_scale = O.sparse_mla_slots_ref(q, kv, s, rows, bias, 1.0)[0]
    assert (wrong_scale - o).abs().max() > 1e-2
    K = O.dequant(kv[rows[0]], s[rows[0]])
    full = torch.softmax(192 ** -0.5 * q[0].float() @ K.t() + bias[0], -1) @ K  # value over all 576 columns
    assert full.shape[-1] != o.shape[-1]
