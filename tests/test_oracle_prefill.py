"""Pins the oracle's prefill-chunk indexer (oracle/dsa_oracle.py prefill_scores_ref, after
trnrt/kernels/dsa_long_select.py:119-133 `emulate_scores`) against exact rational arithmetic on a tiny case, a
brute-force float64 loop, the decode indexer oracle through an identity page table (the same sum with the scale
folded into the head weights), and planted mistakes (a candidate mask off by one, no relu, one accumulator dropped)
that must fail."""

from fractions import Fraction

import pytest
import torch

from oracle import dsa_oracle as O

FP8 = torch.float8_e4m3fn


def _tiny(seed=0):
    """N 3 queries, Hi 5 heads (odd: both accumulators and an unpaired even head), D 4, P 6 keys; small integers and
    powers of two, so every fp32 operation is exact and the result is comparable with Fractions."""
    g = torch.Generator().manual_seed(seed)
    N, Hi, D, P = 3, 5, 4, 6
    q = torch.randint(-3, 4, (N, Hi, D), generator=g).float().to(torch.bfloat16)
    w = torch.randint(-2, 3, (N, Hi), generator=g).float() / 4
    k8 = torch.randint(-8, 9, (P, D), generator=g).float().to(FP8)
    ks = 2.0 ** torch.randint(-3, 2, (P,), generator=g).float()
    npool = torch.tensor([6, 0, 4])
    return q, w, k8, ks, npool, 0.5


def _exact(q, w, k8, ks, npool, scale, stride):
    N, Hi, D = q.shape
    P = k8.shape[0]
    neg = Fraction(float(torch.tensor(O.NEG_INF, dtype=torch.float32)))
    out = []
    for n in range(N):
        row = []
        for p in range(stride):
            if p >= min(int(npool[n]), P):
                row.append(neg)
                continue
            tot = Fraction(0)
            for h in range(Hi):
                dot = sum(Fraction(float(q[n, h, d])) * Fraction(float(k8[p, d].float())) * Fraction(float(ks[p]))
                          for d in range(D))
                tot += Fraction(float(w[n, h])) * max(Fraction(scale) * dot, Fraction(0))
            row.append(tot)
        out.append(row)
    return out


def test_exact_rational_tiny_case():
    q, w, k8, ks, npool, scale = _tiny()
    got = O.prefill_scores_ref(q, w, k8, ks, npool, scale, stride=8)
    want = _exact(q, w, k8, ks, npool, scale, 8)
    for n in range(3):
        for p in range(8):
            assert Fraction(float(got[n, p])) == want[n][p], (n, p)


def test_brute_force_float64():
    g = torch.Generator().manual_seed(3)
    N, Hi, D, P = 5, 7, 128, 70
    q = torch.randn(N, Hi, D, generator=g).to(torch.bfloat16)
    w = torch.randn(N, Hi, generator=g) / 4
    x = torch.randn(P, D, generator=g)
    k8, ks = (x / (x.abs().amax(1, keepdim=True) / 448)).to(FP8), x.abs().amax(1) / 448
    npool = torch.tensor([70, 1, 33, 0, 200])
    scale = 128 ** -0.5
    got = O.prefill_scores_ref(q, w, k8, ks, npool, scale)
    pk = k8.double() * ks.double().view(P, 1)
    for n in range(N):
        for p in range(P):
            if p >= min(int(npool[n]), P):
                assert got[n, p] == O.NEG_INF
                continue
            want = sum(float(w[n, h]) * max(scale * float(q[n, h].double() @ pk[p]), 0.0) for h in range(Hi))
            assert abs(float(got[n, p]) - want) <= 1e-5 * (1 + abs(want)), (n, p)


def test_agrees_with_the_decode_indexer_through_an_identity_table():
    """Each query of the chunk is a decode row whose page table is the identity and whose length is its candidate
    count; the decode oracle folds the scale into the head weights (relu(a x) = a relu(x), a > 0)."""
    g = torch.Generator().manual_seed(4)
    N, Hi, D, P, ps = 4, 16, 128, 128, 32
    q = torch.randn(N, Hi, D, generator=g).to(torch.bfloat16)
    w = torch.randn(N, Hi, generator=g) / 4
    x = torch.randn(P, D, generator=g)
    k8, ks = (x / (x.abs().amax(1, keepdim=True) / 448)).to(FP8), x.abs().amax(1) / 448
    npool = torch.tensor([128, 77, 1, 0])
    scale = 128 ** -0.5
    got = O.prefill_scores_ref(q, w, k8, ks, npool, scale)
    table = torch.arange(P // ps, dtype=torch.int32).view(1, -1).expand(N, -1)
    want = O.indexer_ref(q, w * scale, k8, ks, table, npool, ps, stride=P)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def _planted(kind, q, w, k8, ks, npool, scale, stride):
    N, Hi, _ = q.shape
    P = k8.shape[0]
    s = torch.einsum("nhd,pd->nhp", q.float(), O.dequant(k8, ks)) * scale
    r = s if kind == "no_relu" else torch.relu(s)
    lim = npool.long().clamp(0, P).view(N, 1) + (1 if kind == "mask_off_by_one" else 0)
    heads = range(0, Hi, 2) if kind == "odd_dropped" else range(Hi)
    tot = sum(r[:, h] * w[:, h:h + 1] for h in heads)
    out = torch.full((N, stride), O.NEG_INF)
    out[:, :P] = torch.where(torch.arange(P).view(1, P) < lim, tot, O.NEG_INF)
    return out


@pytest.mark.parametrize("kind", ["no_relu", "mask_off_by_one", "odd_dropped"])
def test_planted_mistakes_fail_the_exact_check(kind):
    q, w, k8, ks, npool, scale = _tiny()
    want = _exact(q, w, k8, ks, npool, scale, 8)
    bad = _planted(kind, q, w, k8, ks, npool, scale, 8)
    assert any(Fraction(float(bad[n, p])) != want[n][p] for n in range(3) for p in range(8)), kind
    good = _planted("none", q, w, k8, ks, npool, scale, 8)
    assert all(Fraction(float(good[n, p])) == want[n][p] for n in range(3) for p in range(8))
