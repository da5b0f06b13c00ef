"""Pins the oracle's indexer (oracle/dsa_oracle.py indexer_ref) against exact rational arithmetic on a tiny paged
cache, a brute-force float64 loop, the scale-folding identity relu(a x) = a relu(x) (a > 0) that both the reference
(trnrt/kernels/dsa_index.py:13-16, trnrt/models/mla.py:629) and the kernel rely on, and planted mistakes (no relu, a
shuffled page table, a squared scale) that must fail."""

from fractions import Fraction

import torch

from oracle import dsa_oracle as O

FP8 = torch.float8_e4m3fn


def _tiny(seed=0):
    """B 2 rows, Hi 3 heads, D 4, pages of 2: every value exact in bf16 / e4m3 / fp32 (small integers, powers of two),
    so the oracle's fp32 result is exact and comparable with Fractions."""
    g = torch.Generator().manual_seed(seed)
    B, Hi, D, ps = 2, 3, 4, 2
    num_pages = 6
    q = torch.randint(-3, 4, (B, Hi, D), generator=g).float().to(torch.bfloat16)
    w = torch.randint(-2, 3, (B, Hi), generator=g).float() / 4
    k8 = torch.randint(-8, 9, (num_pages * ps, D), generator=g).float().to(FP8)
    ks = 2.0 ** torch.randint(-3, 2, (num_pages * ps,), generator=g).float()
    table = torch.tensor([[3, 1, 5], [2, 4, 0]], dtype=torch.int32)
    ctx = [5, 3]
    return q, w, k8, ks, table, ctx, ps


def _exact(q, w, k8, ks, table, ctx, ps, stride):
    B, Hi, D = q.shape
    out = [[None] * stride for _ in range(B)]
    for b in range(B):
        for t in range(stride):
            if t >= ctx[b]:
                out[b][t] = Fraction(float(torch.tensor(O.NEG_INF, dtype=torch.float32)))  # NEG_INF in fp32
                continue
            slot = int(table[b, t // ps]) * ps + t % ps
            tot = Fraction(0)
            for h in range(Hi):
                dot = sum(Fraction(float(q[b, h, d])) * Fraction(float(k8[slot, d].float())) * Fraction(float(ks[slot]))
                          for d in range(D))
                tot += Fraction(float(w[b, h])) * max(dot, Fraction(0))
            out[b][t] = tot
    return out


def test_exact_rational_tiny_case():
    q, w, k8, ks, table, ctx, ps = _tiny()
    stride = 6
    got = O.indexer_ref(q, w, k8, ks, table, torch.tensor(ctx), ps, stride)
    want = _exact(q, w, k8, ks, table, ctx, ps, stride)
    for b in range(2):
        for t in range(stride):
            assert Fraction(float(got[b, t])) == want[b][t], (b, t)


def test_brute_force_float64():
    g = torch.Generator().manual_seed(1)
    B, Hi, D, ps, npg = 3, 8, 128, 64, 12
    q = torch.randn(B, Hi, D, generator=g).to(torch.bfloat16)
    w = torch.randn(B, Hi, generator=g) * 0.25 * D ** -0.5
    x = torch.randn(npg * ps, D, generator=g)
    s = x.abs().amax(-1) / 448
    k8 = (x / s[:, None]).clamp(-448, 448).to(FP8)
    table = (torch.randperm(npg - 1, generator=g)[: B * 3].view(B, 3) + 1).to(torch.int32)
    ctx = torch.tensor([192, 100, 1], dtype=torch.int32)
    got = O.indexer_ref(q, w, k8, s, table, ctx, ps, 192)
    for b in range(B):
        for t in range(192):
            if t >= int(ctx[b]):
                assert float(got[b, t]) == float(torch.tensor(O.NEG_INF, dtype=torch.float32))
                continue
            slot = int(table[b, t // ps]) * ps + t % ps
            kk = k8[slot].double() * float(s[slot])
            ref = sum(float(w[b, h]) * max(0.0, float((q[b, h].double() * kk).sum())) for h in range(Hi))
            assert abs(float(got[b, t]) - ref) <= 1e-5 * (1 + abs(ref)), (b, t)


def test_scale_after_the_dot_is_the_dequantised_key():
    """relu(a x) = a relu(x) for a > 0: scoring the raw e4m3 keys and scaling afterwards (the kernel's order) equals
    scoring the dequantised keys, up to fp32 rounding."""
    g = torch.Generator().manual_seed(2)
    B, Hi, D, ps, npg = 2, 16, 128, 64, 5
    q = torch.randn(B, Hi, D, generator=g).to(torch.bfloat16)
    w = torch.randn(B, Hi, generator=g) * 0.05
    x = torch.randn(npg * ps, D, generator=g) * 3
    s = x.abs().amax(-1) / 448
    k8 = (x / s[:, None]).clamp(-448, 448).to(FP8)
    table = torch.tensor([[1, 2], [3, 4]], dtype=torch.int32)
    ctx = torch.tensor([128, 128])
    a = O.indexer_ref(q, w, k8, s, table, ctx, ps, 128)
    ones = torch.ones_like(s)
    raw = O.indexer_ref(q, w, k8, ones, table, ctx, ps, 128)
    for b in range(B):
        slots = O.token_slots(table[b], torch.arange(128), ps)
        d = (a[b] - raw[b] * s[slots]).abs().max() / a[b].abs().max()  # the reference's error form, test_dsa_index.py:100
        assert d < 1e-5, float(d)


def test_planted_mistakes_fail():
    q, w, k8, ks, table, ctx, ps = _tiny(3)
    w = torch.tensor([[1.0, -2.0, 0.5], [-1.0, 1.0, 1.0]])
    good = O.indexer_ref(q, w, k8, ks, table, torch.tensor(ctx), ps, 6)
    want = _exact(q, w, k8, ks, table, ctx, ps, 6)
    assert all(Fraction(float(good[b, t])) == want[b][t] for b in range(2) for t in range(6))
    # no relu
    no_relu = torch.full_like(good, O.NEG_INF)
    for b in range(2):
        K = O.row_tokens(k8, ks, table[b], ctx[b], ps)
        no_relu[b, : ctx[b]] = torch.einsum("h,ht->t", w[b], torch.einsum("hd,td->ht", q[b].float(), K))
    assert not torch.equal(no_relu, good)
    # rows swapped in the page table
    bad_table = table.flip(0)
    assert not torch.equal(O.indexer_ref(q, w, k8, ks, bad_table, torch.tensor(ctx), ps, 6), good)
    # the scale applied twice
    assert not torch.equal(O.indexer_ref(q, w, k8, ks * ks, table, torch.tensor(ctx), ps, 6), good)
