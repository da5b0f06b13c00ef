"""Pins the oracle's selection (oracle/dsa_oracle.py topk_ref / selection_mask / two_level_ref) against independent
forms: a brute-force Python loop, the reference kernel's radix algorithm (a second, sort-free form), the reference's
literal known answer (trnrt tests/test_dsa_long.py:106-114), the reference's adversarial score kinds
(tests/test_dsa_topk.py:28-53) and its two-level case families (tests/test_dsa_long.py:48-84); a planted wrong tie
rule must fail."""

import json
import os

import pytest
import torch

from oracle import dsa_oracle as O

NEG = O.NEG_INF
HERE = os.path.dirname(os.path.abspath(__file__))


def scores_of(kind: str, rows: int, n: int, g: torch.Generator) -> torch.Tensor:
    """The reference's adversarial score kinds (trnrt tests/test_dsa_topk.py:28-53)."""
    if kind == "randn":
        return torch.randn(rows, n, generator=g)
    if kind == "integers":  # thousands tied at the threshold
        return torch.randint(-3, 4, (rows, n), generator=g).float()
    if kind == "zeros":  # exact zeros of both signs beside tiny values
        s = torch.relu(torch.randn(rows, n, generator=g)) * (torch.rand(rows, n, generator=g) - 0.5) * 1e-6
        s[:, ::3] = 0.0
        s[:, 1::5] = -0.0
        return s
    if kind == "wide":  # underflow to overflow, both signs, infinities
        return torch.sign(torch.randn(rows, n, generator=g)) * torch.exp(torch.randn(rows, n, generator=g) * 30)
    if kind == "invisible":
        s = torch.randn(rows, n, generator=g) * 10
        s[:, n // 3:] += NEG
        return s
    if kind == "ulps":  # one ulp apart at the threshold
        s = torch.randn(rows, n, generator=g)
        s[:, : n // 2] = 1.0 + torch.randint(0, 4, (rows, n // 2), generator=g).float() * 2**-23
        return s
    if kind == "equal":
        return torch.full((rows, n), 0.37)
    raise ValueError(kind)


KINDS = ["randn", "integers", "zeros", "wide", "invisible", "ulps", "equal"]


def brute(s: torch.Tensor, keep: int, vis_only: bool) -> torch.Tensor:
    """The rule written out: candidates in (descending value, ascending index) order, the first keep."""
    R, P = s.shape
    out = torch.zeros(R, P, dtype=torch.bool)
    for r in range(R):
        c = [p for p in range(P) if (not vis_only) or float(s[r, p]) > O.VISIBLE]
        c.sort(key=lambda p: (-float(s[r, p]), p))
        for p in c[:keep]:
            out[r, p] = True
    return out


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("vis_only", [True, False])
def test_sort_rule_is_the_brute_force_rule(kind, vis_only):
    g = torch.Generator().manual_seed(11 + KINDS.index(kind))
    for _ in range(6):
        n = int(torch.randint(2, 80, (1,), generator=g))
        keep = int(torch.randint(1, n + 3, (1,), generator=g))
        s = scores_of(kind, 3, n, g)
        assert torch.equal(O.selection_mask(s, keep, vis_only), brute(s, keep, vis_only)), (kind, n, keep)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("vis_only", [True, False])
def test_radix_form_equals_sort_form(kind, vis_only):
    """Two independent forms of the rule agree (the reference's emulate vs its reference_mask,
    tests/test_dsa_topk.py:109-120)."""
    g = torch.Generator().manual_seed(200 + KINDS.index(kind))
    for _ in range(8):
        n = int(torch.randint(16, 3000, (1,), generator=g))
        keep = int(torch.randint(1, n, (1,), generator=g))
        s = scores_of(kind, 4, n, g)
        got = O.topk_radix_ref(s, keep, vis_only)
        assert torch.equal(got, O.selection_mask(s, keep, vis_only)), (kind, n, keep)
        if not vis_only:
            assert (got.sum(-1) == keep).all()


def test_literal_known_answer():
    case = json.load(open(os.path.join(HERE, "golden", "topk_known_answer.json")))
    s = torch.tensor(case["scores"])
    idx, cnt = O.topk_ref(s, case["keep"])
    assert idx[0, : case["count"]].tolist() == case["selected"] and int(cnt[0]) == case["count"]
    idx2, cnt2 = O.two_level_ref(s, case["keep"], case["sub"])
    assert idx2[0, : case["count"]].tolist() == case["selected"] and int(cnt2[0]) == case["count"]
    assert brute(s, case["keep"], True)[0].nonzero().flatten().tolist() == case["selected"]


def _cases():
    """The reference's two-level families (tests/test_dsa_long.py:48-84): random, integer ties, exact zeros, relu,
    a plateau across sub-block boundaries, equal sub-block maxima, signed zeros and denormal neighbours, with
    candidate prefixes shorter than, equal to and longer than keep."""
    g = torch.Generator().manual_seed(0)
    out = []
    for P in (37, 64, 257, 1000, 4096):
        for keep in (1, 4, 16, 64):
            if keep >= P:
                continue
            N = 6
            npool = torch.tensor([0, 1, keep, keep + 1, P // 2, P])
            cand = torch.arange(P).view(1, P) < npool.view(N, 1)

            def put(s, cand=cand):
                return torch.where(cand, s, torch.tensor(NEG))

            out.append(put(torch.randn(N, P, generator=g)))
            out.append(put(torch.randint(0, 5, (N, P), generator=g).float()))
            out.append(put(torch.zeros(N, P)))
            out.append(put(torch.relu(torch.randn(N, P, generator=g) - 1.5)))
            s = torch.full((N, P), 1.0)
            s[:, P // 3:] = 2.0
            s[:, -3:] = 5.0
            out.append(put(s))
            s = torch.zeros(N, P)
            for p in range(P):
                if (p * 7) % 4 == p % 4:
                    s[:, p] = 3.0
            out.append(put(s))
            s = torch.where(torch.rand(N, P, generator=g) < 0.5, torch.tensor(0.0), torch.tensor(-0.0))
            s = s + torch.where(torch.rand(N, P, generator=g) < 0.1, torch.tensor(1e-45), torch.tensor(0.0))
            out.append(put(s))
            out[-7:] = [(x, keep) for x in out[-7:]]
    return out


@pytest.mark.parametrize("sub", [2, 4, 32])
def test_two_level_equals_flat(sub):
    n = 0
    for s, keep in _cases():
        want = O.topk_ref(s, keep)
        got = O.two_level_ref(s, keep, sub)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), (s.shape, keep, sub)
        n += 1
    assert n > 100


def test_counts_and_lengths():
    g = torch.Generator().manual_seed(3)
    s = torch.randn(5, 300, generator=g)
    lens = [0, 1, 50, 299, 300]
    idx, cnt = O.topk_ref(s, 64, lens)
    assert cnt.tolist() == [0, 1, 50, 64, 64]
    for r, L in enumerate(lens):
        sel = idx[r, : int(cnt[r])]
        assert (sel < max(L, 1)).all()
        assert torch.all(sel[1:] > sel[:-1])  # ascending, distinct
        assert (idx[r, int(cnt[r]):] == 0).all()
        if L > 64:
            assert torch.equal(sel, O.topk_ref(s[r:r + 1, :L], 64)[0][0])


def test_planted_wrong_tie_rule_fails():
    """Positive control: a selection that breaks ties to the HIGHEST index differs from the rule on tied data."""
    g = torch.Generator().manual_seed(5)
    s = scores_of("integers", 4, 500, g)

    def wrong(s, keep):
        r = torch.flip(s, dims=[-1])
        return torch.flip(O.selection_mask(r, keep, True), dims=[-1])

    assert not torch.equal(wrong(s, 100), brute(s, 100, True))
    assert torch.equal(O.selection_mask(s, 100, True), brute(s, 100, True))


def test_pooled_mask_known_answer():
    """dsa_topk._out (trnrt/kernels/dsa_topk.py:89-93): the selection, with tail every non-candidate pool, repeated
    over each pool's kp tokens."""
    s = torch.tensor([[3.0, 1.0, O.NEG_INF, O.NEG_INF]])
    N = float(torch.tensor(O.NEG_INF, dtype=torch.float32))  # NEG_INF as fp32 holds it
    assert O.topk_mask_ref(s, 1, True, 2, True).tolist() == [[0.0, 0.0, N, N, 0.0, 0.0, 0.0, 0.0]]
    assert O.topk_mask_ref(s, 1, True, 2, False).tolist() == [[0.0, 0.0, N, N, N, N, N, N]]
    assert O.topk_mask_ref(s, 3, True, 1, False).tolist() == [[0.0, 0.0, N, N]]  # only the visible ones
