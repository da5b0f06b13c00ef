"""GPU parity of the exact top-k (trnrt_amd.kernels.dsa_topk -> dsa_topk): bit-exact indices and counts against the
oracle (oracle/dsa_oracle.py topk_ref, the rule of trnrt/models/dsa_select.py:33-38) when fed the same scores, on the
reference's adversarial score kinds, the decode shapes (flat rows up to 32K, two-level rows to 1M), ragged lengths and
the mask form."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import say
from tests.test_oracle_topk import KINDS, scores_of
from trnrt_amd.kernels import dsa_topk
from trnrt_amd.models import dsa_long

pytestmark = pytest.mark.gpu


def _exact(s: torch.Tensor, keep: int, lengths=None, vis_only=True):
    lg = None if lengths is None else torch.tensor(lengths, dtype=torch.int32).cuda()
    idx, cnt = dsa_topk.select_indices(s.cuda(), keep, lengths=lg, vis_only=vis_only,
                                       max_len=None if lengths is None else max(lengths))
    torch.cuda.synchronize()
    ri, rc = O.topk_ref(s, keep, lengths, vis_only)
    assert torch.equal(cnt.cpu().long(), rc)
    assert torch.equal(idx.cpu().long(), ri)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,keep", [(3000, 2048), (4096, 2048), (8192, 2048), (32768, 2048), (5000, 17), (777, 1)])
def test_kinds(kind, n, keep):
    say(f"topk {kind} n={n} keep={keep}")
    g = torch.Generator().manual_seed(KINDS.index(kind) * 100003 + n + keep)
    _exact(scores_of(kind, 4, n, g), keep)


@pytest.mark.parametrize("kind", ["randn", "integers", "wide", "equal"])
def test_all_candidates_vis_only_false(kind):
    say(f"topk vis_only=False {kind}")
    g = torch.Generator().manual_seed(31)
    _exact(scores_of(kind, 3, 6000, g), 2048, vis_only=False)


def test_ragged_lengths():
    say("topk ragged lengths")
    g = torch.Generator().manual_seed(8)
    s = torch.randn(6, 20000, generator=g)
    _exact(s, 2048, lengths=[20000, 2048, 2047, 1, 0, 9999])


@pytest.mark.parametrize("n", [65536, 131072])
@pytest.mark.parametrize("kind", ["randn", "integers", "invisible"])
def test_two_level_rows(n, kind):
    say(f"topk two-level n={n} {kind}")
    g = torch.Generator().manual_seed(n % 97)
    _exact(scores_of(kind, 3, n, g), 2048)


@pytest.mark.parametrize("kind", ["equal", "zeros", "wide", "integers"])
def test_long_rows_ties_and_ragged(kind):
    """Rows past 32,768 scores in a small batch (the long chunked selection): every score tied (the candidates past
    the LDS staging, ties taken in chunk and then position order across chunks), wide-range and integer scores, with
    ragged lengths that end inside, at and just past a 2,048-position chunk."""
    say(f"topk long rows {kind}")
    g = torch.Generator().manual_seed(KINDS.index(kind) + 4242)
    s = scores_of(kind, 4, 100000, g)
    _exact(s, 2048, lengths=[100000, 40000, 32769, 34816])


def test_one_million():
    say("topk 1M rows")
    g = torch.Generator().manual_seed(1)
    s = torch.randn(2, 1 << 20, generator=g)
    s[1, ::3] = 0.0
    _exact(s, 2048, lengths=[1 << 20, 700000])


def test_indexer_like_scores_config2_shape():
    """The decode shape of BASELINE config 2 (8 rows of 32,768, keep 2048) on scores formed like the indexer's
    (weighted relu head sums, both signs, dead keys at exactly 0; trnrt tests/test_dsa_topk.py:63-75)."""
    say("topk config-2 shape, pooled-like scores")
    g = torch.Generator().manual_seed(7)
    q = torch.randn(8, 8, 16, generator=g)
    k = torch.randn(32768, 16, generator=g)
    w = torch.randn(8, 8, generator=g)
    rel = torch.relu(torch.einsum("rhd,nd->rhn", q, k))
    rel[..., ::5] = 0.0
    _exact(torch.einsum("rh,rhn->rn", w, rel), 2048)


def test_mask_form_and_select_device():
    say("topk mask form + select_device")
    g = torch.Generator().manual_seed(12)
    s = scores_of("integers", 4, 5000, g)
    m = dsa_topk.select(s.cuda(), 700).cpu()
    want = O.selection_mask(s, 700, True)
    assert torch.equal(m == 0, want) and torch.equal(m < -1e29, ~want)
    idx, cnt = dsa_long.select_device(s.cuda(), 700)
    ri, rc = O.topk_ref(s, 700)
    assert idx.dtype == torch.int64 and torch.equal(idx.cpu(), ri) and torch.equal(cnt.cpu(), rc)


def test_deterministic():
    say("topk determinism")
    g = torch.Generator().manual_seed(2)
    s = scores_of("integers", 8, 32768, g).cuda()
    a = dsa_topk.select_indices(s, 2048)
    b = dsa_topk.select_indices(s, 2048)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("kp,tail", [(4, True), (4, False), (1, True)])
def test_pooled_mask_forms(kp, tail):
    """dsa_topk.select(kp, tail): the pooled indexer's block mask (trnrt/models/glm5_next.py:194-208): pool scores
    with the non-candidates (pools whose last token is not visible) at NEG_INF, keep 512."""
    say(f"topk pooled mask kp={kp} tail={tail}")
    g = torch.Generator().manual_seed(30 + kp)
    R, P, keep = 6, 2048, 512
    s = torch.randn(R, P, generator=g)
    npool = torch.tensor([2048, 1500, 512, 100, 0, 777])
    s[torch.arange(P).view(1, P) >= npool.view(R, 1)] = O.NEG_INF
    m = dsa_topk.select(s.cuda(), keep, kp=kp, tail=tail).cpu()
    assert torch.equal(m, O.topk_mask_ref(s, keep, True, kp, tail))


@pytest.mark.parametrize("P,keep,vis_only,kp,tail", [(5000, 5000, True, 1, False), (5000, 9000, False, 1, False),
                                                     (40000, 40000, True, 4, True), (70000, 80000, True, 2, False),
                                                     (70000, 70000, False, 1, False)])
def test_select_keep_at_least_p(P, keep, vis_only, kp, tail):
    """dsa_topk.select with keep >= P (rows longer than the kernel's 32,768 included): every visible score, or every
    score without vis_only, as the reference's short-cut (trnrt/kernels/dsa_topk.py:510-511, 103-105)."""
    say(f"topk select keep>=P P={P} keep={keep} vis_only={vis_only} kp={kp} tail={tail}")
    g = torch.Generator().manual_seed(P + keep)
    s = torch.randn(3, P, generator=g)
    s[0, P // 3:] = O.NEG_INF
    s[2, ::7] = O.VISIBLE  # exactly VISIBLE: not visible
    m = dsa_topk.select(s.cuda(), keep, vis_only=vis_only, kp=kp, tail=tail).cpu()
    assert torch.equal(m, O.topk_mask_ref(s, keep, vis_only, kp, tail))


@pytest.mark.parametrize("n", [6000, 9000, 16384, 20000, 32768])
@pytest.mark.parametrize("kind", ["randn", "integers", "zeros", "wide", "invisible", "equal"])
def test_many_rows_form(kind, n):
    """520 rows (a prefill chunk's shape): one workgroup per row holding the whole row (2 .. 8 float4 groups per
    thread), every row bit-exact against the oracle, with ragged lengths on some rows."""
    say(f"topk many rows {kind} n={n}")
    g = torch.Generator().manual_seed(KINDS.index(kind) * 7919 + n)
    s = scores_of(kind, 520, n, g)
    lengths = [n] * 520
    lengths[3], lengths[100], lengths[511] = 0, 2047, n - 1
    _exact(s, 2048, lengths)
