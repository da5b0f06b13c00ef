"""GPU parity of the compaction kernels (csrc/dsa_compact.hip) through their operator surfaces: dsa_long.compact
(trnrt/models/dsa_long.py:140-166) bit-exact against oracle compact_ref, and dsa_slots_c.attend
(trnrt/kernels/dsa_slots_c.py:416-447) against oracle slots_compact_ref (bf16-exact operands, fp32 sums: output within
2e-2, lse within 1e-3) and against the uncompacted row form (dsa_decode.attend) on rows with a visible token.
Cases: masks with no ones, fewer and more ones than keep, widths that are not a multiple of the 8-entry thread
chunk, the 262,144-pool width of a 1M context; slot lists of 640 slots at kpool 1 and 4 with sparse, dense, empty and
single-token rows."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, say
from trnrt_amd.kernels import dsa_decode, dsa_slots_c
from trnrt_amd.models import dsa_long

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,M,keep,dens", [(4, 1, 1, 0.5), (16, 2048, 64, 0.01), (16, 2048, 64, 0.5),
                                           (8, 1001, 2048, 0.3), (8, 65536, 2048, 0.02), (3, 262144, 2048, 0.002),
                                           (2, 4096, 16, 1.0), (2, 4096, 16, 0.0)])
def test_compact_matches_oracle(N, M, keep, dens):
    say(f"compact N={N} M={M} keep={keep} density={dens}")
    g = torch.Generator().manual_seed(N * 7 + M)
    sel = (torch.rand(N, M, generator=g) < dens).float()
    idx, cnt = dsa_long.compact(sel.cuda(), keep)
    torch.cuda.synchronize()
    ri, rc = O.compact_ref(sel, keep)
    assert torch.equal(cnt.cpu(), rc)
    assert torch.equal(idx.cpu(), ri)


def _slot_inputs(B, H, NS, kp, seed):
    g = torch.Generator().manual_seed(seed)
    pools = 2048
    kv = (torch.randn(pools * kp, 576, generator=g) * 0.4).to(torch.float8_e4m3fn)
    ks = torch.rand(pools * kp, generator=g) * 0.5 + 0.75
    q = (torch.randn(B, H, 576, generator=g) * 0.5).to(torch.bfloat16)
    rows = torch.randint(0, pools, (B, NS), generator=g)
    bias = torch.full((B, NS, kp), O.NEG_INF)
    # row 0: 64 live pools (every token) + a partial tail pool; row 1: dense; row 2: empty; row 3: one token;
    # the rest: random visibility
    bias[0, torch.randperm(NS, generator=g)[:64]] = 0.0
    bias[0, NS - 1, : max(kp - 1, 1)] = 0.0
    bias[1] = 0.0
    bias[3, 5, 0] = 0.0
    for b in range(4, B):
        bias[b] = torch.where(torch.rand(NS, kp, generator=g) < 0.1, 0.0, O.NEG_INF)
    return q, kv, ks, rows, bias


@pytest.mark.parametrize("kp", [1, 4])
def test_slots_compact_attend(kp):
    say(f"slots_c attend kp={kp}")
    B, H, NS, scale = 6, 64, 640, 0.0417
    q, kv, ks, rows, bias = _slot_inputs(B, H, NS, kp, seed=20 + kp)
    b_arg = bias if kp > 1 else bias.reshape(B, NS)
    o, lse = dsa_slots_c.attend(q.cuda(), kv.cuda(), rows.cuda(), b_arg.cuda(), scale, lse=True, kc_scale=ks.cuda())
    torch.cuda.synchronize()
    ro, rl = O.slots_compact_ref(q.float(), kv, ks, rows, bias, scale)
    assert_attention_close(o.cpu(), ro)
    live = rl > -1e29
    torch.testing.assert_close(lse.cpu()[live], rl[live], atol=1e-3, rtol=1e-4)
    assert torch.all(lse.cpu()[~live] < -1e29)
    # the uncompacted row form on the rows with a visible token: the same tokens and scores
    uo, ul = dsa_decode.attend(q.cuda(), kv.cuda(), rows.cuda(), b_arg.cuda(), scale, kc_scale=ks.cuda(), lse=True)
    torch.cuda.synchronize()
    vis = (bias > O.NEG_INF / 2).reshape(B, -1).any(-1)
    assert_attention_close(o.cpu()[vis], uo.cpu()[vis])
    torch.testing.assert_close(lse.cpu()[vis], ul.cpu()[vis], atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("keep", [1, 100, 2048, 8000])
def test_value_order_with_ties(keep):
    """dsa_long_select.value_order (trnrt/kernels/dsa_long_select.py:74-84) against a host sort of the same entries
    by (score descending, pool ascending): scores drawn from 7 values so most compare equal, counts 0, keep and
    partial, values copied bit for bit (a -0.0 stays -0.0)."""
    from trnrt_amd.kernels import dsa_long_select as LS

    say(f"value order keep={keep}")
    N = 5
    g = torch.Generator().manual_seed(keep)
    pools = torch.stack([torch.sort(torch.randperm(4 * keep + 8, generator=g)[:keep]).values for _ in range(N)])
    vals = torch.tensor([-1.5, -0.0, 0.0, 0.25, 1.0, 3.0, -2.0])[torch.randint(0, 7, (N, keep), generator=g)]
    cnt = torch.tensor([keep, 0, keep // 2, max(keep - 1, 0), 1])[:N]
    live = torch.arange(keep).view(1, -1) < cnt.view(-1, 1)
    pools = torch.where(live, pools, 0)
    vals = torch.where(live, vals, O.NEG_INF)
    vp, vc, vv = LS.value_order(pools.cuda(), cnt.cuda(), vals.cuda())
    torch.cuda.synchronize()
    vp, vv = vp.cpu(), vv.cpu()
    for n in range(N):
        c = int(cnt[n])
        order = sorted(range(c), key=lambda k: (-float(vals[n, k]), int(pools[n, k])))
        assert vp[n, :c].tolist() == [int(pools[n, k]) for k in order]
        assert torch.equal(vv[n, :c].view(torch.int32), vals[n, order].view(torch.int32))
        assert torch.all(vp[n, c:] == 0) and torch.all(vv[n, c:] == O.NEG_INF)
    assert torch.equal(vc.cpu(), cnt)
