"""GPU parity of the pooled (kpool > 1) forms of the path against the oracle: the slots of selected pools with the
query's tail pool (trnrt_amd.models.dsa_long.slots -> dsa_pool_slots, after trnrt/models/dsa_long.py:189-215,
bit-exact), and sparse MLA over pool slots of kp tokens each (dsa_long.attend, after trnrt/kernels/dsa_decode.py:
26-37 with bias [N, S, kp]; 2e-2 abs/rel in bf16)."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, say
from trnrt_amd import workloads as W
from trnrt_amd.models import dsa_long

pytestmark = pytest.mark.gpu


def _selection(N, L, kp, keep, positions, seed):
    g = torch.Generator().manual_seed(seed)
    P = L // kp
    npool = torch.div(positions + 1, kp, rounding_mode="floor")
    sc = torch.randn(N, P, generator=g)
    sc = sc + torch.where(torch.arange(P).view(1, P) < npool.view(N, 1), 0.0, O.NEG_INF)
    pools, cnt = O.topk_ref(sc, keep)
    return pools, cnt, npool


@pytest.mark.parametrize("kp,ps", [(4, 64), (4, 8), (4, 4), (1, 64)])
@pytest.mark.parametrize("shared", [True, False])
def test_slots_bit_exact(kp, ps, shared):
    say(f"pool slots kp={kp} ps={ps} shared={shared}")
    L = 2048
    positions = torch.tensor([0, 3, 4, 5, 100, 1023, 2046, 2047, 777])
    N = positions.shape[0]
    keep = 64 if kp == 4 else 256
    pools, cnt, npool = _selection(N, L, kp, keep, positions, seed=kp * 10 + ps)
    pages = L // ps
    g = torch.Generator().manual_seed(ps)
    table = torch.randperm(4 * pages, generator=g)[:pages].to(torch.int32) + 1
    tb = table if shared else torch.stack([table.roll(i) for i in range(N)])
    rows, bias = dsa_long.slots(pools.cuda(), cnt.cuda(), npool.cuda(), positions.cuda(), tb.cuda(), ps, kp, keep + 5)
    torch.cuda.synchronize()
    want_r, want_b = O.pool_slots_ref(pools, cnt, npool, positions, tb, ps, kp, keep + 5)
    assert torch.equal(rows.cpu(), want_r)
    assert torch.equal(bias.cpu(), want_b)


def test_pooled_attention_vs_oracle():
    """Absorbed MLA over 64 selected pools of 4 tokens plus the tail pool, through a paged FP8 cache."""
    say("pooled attention kp=4")
    cfg = W.Config("pooled", B=6, L=1024, H=32, Hi=16)
    inp = W.make_inputs(cfg, seed=4, lengths=[1024] * 6)
    kp, keep, ps = 4, 64, cfg.page_size
    positions = torch.tensor([1023, 1000, 514, 13, 4, 3])
    pools, cnt, npool = _selection(cfg.B, 1024, kp, keep, positions, seed=5)
    rows, bias = dsa_long.slots(pools.cuda(), cnt.cuda(), npool.cuda(), positions.cuda(), inp.table.cuda(), ps, kp,
                                keep + 1)
    o = dsa_long.attend(inp.q.cuda(), inp.kv_cache.cuda(), rows, bias, cfg.scale, kc_scale=inp.kv_scale.cuda())
    torch.cuda.synchronize()
    tok = (rows.cpu().unsqueeze(-1) * kp + torch.arange(kp)).reshape(cfg.B, -1)
    ref, _ = O.sparse_mla_slots_ref(inp.q, inp.kv_cache, inp.kv_scale, tok, bias.cpu().reshape(cfg.B, -1), cfg.scale)
    assert_attention_close(o, ref)
