"""The attention surfaces called exactly as the reference's callers call them, on the reference's unscaled FP8 latent
cache (trnrt/models/decoder.py:481-486 stores kv clamped and cast, no scale): dsa_decode.attend(q_lat, kc, rows,
bias, scale) (trnrt/models/mla.py:526), dsa_slots_n.attend(q_lat, kc, rows, bias, scale, n) (trnrt/models/mla.py:1208,
1215, n a one-element int tensor), dsa_slots_c.attend(q_lat, kc, rows, bias, scale) (trnrt/models/mla.py:852) and
dsa_long.attend(q_lat, kc, rows, bias, scale) (trnrt/models/dsa_long.py:218-223) -- positional arguments only, no
kc_scale. Each against the oracle with unit scales (output within 2e-2 abs/rel, lse within 1e-3). Also
dsa_slots_n.attend's live-row count: the first n rows against the oracle, the rest untouched (an `out` prefilled with
a sentinel keeps it; a fresh output reads zero there, the reference's host form), n = 0, n = N and n past N."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import assert_attention_close, say
from trnrt_amd.kernels import dsa_decode, dsa_slots_c, dsa_slots_n
from trnrt_amd.models import dsa_long

pytestmark = pytest.mark.gpu


def _unscaled(N, H, NS, kp, R, seed):
    """q_lat bf16 [N, H, R], kc e4m3fn [pools kp, 1, R] (values clamped and cast, the reference's cache), rows [N, NS]
    pool rows, bias [N, NS, kp] 0 / NEG_INF with a few masked tokens and a fully masked row."""
    g = torch.Generator().manual_seed(seed)
    pools = 1024
    kc = (torch.randn(pools * kp, 1, R, generator=g) * 2.0).clamp(-448, 448).to(torch.float8_e4m3fn)
    q = (torch.randn(N, H, R, generator=g) * 0.5).to(torch.bfloat16)
    rows = torch.randint(0, pools, (N, NS), generator=g)
    bias = torch.where(torch.rand(N, NS, kp, generator=g) < 0.85, 0.0, O.NEG_INF)
    bias[2] = O.NEG_INF  # a row with every token masked: the uniform mean, lse NEG_INF
    return q, kc, rows, bias


def _oracle(q, kc, rows, bias, scale):
    N, NS = rows.shape
    kp = bias.shape[-1]
    tok = (rows.long().unsqueeze(-1) * kp + torch.arange(kp)).reshape(N, NS * kp)
    kv = kc.reshape(kc.shape[0], -1)
    return O.sparse_mla_slots_ref(q.float(), kv, torch.ones(kv.shape[0]), tok, bias.reshape(N, -1), scale)


def _close(o, lse, ro, rl):
    assert_attention_close(o.cpu(), ro)
    live = rl > -1e29
    torch.testing.assert_close(lse.cpu()[live], rl[live], atol=1e-3, rtol=1e-4)
    assert torch.all(lse.cpu()[~live] < -1e29)


@pytest.mark.parametrize("kp,R", [(4, 512), (1, 576)])
def test_reference_calls_on_an_unscaled_cache(kp, R):
    say(f"reference calls, unscaled cache kp={kp} R={R}")
    N, H, NS, scale = 5, 64, 160, 0.0417
    q, kc, rows, bias = _unscaled(N, H, NS, kp, R, seed=30 + kp)
    ro, rl = _oracle(q, kc, rows, bias, scale)
    qd, kd, rd, bd = q.cuda(), kc.cuda(), rows.cuda(), bias.cuda()
    n = torch.tensor([N], dtype=torch.int32, device="cuda")

    o = dsa_decode.attend(qd, kd, rd, bd, scale)
    torch.cuda.synchronize()
    assert_attention_close(o.cpu(), ro)
    o, lse = dsa_decode.attend(qd, kd, rd, bd, scale, lse=True)
    torch.cuda.synchronize()
    _close(o, lse, ro, rl)

    o = dsa_long.attend(qd, kd, rd, bd, scale)
    torch.cuda.synchronize()
    assert_attention_close(o.cpu(), ro)

    o = dsa_slots_n.attend(qd, kd, rd, bd, scale, n)
    torch.cuda.synchronize()
    assert_attention_close(o.cpu(), ro)
    o, lse = dsa_slots_n.attend(qd, kd, rd, bd, scale, n, True)
    torch.cuda.synchronize()
    _close(o, lse, ro, rl)

    # the compacted form: a fully masked row attends pool row 0's tokens (the reference's compacted fill), the
    # others their visible tokens, as the uncompacted form
    o, lse = dsa_slots_c.attend(qd, kd, rd, bd, scale, True)
    torch.cuda.synchronize()
    vis = (bias > O.NEG_INF / 2).reshape(N, -1).any(-1)
    assert_attention_close(o.cpu()[vis], ro[vis])
    torch.testing.assert_close(lse.cpu()[vis], rl[vis], atol=1e-3, rtol=1e-4)
    rc, _ = O.slots_compact_ref(q.float(), kc.reshape(kc.shape[0], -1), torch.ones(kc.shape[0]), rows, bias, scale)
    assert_attention_close(o.cpu(), rc)


@pytest.mark.parametrize("n_live", [0, 3, 7, 9])
def test_slots_n_live_rows(n_live):
    """N = 7 rows: the first n against the oracle; the others keep a sentinel in a caller's out (n = 9: every row)."""
    say(f"slots_n live rows n={n_live}")
    N, H, NS, kp, scale = 7, 32, 96, 4, 0.05
    q, kc, rows, bias = _unscaled(N, H, NS, kp, 512, seed=40)
    ro, rl = _oracle(q, kc, rows, bias, scale)
    n = torch.tensor([n_live], dtype=torch.int32, device="cuda")
    out = torch.full((N, H, 512), 7.5, dtype=torch.float32, device="cuda")
    o, lse = dsa_slots_n.attend(q.cuda(), kc.cuda(), rows.cuda(), bias.cuda(), scale, n, True, out=out)
    torch.cuda.synchronize()
    assert o is out
    k = min(n_live, N)
    if k:
        _close(o[:k], lse[:k], ro[:k], rl[:k])
    assert torch.all(o[k:].cpu() == 7.5), "rows past n were written"
    assert torch.all(lse[k:].cpu() == 0.0)
    # a fresh output: zeros past n (the reference's host form)
    o2 = dsa_slots_n.attend(q.cuda(), kc.cuda(), rows.cuda(), bias.cuda(), scale, n_live)
    torch.cuda.synchronize()
    assert torch.all(o2[k:].cpu() == 0.0)
    if k:
        assert torch.equal(o2[:k], o[:k])
