"""Pins the oracle's pooled-indexer keys (oracle/dsa_oracle.py pool_keys_ref, after trnrt/models/glm5_next.py:151-160
`pool_keys`; write_pool_keys_ref, after trnrt/models/mla.py:1262-1296): a float64 loop over the softmax-gated mean,
the known answer of equal gates (the mean of the keys), the pieces' slot layout (a page's pool keys contiguous, in
pool order), and a planted mistake (the pool-position bias dropped) that must fail."""

import torch

from oracle import dsa_oracle as O


def _rows(T, kp, g):
    return (torch.randn(T, kp, 256, generator=g) * 2).to(torch.bfloat16)


def test_float64_loop():
    g = torch.Generator().manual_seed(0)
    kp = 4
    rows = _rows(5, kp, g)
    ape = torch.randn(kp, 128, generator=g)
    got = O.pool_keys_ref(rows, ape).float()
    r = rows.double()
    for n in range(5):
        for d in range(128):
            lg = [float(r[n, t, 128 + d]) + float(ape[t, d].float()) for t in range(kp)]
            m = max(lg)
            e = [torch.tensor(x - m, dtype=torch.float64).exp().item() for x in lg]
            want = sum(e[t] / sum(e) * float(r[n, t, d]) for t in range(kp))
            assert abs(float(got[n, d]) - want) <= 2 ** -7 * (abs(want) + sum(abs(float(r[n, t, d])) for t in range(kp)) / kp) + 1e-30


def test_equal_gates_give_the_mean():
    g = torch.Generator().manual_seed(1)
    rows = _rows(3, 4, g)
    rows[..., 128:] = 0.5  # equal gates: weights 1/4, exact in bf16
    got = O.pool_keys_ref(rows, torch.zeros(4, 128))
    want = (rows[..., :128].float().sum(-2) / 4).to(torch.bfloat16)
    assert torch.equal(got, want)


def test_piece_layout_and_planted_bias():
    g = torch.Generator().manual_seed(2)
    kp, ps, pages = 4, 16, 3
    slots = (pages + 1) * ps
    rows = (torch.randn(slots, 256, generator=g)).to(torch.bfloat16)
    ape = torch.randn(kp, 128, generator=g)
    table = torch.tensor([3, 1, 2], dtype=torch.int32)  # positions 0..47 of one sequence
    positions = torch.arange(48)
    slot_mapping = (table.long()[positions // ps] * ps + positions % ps)
    pk = O.write_pool_keys_ref(torch.zeros(slots, 128 // kp, dtype=torch.bfloat16), rows, None, positions, table,
                               slot_mapping, ape, ps, kp)
    # pool p of the sequence: its key is the kp pieces at its kp token slots, contiguous within the page
    by_page = pk.view(pages + 1, ps // kp, 128)
    for p in range(48 // kp):
        page, j = int(table[p * kp // ps]), (p * kp % ps) // kp
        toks = table.long()[(p * kp + torch.arange(kp)) // ps] * ps + (p * kp + torch.arange(kp)) % ps
        want = O.pool_keys_ref(rows[toks].view(1, kp, 256), ape)[0]
        assert torch.equal(by_page[page, j], want), p
    bad = O.write_pool_keys_ref(torch.zeros(slots, 128 // kp, dtype=torch.bfloat16), rows, None, positions, table,
                                slot_mapping, torch.zeros(kp, 128), ps, kp)
    assert not torch.equal(bad, pk)
