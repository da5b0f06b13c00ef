"""Pins the oracle's cache-store step (oracle/dsa_oracle.py cache_write_ref, after trnrt/models/decoder.py:481-486
`_store`): torch's float -> float8_e4m3fn cast, which the oracle uses, against a round-to-nearest-even encoder
written from the OCP e4m3fn definition (oracle e4m3fn_encode) over every representable value, every midpoint and
the neighbours of each; known-answer rows; the per-token round-trip bound; and planted mistakes (no clamp,
truncation instead of rounding) that must fail."""

import math

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

FP8 = torch.float8_e4m3fn


def _finite_values():
    """Every non-negative finite e4m3fn value, ascending."""
    codes = torch.arange(0x7F, dtype=torch.uint8)
    return codes.view(FP8).float().tolist()


def _probe_values():
    """Each representable value, each midpoint between neighbours, and the fp32 neighbours of every midpoint, both
    signs, plus the subnormal range below the smallest step."""
    vals = _finite_values()
    out = []
    for a, b in zip(vals, vals[1:]):
        mid = (a + b) / 2  # exact in fp32 (e4m3 values have 4 significant bits)
        out += [a, mid, float(np.nextafter(np.float32(mid), np.float32(0))),
                float(np.nextafter(np.float32(mid), np.float32(1e9)))]
    out += [vals[-1], 2.0 ** -12, 2.0 ** -11, 3 * 2.0 ** -11, 1e-30, 0.0]
    return out + [-v for v in out]


def test_torch_cast_is_round_to_nearest_even_e4m3fn():
    probe = _probe_values()
    got = torch.tensor(probe, dtype=torch.float32).to(FP8).view(torch.uint8).tolist()
    want = [O.e4m3fn_encode(v) for v in probe]
    bad = [(v, g, w) for v, g, w in zip(probe, got, want) if g != w]
    assert not bad, bad[:5]


def test_encoder_known_codes():
    assert O.e4m3fn_encode(448.0) == 0x7E
    assert O.e4m3fn_encode(1.0) == 0x38
    assert O.e4m3fn_encode(-0.0) == 0x80
    assert O.e4m3fn_encode(2.0 ** -9) == 0x01  # the smallest subnormal
    assert O.e4m3fn_encode(2.0 ** -10) == 0x00  # a tie between 0 and 2^-9: the even code 0
    assert O.e4m3fn_encode(432.0) == 0x7E  # the tie between 416 (code 0x7D) and 448 (0x7E): even


def test_known_answer_rows():
    # absmax 2 -> s = 2 / 448; x / s = [224, -448, 112, 0, 32, 56, -112, 1] -> all e4m3fn values
    x = torch.tensor([[1.0, -2.0, 0.5, 0.0, 1 / 7, 0.25, -0.5, 1 / 224]])
    cache = torch.zeros(4, 8, dtype=torch.uint8)
    scale = torch.zeros(4)
    c, s = O.cache_write_ref(cache, scale, torch.tensor([2]), x)
    assert s[2] == torch.tensor(2.0 / 448.0) and s[0] == 0 and s[3] == 0
    want = [O.e4m3fn_encode(v) for v in (224.0, -448.0, 112.0, 0.0, 32.0, 56.0, -112.0, 1.0)]
    assert c[2].tolist() == want
    assert c[0].tolist() == [0] * 8 and c[3].tolist() == [0] * 8
    # the reference's form: clamp to +-fp8_max, cast, scale 1
    x2 = torch.tensor([[500.0, -500.0, 1.0, 0.5, 240.0, 250.0, -0.0, 3.0]])
    c2, s2 = O.cache_write_ref(cache, scale, torch.tensor([1]), x2, fp8_max=240.0, per_token=False)
    assert c2[1].tolist() == [O.e4m3fn_encode(v) for v in (240.0, -240.0, 1.0, 0.5, 240.0, 240.0, -0.0, 3.0)]
    assert s2[1] == 1.0


def test_out_of_range_slots_are_skipped():
    cache = torch.full((3, 8), 7, dtype=torch.uint8)
    c, s = O.cache_write_ref(cache, None, torch.tensor([-1, 3, 1]), torch.ones(3, 8))
    assert s is None
    assert c[0].tolist() == [7] * 8 and c[2].tolist() == [7] * 8
    assert c[1].tolist() == [O.e4m3fn_encode(448.0)] * 8


def test_per_token_round_trip_bound():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 576, generator=g) * torch.exp(torch.randn(64, 1, generator=g) * 4)
    cache = torch.zeros(64, 576, dtype=torch.uint8)
    c, s = O.cache_write_ref(cache, torch.zeros(64), torch.arange(64), x)
    back = c.view(FP8).float() * s.view(-1, 1)
    # |x - back| <= half an e4m3 step: 2^-4 relative for normals, 2^-10 s absolute for subnormals
    bound = torch.maximum(x.abs() * 2.0 ** -4, s.view(-1, 1) * 2.0 ** -10)
    assert torch.all((x - back).abs() <= bound * (1 + 1e-6))
    assert torch.all(back.abs().amax(-1) == s * 448.0)  # the row's absmax maps to 448 exactly or by one rounding


def _planted(kind, x, fp8_max):
    xf = x.float()
    if kind == "no_clamp":
        return xf.to(FP8).view(torch.uint8)
    if kind == "truncate":  # round toward zero: the largest code whose value does not exceed |v|
        vals = torch.tensor(_finite_values())
        a = xf.clamp(-fp8_max, fp8_max).abs()
        idx = torch.searchsorted(vals, a, right=True) - 1
        return (idx.to(torch.uint8) | torch.where(xf < 0, 0x80, 0).to(torch.uint8))
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["no_clamp", "truncate"])
def test_planted_mistakes_fail(kind):
    x = torch.tensor([[500.0, 1.0625, 3.3, -7.7, 0.3, 100.0, -448.5, 0.01]])
    cache = torch.zeros(1, 8, dtype=torch.uint8)
    c, _ = O.cache_write_ref(cache, None, torch.tensor([0]), x, fp8_max=448.0, per_token=False)
    assert not torch.equal(_planted(kind, x, 448.0)[0], c[0]), kind
    assert math.isnan(torch.tensor([500.0]).to(FP8).float().item())  # why the clamp exists
