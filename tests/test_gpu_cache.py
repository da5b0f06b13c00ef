"""GPU parity of the cache-store step (trnrt_amd.kernels.dsa_cache.store -> dsa_cache_write) against the oracle
(oracle/dsa_oracle.py cache_write_ref, after trnrt/models/decoder.py:481-486 `_store`): every byte of the cache and
every scale bit-exact, on the same seeded rows, for both cache widths (576 latent, 128 indexer key), bf16 and fp32
rows, the per-token and the reference's unscaled forms, edge rows (zeros, one huge value, tiny values, negative
zeros), slots outside the cache (skipped) and a whole config-2 cache."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests._helpers import say
from trnrt_amd import workloads as W
from trnrt_amd.kernels import dsa_cache

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn


def _rows(T, width, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, width, generator=g) * torch.exp(torch.randn(T, 1, generator=g) * 6)
    x[0] = 0.0  # absmax 0: the 1e-30 floor
    x[1] = 0.0
    x[1, 3] = 3e38  # one huge value
    x[2] = torch.randn(width, generator=g) * 1e-36  # tiny values: a tiny scale, normal quotients
    x[3] = -0.0
    x[4, ::2] = -0.0
    return x.to(dtype)


def _check(T, width, dtype, per_token, fp8_max=448.0, seed=0, num_slots=None):
    num_slots = num_slots or 2 * T + 5
    g = torch.Generator().manual_seed(seed + 1)
    x = _rows(T, width, seed, dtype)
    slots = torch.randperm(num_slots, generator=g)[:T].long()
    slots[5] = -1  # outside: skipped
    slots[6] = num_slots
    cache = torch.randint(0, 256, (num_slots, width), generator=g, dtype=torch.uint8)
    scale = torch.rand(num_slots, generator=g) if per_token else None
    want_c, want_s = O.cache_write_ref(cache, scale, slots, x, fp8_max, per_token)
    gc, gs = cache.cuda(), None if scale is None else scale.cuda()
    dsa_cache.store(gc, slots.cuda(), x.cuda(), fp8_max, scale=gs)
    torch.cuda.synchronize()
    diff = (gc.cpu() != want_c).any(-1).nonzero().flatten().tolist()
    assert not diff, f"rows differ at cache slots {diff[:8]}"
    if per_token:
        assert torch.equal(gs.cpu(), want_s)


@pytest.mark.parametrize("width", [576, 128, 8, 1024])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_per_token_scaled_rows_bit_exact(width, dtype):
    say(f"cache write per-token width={width} dtype={dtype}")
    _check(300, width, dtype, per_token=True, seed=width)


@pytest.mark.parametrize("fp8_max", [448.0, 240.0])
def test_reference_form_clamp_and_cast(fp8_max):
    say(f"cache write unscaled fp8_max={fp8_max}")
    _check(300, 576, torch.bfloat16, per_token=False, fp8_max=fp8_max, seed=3)
    _check(300, 128, torch.float32, per_token=False, fp8_max=fp8_max, seed=4)


def test_whole_config2_caches():
    """A whole config-2 cache of each width (262,144 + 64 rows of 576 and of 128) against the oracle on the host,
    whose IEEE fp32 division and cast are the reference's arithmetic."""
    say("cache write config 2 caches")
    cfg = W.CONFIGS[2]
    g = torch.Generator().manual_seed(11)
    n = cfg.B * cfg.L + cfg.page_size
    for width in (cfg.dqk, cfg.D):
        x = torch.randn(n, width, generator=g)
        want_q, want_s = W.quantize_rows(x)
        cache = torch.empty(n, width, dtype=FP8, device="cuda")
        scale = torch.empty(n, device="cuda")
        dsa_cache.store(cache, torch.arange(n, device="cuda"), x.cuda(), scale=scale)
        torch.cuda.synchronize()
        assert torch.equal(cache.cpu().view(torch.uint8), want_q.view(torch.uint8))
        assert torch.equal(scale.cpu(), want_s)


def test_slots_through_a_page_table():
    """The decode step's store: one new token per row at position ctx_len, its slot through the row's table."""
    say("cache write through page tables")
    cfg = W.Config("t", B=4, L=300, H=16, Hi=16)
    inp = W.make_inputs(cfg, seed=2, lengths=[300, 64, 1, 129])
    pos = torch.tensor([299, 63, 0, 128])
    slots = dsa_cache.slots_of(pos.cuda(), inp.table.cuda(), cfg.page_size)
    want = O.token_slots(inp.table[0], pos[:1], cfg.page_size)
    assert int(slots[0]) == int(want[0])
    x = torch.randn(4, cfg.dqk).to(torch.bfloat16)
    cache, scale = inp.kv_cache.clone(), inp.kv_scale.clone()
    want_c, want_s = O.cache_write_ref(cache, scale, slots.cpu(), x)
    gc, gs = cache.cuda(), scale.cuda()
    dsa_cache.store(gc, slots, x.cuda(), scale=gs)
    torch.cuda.synchronize()
    assert torch.equal(gc.cpu().view(torch.uint8), want_c.view(torch.uint8))
    assert torch.equal(gs.cpu(), want_s)


def test_argument_checks():
    cache = torch.zeros(8, 576, dtype=FP8, device="cuda")
    x = torch.zeros(2, 576, device="cuda")
    with pytest.raises(ValueError):
        dsa_cache.store(cache, torch.arange(2, device="cuda"), torch.zeros(2, 512, device="cuda"))
    with pytest.raises(NotImplementedError):
        dsa_cache.store(torch.zeros(8, 576, device="cuda"), torch.arange(2, device="cuda"), x)
    with pytest.raises(NotImplementedError):
        dsa_cache.store(torch.zeros(8, 20, dtype=FP8, device="cuda"), torch.arange(2, device="cuda"),
                        torch.zeros(2, 20, device="cuda"))
    with pytest.raises(ValueError):
        dsa_cache.store(cache, torch.arange(2, device="cuda"), x, fp8_max=500.0)
