"""The decode layer steps captured in a HIP graph (torch.cuda.CUDAGraph): the step allocates nothing and clears
nothing with a memset (the top-k histograms are left at zero by the kernels themselves), so a captured step replays
the same launches. Each replay is checked against an eager step on the same inputs, with eager work and
synchronisations between the replays, and after the inputs change in place."""

import pytest
import torch

from tests._helpers import say
from trnrt_amd import workloads as W
from trnrt_amd.kernels import dsa_cache
from trnrt_amd.kernels.dsa_layer import DecodeLayer, PooledDecodeLayer

pytestmark = pytest.mark.gpu


def _capture(step):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    return g


def _replays_match(g, step, outs, change):
    """Replays against eager steps: three replays with eager work between, then one after change() edits the
    inputs in place."""
    step()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    for r in range(3):
        for o in outs:
            o.fill_(7)  # eager work on the same buffers between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o, w), f"replay {r}"
    change()
    step()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    for o in outs:
        o.fill_(7)
    g.replay()
    torch.cuda.synchronize()
    for o, w in zip(outs, want):
        assert torch.equal(o, w), "replay after the inputs changed"


def test_decode_layer_graph_replay():
    cfg = W.Config("graph", B=3, L=8192, H=64, Hi=64)
    say("decode layer graph replay")
    g = W.make_inputs(cfg, seed=9, lengths=[8192, 5000, 300], device="cuda")
    L = DecodeLayer(cfg.B, cfg.Hi, cfg.H, g.max_pages, cfg.page_size, g.num_pages, cfg.keep, cfg.scale)
    args = (g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len)

    def step():
        L.step(*args, check=False)

    gr = _capture(step)

    def change():
        g.q.mul_(-1)
        g.q_idx.mul_(0.5)

    _replays_match(gr, step, [L.scores, L.idx, L.cnt, L.out, L.lse], change)


def test_pooled_layer_graph_replay():
    cfg = W.PooledConfig("graph-pooled", B=3, L=4096)
    say("pooled layer graph replay")
    inp = W.make_pooled_inputs(cfg, seed=10, device="cuda")
    ps, kp = cfg.page_size, cfg.kp
    pos = torch.tensor([4095, 3001, 6], dtype=torch.int32, device="cuda")
    slot_mapping = dsa_cache.slots_of(pos, inp.table, ps)
    npool = torch.div(pos + 1, kp, rounding_mode="floor").to(torch.int32)
    layer = PooledDecodeLayer(cfg.B, cfg.Hi, cfg.H, cfg.dqk, inp.table.shape[1], ps, inp.pool_key.shape[0] // ps, kp,
                              cfg.keep, cfg.scale)

    def step():
        dsa_cache.write_pool_keys(inp.pool_key, inp.rows, pos, inp.table, slot_mapping, inp.ape, ps, kp,
                                  rows_scale=inp.rows_scale)
        layer.step(inp.q_idx, inp.w, inp.pool_key, inp.q, inp.kv_cache, inp.kv_scale, inp.table, npool, pos,
                   check=False)

    gr = _capture(step)

    def change():
        inp.q.mul_(-1)
        inp.w.mul_(2)

    _replays_match(gr, step, [layer.scores, layer.pools, layer.cnt, layer.out, layer.lse], change)
