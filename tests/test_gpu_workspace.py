"""One decode workspace (or the allocation-free entry point's scratch) reused across batch sizes and across the two
forms of the layer: a one-launch call whose rows leave counts in the status words (a crowded row takes the
two-exchange selection), then a larger batch through the separate kernels (a row past 32,768 tokens), whose top-k
reads the row histograms that follow the barrier and status words. Every stage of both calls against the oracle
(scores within 1e-2 row-relative of indexer_ref, indices and counts bit-exact against topk_ref over the kernel's own
scores, the bf16 output within 2e-2 and lse within 1e-3 of the oracle attention). Also: a barrier give-up counted in
the status words is reported by dsa_layer_status and raised by the Python layer (set from the host: no kernel is made
to wait), and cleared."""

from types import SimpleNamespace

import pytest
import torch

from tests._helpers import say
from tests.test_gpu_fused import SYNC_WORDS, XCD_WORDS, _check_full, sync_block
from trnrt_amd import _lib
from trnrt_amd import workloads as W
from trnrt_amd.kernels.dsa_layer import DecodeLayer

pytestmark = pytest.mark.gpu


def _crowded_inputs():
    """4 rows; row 0's largest scores crowd into its first 2,048 positions (their key scales raised a thousandfold),
    more than two workgroups' key lists hold, so the one-launch layer selects it in the two-exchange form."""
    cfg = W.Config("ws-crowded", B=4, L=32768, H=64, Hi=64)
    inp = W.make_inputs(cfg, seed=21, lengths=[32768, 30000, 9000, 32768])
    ps = cfg.page_size
    pos = torch.arange(2048)
    slots = inp.table[0, pos // ps].long() * ps + pos % ps
    inp.k_scale[slots] *= 1000.0
    return inp


def _long_inputs():
    """8 rows, one past 32,768 tokens (the separate kernels), row 4 four tokens shorter than keep: in a layout whose
    status words followed the histograms of a 4-row call, that row's histogram would start with them."""
    cfg = W.Config("ws-long", B=8, L=40000, H=64, Hi=64)
    return W.make_inputs(cfg, seed=22, lengths=[40000, 32768, 9000, 300, 2044, 31000, 12000, 5000])


def _layer(inp, g, ws=None):
    cfg = inp.cfg
    L = DecodeLayer(cfg.B, cfg.Hi, cfg.H, g.max_pages, cfg.page_size, g.num_pages, cfg.keep, cfg.scale,
                    max_len=max(inp.lengths))
    if ws is not None:
        assert ws.numel() >= L.workspace.numel()
        L.workspace = ws
    return L


def test_workspace_reused_from_one_launch_to_separate_kernels():
    a, b = _crowded_inputs(), _long_inputs()
    ga, gb = a.to("cuda"), b.to("cuda")
    Lb = _layer(b, gb)
    La = _layer(a, ga, ws=Lb.workspace)  # the larger call's workspace, used by the smaller call first
    say("workspace reuse: B=4 one launch (a crowded row), then B=8 separate kernels (a 40,000-token row)")
    La.step(ga.q_idx, ga.w_k, ga.k_cache, ga.k_scale, ga.q, ga.kv_cache, ga.kv_scale, ga.table, ga.ctx_len)
    torch.cuda.synchronize()
    assert La.status() == {"gave_up": 0, "two_exchange": 1}
    _check_full(a, La)
    Lb.step(gb.q_idx, gb.w_k, gb.k_cache, gb.k_scale, gb.q, gb.kv_cache, gb.kv_scale, gb.table, gb.ctx_len,
            verify=True)
    torch.cuda.synchronize()
    assert int(Lb.cnt[4]) == 2044
    _check_full(b, Lb)
    ws = Lb.workspace.view(torch.int32).cpu()
    ctr, sync = sync_block(ws)
    assert torch.all(ctr % 256 == 0) and torch.all(sync[:, 1] == 0)
    assert torch.all(ws[SYNC_WORDS:SYNC_WORDS + 8 * 4096] == 0), "row histograms left non-zero"
    assert Lb.status(clear=True) == {"gave_up": 0, "two_exchange": 1}
    assert Lb.status() == {"gave_up": 0, "two_exchange": 0}


def _noalloc(g, inp):
    cfg = inp.cfg
    stride = g.max_pages * cfg.page_size
    dev = g.q.device
    r = SimpleNamespace(
        scores=torch.empty(cfg.B, stride, dtype=torch.float32, device=dev),
        idx=torch.empty(cfg.B, cfg.keep, dtype=torch.int32, device=dev),
        cnt=torch.empty(cfg.B, dtype=torch.int32, device=dev),
        out=torch.empty(cfg.B, cfg.H, 512, dtype=torch.bfloat16, device=dev),
        lse=torch.empty(cfg.B, cfg.H, dtype=torch.float32, device=dev))
    st = _lib.lib().dsa_decode_layer_noalloc(
        g.q_idx.data_ptr(), g.w_k.data_ptr(), g.k_cache.data_ptr(), g.k_scale.data_ptr(), g.q.data_ptr(),
        g.kv_cache.data_ptr(), g.kv_scale.data_ptr(), g.table.data_ptr(), g.ctx_len.data_ptr(), r.scores.data_ptr(),
        r.idx.data_ptr(), r.cnt.data_ptr(), r.out.data_ptr(), r.lse.data_ptr(), cfg.B, cfg.Hi, cfg.H, g.max_pages,
        cfg.page_size, g.num_pages, stride, max(inp.lengths), cfg.keep, cfg.scale, 0,
        torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "dsa_decode_layer_noalloc")
    torch.cuda.synchronize()
    return r


def test_noalloc_scratch_reused_from_one_launch_to_separate_kernels():
    a, b = _crowded_inputs(), _long_inputs()
    ga, gb = a.to("cuda"), b.to("cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.layer_status(None, stream, clear=True)
    say("noalloc reuse: B=4 one launch (a crowded row), then B=8 separate kernels (a 40,000-token row)")
    ra = _noalloc(ga, a)
    assert _lib.layer_status(None, stream) == (0, 1)
    _check_full(a, ra)
    rb = _noalloc(gb, b)
    assert int(rb.cnt[4]) == 2044
    _check_full(b, rb)
    assert _lib.layer_status(None, stream, clear=True) == (0, 1)


def test_gave_up_count_is_reported_and_cleared():
    """A give-up count written into XCD 3's status word from the host (the kernels are not made to wait): the
    next verified step raises RuntimeError and clears it; the step after is clean, and its outputs are the same."""
    cfg = W.CONFIGS[1]
    inp = W.make_inputs(cfg, seed=23)
    g = inp.to("cuda")
    L = _layer(inp, g)
    say("status: a give-up set from the host")
    L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len, verify=True)
    out0 = L.out.clone()
    L.workspace.view(torch.int32)[3 * XCD_WORDS + 2] = 5
    assert L.status()["gave_up"] == 5
    with pytest.raises(RuntimeError, match="gave up"):
        L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len, verify=True)
    assert L.status()["gave_up"] == 0
    L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len, verify=True)
    assert torch.equal(L.out, out0)
    _check_full(inp, L)
