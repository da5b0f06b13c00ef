"""The allocation-free decode layer entry point (dsa_decode_layer_noalloc: no workspace argument, the library's own
static device scratch) against the workspace entry point (dsa_decode_layer) through the C ABI: calls in a row on
the same scratch, the second with a smaller input (fewer rows, shorter contexts, fewer heads) and a third with more
rows again (its zero region covers what the second call left past its own), each checked to the
parity bar against the workspace entry point's outputs on the same inputs (indices and counts bit-exact, scores within
1e-2 row-relative, the bf16 output within 2e-2 and lse within 1e-3), and a size beyond the scratch refused before
any GPU work."""

import pytest
import torch

from tests._helpers import assert_attention_close, row_rel_err, say
from trnrt_amd import _lib
from trnrt_amd import workloads as W
from trnrt_amd.kernels.dsa_layer import DecodeLayer

pytestmark = pytest.mark.gpu


def _noalloc_step(g, max_len):
    cfg = g.cfg
    stride = g.max_pages * cfg.page_size
    dev = g.q.device
    scores = torch.empty(cfg.B, stride, dtype=torch.float32, device=dev)
    idx = torch.empty(cfg.B, cfg.keep, dtype=torch.int32, device=dev)
    cnt = torch.empty(cfg.B, dtype=torch.int32, device=dev)
    out = torch.empty(cfg.B, cfg.H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(cfg.B, cfg.H, dtype=torch.float32, device=dev)
    st = _lib.lib().dsa_decode_layer_noalloc(
        g.q_idx.data_ptr(), g.w_k.data_ptr(), g.k_cache.data_ptr(), g.k_scale.data_ptr(), g.q.data_ptr(),
        g.kv_cache.data_ptr(), g.kv_scale.data_ptr(), g.table.data_ptr(), g.ctx_len.data_ptr(), scores.data_ptr(),
        idx.data_ptr(), cnt.data_ptr(), out.data_ptr(), lse.data_ptr(), cfg.B, cfg.Hi, cfg.H, g.max_pages,
        cfg.page_size, g.num_pages, stride, max_len, cfg.keep, cfg.scale, 0,
        torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "dsa_decode_layer_noalloc")
    return scores, idx, cnt, out, lse


def _compare(cfg, lengths, seed):
    say(f"noalloc layer B={cfg.B} H={cfg.H} lengths={lengths}")
    g = W.make_inputs(cfg, seed=seed, lengths=lengths).to("cuda")
    max_len = max(lengths)
    sc, idx, cnt, out, lse = _noalloc_step(g, max_len)
    L = DecodeLayer(cfg.B, cfg.Hi, cfg.H, g.max_pages, cfg.page_size, g.num_pages, cfg.keep, cfg.scale,
                    max_len=max_len)
    L.step(g.q_idx, g.w_k, g.k_cache, g.k_scale, g.q, g.kv_cache, g.kv_scale, g.table, g.ctx_len)
    torch.cuda.synchronize()
    ref = L.scores.cpu()
    live = ref > -1e29
    assert row_rel_err(sc.cpu(), ref, live) <= 1e-2
    assert torch.all(sc.cpu()[~live] == ref[~live])
    assert torch.equal(idx.cpu(), L.idx.cpu()) and torch.equal(cnt.cpu(), L.cnt.cpu())
    assert_attention_close(out, L.out)
    torch.testing.assert_close(lse.cpu(), L.lse.cpu(), atol=1e-3, rtol=1e-4)


def test_noalloc_layer_matches_workspace_layer_twice():
    # first call: 4 rows of up to 12,000 tokens, 64 + 64 heads; second: 2 shorter rows, 16 + 16 heads; third: 6 rows
    _compare(W.Config("noalloc-a", B=4, L=12000, H=64, Hi=64), [12000, 9000, 2048, 700], seed=11)
    _compare(W.Config("noalloc-b", B=2, L=4096, H=16, Hi=16), [4096, 1500], seed=12)
    _compare(W.Config("noalloc-c", B=6, L=8192, H=64, Hi=64), [8192, 5000, 300, 8000, 2049, 4096], seed=13)


def test_noalloc_layer_refuses_more_than_its_scratch():
    # 512 rows of 32,768 tokens need more workspace than the scratch holds: refused before any GPU work
    need = _lib.workspace_bytes(_lib.DSA_WS_LAYER, 512, 64, 2048, 32768)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    p = 16  # never dereferenced
    st = _lib.lib().dsa_decode_layer_noalloc(p, p, p, p, p, p, p, p, p, p, p, p, p, p, 512, 64, 64, 512, 64, 1 << 16,
                                             32768, 32768, 2048, 0.07, 0, None)
    assert st == _lib.DSA_ESCRATCH
    with pytest.raises(ValueError):
        _lib.check(st, "dsa_decode_layer_noalloc")
