"""The Python operator surface on the CPU host: there is no CPU path (host tensors raise instead of falling back),
and shape errors raise the reference's exception kinds before any GPU work."""

import pytest
import torch

from trnrt_amd.kernels import dsa_decode, dsa_index, dsa_topk
from trnrt_amd.models import dsa_long


def test_page_groups_layout():
    """ppg[p, b, g] is page p NG + g of row b; not a multiple of 128 pages -> ValueError
    (trnrt/kernels/dsa_index.py:234-240)."""
    table = torch.arange(2 * 256, dtype=torch.int32).view(2, 256)
    ppg = dsa_index.page_groups(table)
    assert ppg.shape == (128, 2, 2) and ppg.dtype == torch.int32
    assert torch.equal(ppg[5, 1], table[1, 10:12])
    assert torch.equal(dsa_index._table(ppg, 2), table)
    with pytest.raises(ValueError, match="multiple of 128"):
        dsa_index.page_groups(table[:, :200])


def test_host_tensors_raise():
    s = torch.randn(2, 100)
    with pytest.raises(RuntimeError, match="GPU only"):
        dsa_topk.select_indices(s, 10)
    with pytest.raises(RuntimeError, match="GPU only"):
        dsa_long.select_device(s, 10)
    with pytest.raises(RuntimeError, match="GPU only"):
        dsa_index.decode_scores(torch.zeros(1, 4, 128, dtype=torch.bfloat16), torch.zeros(1, 4),
                                torch.zeros(64, 128, dtype=torch.uint8), torch.ones(64),
                                torch.zeros(1, 1, dtype=torch.int32), None, 64)
    with pytest.raises(RuntimeError, match="GPU only"):
        dsa_decode.attend(torch.zeros(1, 16, 576), torch.zeros(64, 576, dtype=torch.uint8),
                          torch.zeros(1, 8, dtype=torch.int32), torch.zeros(1, 8), 0.1, kc_scale=torch.ones(64))


def test_pooled_forms_host_checks():
    with pytest.raises(ValueError):
        dsa_topk.select(torch.randn(2, 64), 8, vis_only=False, kp=4, tail=True)  # tail needs vis_only
    with pytest.raises(RuntimeError, match="GPU only"):
        dsa_topk.select(torch.randn(2, 64), 8, kp=4)
    with pytest.raises(ValueError):
        dsa_long.npools(torch.tensor([3]), 3)
    assert torch.equal(dsa_long.npools(torch.tensor([0, 5, 7]), 4), torch.tensor([0, 1, 2]))
    assert torch.equal(dsa_long.npools(torch.tensor([0, 5]), 1), torch.tensor([1, 6]))
