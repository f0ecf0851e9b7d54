"""Host logic of ``linatt_amd.delta_rule`` that runs without a GPU."""

import pytest
import torch


def test_varlen_layout():
    """The packed -> padded-batch index map behind ``cu_seqlens`` and its
    refusals (host logic of ``linatt_amd.delta_rule``)."""
    from linatt_amd.delta_rule import _seq_layout
    dst, N, Tmax = _seq_layout(torch.tensor([0, 3, 3, 4, 9]), 9, "cpu")
    assert (N, Tmax) == (4, 5)
    # sequence n occupies row n of a (N, Tmax) batch, from column 0
    assert dst.tolist() == [0, 1, 2, 10, 15, 16, 17, 18, 19]
    for bad in ([1, 9], [0, 8], [0, 5, 3, 9], [0], [0, 0]):
        T = 9 if bad != [0, 0] else 0
        with pytest.raises(ValueError):
            _seq_layout(torch.tensor(bad), T, "cpu")
