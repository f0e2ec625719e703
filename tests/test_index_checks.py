"""The pre-launch index checks of the Python layer (no GPU): the switch and the range rule."""

import pytest
import torch

from mini_infra_qwen3_amd import data_plane


def test_switch_returns_the_previous_setting():
    first = data_plane.set_index_checks(True)
    try:
        assert data_plane.set_index_checks(False) is True
        assert data_plane.set_index_checks(True) is False
    finally:
        data_plane.set_index_checks(first)


def test_range_rule():
    previous = data_plane.set_index_checks(True)
    try:
        data_plane._check_range("ids", torch.tensor([0, 3, 9]), 10)
        data_plane._check_range("slots", torch.tensor([-1, 159]), 160, allow_minus_one=True)
        data_plane._check_range("ids", torch.zeros((2, 0), dtype=torch.long), 10)
        with pytest.raises(IndexError, match="index 10"):
            data_plane._check_range("ids", torch.tensor([[1, 10]]), 10)
        with pytest.raises(IndexError, match="index -1"):
            data_plane._check_range("ids", torch.tensor([2, -1]), 10)
        with pytest.raises(IndexError, match="index -2"):
            data_plane._check_range("slots", torch.tensor([-2]), 160, allow_minus_one=True)
        data_plane.set_index_checks(False)
        data_plane._check_range("ids", torch.tensor([99]), 10)  # off: the kernels' rule applies
    finally:
        data_plane.set_index_checks(previous)
