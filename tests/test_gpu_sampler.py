"""Greedy sampling (reference src/mini_infra/worker/sampler.py:9-23, a torch.argmax over the last
position's logits) against torch.argmax on the CPU and numpy's argmax, which agree on every case
below: first index on ties, -0 equal to +0, NaN above every number with the first NaN winning.
Index work, so bit-exact."""

import numpy as np
import pytest
import torch

from mini_infra_qwen3_amd import data_plane
from mini_infra_qwen3_amd.worker.sampler import greedy_sample

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
VOCAB = 151936


def expect(logits_gpu):
    cpu = logits_gpu.float().cpu()
    want = torch.argmax(cpu, dim=-1)
    assert want.tolist() == np.argmax(cpu.numpy(), axis=-1).tolist()
    return want


def check(logits_gpu):
    got = data_plane.argmax_rows(logits_gpu)
    assert got.dtype == torch.int64 and got.shape == (logits_gpu.shape[0],)
    assert got.cpu().tolist() == expect(logits_gpu).tolist()


@pytest.mark.parametrize("rows", [1, 3, 64, 257])
def test_random_rows_of_the_vocabulary(rows):
    g = torch.Generator().manual_seed(rows)
    check(torch.randn(rows, VOCAB, generator=g).to(torch.bfloat16).to(DEV))


def test_ties_go_to_the_first_index():
    g = torch.Generator().manual_seed(1)
    logits = torch.randint(-4, 4, (32, VOCAB), generator=g).to(torch.bfloat16)
    # Plant the row maximum at several places, the first one in a different lane each row.
    for r in range(32):
        cols = torch.randperm(VOCAB, generator=g)[:1 + r % 7]
        logits[r, cols] = 9.0
    logits[31, :] = 2.0
    check(logits.to(DEV))


def test_infinities_zeros_and_nans():
    rows = []
    rows.append(torch.full((VOCAB,), float("-inf")))                   # all -inf -> 0
    r = torch.full((VOCAB,), float("-inf")); r[12345] = -1e30; rows.append(r)
    r = torch.randn(VOCAB); r[777] = float("inf"); r[99999] = float("inf"); rows.append(r)
    r = -torch.rand(VOCAB) - 1; r[5000] = -0.0; r[7000] = 0.0; rows.append(r)  # -0 first, equal to +0
    r = -torch.rand(VOCAB) - 1; r[5000] = 0.0; r[7000] = -0.0; rows.append(r)
    r = torch.randn(VOCAB); r[4242] = float("nan"); r[100] = float("inf"); rows.append(r)
    r = torch.randn(VOCAB); r[150000] = float("nan"); r[60000] = float("nan"); rows.append(r)
    r = torch.full((VOCAB,), float("nan")); rows.append(r)              # all NaN -> 0
    r = torch.randn(VOCAB); r[-1] = 50.0; rows.append(r)                 # last element
    r = torch.randn(VOCAB); r[0] = 50.0; rows.append(r)
    check(torch.stack(rows).to(torch.bfloat16).to(DEV))


@pytest.mark.parametrize("cols", [1, 5, 8, 13, 1000, 1029, 8192 + 3, VOCAB - 1])
def test_widths_and_tails(cols):
    g = torch.Generator().manual_seed(cols)
    logits = torch.randint(-3, 3, (9, cols), generator=g).to(torch.bfloat16)
    check(logits.to(DEV))


def test_row_views_and_unaligned_rows():
    g = torch.Generator().manual_seed(5)
    base = torch.randint(-6, 6, (7, 3, VOCAB + 8), generator=g).to(torch.bfloat16).to(DEV)
    check(base[:, -1, :VOCAB])     # strided rows, 16-byte aligned
    check(base[:, 1, 1:VOCAB + 1])  # rows start 2 bytes off: the per-element loads
    check(base[:, 0, 3:1003])
    check(base[2:3, 2, :])          # one row


def test_greedy_sample_last_position():
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(6, 4, VOCAB, generator=g).to(torch.bfloat16).to(DEV)
    token, last = greedy_sample(logits)
    assert token.shape == (6, 1) and token.dtype == torch.int64
    assert last.data_ptr() == logits[:, -1, :].data_ptr()
    assert token.squeeze(-1).cpu().tolist() == expect(logits[:, -1, :]).tolist()


def test_rejects_what_it_does_not_cover():
    with pytest.raises(ValueError):
        data_plane.argmax_rows(torch.zeros(4, 16, dtype=torch.float32, device=DEV))
    with pytest.raises(ValueError):
        data_plane.argmax_rows(torch.zeros(2, 4, 16, dtype=torch.bfloat16, device=DEV))
    assert data_plane.argmax_rows(torch.zeros(0, 16, dtype=torch.bfloat16, device=DEV)).shape == (0,)
