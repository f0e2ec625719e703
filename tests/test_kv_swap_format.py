"""KV block record format on the CPU: the file header byte layout, header validation, and the
oracle's record restatement pinned by a known-answer pool and a round trip.

The record format has no counterpart in the reference's code (it is the data side of the "swap"
preemption mode the reference only plans: src/mini_infra/core/types.py:110-114), so the
known-answer tests below are the specification."""

import numpy as np
import pytest
import torch

from mini_infra_qwen3_amd.worker.kv_swap import HEADER_BYTES, KVBlockHeader, _runs
from oracle import closed_form


def test_header_bytes_are_the_documented_layout():
    header = KVBlockHeader(28, 16, 8, 128, torch.bfloat16, 3, 0xDEADBEEF)
    want = (b"MIKVBLK1" + bytes.fromhex(
        "40000000" "01000000" "1c000000" "10000000" "08000000" "80000000" "01000000" "02000000"
        "0300000000000000" "00001c0000000000" "efbeadde" "00000000"))
    assert HEADER_BYTES == 64 and len(want) == 64
    assert header.encode() == want
    assert header.record_bytes == 1_835_008 == 2 * 28 * 16 * 8 * 128 * 2
    assert KVBlockHeader.decode(want) == header
    assert header.record_shape == (28, 2, 16, 8, 128)


@pytest.mark.parametrize("dtype,code,elt", [(torch.float16, 2, 2), (torch.float32, 3, 4)])
def test_header_dtype_codes(dtype, code, elt):
    raw = KVBlockHeader(2, 32, 4, 64, dtype, 7).encode()
    assert int.from_bytes(raw[32:36], "little") == code and int.from_bytes(raw[36:40], "little") == elt
    assert int.from_bytes(raw[48:56], "little") == 2 * 2 * 32 * 4 * 64 * elt
    assert KVBlockHeader.decode(raw).dtype == dtype


def test_header_rejects_what_it_does_not_describe():
    good = bytearray(KVBlockHeader(28, 16, 8, 128, torch.bfloat16, 3).encode())
    for offset, value, what in ((0, b"XIKVBLK1", "magic"), (12, (2).to_bytes(4, "little"), "version"),
                                (8, (65).to_bytes(4, "little"), "version"), (32, (9).to_bytes(4, "little"), "dtype"),
                                (36, (4).to_bytes(4, "little"), "inconsistent"),
                                (48, (12345).to_bytes(8, "little"), "inconsistent"),
                                (16, (0).to_bytes(4, "little"), "inconsistent")):
        bad = bytearray(good)
        bad[offset:offset + len(value)] = value
        with pytest.raises(ValueError, match=what):
            KVBlockHeader.decode(bytes(bad))
    with pytest.raises(ValueError, match="64 bytes"):
        KVBlockHeader.decode(bytes(good[:63]))
    with pytest.raises(ValueError):
        KVBlockHeader(1, 16, 8, 128, torch.int8, 1).encode()


def test_runs_of_consecutive_slots():
    assert _runs([]) == []
    assert _runs([4, 5, 6, 9, 10, 2]) == [(4, 0, 3), (9, 3, 2), (2, 5, 1)]
    assert _runs([7]) == [(7, 0, 1)]


def arange_pools(layers, nb, bs, h, d):
    """Element value encodes its own address: ((layer * 2 + kv) * nb + block) * E + offset."""
    e = bs * h * d
    keys = [np.arange((2 * l) * nb * e, (2 * l + 1) * nb * e, dtype=np.int64).reshape(nb, bs, h, d)
            for l in range(layers)]
    values = [np.arange((2 * l + 1) * nb * e, (2 * l + 2) * nb * e, dtype=np.int64).reshape(nb, bs, h, d)
              for l in range(layers)]
    return keys, values


def test_oracle_records_known_answer():
    layers, nb, bs, h, d = 3, 11, 4, 2, 3
    keys, values = arange_pools(layers, nb, bs, h, d)
    ids = [5, 0, 10, 5, -1, 11]
    rec = closed_form.pack_records(keys, values, ids)
    e = bs * h * d
    offset = np.arange(e).reshape(bs, h, d)
    for i, bid in enumerate(ids):
        read = bid if 0 <= bid < nb else 0  # an id outside the pool reads the null block 0
        for l in range(layers):
            for kv in range(2):
                assert (rec[i, l, kv] == ((l * 2 + kv) * nb + read) * e + offset).all()
    # flat byte order: record i, layer l, K then V, then the block's own [bs, H, D] order
    flat = rec.reshape(-1)
    assert flat[(1 * layers * 2 + 2 * 2 + 1) * e + 7] == ((2 * 2 + 1) * nb + 0) * e + 7


def test_oracle_unpack_inverts_pack_into_other_blocks():
    keys, values = arange_pools(2, 9, 2, 2, 4)
    src, dst = [1, 4, 7], [8, 2, 3]
    rec = closed_form.pack_records(keys, values, src)
    new_keys, new_values = closed_form.unpack_records(keys, values, rec, dst + [99])
    assert closed_form.unpack_records(keys, values, rec[:0], [])[0][0].tobytes() == keys[0].tobytes()
    for l in range(2):
        for s, t in zip(src, dst):
            assert (new_keys[l][t] == keys[l][s]).all() and (new_values[l][t] == values[l][s]).all()
        untouched = [b for b in range(9) if b not in dst]
        assert (new_keys[l][untouched] == keys[l][untouched]).all()
        assert (new_values[l][untouched] == values[l][untouched]).all()
