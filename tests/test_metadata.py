"""Host metadata packing: known answers from the reference's suite and agreement with the
oracle's per-token loops on seeded random cases."""

import random

import numpy as np
import pytest

from mini_infra_qwen3_amd.core import KVCacheManager
from mini_infra_qwen3_amd.worker.metadata import (
    pack_decode_rows,
    pack_mixed_rows,
    pack_prefill_rows,
    padded_mixed_shape,
    padded_tables,
    prefill_scatter_indices,
)
from oracle import closed_form, torch_ref


def test_decode_rows_known_answer():
    """tests/unit/test_paged_kv_cache.py:96-106: A at position 5 in blocks [9, 4], B at 2 in [7]."""
    rows = pack_decode_rows([[9, 4], [7]], last_tokens=[11, 22], positions=[5, 2], block_size=4)
    assert rows[:, 0].tolist() == [11, 22] and rows[:, 1].tolist() == [5, 2]
    assert rows[:, 2].tolist() == [4 * 4 + 1, 7 * 4 + 2]
    assert rows[:, 3].tolist() == [6, 3]
    assert rows[:, 4:].tolist() == [[9, 4], [7, 0]]


def test_decode_rows_smoke_known_answer():
    """verification/smoke.py:320-336: position 6 of a 2-block table -> block[1] * 4 + 2, context 7."""
    rows = pack_decode_rows([[1, 2]], [7], [6], 4)
    assert rows[0, 2] == 2 * 4 + 2 and rows[0, 3] == 7


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("block_size", [1, 3, 4, 16])
def test_decode_rows_match_reference_loop(seed, block_size):
    rng = random.Random(seed)
    manager = KVCacheManager(block_size, num_blocks=512)
    positions = []
    for i in range(rng.randint(1, 9)):
        n = rng.randint(1, 60)
        assert manager.allocate_slots(i, n)
        positions.append(n - 1)
    tables = [manager.block_table(i) for i in range(len(positions))]
    tokens = [rng.randint(0, 1000) for _ in positions]
    ours = pack_decode_rows(tables, tokens, positions, block_size)
    ref = torch_ref.prepare_decode_rows(tables, tokens, positions, block_size).numpy()
    assert np.array_equal(ours, ref)


@pytest.mark.parametrize("seed", range(5))
@pytest.mark.parametrize("block_size", [1, 3, 4, 16])
def test_scatter_indices_match_reference_loop(seed, block_size):
    rng = random.Random(100 + seed)
    manager = KVCacheManager(block_size, num_blocks=1024)
    manager.allocate_slots(999, rng.randint(0, 40))  # make tables non-contiguous
    chunk_lens, starts = [], []
    for i in range(rng.randint(1, 6)):
        start = rng.randint(0, 50)
        n = rng.randint(1, 40)
        assert manager.allocate_slots(i, start + n)
        starts.append(start)
        chunk_lens.append(n)
    tables = [manager.block_table(i) for i in range(len(starts))]
    padded = max(chunk_lens) + rng.randint(0, 3)
    ours = prefill_scatter_indices(tables, chunk_lens, starts, padded, block_size)
    ref = np.array(torch_ref.store_prefill_indices(tables, chunk_lens, starts, padded, block_size), dtype=np.int64)
    assert np.array_equal(ours, ref.reshape(3, -1))
    # every slot is where the closed form puts logical position start + t
    k = 0
    for row, (table, n, start) in enumerate(zip(tables, chunk_lens, starts)):
        for t in range(n):
            assert ours[2, k] == closed_form.slot_of(table, start + t, block_size)
            k += 1
    assert len(set(ours[2].tolist())) == ours.shape[1]


def test_prefill_rows_layout():
    """Row layout of src/mini_infra/worker/paged_runner.py:57-72 on a two-row chunk step."""
    rows = pack_prefill_rows([[5, 6, 7], [8]], start_positions=[5, 2], block_tables=[[3, 4, 9], [6, 1]],
                             block_size=4, pad_token_id=0)
    width = 3
    assert rows[:, :width].tolist() == [[5, 6, 7], [0, 0, 8]]
    assert rows[:, width:2 * width].tolist() == [[5, 6, 7], [0, 0, 2]]
    assert rows[:, 2 * width:2 * width + 2].tolist() == [[5, 3], [2, 1]]
    assert rows[:, 2 * width + 2:].tolist() == [[3, 4], [6, 0]]  # ceil(5/4)=2 and ceil(2/4)=1 blocks


def test_tables_cover_positions():
    with pytest.raises(ValueError):
        pack_decode_rows([[1]], [0], [4], 4)
    with pytest.raises(ValueError):
        prefill_scatter_indices([[1]], [2], [3], 2, 4)
    assert padded_tables([[1, 2], []]).tolist() == [[1, 2], [0, 0]]


# ------------------------------------------------------------------ padded graph buckets
def test_decode_rows_padded_to_a_bucket():
    """Pad rows append nothing (slot -1) and attend to nothing (context 0); live rows are the
    unpadded packing with null-padded tables."""
    tables, toks, pos = [[9, 4], [7]], [11, 22], [5, 2]
    plain = pack_decode_rows(tables, toks, pos, block_size=4)
    padded = pack_decode_rows(tables, toks, pos, block_size=4, rows=4, blocks=5)
    assert padded.shape == (4, 9)
    assert (padded[:2, :4] == plain[:, :4]).all()
    assert padded[:2, 4:].tolist() == [[9, 4, 0, 0, 0], [7, 0, 0, 0, 0]]
    assert padded[2:].tolist() == [[0, 0, -1, 0] + [0] * 5] * 2
    with pytest.raises(ValueError):
        pack_decode_rows(tables, toks, pos, block_size=4, rows=1)
    with pytest.raises(ValueError):
        pack_decode_rows(tables, toks, pos, block_size=4, blocks=1)


def test_prefill_rows_widened_to_a_bucket():
    """A chunk widened to a bucket: more left padding (pad id, position 0), the same start / length,
    history tables null-padded."""
    chunks, starts, tables = [[5, 6, 7], [8]], [4, 0], [[3, 9, 2], [1]]
    plain = pack_prefill_rows(chunks, starts, tables, block_size=4, pad_token_id=99)
    wide = pack_prefill_rows(chunks, starts, tables, block_size=4, pad_token_id=99, width=6, history_blocks=3)
    assert plain.shape == (2, 2 * 3 + 2 + 1) and wide.shape == (2, 2 * 6 + 2 + 3)
    assert wide[0, :6].tolist() == [99, 99, 99, 5, 6, 7] and wide[1, :6].tolist() == [99] * 5 + [8]
    assert wide[0, 6:12].tolist() == [0, 0, 0, 4, 5, 6] and wide[1, 6:12].tolist() == [0] * 6
    assert wide[:, 12:14].tolist() == [[4, 3], [0, 1]]
    assert wide[:, 14:].tolist() == [[3, 0, 0], [0, 0, 0]]
    for w, h in ((2, 3), (6, 0)):
        with pytest.raises(ValueError):
            pack_prefill_rows(chunks, starts, tables, block_size=4, pad_token_id=99, width=w, history_blocks=h)


@pytest.mark.parametrize("sizes", [None, (9, 4, 5, 6)])
def test_mixed_rows_ragged_layout(sizes):
    """The mixed buffer: chunk tokens back to back (then pad tokens up to C), decode tokens, their
    positions, per chunk row (start, length, first token, history table), and the decode rows of
    ``pack_decode_rows`` (optionally at a bucket's fixed sizes)."""
    chunks, starts, pf_tables = [[5, 6, 7], [8, 9]], [4, 0], [[3, 9, 2], [1]]
    dec_tables, toks, pos = [[9, 4], [7], [6, 2, 1]], [11, 22, 33], [5, 2, 9]
    kw = {} if sizes is None else dict(zip(("chunk_tokens", "history_blocks", "decode_rows", "decode_blocks"), sizes))
    flat, (p, c, nb, d, mb) = pack_mixed_rows(chunks, starts, pf_tables, toks, pos, dec_tables, 4, 99, **kw)
    dc = pack_decode_rows(dec_tables, toks, pos, 4, rows=kw.get("decode_rows"), blocks=kw.get("decode_blocks"))
    assert (p, c, nb) == ((2, 5, 1) if sizes is None else (2, 9, 4))
    assert (d, mb) == (dc.shape[0], dc.shape[1] - 4)
    t = c + d
    assert flat.shape == (2 * t + p * (3 + nb) + d * (2 + mb),)
    assert flat[:c].tolist() == [5, 6, 7, 8, 9] + [99] * (c - 5)
    assert (flat[c:t] == dc[:, 0]).all()
    assert flat[t:t + c].tolist() == [4, 5, 6, 0, 1] + [0] * (c - 5)
    assert (flat[t + c:2 * t] == dc[:, 1]).all()
    meta = flat[2 * t:2 * t + p * (3 + nb)].reshape(p, 3 + nb)
    assert meta[:, :3].tolist() == [[4, 3, 0], [0, 2, 3]]
    assert meta[0, 3:].tolist() == [3] + [0] * (nb - 1)  # ceil(4 / 4) = 1 history block
    assert meta[1, 3:].tolist() == [0] * nb
    assert (flat[2 * t + p * (3 + nb):].reshape(d, 2 + mb) == dc[:, 2:]).all()
    with pytest.raises(ValueError):
        pack_mixed_rows(chunks, starts, pf_tables, toks, pos, dec_tables, 4, 99, chunk_tokens=4)
    with pytest.raises(ValueError):
        pack_mixed_rows([[5], []], [0, 0], [[1], [2]], toks, pos, dec_tables, 4, 99)


def test_ragged_scatter_indices_follow_the_rows_first_tokens():
    """With row_first, token t of row i is position row_first[i] + t of the one cached row; the
    slots are the plain index's."""
    tables, lens, starts = [[3, 9, 2], [1, 5]], [3, 4], [4, 2]
    plain = prefill_scatter_indices(tables, lens, starts, 6, 4)
    ragged = prefill_scatter_indices(tables, lens, starts, 99, 4, row_first=[0, 3])
    assert (ragged[2] == plain[2]).all()
    assert ragged[0].tolist() == [0] * 7
    assert ragged[1].tolist() == [0, 1, 2, 3, 4, 5, 6]
    assert plain[1].tolist() == [3, 4, 5, 2, 3, 4, 5]


def test_padded_mixed_shape_known_answers():
    """Chunk tokens up to the next multiple of 128 (or the quantum given), decode rows up to the next
    power of two, no decode rows stays none; nonsense shapes raise."""
    cases = {(1, 0): (128, 0), (128, 1): (128, 1), (129, 2): (256, 2), (983, 3): (1024, 4), (1024, 8): (1024, 8),
             (1025, 9): (1152, 16), (39, 13): (128, 16), (2048, 33): (2048, 64)}
    for (width, rows), want in cases.items():
        assert padded_mixed_shape(width, rows) == want
    assert padded_mixed_shape(70, 5, quantum=64) == (128, 8)
    for bad in ((0, 1), (5, -1), (5, 1, 0)):
        with pytest.raises(ValueError):
            padded_mixed_shape(*bad)


@pytest.mark.parametrize("seed,block_size", [(0, 16), (1, 4), (2, 1)])
def test_prefill_rows_slot_columns_match_reference_loop(seed, block_size):
    """The optional slot columns: padded position p of row i holds the pool slot of its token
    (the reference's per-token slot, src/mini_infra/worker/paged_runner.py:123-128), -1 on left
    padding and past the end of the table; the other columns are the plain packing's."""
    rng = random.Random(seed)
    rows = 4
    lens = [rng.randint(1, 40) for _ in range(rows)]
    starts = [rng.randint(0, 70) for _ in range(rows)]
    tables, next_block = [], 1
    for s, n in zip(starts, lens):
        need = -(-(s + n) // block_size) - (1 if rng.random() < 0.3 and n > block_size else 0)  # some too short
        tables.append(list(range(next_block, next_block + need)))
        next_block += need + rng.randint(0, 3)
    ids = [[rng.randint(5, 99) for _ in range(n)] for n in lens]
    width, hist = 48, max(-(-s // block_size) for s in starts) + 2
    plain = pack_prefill_rows(ids, starts, tables, block_size, 0, width=width, history_blocks=hist)
    packed = pack_prefill_rows(ids, starts, tables, block_size, 0, width=width, history_blocks=hist, slots=True)
    assert packed.shape == (rows, plain.shape[1] + width)
    assert np.array_equal(packed[:, :plain.shape[1]], plain)
    slots = packed[:, plain.shape[1]:]
    for i, (s, n, table) in enumerate(zip(starts, lens, tables)):
        for p in range(width):
            t = p - (width - n)
            logical = s + t
            if t < 0 or logical // block_size >= len(table):
                want = -1
            else:
                want = table[logical // block_size] * block_size + logical % block_size
            assert slots[i, p] == want, (i, p)
