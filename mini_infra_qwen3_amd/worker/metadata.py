"""Host-side packing of paged-attention metadata, vectorised with numpy.

The reference builds these int64 rows with per-token / per-row Python loops
(src/mini_infra/worker/paged_runner.py:57-72, :118-128, :154-161); the values here are
identical, computed per block row with array operations so host time stays flat as the
batch and prompt lengths grow.  Everything returns numpy int64 arrays that the runner
uploads with a single host-to-device copy.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np

from mini_infra_qwen3_amd.core.block_manager import NULL_BLOCK_ID


def padded_tables(block_tables: Sequence[Sequence[int]], width: int | None = None) -> np.ndarray:
    """Ragged block tables -> ``[B, width]`` int64, right-padded with the null block."""
    lengths = [len(t) for t in block_tables]
    width = max(lengths, default=0) if width is None else width
    out = np.full((len(block_tables), width), NULL_BLOCK_ID, dtype=np.int64)
    for row, (table, n) in enumerate(zip(block_tables, lengths)):
        n = min(n, width)
        if n:
            out[row, :n] = np.asarray(table[:n], dtype=np.int64)
    return out


def pack_decode_rows(block_tables: Sequence[Sequence[int]], last_tokens: Sequence[int],
                     positions: Sequence[int], block_size: int, rows: int | None = None,
                     blocks: int | None = None) -> np.ndarray:
    """``[B, 4 + max_blocks]``: token, position, slot, context length, null-padded block table.

    Same columns as the reference's decode packing (src/mini_infra/worker/paged_runner.py:154-162).
    ``rows`` / ``blocks`` (at least B / the longest table) fix the shape of a padded bucket: pad
    rows are token 0, position 0, slot -1 (no append) and context 0 (zero output).
    """
    n = len(block_tables)
    width = max((len(t) for t in block_tables), default=0) if blocks is None else blocks
    total = n if rows is None else rows
    if total < n:
        raise ValueError(f"{n} decode rows do not fit {total}")
    tables = padded_tables(block_tables, width)
    if blocks is not None and any(len(t) > blocks for t in block_tables):
        raise ValueError(f"a block table is longer than {blocks}")
    pos = np.asarray(positions, dtype=np.int64)
    logical = pos // block_size
    if np.any(logical >= np.array([len(t) for t in block_tables], dtype=np.int64)):
        raise ValueError("a block table does not cover its decode position")
    out = np.zeros((total, 4 + width), dtype=np.int64)
    out[n:, 2] = -1
    out[:n, 0] = np.asarray(last_tokens, dtype=np.int64)
    out[:n, 1] = pos
    out[:n, 2] = tables[np.arange(n), logical] * block_size + pos % block_size
    out[:n, 3] = pos + 1
    out[:n, 4:] = tables
    return out


def prefill_scatter_indices(block_tables: Sequence[Sequence[int]], chunk_lens: Sequence[int],
                            start_positions: Sequence[int], padded_length: int, block_size: int,
                            row_first: Sequence[int] | None = None) -> np.ndarray:
    """``[3, N]`` (token_rows, token_positions, slots) of the valid chunk tokens, row-major.

    Token t of row i sits at padded position ``padded_length - chunk_lens[i] + t`` and goes to
    logical position ``start_positions[i] + t`` (src/mini_infra/worker/paged_runner.py:118-128).
    With ``row_first`` (ragged rows, all in one cached row): token t of row i sits at position
    ``row_first[i] + t`` of row 0.
    """
    lens = np.asarray(chunk_lens, dtype=np.int64)
    starts = np.asarray(start_positions, dtype=np.int64)
    total = int(lens.sum())
    out = np.empty((3, total), dtype=np.int64)
    if total == 0:
        return out
    rows = np.repeat(np.arange(len(lens), dtype=np.int64), lens)
    offsets = np.arange(total, dtype=np.int64) - np.repeat(np.cumsum(lens) - lens, lens)  # t within its row
    logical = np.repeat(starts, lens) + offsets
    width = max(int(((starts + lens + block_size - 1) // block_size).max()), 1)
    tables = padded_tables(block_tables, width)
    covered = np.array([len(t) for t in block_tables], dtype=np.int64)
    if np.any(logical // block_size >= covered[rows]):
        raise ValueError("a block table does not cover its chunk")
    out[2] = tables[rows, logical // block_size] * block_size + logical % block_size
    if row_first is None:
        out[0] = rows
        out[1] = padded_length - np.repeat(lens, lens) + offsets
    else:
        out[0] = 0
        out[1] = np.repeat(np.asarray(row_first, dtype=np.int64), lens) + offsets
    return out


def pack_prefill_rows(chunk_token_ids: Sequence[Sequence[int]], start_positions: Sequence[int],
                      block_tables: Sequence[Sequence[int]], block_size: int, pad_token_id: int,
                      width: int | None = None, history_blocks: int | None = None,
                      slots: bool = False) -> np.ndarray:
    """``[B, 2 L + 2 + max_history_blocks]``: left-padded ids | positions | start, len | history table.

    Same row layout as the reference's chunked-prefill packing
    (src/mini_infra/worker/paged_runner.py:57-72); history blocks are the first
    ``ceil(start / block_size)`` entries of each table, null-padded.  ``width`` / ``history_blocks``
    (at least the longest chunk / history) fix the shape of a padded bucket: wider left padding
    (pad tokens at position 0) and null-padded tables.  ``slots``: L more columns, the pool slot of
    each padded position's token (``table[p // block_size] * block_size + p % block_size`` at its
    logical position p), -1 for left padding and for tokens past the end of the table.
    """
    lens = [len(ids) for ids in chunk_token_ids]
    if not lens or min(lens) < 1:
        raise ValueError("every chunk must hold at least one token")
    hist = [-(-s // block_size) for s in start_positions]
    if width is None:
        width = max(lens)
    if history_blocks is None:
        history_blocks = max(hist)
    if width < max(lens) or history_blocks < max(hist):
        raise ValueError(f"chunks of {max(lens)} tokens / {max(hist)} history blocks do not fit "
                         f"width {width} / {history_blocks} blocks")
    max_hist = history_blocks
    out = np.zeros((len(lens), 2 * width + 2 + max_hist + (width if slots else 0)), dtype=np.int64)
    out[:, :width] = pad_token_id
    if slots:
        base = 2 * width + 2 + max_hist
        out[:, base:] = -1
        for row, (n, start, table) in enumerate(zip(lens, start_positions, block_tables)):
            logical = np.arange(start, start + n, dtype=np.int64)
            covered = logical < len(table) * block_size
            ids = np.asarray(table, dtype=np.int64)
            cols = base + width - n + np.nonzero(covered)[0]
            lc = logical[covered]
            out[row, cols] = ids[lc // block_size] * block_size + lc % block_size
    for row, (ids, n, start, table, h) in enumerate(zip(chunk_token_ids, lens, start_positions, block_tables, hist)):
        out[row, width - n:width] = np.asarray(ids, dtype=np.int64)
        out[row, 2 * width - n:2 * width] = np.arange(start, start + n, dtype=np.int64)
        out[row, 2 * width] = start
        out[row, 2 * width + 1] = n
        if h:
            if len(table) < h:
                raise ValueError("a block table does not cover its history")
            out[row, 2 * width + 2:2 * width + 2 + h] = np.asarray(table[:h], dtype=np.int64)
    return out


MIXED_WIDTH_QUANTUM = 128  # chunk width step of a padded mixed step


def padded_mixed_shape(chunk_tokens: int, decode_rows: int, quantum: int = MIXED_WIDTH_QUANTUM) -> tuple[int, int]:
    """The (chunk tokens, decode rows) a mixed step with reference numerics runs at: its chunks'
    tokens rounded up to a multiple of ``quantum``, the decode rows up to a power of two (none
    stays none).  The reference plans mixed steps but does not define them
    (src/mini_infra/core/scheduler.py:310-311); their GEMMs run over all C + D rows, and a GEMM's
    rows can round differently at another M.  With C and D on these steps every step shape is one of
    a few buckets, each of which a HIP graph replays with the same GEMM calls, and so the same bits,
    as the eager forward of that shape."""
    if chunk_tokens <= 0 or decode_rows < 0 or quantum <= 0:
        raise ValueError(f"bad mixed step shape: {chunk_tokens} chunk tokens, decode rows {decode_rows}, "
                         f"quantum {quantum}")
    return -(-chunk_tokens // quantum) * quantum, (1 << (decode_rows - 1).bit_length()) if decode_rows else 0


def pack_mixed_rows(chunk_token_ids: Sequence[Sequence[int]], start_positions: Sequence[int],
                    prefill_tables: Sequence[Sequence[int]], last_tokens: Sequence[int], positions: Sequence[int],
                    decode_tables: Sequence[Sequence[int]], block_size: int, pad_token_id: int,
                    chunk_tokens: int | None = None, history_blocks: int | None = None,
                    decode_rows: int | None = None,
                    decode_blocks: int | None = None) -> tuple[np.ndarray, tuple[int, int, int, int, int]]:
    """One int64 buffer for a mixed chunk + decode step, uploaded at once.

    Layout (T = C + D): tokens ``[T]`` | positions ``[T]`` | per chunk row (start, length, first
    token, history table) ``[P, 3 + nb]`` | per decode row (slot, context length, block table)
    ``[D, 2 + mb]``.  The first C tokens are the chunks back to back (ragged rows: row b's tokens
    from token ``first``, at logical positions start ..), then pad tokens (position 0) up to C; the
    last D are the decode tokens of ``pack_decode_rows``.  History tables are the first
    ``ceil(start / block_size)`` entries of each table, null-padded, as ``pack_prefill_rows`` takes
    them.  The optional sizes fix C, nb, D and mb for a padded bucket.  Returns the buffer and
    (P, C, nb, D, mb).
    """
    lens = [len(ids) for ids in chunk_token_ids]
    if not lens or min(lens) < 1:
        raise ValueError("every chunk must hold at least one token")
    hist = [-(-s // block_size) for s in start_positions]
    total = sum(lens)
    chunk_tokens = total if chunk_tokens is None else chunk_tokens
    nb = max(hist) if history_blocks is None else history_blocks
    if chunk_tokens < total or nb < max(hist):
        raise ValueError(f"{total} chunk tokens / {max(hist)} history blocks do not fit {chunk_tokens} / {nb}")
    decode = pack_decode_rows(decode_tables, last_tokens, positions, block_size, rows=decode_rows,
                              blocks=decode_blocks)
    rows = len(lens)
    ids = np.full(chunk_tokens, pad_token_id, dtype=np.int64)
    pos = np.zeros(chunk_tokens, dtype=np.int64)
    meta = np.zeros((rows, 3 + nb), dtype=np.int64)
    first = 0
    for row, (toks, n, start, table, h) in enumerate(zip(chunk_token_ids, lens, start_positions, prefill_tables,
                                                         hist)):
        ids[first:first + n] = np.asarray(toks, dtype=np.int64)
        pos[first:first + n] = np.arange(start, start + n, dtype=np.int64)
        meta[row, :3] = (start, n, first)
        if h:
            if len(table) < h:
                raise ValueError("a block table does not cover its history")
            meta[row, 3:3 + h] = np.asarray(table[:h], dtype=np.int64)
        first += n
    flat = np.concatenate([ids, decode[:, 0], pos, decode[:, 1], meta.ravel(), decode[:, 2:].ravel()])
    return flat, (rows, chunk_tokens, nb, decode.shape[0], decode.shape[1] - 4)


__all__ = ["MIXED_WIDTH_QUANTUM", "pack_decode_rows", "pack_mixed_rows", "pack_prefill_rows", "padded_mixed_shape",
           "padded_tables", "prefill_scatter_indices"]
