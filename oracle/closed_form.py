"""What the mathematics fixes for the paged-KV path (oracle; test infrastructure only).

Written independently of ``oracle.torch_ref`` (numpy indexing and explicit fp64 loops) so
that tests can pin the restatement against it: a dropped term, a wrong index or a
transposed head mapping in either shows up as a mismatch.
"""

from __future__ import annotations

import math

import numpy as np


def scatter_rows(pool_bits: np.ndarray, src_bits: np.ndarray, rows, positions, slots) -> np.ndarray:
    """Closed form of the reshape-and-cache scatter on raw element bits.

    pool_bits ``[num_blocks, bs, H, D]``; src_bits ``[B, H, L, D]``.  Returns a new pool with
    ``pool.reshape(-1, H, D)[slots[i]] = src[rows[i], :, positions[i], :]`` for every i and every
    other row unchanged (reference contract, src/mini_infra/worker/paged_kv_cache.py:81-87).
    """
    out = pool_bits.copy()
    flat = out.reshape(-1, out.shape[2], out.shape[3])
    for r, p, s in zip(rows, positions, slots):
        flat[int(s)] = src_bits[int(r), :, int(p), :]
    return out


def gather_rows(pool_bits: np.ndarray, block_ids: np.ndarray) -> np.ndarray:
    """Closed form of the block gather: ``out[b, j * bs + t] = pool[block_ids[b, j], t]``.

    Returns ``[B, nb * bs, H, D]`` (src/mini_infra/worker/paged_kv_cache.py:57-62).
    """
    batch, nb = block_ids.shape
    _, bs, heads, dim = pool_bits.shape
    out = np.empty((batch, nb * bs, heads, dim), dtype=pool_bits.dtype)
    for b in range(batch):
        for j in range(nb):
            out[b, j * bs:(j + 1) * bs] = pool_bits[int(block_ids[b, j])]
    return out


def pack_records(key_bits, value_bits, block_ids) -> np.ndarray:
    """Closed form of the KV block record format (the swap / wire format of whole physical blocks
    for the "swap" preemption mode the reference plans, src/mini_infra/core/types.py:110-114,
    over the pool layout of src/mini_infra/worker/paged_kv_cache.py:23-52).

    key_bits / value_bits: per-layer ``[num_blocks, bs, H, D]`` arrays.  Record i is block
    ``block_ids[i]`` of every layer: ``rec[i, l, 0] = key[l][id]``, ``rec[i, l, 1] = value[l][id]``;
    an id outside ``[0, num_blocks)`` reads the null block 0 (the library's rule for every read
    through a block id).  Explicit loops, one block at a time.
    """
    layers = len(key_bits)
    nb = key_bits[0].shape[0]
    out = np.zeros((len(block_ids), layers, 2, *key_bits[0].shape[1:]), dtype=key_bits[0].dtype)
    for i, bid in enumerate(block_ids):
        bid = int(bid)
        if not 0 <= bid < nb:
            bid = 0
        for layer in range(layers):
            out[i, layer, 0] = key_bits[layer][bid]
            out[i, layer, 1] = value_bits[layer][bid]
    return out


def unpack_records(key_bits, value_bits, records: np.ndarray, block_ids):
    """Inverse of ``pack_records``: new per-layer pools with block ``block_ids[i]`` of every layer
    set from record i (ids outside ``[0, num_blocks)`` skipped), every other block unchanged."""
    keys = [k.copy() for k in key_bits]
    values = [v.copy() for v in value_bits]
    nb = keys[0].shape[0]
    for i, bid in enumerate(block_ids):
        bid = int(bid)
        if not 0 <= bid < nb:
            continue
        for layer in range(len(keys)):
            keys[layer][bid] = records[i, layer, 0]
            values[layer][bid] = records[i, layer, 1]
    return keys, values


def slot_of(table, position: int, block_size: int) -> int:
    """Physical slot of a logical position (src/mini_infra/worker/paged_kv_cache.py:19)."""
    return int(table[position // block_size]) * block_size + position % block_size


def decode_attention_fp64(query: np.ndarray, key_pool: np.ndarray, value_pool: np.ndarray,
                          block_tables: np.ndarray, context_lens: np.ndarray, scale: float) -> np.ndarray:
    """Textbook single-query GQA attention over a paged context, in fp64 with explicit loops.

    query ``[B, H, D]``; pools ``[num_blocks, bs, Hkv, D]``; query head h reads kv head
    ``h // (H // Hkv)``; positions ``t < min(ctx, max_blocks * bs)`` only.  Returns ``[B, H, D]``.
    """
    batch, heads, dim = query.shape
    _, bs, kv_heads, _ = key_pool.shape
    group = heads // kv_heads
    q = query.astype(np.float64)
    kp = key_pool.astype(np.float64)
    vp = value_pool.astype(np.float64)
    out = np.zeros((batch, heads, dim), dtype=np.float64)
    for b in range(batch):
        n = min(int(context_lens[b]), block_tables.shape[1] * bs)
        for h in range(heads):
            g = h // group
            scores = []
            for t in range(n):
                k = kp[int(block_tables[b, t // bs]), t % bs, g]
                scores.append(float(np.dot(q[b, h], k)) * scale)
            top = max(scores)
            weights = [math.exp(s - top) for s in scores]
            total = sum(weights)
            acc = np.zeros(dim, dtype=np.float64)
            for t, w in enumerate(weights):
                acc += w * vp[int(block_tables[b, t // bs]), t % bs, g]
            out[b, h] = acc / total
    return out


def prefill_attention_fp64(query: np.ndarray, keys: np.ndarray, values: np.ndarray, visible: np.ndarray,
                           scale: float) -> np.ndarray:
    """Masked GQA attention in fp64: query ``[H, L, D]``, keys/values ``[Hkv, S, D]``,
    visible ``[L, S]`` bool.  Rows with nothing visible return zeros.  Returns ``[H, L, D]``."""
    heads, q_len, dim = query.shape
    kv_heads = keys.shape[0]
    group = heads // kv_heads
    out = np.zeros((heads, q_len, dim), dtype=np.float64)
    for h in range(heads):
        k = keys[h // group].astype(np.float64)
        v = values[h // group].astype(np.float64)
        s = (query[h].astype(np.float64) @ k.T) * scale
        for i in range(q_len):
            idx = np.nonzero(visible[i])[0]
            if idx.size == 0:
                continue
            row = s[i, idx]
            w = np.exp(row - row.max())
            out[h, i] = (w[:, None] * v[idx]).sum(axis=0) / w.sum()
    return out
