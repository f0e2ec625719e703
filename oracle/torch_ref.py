"""CPU restatement of the reference's paged-KV torch path (oracle; test infrastructure only).

Each function follows one reference function op for op, so that bf16 rounding happens at
the same points.  Pinned by tests/test_oracle.py against the reference's known-answer
tests, the closed forms in ``oracle.closed_form`` and the committed golden fixtures.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn.functional as F

NULL_BLOCK_ID = 0


# ----------------------------------------------------------------------------- pool ops
def make_pools(num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
               dtype: torch.dtype = torch.bfloat16, device="cpu") -> list[tuple[torch.Tensor, torch.Tensor]]:
    """Zero-filled per-layer (K, V) pools. src/mini_infra/worker/paged_kv_cache.py:23-41."""
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    return [(torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device))
            for _ in range(num_layers)]


def write_prefill(kv_pools, prefill_cache, token_rows, token_positions, slot_mapping) -> None:
    """In-place scatter of prefill K/V into slots. src/mini_infra/worker/paged_kv_cache.py:74-95.

    Per layer: advanced-index gather ``src[token_rows, :, token_positions, :]`` -> ``[N, H, D]``,
    then ``pool.view(-1, H, D).index_copy_(0, slot_mapping, ...)``.
    """
    for (key_pool, value_pool), (key, value) in zip(kv_pools, prefill_cache):
        heads, dim = key_pool.shape[2], key_pool.shape[3]
        key_rows = key[token_rows, :, token_positions, :]
        value_rows = value[token_rows, :, token_positions, :]
        key_pool.view(-1, heads, dim).index_copy_(0, slot_mapping, key_rows)
        value_pool.view(-1, heads, dim).index_copy_(0, slot_mapping, value_rows)


def gather_blocks(kv_pools, block_ids: torch.Tensor):
    """History views by block table. src/mini_infra/worker/paged_kv_cache.py:54-72.

    Returns per layer ``(key, value)`` of shape ``[B, H, nb * bs, D]`` (transposed views of the
    materialised ``[B, nb * bs, H, D]`` gather).
    """
    batch, nb = block_ids.shape
    out = []
    for key_pool, value_pool in kv_pools:
        _, bs, heads, dim = key_pool.shape
        shape = (batch, nb * bs, heads, dim)
        out.append((key_pool[block_ids].view(shape).transpose(1, 2),
                    value_pool[block_ids].view(shape).transpose(1, 2)))
    return tuple(out)


# ------------------------------------------------------------------------ host packing
def store_prefill_indices(block_tables: Sequence[Sequence[int]], chunk_lens: Sequence[int],
                          start_positions: Sequence[int], padded_length: int, block_size: int):
    """(token_rows, token_positions, slots) as lists. src/mini_infra/worker/paged_runner.py:118-128."""
    rows, positions, slots = [], [], []
    for row, (table, chunk_len, start) in enumerate(zip(block_tables, chunk_lens, start_positions)):
        for t in range(chunk_len):
            logical = start + t
            rows.append(row)
            positions.append(padded_length - chunk_len + t)
            slots.append(table[logical // block_size] * block_size + logical % block_size)
    return rows, positions, slots


def prepare_decode_rows(block_tables: Sequence[Sequence[int]], last_tokens: Sequence[int],
                        positions: Sequence[int], block_size: int) -> torch.Tensor:
    """Packed ``[B, 4 + max_blocks]`` decode metadata. src/mini_infra/worker/paged_runner.py:138-166.

    Columns: token, position, slot, context length (= position + 1), then the block table
    right-padded with the null block.
    """
    max_blocks = max(len(t) for t in block_tables)
    rows = []
    for table, token, pos in zip(block_tables, last_tokens, positions):
        slot = table[pos // block_size] * block_size + pos % block_size
        rows.append([token, pos, slot, pos + 1] + list(table) + [NULL_BLOCK_ID] * (max_blocks - len(table)))
    return torch.tensor(rows, dtype=torch.long)


# --------------------------------------------------------------------------- attention
def repeat_kv(x: torch.Tensor, groups: int) -> torch.Tensor:
    """GQA expansion, q head h -> kv head h // groups. src/mini_infra/model/qwen3.py:147-156."""
    return x if groups == 1 else x.repeat_interleave(groups, dim=1)


def attend(query, key, value, attn_bias, scaling: float) -> torch.Tensor:
    """GQA attention with the reference's rounding points. src/mini_infra/model/qwen3.py:219-255.

    query ``[B, H, q, D]``, key/value ``[B, Hkv, kv, D]``, attn_bias ``[B, 1, q, kv]`` (model dtype).
    Scores and the scale product are in the model dtype, softmax in fp32, probabilities cast
    back, PV in the model dtype.  Returns ``[B, q, H * D]``.
    """
    batch, heads, q_len, _ = query.shape
    groups = heads // key.shape[1]
    k = repeat_kv(key, groups)
    v = repeat_kv(value, groups)
    # Operands made contiguous first (same values; bf16 batched products on a transposed right
    # operand are avoided on ROCm).
    scores = torch.matmul(query.contiguous(), k.transpose(2, 3).contiguous()) * scaling
    scores = scores + attn_bias
    probs = F.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
    out = torch.matmul(probs, v.contiguous())
    return out.transpose(1, 2).contiguous().view(batch, q_len, -1)


# ----------------------------------------------------- attention / RMSNorm, exact sums
# The reference's rounding points (bf16 scores, fp32 softmax cast to bf16 before P V, bf16
# output; fp32 RMSNorm) with every sum exact instead of an fp32 sum in ATen's order: the
# definitions the HIP kernels' "exact" forms compute (csrc/exact_attention.hip,
# csrc/mi_common.h rms_inv).  Products of bf16 values are exact in fp64; fp64 sums of the terms
# here are exact or off far below what the final roundings see.  Pinned by tests/test_oracle.py:
# fp64 closed forms, agreement with ``attend`` (the op-for-op restatement) within one bf16 ulp
# per rounding point, and independence from the key order.

_SPLIT = 1572864.0  # 1.5 * 2^20: (x + _SPLIT) - _SPLIT rounds |x| <= 1 to a multiple of 2^-32 in fp64


def exact_sum(values: torch.Tensor, dim: int = -1, keepdim: bool = False) -> torch.Tensor:
    """fp64 sum of fp32 values in [0, 1] that does not depend on the order: each value splits into
    its multiple of 2^-32 (these add exactly for up to 2^20 terms) and a remainder below 2^-33."""
    x = values.double()
    hi = (x + _SPLIT) - _SPLIT
    lo = x - hi
    return hi.sum(dim, keepdim=keepdim) + lo.sum(dim, keepdim=keepdim)


def rms_norm_exact(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm (src/mini_infra/model/qwen3.py:67-78) with an exact sum of squares:
    var = fp32(sum(x^2) / N), r = fp32(1 / sqrt_f64(fp32(var + eps))), out = w * bf16(x * r)."""
    xf = x.float()
    var = (x.double().pow(2).sum(dim=-1, keepdim=True) / x.shape[-1]).float()
    r = (1.0 / torch.sqrt((var + eps).double())).float()
    return weight * (xf * r).to(x.dtype)


def attend_exact(query, key, value, attn_bias, scaling: float) -> torch.Tensor:
    """``attend`` (src/mini_infra/model/qwen3.py:219-255) with exact sums.  Per row and visible key t
    (``attn_bias == 0``; the reference's finfo.min bias gives the others exactly zero weight):
    s_t = bf16(bf16(fp32(q . k_t)) * scale), m = max s, e_t = fp32(exp_f64(fp32(s_t - m))),
    l = fp32(exact_sum(e)), p_t = bf16(fp32(e_t / l)), out = bf16(fp32(sum_t p_t v_t)).
    A row with no visible key (left padding) is zero; the reference's uniform average over masked
    keys there is never read.  Returns ``[B, q, H * D]``."""
    batch, heads, q_len, dim = query.shape
    groups = heads // key.shape[1]
    k = repeat_kv(key, groups).double()
    v = repeat_kv(value, groups).double()
    kv_len = k.shape[2]
    allowed = (attn_bias == 0).expand(batch, 1, q_len, kv_len)
    s = torch.matmul(query.double(), k.transpose(2, 3)).float().to(torch.bfloat16).float()
    s = (s * torch.tensor(scaling, dtype=torch.float32, device=s.device)).to(torch.bfloat16).float()
    s = s.masked_fill(~allowed, float("-inf"))
    m = s.amax(dim=-1, keepdim=True)
    none = torch.isinf(m)
    e = torch.exp((s - torch.where(none, torch.zeros_like(m), m)).double()).float()
    l = exact_sum(e, -1, keepdim=True).float()
    p = (e.double() / torch.where(none, torch.ones_like(l), l).double()).float().to(torch.bfloat16)
    out = torch.matmul(p.double(), v).float().to(query.dtype)
    out = out.masked_fill(none, 0)
    return out.transpose(1, 2).contiguous().view(batch, q_len, heads * dim)


def paged_bias(block_tables: torch.Tensor, context_lens: torch.Tensor, block_size: int,
               dtype: torch.dtype) -> torch.Tensor:
    """Additive decode bias ``[B, 1, 1, max_len]``. src/mini_infra/model/qwen3.py:513-528."""
    batch = block_tables.shape[0]
    max_len = block_tables.shape[1] * block_size
    positions = torch.arange(max_len, device=block_tables.device)
    allowed = (positions.unsqueeze(0) < context_lens.unsqueeze(1)).view(batch, 1, 1, max_len)
    bias = torch.zeros(allowed.shape, dtype=dtype, device=block_tables.device)
    bias.masked_fill_(~allowed, torch.finfo(dtype).min)
    return bias


def apply_paged_kv_pool(key, value, kv_pool, slot_mapping, block_tables):
    """Decode append + history gather. src/mini_infra/model/qwen3.py:257-292.

    key/value ``[B, Hkv, 1, D]``; the new rows are written to ``slot_mapping`` in place, then the
    ``[B, Hkv, max_blocks * bs, D]`` history is gathered through ``block_tables``.
    """
    batch = key.shape[0]
    key_pool, value_pool = kv_pool
    _, bs, heads, dim = key_pool.shape
    key_pool.view(-1, heads, dim).index_copy_(0, slot_mapping, key.squeeze(2))
    value_pool.view(-1, heads, dim).index_copy_(0, slot_mapping, value.squeeze(2))
    shape = (batch, block_tables.shape[1] * bs, heads, dim)
    return (key_pool[block_tables].view(shape).transpose(1, 2),
            value_pool[block_tables].view(shape).transpose(1, 2))


def paged_decode_step(query, key, value, kv_pool, slot_mapping, block_tables, context_lens,
                      scaling: float) -> torch.Tensor:
    """One layer of the reference paged decode: append, gather, bias, attend -> ``[B, 1, H * D]``.

    Composition of qwen3.py:282-292 (append/gather), :513-528 (bias) and :219-255 (attend).
    query ``[B, H, 1, D]``; key/value ``[B, Hkv, 1, D]``.
    """
    hist_k, hist_v = apply_paged_kv_pool(key, value, kv_pool, slot_mapping, block_tables)
    bias = paged_bias(block_tables, context_lens, kv_pool[0].shape[1], query.dtype)
    return attend(query, hist_k, hist_v, bias, scaling)


def paged_decode_attention(query, key_pool, value_pool, block_tables, context_lens, scaling: float,
                           exact: bool = False) -> torch.Tensor:
    """Kernel-3 oracle (no append): gather + bias + attend (``attend_exact`` with ``exact``).
    query ``[B, H, D]`` -> ``[B, H * D]``."""
    batch = query.shape[0]
    _, bs, heads, dim = key_pool.shape
    shape = (batch, block_tables.shape[1] * bs, heads, dim)
    hist_k = key_pool[block_tables].view(shape).transpose(1, 2)
    hist_v = value_pool[block_tables].view(shape).transpose(1, 2)
    bias = paged_bias(block_tables, context_lens, bs, query.dtype)
    return (attend_exact if exact else attend)(query.unsqueeze(2), hist_k, hist_v, bias, scaling).view(batch, -1)


def chunk_allowed_mask(start_lens: Sequence[int], chunk_lens: Sequence[int], num_history_blocks: int,
                       block_size: int, padded_chunk_len: int) -> torch.Tensor:
    """``[B, 1, L, hist + L]`` visibility of a chunked-prefill step.

    History slot k is visible iff k < start (src/mini_infra/worker/paged_runner.py:83-89); chunk
    key j is visible to chunk query i iff j <= i (causal, src/mini_infra/model/qwen3.py:477-484) and
    j is not left padding.
    """
    hist = num_history_blocks * block_size
    batch = len(start_lens)
    kv_len = hist + padded_chunk_len
    starts = torch.tensor(list(start_lens), dtype=torch.long).view(batch, 1)
    lens = torch.tensor(list(chunk_lens), dtype=torch.long).view(batch, 1)
    chunk_pos = torch.arange(padded_chunk_len).unsqueeze(0)
    attention_mask = chunk_pos >= padded_chunk_len - lens
    if hist:
        attention_mask = torch.cat((torch.arange(hist).unsqueeze(0) < starts, attention_mask), dim=1)
    query_pos = torch.arange(hist, kv_len)
    key_pos = torch.arange(kv_len)
    causal = key_pos.unsqueeze(0) <= query_pos.unsqueeze(1)
    return causal.view(1, 1, padded_chunk_len, kv_len) & attention_mask.view(batch, 1, 1, kv_len)


def chunked_prefill_attention(query, chunk_key, chunk_value, kv_pool, history_block_ids: torch.Tensor,
                              start_lens: Sequence[int], chunk_lens: Sequence[int], scaling: float,
                              exact: bool = False) -> torch.Tensor:
    """One layer of a chunked-prefill step with history -> ``[B, L, H * D]``.

    History gather (paged_kv_cache.py:54-72), concat with the chunk (qwen3.py:325-330), visibility
    bias (qwen3.py:560-561) and attend (qwen3.py:219-255).  query ``[B, H, L, D]``, chunk K/V
    ``[B, Hkv, L, D]`` (left-padded), history_block_ids ``[B, nb]``.
    """
    dtype = query.dtype
    nb = history_block_ids.shape[1]
    bs = kv_pool[0].shape[1]
    if nb:
        (hist_k, hist_v), = gather_blocks([kv_pool], history_block_ids)
        key = torch.cat((hist_k, chunk_key), dim=2)
        value = torch.cat((hist_v, chunk_value), dim=2)
    else:
        key, value = chunk_key, chunk_value
    allowed = chunk_allowed_mask(start_lens, chunk_lens, nb, bs, query.shape[2]).to(query.device)
    bias = torch.zeros(allowed.shape, dtype=dtype, device=query.device)
    bias.masked_fill_(~allowed, torch.finfo(dtype).min)
    return (attend_exact if exact else attend)(query, key, value, bias, scaling)
