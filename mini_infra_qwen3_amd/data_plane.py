"""Torch-tensor front end of the C ABI: shape/device checks, strides, stream, error mapping.

Every function here enqueues hand-written HIP kernels from libmi_paged.so on the current
torch stream of the tensors' device.  They accept only GPU tensors: there is no CPU or
torch fallback, and a missing library raises ``NativeLibraryError``.
"""

from __future__ import annotations

import os
from collections.abc import Sequence

import torch

from mini_infra_qwen3_amd import _native

__all__ = [
    "KERNEL_BLOCK_SIZE",
    "argmax_rows",
    "chunked_prefill_attention",
    "gather_blocks",
    "mixed_paged_attention",
    "pack_blocks",
    "paged_decode_attention",
    "paged_decode_attention_fused",
    "paged_decode_exact_workspace_bytes",
    "paged_decode_workspace_bytes",
    "qk_norm_rope",
    "reshape_and_cache",
    "rms_norm",
    "set_index_checks",
    "silu_mul",
    "unpack_blocks",
]


def _require_gpu(name: str, tensor: torch.Tensor, device: torch.device | None = None) -> None:
    if tensor.device.type != "cuda":
        raise RuntimeError(
            f"{name} is on {tensor.device}: the paged-KV data plane runs only on the GPU (no CPU fallback)"
        )
    if device is not None and tensor.device != device:
        raise ValueError(f"{name} is on {tensor.device}, expected {device}")


def _require_index(name: str, tensor: torch.Tensor, ndim: int) -> None:
    if tensor.dtype != torch.long or tensor.ndim != ndim:
        raise ValueError(f"{name} must be an int64 tensor with {ndim} dims, got {tensor.dtype} {tuple(tensor.shape)}")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_INDEX_CHECKS = os.environ.get("MI_CHECK_INDICES", "") == "1"


def set_index_checks(enabled: bool) -> bool:
    """Turns the pre-launch index checks on or off; returns the previous setting.

    On, every entry point raises ``IndexError`` -- as the reference's tensor indexing does for ids
    >= num_blocks -- when a block id or slot it is given lies outside the pool (slot -1, the
    "no write" marker of padding rows, is allowed), at the cost of one device reduction and host
    synchronisation per index tensor.  Off (the default; ``MI_CHECK_INDICES=1`` in the environment
    turns it on at import), the kernels' rule applies: reads through such ids read the null block
    0, writes to such slots or blocks are skipped.
    """
    global _INDEX_CHECKS
    previous, _INDEX_CHECKS = _INDEX_CHECKS, bool(enabled)
    return previous


def _check_range(name: str, ids: torch.Tensor, limit: int, allow_minus_one: bool = False) -> None:
    if not _INDEX_CHECKS or ids.numel() == 0:
        return
    bad = (ids >= limit) | (ids < (-1 if allow_minus_one else 0))
    if bool(bad.any()):
        first = int(ids[bad].flatten()[0])
        raise IndexError(f"{name}: index {first} is out of bounds for size {limit}")


def reshape_and_cache(
    key_src: Sequence[torch.Tensor],
    value_src: Sequence[torch.Tensor],
    slot_mapping: torch.Tensor,
    key_pools: Sequence[torch.Tensor],
    value_pools: Sequence[torch.Tensor],
    token_rows: torch.Tensor | None = None,
    token_positions: torch.Tensor | None = None,
) -> None:
    """Scatters K/V rows of every layer into pool slots (kernel 1), in one launch.

    key_src[l] / value_src[l]: ``[B, H_kv, L, D]`` (any strides with D contiguous), one per layer.
    slot_mapping / token_rows / token_positions: ``[N]`` int64; token ``i`` copies
    ``src[token_rows[i], :, token_positions[i], :]`` into ``pool.view(-1, H_kv, D)[slot_mapping[i]]``.
    ``token_rows=None`` means row ``i`` and ``token_positions=None`` position 0 (decode form).
    Pools: ``[num_blocks, block_size, H_kv, D]`` contiguous, same dtype as the sources.
    """
    num_layers = len(key_pools)
    if not (len(key_src) == len(value_src) == len(value_pools) == num_layers):
        raise ValueError("reshape_and_cache: per-layer lists differ in length")
    if num_layers == 0:
        return
    device = key_pools[0].device
    _require_gpu("slot_mapping", slot_mapping, device)
    _require_index("slot_mapping", slot_mapping, 1)
    num_tokens = slot_mapping.shape[0]
    pool0 = key_pools[0]
    if pool0.ndim != 4:
        raise ValueError(f"pools must be [num_blocks, block_size, H_kv, D], got {tuple(pool0.shape)}")
    num_blocks, block_size, num_kv_heads, head_dim = pool0.shape
    for name, tensors in (("key_pools", key_pools), ("value_pools", value_pools)):
        for t in tensors:
            _require_gpu(name, t, device)
            if t.shape != pool0.shape or t.dtype != pool0.dtype or not t.is_contiguous():
                raise ValueError(f"{name}: every pool must be contiguous {tuple(pool0.shape)} {pool0.dtype}")
    k0, v0 = key_src[0], value_src[0]
    for name, tensors, ref in (("key_src", key_src, k0), ("value_src", value_src, v0)):
        for t in tensors:
            _require_gpu(name, t, device)
            if t.ndim != 4 or t.shape[1] != num_kv_heads or t.shape[3] != head_dim or t.dtype != pool0.dtype:
                raise ValueError(f"{name} must be [B, {num_kv_heads}, L, {head_dim}] {pool0.dtype}, got "
                                 f"{tuple(t.shape)} {t.dtype}")
            if t.stride() != ref.stride() or t.shape != ref.shape or t.stride(3) != 1:
                raise ValueError(f"{name}: all layers need the same shape and strides, with D contiguous")
    if k0.shape[:3] != v0.shape[:3]:
        raise ValueError("reshape_and_cache: key and value sources differ in shape")

    index_stride = slot_mapping.stride(0) if num_tokens > 1 else 1
    for name, t in (("token_rows", token_rows), ("token_positions", token_positions)):
        if t is not None:
            _require_gpu(name, t, device)
            _require_index(name, t, 1)
            if t.shape[0] != num_tokens:
                raise ValueError(f"{name} has {t.shape[0]} entries, slot_mapping {num_tokens}")
    strides = {t.stride(0) for t in (slot_mapping, token_rows, token_positions) if t is not None and num_tokens > 1}
    if len(strides) > 1:
        slot_mapping = slot_mapping.contiguous()
        token_rows = token_rows.contiguous() if token_rows is not None else None
        token_positions = token_positions.contiguous() if token_positions is not None else None
        index_stride = 1
    if num_tokens == 0:
        return
    _check_range("slot_mapping", slot_mapping, num_blocks * block_size, allow_minus_one=True)
    if token_rows is not None:
        _check_range("token_rows", token_rows, k0.shape[0])
    if token_positions is not None:
        _check_range("token_positions", token_positions, k0.shape[2])

    lib = _native.load()
    rc = lib.mi_reshape_and_cache(
        _native.pointer_array([t.data_ptr() for t in key_src]),
        _native.pointer_array([t.data_ptr() for t in value_src]),
        k0.stride(0), k0.stride(1), k0.stride(2),
        v0.stride(0), v0.stride(1), v0.stride(2),
        token_rows.data_ptr() if token_rows is not None else None,
        token_positions.data_ptr() if token_positions is not None else None,
        slot_mapping.data_ptr(),
        index_stride,
        num_tokens,
        k0.shape[0],
        k0.shape[2],
        _native.pointer_array([t.data_ptr() for t in key_pools]),
        _native.pointer_array([t.data_ptr() for t in value_pools]),
        num_layers,
        num_blocks * block_size,
        num_kv_heads,
        head_dim,
        pool0.element_size(),
        _stream(device),
    )
    _native.check(rc, "mi_reshape_and_cache")


def gather_blocks(
    key_pools: Sequence[torch.Tensor],
    value_pools: Sequence[torch.Tensor],
    block_ids: torch.Tensor,
    key_out: Sequence[torch.Tensor],
    value_out: Sequence[torch.Tensor],
) -> None:
    """Copies whole pool blocks by block table for every layer (kernel 2), in one launch.

    block_ids: ``[B, nb]`` int64 (rows may be strided); outputs: contiguous ``[B, nb * block_size, H_kv, D]``.
    """
    num_layers = len(key_pools)
    if not (len(value_pools) == len(key_out) == len(value_out) == num_layers):
        raise ValueError("gather_blocks: per-layer lists differ in length")
    if num_layers == 0:
        return
    pool0 = key_pools[0]
    device = pool0.device
    _require_gpu("block_ids", block_ids, device)
    _require_index("block_ids", block_ids, 2)
    if block_ids.stride(1) != 1:
        block_ids = block_ids.contiguous()
    batch, nb = block_ids.shape
    num_blocks, block_size, num_kv_heads, head_dim = pool0.shape
    expect = (batch, nb * block_size, num_kv_heads, head_dim)
    for name, tensors, shape in (("key_pools", key_pools, pool0.shape), ("value_pools", value_pools, pool0.shape),
                                 ("key_out", key_out, expect), ("value_out", value_out, expect)):
        for t in tensors:
            _require_gpu(name, t, device)
            if tuple(t.shape) != tuple(shape) or t.dtype != pool0.dtype or not t.is_contiguous():
                raise ValueError(f"{name}: expected contiguous {tuple(shape)} {pool0.dtype}, got "
                                 f"{tuple(t.shape)} {t.dtype}")
    if batch == 0 or nb == 0:
        return
    _check_range("block_ids", block_ids, num_blocks)
    lib = _native.load()
    rc = lib.mi_gather_blocks(
        _native.pointer_array([t.data_ptr() for t in key_pools]),
        _native.pointer_array([t.data_ptr() for t in value_pools]),
        num_blocks,
        block_ids.data_ptr(),
        block_ids.stride(0) if batch > 1 else nb,
        batch,
        nb,
        _native.pointer_array([t.data_ptr() for t in key_out]),
        _native.pointer_array([t.data_ptr() for t in value_out]),
        num_layers,
        block_size * num_kv_heads * head_dim * pool0.element_size(),
        _stream(device),
    )
    _native.check(rc, "mi_gather_blocks")


KERNEL_BLOCK_SIZE = 16  # token rows per block the attention kernels are specialised for


def _as_kernel_blocks(key_pool: torch.Tensor, value_pool: torch.Tensor, tables: torch.Tensor):
    """A pool of block_size 16 k is the same memory as a pool of 16-token blocks, block i holding
    sub-blocks k i .. k i + k - 1.  Returns the pools viewed that way and the table of sub-block
    ids (entry j of a row -> table[j // k] * k + j % k; ids outside the pool stay outside, so they
    still read the null block).  Other block sizes pass through (the kernels reject them)."""
    block_size = key_pool.shape[1]
    if block_size == KERNEL_BLOCK_SIZE or block_size % KERNEL_BLOCK_SIZE != 0:
        return key_pool, value_pool, tables
    k = block_size // KERNEL_BLOCK_SIZE
    n = key_pool.shape[0]
    kp = key_pool.view(n * k, KERNEL_BLOCK_SIZE, *key_pool.shape[2:])
    vp = value_pool.view(n * k, KERNEL_BLOCK_SIZE, *value_pool.shape[2:])
    sub = torch.arange(k, dtype=tables.dtype, device=tables.device)
    return kp, vp, (tables.unsqueeze(-1) * k + sub).reshape(tables.shape[0], tables.shape[1] * k)


def paged_decode_workspace_bytes(batch: int, max_blocks: int, num_heads: int, head_dim: int, block_size: int,
                                 num_kv_heads: int) -> int:
    """Workspace for ``paged_decode_attention`` on ``[batch, max_blocks]`` tables of a pool with
    ``block_size``-token blocks (multiples of 16 count as 16-token sub-blocks) and ``num_kv_heads``
    KV heads."""
    if block_size > KERNEL_BLOCK_SIZE and block_size % KERNEL_BLOCK_SIZE == 0:
        max_blocks, block_size = max_blocks * (block_size // KERNEL_BLOCK_SIZE), KERNEL_BLOCK_SIZE
    return int(_native.load().mi_paged_decode_workspace_bytes(batch, max_blocks, num_heads, num_kv_heads, head_dim,
                                                                        block_size))


def paged_decode_exact_workspace_bytes(batch: int, max_blocks: int, num_heads: int, num_kv_heads: int,
                                       block_size: int = KERNEL_BLOCK_SIZE) -> int:
    """Workspace of the reference-numerics decode's split form (0: the launch runs unsplit)."""
    if block_size > KERNEL_BLOCK_SIZE and block_size % KERNEL_BLOCK_SIZE == 0:
        max_blocks = max_blocks * (block_size // KERNEL_BLOCK_SIZE)
    return int(_native.load().mi_paged_decode_exact_workspace_bytes(batch, max_blocks, num_heads, num_kv_heads))


def _exact_workspace(workspace: torch.Tensor | None, need: int, device: torch.device) -> tuple[int | None, int]:
    """(pointer, bytes) of a 256-byte aligned workspace of at least ``need`` bytes: ``workspace``
    when it qualifies, else a new buffer (None, 0 when nothing is needed)."""
    if need <= 0:
        return None, 0
    if workspace is None or workspace.numel() * workspace.element_size() < need or workspace.data_ptr() % 256:
        workspace = torch.empty(need, dtype=torch.uint8, device=device)
    _require_gpu("workspace", workspace, device)
    return workspace.data_ptr(), workspace.numel() * workspace.element_size()


def paged_decode_attention(
    query: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    exact: bool = False,
) -> torch.Tensor:
    """Paged GQA decode attention straight from the pool (kernel 3).

    query: ``[B, H, D]`` bf16 (D contiguous); pools ``[num_blocks, block_size, H_kv, D]`` bf16
    contiguous, block_size 16 or a multiple of it; block_tables ``[B, max_blocks]`` int64
    (null-padded); context_lens ``[B]`` int64 (includes the new token).  Returns ``out``
    ``[B, H * D]`` bf16.  ``workspace`` (optional, uint8, reused across calls) holds the
    split-context partials; it is allocated here when missing or too small.  ``exact``: the
    reference-numerics kernel (``mi_paged_decode_attention_exact``: the reference's rounding
    points with exact sums), whose split form for small batches uses the workspace the same way.
    """
    device = key_pool.device
    for name, t in (("query", query), ("key_pool", key_pool), ("value_pool", value_pool),
                    ("block_tables", block_tables), ("context_lens", context_lens)):
        _require_gpu(name, t, device)
    _require_index("block_tables", block_tables, 2)
    _require_index("context_lens", context_lens, 1)
    if query.ndim != 3 or query.dtype != torch.bfloat16 or query.stride(2) != 1:
        raise ValueError(f"query must be [B, H, D] bf16 with D contiguous, got {tuple(query.shape)} {query.dtype}")
    if key_pool.dtype != torch.bfloat16 or value_pool.shape != key_pool.shape or value_pool.dtype != key_pool.dtype:
        raise ValueError("pools must be bf16 with identical shapes")
    if not (key_pool.is_contiguous() and value_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    batch, num_heads, head_dim = query.shape
    num_blocks, block_size, num_kv_heads, pool_head_dim = key_pool.shape
    if pool_head_dim != head_dim:
        raise ValueError(f"query head_dim {head_dim} != pool head_dim {pool_head_dim}")
    if block_tables.shape[0] != batch or context_lens.shape[0] != batch:
        raise ValueError("block_tables / context_lens batch differs from query batch")
    _check_range("block_tables", block_tables, num_blocks)
    key_pool, value_pool, block_tables = _as_kernel_blocks(key_pool, value_pool, block_tables)
    num_blocks, block_size = key_pool.shape[:2]
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    max_blocks = block_tables.shape[1]
    if out is None:
        out = torch.empty((batch, num_heads * head_dim), dtype=torch.bfloat16, device=device)
    elif out.shape != (batch, num_heads * head_dim) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"out must be [B, H * D] bf16 with unit inner stride, got {tuple(out.shape)}")
    if batch == 0:
        return out
    lib = _native.load()
    stream = _stream(device)
    if exact:
        ws_ptr, ws_bytes = _exact_workspace(
            workspace, paged_decode_exact_workspace_bytes(batch, max_blocks, num_heads, num_kv_heads), device)
        rc = lib.mi_paged_decode_attention_exact(
            out.data_ptr(), out.stride(0), query.data_ptr(), query.stride(0), query.stride(1), None, 0, None, 0, None,
            None, None, None, 0.0, None, 0, key_pool.data_ptr(), value_pool.data_ptr(), num_blocks,
            block_tables.data_ptr(), block_tables.stride(0) if batch > 1 else max(max_blocks, 1), max_blocks,
            context_lens.data_ptr(), context_lens.stride(0) if batch > 1 else 1, batch, num_heads, num_kv_heads,
            head_dim, block_size, float(scale), ws_ptr, ws_bytes, stream)
        _native.check(rc, "mi_paged_decode_attention_exact")
        return out
    need = paged_decode_workspace_bytes(batch, max_blocks, num_heads, head_dim, block_size, num_kv_heads)
    ws_ptr, ws_bytes = None, 0
    if need > 0:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=device)
        _require_gpu("workspace", workspace, device)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    rc = lib.mi_paged_decode_attention(
        out.data_ptr(), out.stride(0),
        query.data_ptr(), query.stride(0), query.stride(1),
        key_pool.data_ptr(), value_pool.data_ptr(), num_blocks,
        block_tables.data_ptr(), block_tables.stride(0) if batch > 1 else max(max_blocks, 1), max_blocks,
        context_lens.data_ptr(), context_lens.stride(0) if batch > 1 else 1,
        batch, num_heads, num_kv_heads, head_dim, block_size, float(scale),
        ws_ptr, ws_bytes, stream,
    )
    _native.check(rc, "mi_paged_decode_attention")
    return out


def paged_decode_attention_fused(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
    slot_mapping: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    exact: bool = False,
) -> torch.Tensor:
    """``qk_norm_rope`` (decode form: the new K/V rows go to ``slot_mapping``) followed by
    ``paged_decode_attention``, in one launch where the per-sequence kernel serves the batch
    (with ``exact``: always one launch of the reference-numerics kernel).

    q ``[B, Hq * 128]``, k / v ``[B, Hkv * 128]``: the new tokens' projection rows (row views are
    fine); cos / sin ``[B, 128]``; the rest as in the two functions.  Same results, bit for bit.
    Returns ``out`` ``[B, Hq * 128]``.
    """
    device = key_pool.device
    for name, t in (("q", q), ("k", k), ("v", v), ("q_weight", q_weight), ("k_weight", k_weight), ("cos", cos),
                    ("sin", sin)):
        _require_bf16_rows(name, t, device)
    for name, t in (("key_pool", key_pool), ("value_pool", value_pool), ("block_tables", block_tables),
                    ("context_lens", context_lens), ("slot_mapping", slot_mapping)):
        _require_gpu(name, t, device)
    _require_index("block_tables", block_tables, 2)
    _require_index("context_lens", context_lens, 1)
    _require_index("slot_mapping", slot_mapping, 1)
    if key_pool.dtype != torch.bfloat16 or value_pool.shape != key_pool.shape or value_pool.dtype != key_pool.dtype \
            or not key_pool.is_contiguous() or not value_pool.is_contiguous():
        raise ValueError("pools must be contiguous bf16 with identical shapes")
    head_dim = q_weight.shape[-1]
    batch = q.numel() // q.shape[-1]
    q2, k2, v2 = q.reshape(batch, -1), k.reshape(batch, -1), v.reshape(batch, -1)
    num_heads, num_kv_heads = q2.shape[1] // head_dim, k2.shape[1] // head_dim
    cos2, sin2 = cos.reshape(batch, head_dim).contiguous(), sin.reshape(batch, head_dim).contiguous()
    if v2.shape != k2.shape or k_weight.shape != q_weight.shape or key_pool.shape[2:] != (num_kv_heads, head_dim):
        raise ValueError("q / k / v / weights / pools have inconsistent head sizes")
    if block_tables.shape[0] != batch or context_lens.shape[0] != batch or slot_mapping.shape[0] != batch:
        raise ValueError("block_tables / context_lens / slot_mapping batch differs from the tokens'")
    _check_range("block_tables", block_tables, key_pool.shape[0])
    _check_range("slot_mapping", slot_mapping, key_pool.shape[0] * key_pool.shape[1], allow_minus_one=True)
    key_pool, value_pool, block_tables = _as_kernel_blocks(key_pool, value_pool, block_tables)
    num_blocks, block_size = key_pool.shape[:2]
    if block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()
    max_blocks = block_tables.shape[1]
    if out is None:
        out = torch.empty((batch, num_heads * head_dim), dtype=torch.bfloat16, device=device)
    elif out.shape != (batch, num_heads * head_dim) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"out must be [B, H * D] bf16 with unit inner stride, got {tuple(out.shape)}")
    if batch == 0:
        return out
    if exact:
        ws_ptr, ws_bytes = _exact_workspace(
            workspace, paged_decode_exact_workspace_bytes(batch, max_blocks, num_heads, num_kv_heads), device)
        rc = _native.load().mi_paged_decode_attention_exact(
            out.data_ptr(), out.stride(0), q2.data_ptr(), q2.stride(0), head_dim, k2.data_ptr(), k2.stride(0),
            v2.data_ptr(), v2.stride(0), q_weight.data_ptr(), k_weight.data_ptr(), cos2.data_ptr(), sin2.data_ptr(),
            float(eps), slot_mapping.data_ptr(), slot_mapping.stride(0) if batch > 1 else 1, key_pool.data_ptr(),
            value_pool.data_ptr(), num_blocks, block_tables.data_ptr(),
            block_tables.stride(0) if batch > 1 else max(max_blocks, 1), max_blocks, context_lens.data_ptr(),
            context_lens.stride(0) if batch > 1 else 1, batch, num_heads, num_kv_heads, head_dim, block_size,
            float(scale), ws_ptr, ws_bytes, _stream(device))
        _native.check(rc, "mi_paged_decode_attention_exact")
        return out
    q_scratch = torch.empty((batch, num_heads, head_dim), dtype=torch.bfloat16, device=device)
    need = paged_decode_workspace_bytes(batch, max_blocks, num_heads, head_dim, block_size, num_kv_heads)
    ws_ptr, ws_bytes = None, 0
    if need > 0:
        if workspace is None or workspace.numel() * workspace.element_size() < need:
            workspace = torch.empty(need, dtype=torch.uint8, device=device)
        _require_gpu("workspace", workspace, device)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    rc = _native.load().mi_paged_decode_attention_fused(
        out.data_ptr(), out.stride(0), q2.data_ptr(), q2.stride(0), k2.data_ptr(), k2.stride(0), v2.data_ptr(),
        v2.stride(0), q_weight.data_ptr(), k_weight.data_ptr(), cos2.data_ptr(), sin2.data_ptr(), float(eps),
        slot_mapping.data_ptr(), slot_mapping.stride(0) if batch > 1 else 1, key_pool.data_ptr(), value_pool.data_ptr(),
        num_blocks, block_tables.data_ptr(), block_tables.stride(0) if batch > 1 else max(max_blocks, 1), max_blocks,
        context_lens.data_ptr(), context_lens.stride(0) if batch > 1 else 1, batch, num_heads, num_kv_heads,
        head_dim, block_size, float(scale), q_scratch.data_ptr(), ws_ptr, ws_bytes, _stream(device))
    _native.check(rc, "mi_paged_decode_attention_fused")
    return out


def chunked_prefill_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    history_blocks: torch.Tensor,
    start_lens: torch.Tensor,
    chunk_lens: torch.Tensor,
    scale: float,
    out: torch.Tensor | None = None,
    exact: bool = False,
) -> torch.Tensor:
    """Chunked-prefill attention with the history read from the pool (kernel 4, MFMA; with
    ``exact`` the reference-numerics kernel ``mi_chunked_prefill_attention_exact``).

    query ``[B, H, L, D]``; key / value ``[B, H_kv, L, D]`` (left-padded chunk, D contiguous, any
    other strides); pools ``[num_blocks, block_size, H_kv, D]``, block_size 16 or a multiple of it;
    history_blocks ``[B, nb]`` int64 (may have ``nb = 0``); start_lens / chunk_lens ``[B]`` int64
    (views with a common stride are fine).
    Returns ``out`` ``[B, L, H * D]`` bf16; left-padding rows are zero.
    """
    device = query.device
    for name, t in (("query", query), ("key", key), ("value", value), ("key_pool", key_pool),
                    ("value_pool", value_pool), ("history_blocks", history_blocks), ("start_lens", start_lens),
                    ("chunk_lens", chunk_lens)):
        _require_gpu(name, t, device)
    _require_index("history_blocks", history_blocks, 2)
    _require_index("start_lens", start_lens, 1)
    _require_index("chunk_lens", chunk_lens, 1)
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.ndim != 4 or t.dtype != torch.bfloat16 or t.stride(3) != 1:
            raise ValueError(f"{name} must be 4-d bf16 with the last dim contiguous, got {tuple(t.shape)} {t.dtype}")
    batch, num_heads, padded_len, head_dim = query.shape
    num_blocks, block_size, num_kv_heads, _ = key_pool.shape
    if key.shape != (batch, num_kv_heads, padded_len, head_dim) or value.shape != key.shape:
        raise ValueError(f"key/value must be [{batch}, {num_kv_heads}, {padded_len}, {head_dim}]")
    if key_pool.dtype != torch.bfloat16 or value_pool.shape != key_pool.shape or not key_pool.is_contiguous() \
            or not value_pool.is_contiguous():
        raise ValueError("pools must be contiguous bf16 with identical shapes")
    if history_blocks.shape[0] != batch or start_lens.shape[0] != batch or chunk_lens.shape[0] != batch:
        raise ValueError("history_blocks / start_lens / chunk_lens batch differs from query batch")
    _check_range("history_blocks", history_blocks, key_pool.shape[0])
    key_pool, value_pool, history_blocks = _as_kernel_blocks(key_pool, value_pool, history_blocks)
    num_blocks, block_size = key_pool.shape[:2]
    if history_blocks.stride(1) != 1:
        history_blocks = history_blocks.contiguous()
    if batch > 1 and start_lens.stride(0) != chunk_lens.stride(0):
        start_lens, chunk_lens = start_lens.contiguous(), chunk_lens.contiguous()
    lens_stride = start_lens.stride(0) if batch > 1 else 1
    nb = history_blocks.shape[1]
    if out is None:
        out = torch.empty((batch, padded_len, num_heads * head_dim), dtype=torch.bfloat16, device=device)
    elif out.shape != (batch, padded_len, num_heads * head_dim) or out.dtype != torch.bfloat16 or out.stride(2) != 1:
        raise ValueError(f"out must be [B, L, H * D] bf16 with unit inner stride, got {tuple(out.shape)}")
    if batch == 0 or padded_len == 0:
        return out
    entry = _native.load().mi_chunked_prefill_attention_exact if exact else _native.load().mi_chunked_prefill_attention
    rc = entry(
        out.data_ptr(), out.stride(0), out.stride(1),
        query.data_ptr(), query.stride(0), query.stride(1), query.stride(2),
        key.data_ptr(), key.stride(0), key.stride(1), key.stride(2),
        value.data_ptr(), value.stride(0), value.stride(1), value.stride(2),
        key_pool.data_ptr(), value_pool.data_ptr(), num_blocks,
        history_blocks.data_ptr() if nb else None, history_blocks.stride(0) if nb else 0, nb,
        start_lens.data_ptr(), chunk_lens.data_ptr(), lens_stride,
        batch, padded_len, num_heads, num_kv_heads, head_dim, block_size, float(scale),
        _stream(device),
    )
    _native.check(rc, "mi_chunked_prefill_attention_exact" if exact else "mi_chunked_prefill_attention")
    return out


def mixed_paged_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    key_pool: torch.Tensor,
    value_pool: torch.Tensor,
    prefill_rows: int,
    prefill_width: int,
    history_blocks: torch.Tensor,
    start_lens: torch.Tensor,
    chunk_lens: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    slot_mapping: torch.Tensor,
    scale: float,
    out: torch.Tensor | None = None,
    exact: bool = False,
    chunk_first: torch.Tensor | None = None,
    chunk_tokens: int | None = None,
) -> torch.Tensor:
    """The attention of a mixed chunk + decode step in one launch (``mi_mixed_paged_attention``, or
    ``mi_mixed_paged_attention_exact`` with ``exact``), which also appends the decode tokens' K/V.

    A flattened batch of T = C + D tokens: query ``[T, H, D]``, key / value ``[T, H_kv, D]``
    (token-major, D contiguous; the rotated q / k of ``qk_norm_rope``).  Tokens ``[0, C)`` are P
    chunk rows with ``history_blocks`` ``[P, nb]`` (nb may be 0), ``start_lens`` / ``chunk_lens``
    ``[P]`` as in ``chunked_prefill_attention``, each seen as a left-padded chunk of width L (at least
    every chunk length).  Without ``chunk_first``, C = P L and row b is tokens ``[b L, b L + L)``;
    with ``chunk_first`` ``[P]`` (ragged rows) C = ``chunk_tokens`` and row b's real tokens start at
    token ``chunk_first[b]``, with no padding stored (a token that no row covers gets a zero row;
    at least one row when ``chunk_tokens`` > 0).  The last D tokens are decode rows
    with ``block_tables`` ``[D, mb]``, ``context_lens`` ``[D]`` (tokens including the new one) and
    ``slot_mapping`` ``[D]`` (where the new K/V go; -1: none).  Pools ``[num_blocks, block_size,
    H_kv, D]``, block_size 16 or a multiple.  Returns ``out`` ``[T, H * D]`` bf16.
    """
    device = query.device
    for name, t in (("query", query), ("key", key), ("value", value), ("key_pool", key_pool),
                    ("value_pool", value_pool), ("history_blocks", history_blocks), ("start_lens", start_lens),
                    ("chunk_lens", chunk_lens), ("block_tables", block_tables), ("context_lens", context_lens),
                    ("slot_mapping", slot_mapping)):
        _require_gpu(name, t, device)
    for name, t, nd in (("history_blocks", history_blocks, 2), ("start_lens", start_lens, 1),
                        ("chunk_lens", chunk_lens, 1), ("block_tables", block_tables, 2),
                        ("context_lens", context_lens, 1), ("slot_mapping", slot_mapping, 1)):
        _require_index(name, t, nd)
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.ndim != 3 or t.dtype != torch.bfloat16 or t.stride(2) != 1:
            raise ValueError(f"{name} must be [T, heads, D] bf16 with D contiguous, got {tuple(t.shape)} {t.dtype}")
    tokens, num_heads, head_dim = query.shape
    num_blocks, block_size, num_kv_heads, _ = key_pool.shape
    rows, width = int(prefill_rows), int(prefill_width)
    decode_rows = int(context_lens.shape[0])
    if chunk_first is None:
        if rows < 0 or width < 0 or tokens != rows * width + decode_rows:
            raise ValueError(f"{tokens} tokens are not {rows} chunk rows x {width} + {decode_rows} decode rows")
        chunk_tokens = rows * width
    else:
        _require_gpu("chunk_first", chunk_first, device)
        _require_index("chunk_first", chunk_first, 1)
        if chunk_tokens is None or rows < 0 or width < 0 or chunk_first.shape[0] != rows or \
                tokens != int(chunk_tokens) + decode_rows or (rows == 0 and int(chunk_tokens) > 0):
            raise ValueError(f"{tokens} tokens are not {chunk_tokens} ragged chunk tokens of {rows} rows + "
                             f"{decode_rows} decode rows")
        chunk_first = chunk_first.contiguous()
    if key.shape != (tokens, num_kv_heads, head_dim) or value.shape != key.shape:
        raise ValueError(f"key/value must be [{tokens}, {num_kv_heads}, {head_dim}]")
    if key_pool.dtype != torch.bfloat16 or value_pool.shape != key_pool.shape or not key_pool.is_contiguous() \
            or not value_pool.is_contiguous():
        raise ValueError("pools must be contiguous bf16 with identical shapes")
    if history_blocks.shape[0] != rows or start_lens.shape[0] != rows or chunk_lens.shape[0] != rows:
        raise ValueError("history_blocks / start_lens / chunk_lens must have one row per chunk row")
    if block_tables.shape[0] != decode_rows or slot_mapping.shape[0] != decode_rows:
        raise ValueError("block_tables / slot_mapping must have one row per decode row")
    _check_range("history_blocks", history_blocks, key_pool.shape[0])
    _check_range("block_tables", block_tables, key_pool.shape[0])
    _check_range("slot_mapping", slot_mapping, key_pool.shape[0] * key_pool.shape[1], allow_minus_one=True)
    kp, vp, history_blocks = _as_kernel_blocks(key_pool, value_pool, history_blocks)
    _, _, block_tables = _as_kernel_blocks(key_pool, value_pool, block_tables)
    num_blocks, block_size = kp.shape[:2]
    if history_blocks.stride(-1) != 1:
        history_blocks = history_blocks.contiguous()
    if block_tables.stride(-1) != 1:
        block_tables = block_tables.contiguous()
    if rows > 1 and start_lens.stride(0) != chunk_lens.stride(0):
        start_lens, chunk_lens = start_lens.contiguous(), chunk_lens.contiguous()
    lens_stride = start_lens.stride(0) if rows > 1 else 1
    nb, mb = history_blocks.shape[1], block_tables.shape[1]
    if out is None:
        out = torch.empty((tokens, num_heads * head_dim), dtype=torch.bfloat16, device=device)
    elif out.shape != (tokens, num_heads * head_dim) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError(f"out must be [T, H * D] bf16 with unit inner stride, got {tuple(out.shape)}")
    if tokens == 0:
        return out
    name = "mi_mixed_paged_attention_exact" if exact else "mi_mixed_paged_attention"
    rc = getattr(_native.load(), name)(
        out.data_ptr(), out.stride(0),
        query.data_ptr(), query.stride(0), query.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        kp.data_ptr(), vp.data_ptr(), num_blocks,
        rows, width, int(chunk_tokens), chunk_first.data_ptr() if chunk_first is not None and rows else None,
        history_blocks.data_ptr() if nb and rows else None, history_blocks.stride(0) if nb else 0,
        nb if rows else 0, start_lens.data_ptr() if rows else None, chunk_lens.data_ptr() if rows else None,
        lens_stride,
        decode_rows, block_tables.data_ptr() if mb and decode_rows else None, block_tables.stride(0) if mb else 0,
        mb if decode_rows else 0, context_lens.data_ptr() if decode_rows else None,
        context_lens.stride(0) if decode_rows else 1, slot_mapping.data_ptr() if decode_rows else None,
        slot_mapping.stride(0) if decode_rows else 1,
        num_heads, num_kv_heads, head_dim, block_size, float(scale), _stream(device),
    )
    _native.check(rc, name)
    return out


# ----------------------------------------------------------------------------- fused layer ops
def _require_bf16_rows(name: str, tensor: torch.Tensor, device: torch.device) -> None:
    _require_gpu(name, tensor, device)
    if tensor.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {tensor.dtype}")
    if tensor.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last dimension")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm over the last dim, optionally of ``x + residual`` (one launch).

    Returns ``(normed, h)`` with ``h = x + residual`` (or ``x`` itself without a residual): the
    next residual of a decoder layer.  bf16, contiguous rows.
    """
    device = x.device
    _require_bf16_rows("x", x, device)
    _require_bf16_rows("weight", weight, device)
    x = x.contiguous()
    hidden = x.shape[-1]
    if weight.shape != (hidden,):
        raise ValueError(f"weight {tuple(weight.shape)} does not match hidden size {hidden}")
    out = torch.empty_like(x)
    res_out = x
    res_ptr = None
    if residual is not None:
        _require_bf16_rows("residual", residual, device)
        if residual.shape != x.shape:
            raise ValueError(f"residual {tuple(residual.shape)} differs from x {tuple(x.shape)}")
        residual = residual.contiguous()
        res_out = torch.empty_like(x)
        res_ptr = residual.data_ptr()
    lib = _native.load()
    rc = lib.mi_rms_norm(out.data_ptr(), x.data_ptr(), res_ptr, res_out.data_ptr() if res_ptr else None,
                         weight.contiguous().data_ptr(), x.numel() // hidden, hidden, float(eps), _stream(device))
    _native.check(rc, "mi_rms_norm")
    return out, res_out


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_weight: torch.Tensor,
                 k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float,
                 slot_mapping: torch.Tensor | None = None, key_pool: torch.Tensor | None = None,
                 value_pool: torch.Tensor | None = None, k_out: torch.Tensor | None = None,
                 v_out: torch.Tensor | None = None, rows: bool | None = None):
    """Per-head RMSNorm + RoPE of q and k, v passed through (one launch).

    q ``[..., Hq * 128]``, k / v ``[..., Hkv * 128]`` over the same T tokens (row views of a
    projection are fine); cos / sin ``[T, 128]`` (any leading shape with T tokens).
    Returns ``q_out [T, Hq, 128]`` and, with ``rows``, ``k_out`` / ``v_out [T, Hkv, 128]``; with
    ``slot_mapping`` ``[T]`` k and v are (also) written into ``key_pool`` / ``value_pool``
    ``[num_blocks, block_size, Hkv, 128]`` at those slots (-1: skipped).  ``rows`` defaults to
    "no slot_mapping"; without rows ``(q_out, None, None)`` is returned (the decode form).
    ``k_out`` / ``v_out`` (optional): contiguous ``[T, Hkv, 128]`` buffers to write instead of new
    ones.
    """
    device = q.device
    for name, t in (("q", q), ("k", k), ("v", v), ("q_weight", q_weight), ("k_weight", k_weight),
                    ("cos", cos), ("sin", sin)):
        _require_bf16_rows(name, t, device)
    head_dim = q_weight.shape[-1]
    tokens = q.numel() // q.shape[-1]
    num_heads, num_kv_heads = q.shape[-1] // head_dim, k.shape[-1] // head_dim
    q2, k2, v2 = q.reshape(tokens, -1), k.reshape(tokens, -1), v.reshape(tokens, -1)
    cos2, sin2 = cos.reshape(tokens, head_dim).contiguous(), sin.reshape(tokens, head_dim).contiguous()
    if v.shape[-1] != k.shape[-1] or k_weight.shape != q_weight.shape:
        raise ValueError("k / v / weights have inconsistent head sizes")
    q_out = torch.empty((tokens, num_heads, head_dim), dtype=q.dtype, device=device)
    lib = _native.load()
    if rows is None:
        rows = slot_mapping is None
    if rows:
        for name, given in (("k_out", k_out), ("v_out", v_out)):
            if given is not None:
                _require_gpu(name, given, device)
                if given.shape != (tokens, num_kv_heads, head_dim) or given.dtype != q.dtype \
                        or not given.is_contiguous():
                    raise ValueError(f"{name} must be contiguous [{tokens}, {num_kv_heads}, {head_dim}] {q.dtype}")
        k_out = torch.empty((tokens, num_kv_heads, head_dim), dtype=q.dtype, device=device) if k_out is None else k_out
        v_out = torch.empty((tokens, num_kv_heads, head_dim), dtype=q.dtype, device=device) if v_out is None else v_out
    else:
        k_out = v_out = None
    if slot_mapping is None:
        rc = lib.mi_qk_norm_rope(q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), q2.data_ptr(), q2.stride(0),
                                 k2.data_ptr(), k2.stride(0), v2.data_ptr(), v2.stride(0), q_weight.data_ptr(),
                                 k_weight.data_ptr(), cos2.data_ptr(), sin2.data_ptr(), tokens, num_heads,
                                 num_kv_heads, head_dim, float(eps), None, 1, None, None, 0, _stream(device))
    else:
        _require_gpu("slot_mapping", slot_mapping, device)
        _require_index("slot_mapping", slot_mapping, 1)
        if slot_mapping.shape[0] != tokens:
            raise ValueError(f"slot_mapping has {slot_mapping.shape[0]} entries for {tokens} tokens")
        for name, pool in (("key_pool", key_pool), ("value_pool", value_pool)):
            if pool is None:
                raise ValueError(f"{name} is required with slot_mapping")
            _require_bf16_rows(name, pool, device)
            if not pool.is_contiguous() or pool.shape[-2:] != (num_kv_heads, head_dim):
                raise ValueError(f"{name} must be contiguous [num_blocks, block_size, {num_kv_heads}, {head_dim}]")
        num_slots = key_pool.numel() // (num_kv_heads * head_dim)
        _check_range("slot_mapping", slot_mapping, num_slots, allow_minus_one=True)
        rc = lib.mi_qk_norm_rope(q_out.data_ptr(), k_out.data_ptr() if rows else None,
                                 v_out.data_ptr() if rows else None, q2.data_ptr(), q2.stride(0), k2.data_ptr(),
                                 k2.stride(0), v2.data_ptr(), v2.stride(0), q_weight.data_ptr(), k_weight.data_ptr(),
                                 cos2.data_ptr(), sin2.data_ptr(), tokens, num_heads, num_kv_heads, head_dim,
                                 float(eps), slot_mapping.data_ptr(), slot_mapping.stride(0), key_pool.data_ptr(),
                                 value_pool.data_ptr(), num_slots, _stream(device))
    _native.check(rc, "mi_qk_norm_rope")
    return q_out, k_out, v_out


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``bf16(bf16(silu(gate)) * up)`` elementwise (one launch); gate / up ``[..., I]`` row views."""
    device = gate.device
    _require_bf16_rows("gate", gate, device)
    _require_bf16_rows("up", up, device)
    if gate.shape != up.shape:
        raise ValueError(f"gate {tuple(gate.shape)} and up {tuple(up.shape)} differ")
    cols = gate.shape[-1]
    rows = gate.numel() // cols
    g2, u2 = gate.reshape(rows, cols), up.reshape(rows, cols)
    out = torch.empty(gate.shape, dtype=gate.dtype, device=device)
    rc = _native.load().mi_silu_mul(out.data_ptr(), cols, g2.data_ptr(), g2.stride(0), u2.data_ptr(), u2.stride(0),
                                    rows, cols, _stream(device))
    _native.check(rc, "mi_silu_mul")
    return out


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """Greedy token of each row of bf16 ``logits [rows, vocab]`` (any row stride): int64 ``[rows]``.

    Same answer as ``torch.argmax(logits, dim=-1)`` -- first index on ties, NaN above every number --
    in one launch (the sampler of reference src/mini_infra/worker/sampler.py:9-23).
    """
    device = logits.device
    _require_bf16_rows("logits", logits, device)
    if logits.dim() != 2:
        raise ValueError(f"logits must be [rows, vocab], got {tuple(logits.shape)}")
    rows, cols = logits.shape
    out = torch.empty(rows, dtype=torch.int64, device=device)
    if rows == 0:
        return out
    row_stride = logits.stride(0) if rows > 1 else cols
    rc = _native.load().mi_argmax_rows(out.data_ptr(), logits.data_ptr(), rows, cols, row_stride, _stream(device))
    _native.check(rc, "mi_argmax_rows")
    return out


def _record_pools(key_pools: Sequence[torch.Tensor], value_pools: Sequence[torch.Tensor]):
    """Validates per-layer pools ``[num_blocks, bs, H, D]`` (one shape and dtype, contiguous)."""
    if len(key_pools) != len(value_pools) or not key_pools:
        raise ValueError("key_pools and value_pools must be equal-length, non-empty per-layer lists")
    pool0 = key_pools[0]
    device = pool0.device
    for name, tensors in (("key_pools", key_pools), ("value_pools", value_pools)):
        for t in tensors:
            _require_gpu(name, t, device)
            if t.shape != pool0.shape or t.dtype != pool0.dtype or not t.is_contiguous() or t.dim() != 4:
                raise ValueError(f"{name}: expected contiguous {tuple(pool0.shape)} {pool0.dtype}, got "
                                 f"{tuple(t.shape)} {t.dtype}")
    block_bytes = pool0[0].numel() * pool0.element_size()
    return pool0, device, block_bytes


def pack_blocks(key_pools: Sequence[torch.Tensor], value_pools: Sequence[torch.Tensor], block_ids: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Packs whole physical blocks of every layer into contiguous records (one launch).

    Returns ``records [n, num_layers, 2, bs, H, D]`` with ``records[i, l, 0] = key_pools[l][block_ids[i]]``
    and ``records[i, l, 1] = value_pools[l][block_ids[i]]``: the wire / swap format.  block_ids:
    ``[n]`` int64 on the pools' device; ids outside ``[0, num_blocks)`` read the null block 0.
    """
    pool0, device, block_bytes = _record_pools(key_pools, value_pools)
    _require_gpu("block_ids", block_ids, device)
    _require_index("block_ids", block_ids, 1)
    block_ids = block_ids.contiguous()
    shape = (block_ids.shape[0], len(key_pools), 2, *pool0.shape[1:])
    if out is None:
        out = torch.empty(shape, dtype=pool0.dtype, device=device)
    else:
        _require_gpu("out", out, device)
        if tuple(out.shape) != shape or out.dtype != pool0.dtype or not out.is_contiguous():
            raise ValueError(f"out: expected contiguous {shape} {pool0.dtype}, got {tuple(out.shape)} {out.dtype}")
    if block_ids.shape[0] == 0:
        return out
    _check_range("block_ids", block_ids, pool0.shape[0])
    rc = _native.load().mi_pack_blocks(
        out.data_ptr(), _native.pointer_array([t.data_ptr() for t in key_pools]),
        _native.pointer_array([t.data_ptr() for t in value_pools]), pool0.shape[0], block_ids.data_ptr(),
        block_ids.shape[0], len(key_pools), block_bytes, _stream(device))
    _native.check(rc, "mi_pack_blocks")
    return out


def unpack_blocks(records: torch.Tensor, key_pools: Sequence[torch.Tensor], value_pools: Sequence[torch.Tensor],
                  block_ids: torch.Tensor) -> None:
    """Writes records (the layout ``pack_blocks`` returns) into physical blocks ``block_ids`` of every
    layer (one launch).  block_ids: ``[n]`` int64, unique; ids outside ``[0, num_blocks)`` are skipped."""
    pool0, device, block_bytes = _record_pools(key_pools, value_pools)
    _require_gpu("records", records, device)
    _require_gpu("block_ids", block_ids, device)
    _require_index("block_ids", block_ids, 1)
    block_ids = block_ids.contiguous()
    shape = (block_ids.shape[0], len(key_pools), 2, *pool0.shape[1:])
    if tuple(records.shape) != shape or records.dtype != pool0.dtype or not records.is_contiguous():
        raise ValueError(f"records: expected contiguous {shape} {pool0.dtype}, got {tuple(records.shape)} "
                         f"{records.dtype}")
    if block_ids.shape[0] == 0:
        return
    _check_range("block_ids", block_ids, pool0.shape[0])
    rc = _native.load().mi_unpack_blocks(
        _native.pointer_array([t.data_ptr() for t in key_pools]),
        _native.pointer_array([t.data_ptr() for t in value_pools]), pool0.shape[0], records.data_ptr(),
        block_ids.data_ptr(), block_ids.shape[0], len(key_pools), block_bytes, _stream(device))
    _native.check(rc, "mi_unpack_blocks")
