"""Qwen3 with the paged-KV data plane in its attention.

Parameter names, shapes and the dense numerics (RMSNorm in fp32, bf16 RoPE tables, q/k norm,
SwiGLU, tied lm_head) follow the reference model (src/mini_infra/model/qwen3.py:55-625), so its
state_dict loads unchanged.  The attention differs in how it reaches K/V:

* decode (``PagedAttentionMetadata``, one token per sequence): q/k norm + RoPE, the append of the
  new K/V rows into their pool slots and paged GQA decode attention over the context in the pool
  -- one launch for small batches (the per-sequence kernel does the first two in its prologue),
  two for large ones (replaces qwen3.py:257-292 + :219-255, no gather, no repeat_interleave);
* prefill (``PagedPrefillMetadata``, or no metadata for a whole left-padded prompt): the MFMA
  chunked-prefill kernel attends causally within the chunk and reads the history straight from
  the pool through the block table (replaces the gather + concat + _attend chain);
* mixed (``PagedMixedMetadata``): prefill chunks and decode tokens in one forward, the batching
  the reference plans next (src/mini_infra/core/scheduler.py:310-311).  The GEMMs, norms and MLP
  run once over all tokens; q/k norm + RoPE and attention run in their prefill and decode forms
  on the two token ranges, writing one output buffer.

Dense GEMMs (projections, MLP, lm_head) stay on PyTorch-ROCm; the elementwise chains around them
run as fused launches of the same library (``data_plane.rms_norm`` with the residual add,
``qk_norm_rope`` with the decode append, ``silu_mul``), keeping the reference's bf16 rounding points.

Numerics (``Qwen3ForCausalLM(config, exact=...)``):

* ``exact=True`` (the default) is bit-identical to the reference op chain evaluated with exact
  sums (``oracle.qwen3_ref.ReferenceQwen3(exact=True)``): attention runs the reference-numerics
  kernels (the reference's rounding points, exact sums), RMSNorm sums exactly, and every GEMM is
  the call the reference makes -- q, k, v, gate and up as separate projections, since hipBLASLt's
  result for a row can depend on the GEMM's N and M.  Greedy decoding then reproduces the
  reference's tokens exactly.  (Running the separate projections of one input concurrently on
  side streams, fork and join captured in the step's HIP graph, measured slower on MI355X: decode
  steps 3.92 ms against 3.45 in the continuous-batching run.)
* ``exact=False`` runs the bandwidth kernels (fp32 online softmax, MFMA prefill) and q/k/v and
  gate/up each as one GEMM over row-concatenated weights (the outputs split as column views):
  within bf16 tolerance of the reference, not bit-identical.
"""

from __future__ import annotations

from typing import NamedTuple

import torch
import torch.nn.functional as F
from torch import nn

from mini_infra_qwen3_amd import data_plane
from mini_infra_qwen3_amd.model.config import Qwen3Config

PastKeyValue = tuple[torch.Tensor, torch.Tensor]


class PagedAttentionMetadata(NamedTuple):
    """Paged decode step addressing (reference qwen3.py:27-42).

    slot_mapping ``[B]``, block_tables ``[B, max_blocks]`` (null-padded), context_lens ``[B]`` (new
    token included) -- int64, possibly column views of one packed tensor; kv_pools per layer.
    ``table_rows`` (not in the reference): when given, ``block_tables`` is a persistent
    ``[rows, width]`` table matrix on the device and row b of the step uses its row
    ``table_rows[b]`` (the forward gathers them once).
    """

    slot_mapping: torch.Tensor
    block_tables: torch.Tensor
    context_lens: torch.Tensor
    kv_pools: tuple[PastKeyValue, ...] = ()
    table_rows: torch.Tensor | None = None


class PagedPrefillMetadata(NamedTuple):
    """Chunked-prefill addressing: row b is a left-padded chunk of ``chunk_lens[b]`` tokens that
    starts at logical position ``start_lens[b]``; its history is the first ``start_lens[b]`` slots of
    ``history_block_tables[b]`` (``[B, nb]`` int64, null-padded; ``nb`` may be 0)."""

    history_block_tables: torch.Tensor
    start_lens: torch.Tensor
    chunk_lens: torch.Tensor
    kv_pools: tuple[PastKeyValue, ...] = ()
    # optional per-layer (K, V) buffers, contiguous [B * L, H_kv, D], that receive the chunk's K/V
    # (the present) instead of new allocations
    kv_out: tuple[PastKeyValue, ...] = ()
    # optional [B, L] int64: the pool slot of each padded position's token (-1: none).  The chunk's
    # K/V rows then also go straight into the pool (the reference's later store_prefill, when the
    # block tables already cover the chunk: src/mini_infra/worker/paged_runner.py:49,104-136)
    slot_mapping: torch.Tensor | None = None


class PagedMixedMetadata(NamedTuple):
    """A mixed chunk + decode step over a flattened ``[1, T]`` batch, T = C + D: tokens ``[0, C)``
    are the ``prefill_rows`` (P) chunk rows addressed by ``prefill``, the last D tokens one new token
    per decoding sequence, addressed by ``decode``.  With ``chunk_first`` (``[P]``, ragged rows) row
    b's tokens are tokens ``chunk_first[b]`` .. of ``[0, chunk_tokens)`` (pad tokens may follow the
    rows), and the attention sees each row left-padded to ``prefill_width`` (at least every chunk
    length).  Without it, C = P L with L = ``prefill_width``: row b is tokens ``[b L, b L + L)``,
    left-padded.  ``prefill.kv_out`` (optional) holds per-layer ``[T, H_kv, D]`` buffers for all T
    tokens' K/V.  Host-side facts of the step for its caller (the forward ignores them):
    ``live_decode_rows``, how many of the D decode rows are real (the rest pad; None: all), and
    ``chunk_first_host``, ``chunk_first`` as host integers."""

    prefill: PagedPrefillMetadata
    decode: PagedAttentionMetadata
    prefill_rows: int
    prefill_width: int
    kv_pools: tuple[PastKeyValue, ...] = ()
    chunk_first: torch.Tensor | None = None
    chunk_tokens: int = 0
    live_decode_rows: int | None = None
    chunk_first_host: tuple[int, ...] | None = None

    @property
    def chunk_span(self) -> int:
        """C: the tokens of the chunk rows (ragged or padded)."""
        return self.chunk_tokens if self.chunk_first is not None else self.prefill_rows * self.prefill_width


class RMSNorm(nn.Module):
    """RMSNorm weight holder (reference qwen3.py:55-78).  The norm itself runs fused with the
    preceding residual add in ``data_plane.rms_norm`` (fp32 inside, reference rounding points)."""

    def __init__(self, hidden_size: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """(normed, x + residual): the normalised input of the next block and the new residual."""
        return data_plane.rms_norm(x, self.weight, self.eps, residual)


class RotaryEmbedding(nn.Module):
    """cos / sin tables for positions, fp32 angles cast to the model dtype (reference qwen3.py:81-109)."""

    def __init__(self, head_dim: int, rope_theta: float):
        super().__init__()
        self.head_dim = head_dim
        self.rope_theta = rope_theta
        self.register_buffer("inv_freq", self._frequencies("cpu"), persistent=False)

    def _frequencies(self, device) -> torch.Tensor:
        exponents = torch.arange(0, self.head_dim, 2, dtype=torch.float32, device=device) / self.head_dim
        return 1.0 / (self.rope_theta ** exponents)

    def _apply(self, fn, *args, **kwargs):
        # The frequencies stay fp32 whatever dtype the model is cast to: a bf16 inv_freq moves the
        # angles of late positions by whole radians (the reference loader restores the fp32 buffer
        # after model.to(dtype): src/mini_infra/model/loader.py:65-68).
        super()._apply(fn, *args, **kwargs)
        self.inv_freq = self._frequencies(self.inv_freq.device)
        return self

    def forward(self, position_ids: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        freqs = position_ids.float().unsqueeze(-1) * self.inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(dtype), emb.sin().to(dtype)


def _concat_weight(owner: nn.Module, linears: tuple[nn.Linear, ...]) -> torch.Tensor:
    """Row-concatenated weights of bias-free linears that read the same input, so their
    projections run as one GEMM (one launch) whose output columns are views of each.  Cached on
    the owner and rebuilt when any weight moves or is modified in place (storage or version)."""
    key = tuple((l.weight.data_ptr(), l.weight._version, l.weight.dtype) for l in linears)
    cached = owner.__dict__.get("_concat_cache")
    if cached is None or cached[0] != key:
        with torch.no_grad():
            fused = torch.cat([l.weight for l in linears], dim=0)
        owner.__dict__["_concat_cache"] = (key, fused)
        return fused
    return cached[1]


class Qwen3Attention(nn.Module):
    def __init__(self, config: Qwen3Config, exact: bool = True):
        super().__init__()
        self.exact = exact
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.scaling = config.head_dim ** -0.5
        self.q_proj = nn.Linear(config.hidden_size, self.num_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(config.hidden_size, self.num_kv_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(config.hidden_size, self.num_kv_heads * self.head_dim, bias=False)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, config.hidden_size, bias=False)
        self.q_norm = RMSNorm(config.head_dim, config.rms_norm_eps)
        self.k_norm = RMSNorm(config.head_dim, config.rms_norm_eps)

    def forward(self, hidden, cos, sin, kv_pool: PastKeyValue, metadata, workspace=None, kv_out=None):
        """q/k/v projections (one PyTorch GEMM over the concatenated weights), then one fused launch for q/k RMSNorm + RoPE (plus,
        when decoding, the K/V append into the pool), then paged attention."""
        batch, length, _ = hidden.shape
        nq, nkv = self.num_heads * self.head_dim, self.num_kv_heads * self.head_dim
        if self.exact:
            q, k, v = self.q_proj(hidden), self.k_proj(hidden), self.v_proj(hidden)
        else:
            qkv = F.linear(hidden, _concat_weight(self, (self.q_proj, self.k_proj, self.v_proj)))
            q, k, v = qkv[..., :nq], qkv[..., nq:nq + nkv], qkv[..., nq + nkv:]
        key_pool, value_pool = kv_pool
        eps = self.q_norm.eps
        if isinstance(metadata, PagedMixedMetadata):
            return self._mixed(q[0], k[0], v[0], cos[0], sin[0], kv_pool, metadata, workspace, kv_out)
        if isinstance(metadata, PagedAttentionMetadata):
            out = data_plane.paged_decode_attention_fused(
                q, k, v, self.q_norm.weight, self.k_norm.weight, cos, sin, eps, metadata.slot_mapping, key_pool,
                value_pool, metadata.block_tables, metadata.context_lens, self.scaling, workspace=workspace,
                exact=self.exact,
            ).view(batch, 1, -1)
            present = kv_pool
        else:
            k_buf, v_buf = kv_out if kv_out is not None else (None, None)
            slots = metadata.slot_mapping
            q_rot, k_rot, v_rows = data_plane.qk_norm_rope(
                q, k, v, self.q_norm.weight, self.k_norm.weight, cos, sin, eps,
                slot_mapping=None if slots is None else slots.reshape(-1), key_pool=key_pool, value_pool=value_pool,
                k_out=k_buf, v_out=v_buf, rows=True)
            # token-major [B, L, H, D] buffers seen as [B, H, L, D] (strided views, no copies)
            q_rot = q_rot.view(batch, length, self.num_heads, self.head_dim).transpose(1, 2)
            k_rot = k_rot.view(batch, length, self.num_kv_heads, self.head_dim).transpose(1, 2)
            v_rows = v_rows.view(batch, length, self.num_kv_heads, self.head_dim).transpose(1, 2)
            out = data_plane.chunked_prefill_attention(
                q_rot, k_rot, v_rows, key_pool, value_pool, metadata.history_block_tables, metadata.start_lens,
                metadata.chunk_lens, self.scaling, exact=self.exact,
            )
            present = (k_rot, v_rows)
        return self.o_proj(out), present

    def _mixed(self, q, k, v, cos, sin, kv_pool: PastKeyValue, metadata: PagedMixedMetadata, workspace, kv_out=None):
        """One q/k norm + RoPE launch over all T tokens, then one attention launch for the chunk rows
        (tokens ``[0, C)``) and the decode rows (the rest), which also appends the decode tokens'
        K/V to the pool.  ``kv_out`` (optional): ``[T, H_kv, D]`` buffers for the rotated K / V.  The
        chunk K/V come back as ``[P, H_kv, L, D]`` rows, or for ragged rows as one ``[1, H_kv, C, D]``
        row."""
        key_pool, value_pool = kv_pool
        rows, width = metadata.prefill_rows, metadata.prefill_width
        n = metadata.chunk_span
        k_buf, v_buf = kv_out if kv_out is not None else (None, None)
        q_rot, k_rot, v_rows = data_plane.qk_norm_rope(q, k, v, self.q_norm.weight, self.k_norm.weight, cos, sin,
                                                       self.q_norm.eps, k_out=k_buf, v_out=v_buf)
        prefill, decode = metadata.prefill, metadata.decode
        out = data_plane.mixed_paged_attention(
            q_rot, k_rot, v_rows, key_pool, value_pool, rows, width, prefill.history_block_tables, prefill.start_lens,
            prefill.chunk_lens, decode.block_tables, decode.context_lens, decode.slot_mapping, self.scaling,
            exact=self.exact, chunk_first=metadata.chunk_first, chunk_tokens=n)
        per_row = (1, n) if metadata.chunk_first is not None else (rows, width)
        k_chunk = k_rot[:n].view(*per_row, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v_chunk = v_rows[:n].view(*per_row, self.num_kv_heads, self.head_dim).transpose(1, 2)
        return self.o_proj(out.unsqueeze(0)), (k_chunk, v_chunk)


class Qwen3MLP(nn.Module):
    def __init__(self, config: Qwen3Config, exact: bool = True):
        super().__init__()
        self.exact = exact
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.exact:
            return self.down_proj(data_plane.silu_mul(self.gate_proj(x), self.up_proj(x)))
        inter = self.gate_proj.out_features
        gate_up = F.linear(x, _concat_weight(self, (self.gate_proj, self.up_proj)))
        return self.down_proj(data_plane.silu_mul(gate_up[..., :inter], gate_up[..., inter:]))


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, config: Qwen3Config, exact: bool = True):
        super().__init__()
        self.self_attn = Qwen3Attention(config, exact)
        self.mlp = Qwen3MLP(config, exact)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, hidden, residual, cos, sin, kv_pool, metadata, workspace=None, kv_out=None):
        """Pre-norm block in residual-stream form: takes the previous block's output and the
        residual before it (None for the first layer), returns the MLP output and the residual
        (the reference's hidden state is their sum, formed by the next norm's fused add)."""
        x, residual = self.input_layernorm(hidden, residual)
        attn, present = self.self_attn(x, cos, sin, kv_pool, metadata, workspace, kv_out)
        x, residual = self.post_attention_layernorm(attn, residual)
        return self.mlp(x), residual, present


class Qwen3Model(nn.Module):
    def __init__(self, config: Qwen3Config, exact: bool = True):
        super().__init__()
        config.validate()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([Qwen3DecoderLayer(config, exact) for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(config.head_dim, config.rope_theta)
        # Stand-in pool for prefill without history (the kernel reads no pool rows then).
        self.register_buffer(
            "_empty_pool", torch.zeros(1, 16, config.num_key_value_heads, config.head_dim), persistent=False
        )

    def forward(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
                position_ids: torch.Tensor | None = None,
                attn_metadata: PagedAttentionMetadata | PagedPrefillMetadata | PagedMixedMetadata | None = None,
                last_only: bool = False):
        """Returns (final hidden states ``[B, L, hidden]``, or ``[B, 1, hidden]`` of the last position
        with ``last_only``, and the per-layer present K/V).

        Decode (``PagedAttentionMetadata``): input_ids / position_ids ``[B, 1]``.  Prefill: a
        left-padded ``[B, L]`` chunk; without metadata, ``attention_mask`` (left padding, True on
        real tokens) gives the chunk lengths and there is no history.  Mixed (``PagedMixedMetadata``):
        ``[1, P L + D]``; with ``last_only`` the rows are the P chunks' last positions, then the D
        decode tokens (``[P + D, 1, hidden]``), and the present K/V are the chunks'.
        """
        if input_ids.ndim != 2 or input_ids.shape[1] < 1:
            raise ValueError("input_ids must be a non-empty [batch, sequence] tensor")
        batch, length = input_ids.shape
        device = input_ids.device
        hidden = self.embed_tokens(input_ids)
        workspace = None
        if isinstance(attn_metadata, PagedMixedMetadata):
            metadata = attn_metadata
            pools = metadata.kv_pools
            rows = metadata.prefill_rows
            decode_rows = metadata.decode.slot_mapping.shape[0]
            if batch != 1 or length != metadata.chunk_span + decode_rows or rows < 1 or decode_rows < 1:
                raise ValueError(f"mixed step takes input_ids [1, C + D] with P, D >= 1, got {tuple(input_ids.shape)}")
            if position_ids is None:
                raise ValueError("a mixed step needs position_ids")
            if len(pools) != len(self.layers):
                raise ValueError("kv_pools has a different number of layers than the model")
            need = data_plane.paged_decode_workspace_bytes(decode_rows, metadata.decode.block_tables.shape[1],
                                                          self.config.num_attention_heads, self.config.head_dim,
                                                          pools[0][0].shape[1], self.config.num_key_value_heads)
            if need:
                workspace = torch.empty(need, dtype=torch.uint8, device=device)
        elif isinstance(attn_metadata, PagedAttentionMetadata):
            if length != 1:
                raise ValueError("paged decode takes input_ids of shape [batch, 1]")
            if position_ids is None:
                raise ValueError("paged decode needs position_ids")
            if len(attn_metadata.kv_pools) != len(self.layers):
                raise ValueError("kv_pools has a different number of layers than the model")
            metadata = attn_metadata
            if metadata.table_rows is not None:  # this step's rows of the persistent table matrix
                metadata = metadata._replace(block_tables=metadata.block_tables.index_select(0, metadata.table_rows),
                                             table_rows=None)
            pools = attn_metadata.kv_pools
            # one buffer serves either decode form: the bandwidth kernel's split-context partials or
            # the reference-numerics kernel's split form
            need = max(data_plane.paged_decode_workspace_bytes(batch, metadata.block_tables.shape[1],
                                                              self.config.num_attention_heads, self.config.head_dim,
                                                              pools[0][0].shape[1], self.config.num_key_value_heads),
                       data_plane.paged_decode_exact_workspace_bytes(batch, metadata.block_tables.shape[1],
                                                                     self.config.num_attention_heads,
                                                                     self.config.num_key_value_heads,
                                                                     pools[0][0].shape[1]))
            if need:
                workspace = torch.empty(need, dtype=torch.uint8, device=device)
        else:
            if attn_metadata is None:
                if attention_mask is None:
                    chunk_lens = torch.full((batch,), length, dtype=torch.long, device=device)
                else:
                    chunk_lens = attention_mask.to(device=device).long().sum(dim=-1)
                pool = self._empty_pool.to(hidden.dtype)
                metadata = PagedPrefillMetadata(torch.zeros((batch, 0), dtype=torch.long, device=device),
                                                torch.zeros(batch, dtype=torch.long, device=device), chunk_lens)
                pools = tuple((pool, pool) for _ in self.layers)
            elif isinstance(attn_metadata, PagedPrefillMetadata):
                metadata = attn_metadata
                pools = attn_metadata.kv_pools
                if len(pools) != len(self.layers):
                    raise ValueError("kv_pools has a different number of layers than the model")
            else:
                raise NotImplementedError(f"{type(attn_metadata).__name__}: only the paged path is built here")
            if position_ids is None:  # real tokens count from start, left padding sits at position 0
                offset = torch.arange(length, device=device).unsqueeze(0) - (length - metadata.chunk_lens).unsqueeze(1)
                position_ids = torch.where(offset >= 0, offset + metadata.start_lens.unsqueeze(1), 0)
        cos, sin = self.rotary_emb(position_ids, hidden.dtype)
        presents: list[PastKeyValue] = []
        residual = None
        holder = metadata.prefill if isinstance(metadata, PagedMixedMetadata) else metadata
        kv_outs = getattr(holder, "kv_out", ()) or (None,) * len(self.layers)
        for layer, kv_pool, kv_out in zip(self.layers, pools, kv_outs):
            hidden, residual, present = layer(hidden, residual, cos, sin, kv_pool, metadata, workspace, kv_out)
            presents.append(present)
        if last_only and isinstance(metadata, PagedMixedMetadata):
            n = metadata.chunk_span
            if metadata.chunk_first is not None:  # each ragged row's last token
                # clamped like the attention clamps a row's first token: a row of length 0 (the
                # zero-filled buffer a mixed graph is captured over) reads token 0, and no sampler
                # reads its logit
                last = (metadata.chunk_first + metadata.prefill.chunk_lens - 1).clamp(0, max(n - 1, 0))
                hidden = torch.cat((hidden[0].index_select(0, last), hidden[0, n:])).unsqueeze(1)
                residual = torch.cat((residual[0].index_select(0, last), residual[0, n:])).unsqueeze(1)
            else:
                width = metadata.prefill_width
                hidden = torch.cat((hidden[0, width - 1:n:width], hidden[0, n:])).unsqueeze(1)
                residual = torch.cat((residual[0, width - 1:n:width], residual[0, n:])).unsqueeze(1)
        elif last_only:  # the norm is row-wise: only the position the sampler reads
            hidden, residual = hidden[:, -1:, :], residual[:, -1:, :]
        return self.norm(hidden, residual)[0], presents


class Qwen3ForCausalLM(nn.Module):
    def __init__(self, config: Qwen3Config, exact: bool = True):
        """``exact``: reference numerics (bit-identical to the reference op chain with exact sums;
        the reference's GEMM calls); ``False``: the bandwidth kernels and fused GEMMs."""
        super().__init__()
        self.config = config
        self.model = Qwen3Model(config, exact)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    @property
    def exact(self) -> bool:
        return self.model.layers[0].self_attn.exact if len(self.model.layers) else True

    def set_exact(self, exact: bool) -> "Qwen3ForCausalLM":
        """Switches every layer between reference numerics and the bandwidth kernels (same weights)."""
        for layer in self.model.layers:
            layer.self_attn.exact = exact
            layer.mlp.exact = exact
        return self

    def forward(self, input_ids, attention_mask=None, position_ids=None, attn_metadata=None,
                last_logits_only: bool = False):
        """(logits, present K/V).  ``last_logits_only`` projects only the last position (``[B, 1, V]``):
        greedy sampling reads nothing else (reference sampler.py:9-23)."""
        hidden, presents = self.model(input_ids, attention_mask, position_ids, attn_metadata, last_logits_only)
        return self.lm_head(hidden), presents


def init_random_(model: Qwen3ForCausalLM, seed: int, std: float = 0.02, untied_head_seed: int | None = None) -> None:
    """Random weights: every matrix N(0, std) from one seeded generator, norms at 1.  With
    ``untied_head_seed`` the lm_head gets its own N(0, 1) draw (a model whose greedy output depends
    on the context, as the reference's diverse test model: tests/unit/conftest.py:13-25)."""
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.fill_(1.0)
            else:
                p.copy_(torch.randn(p.shape, generator=gen) * std)
        if untied_head_seed is not None:
            head_gen = torch.Generator().manual_seed(untied_head_seed)
            model.lm_head.weight = nn.Parameter(
                torch.randn(model.lm_head.weight.shape, generator=head_gen).to(model.lm_head.weight.device,
                                                                               model.lm_head.weight.dtype))


__all__ = [
    "PagedAttentionMetadata",
    "PagedMixedMetadata",
    "PagedPrefillMetadata",
    "Qwen3Attention",
    "Qwen3ForCausalLM",
    "Qwen3Model",
    "init_random_",
]
