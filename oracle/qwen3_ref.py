"""CPU restatement of the reference's Qwen3 forward and PagedRunner (oracle; test infrastructure only).

Functional form over a state_dict with the reference's parameter names.  Follows
src/mini_infra/model/qwen3.py:55-625 (RMSNorm, RoPE, q/k norm, SwiGLU, dense-cache and paged
attention paths) and src/mini_infra/worker/paged_runner.py:32-189 (chunked prefill through
gather_blocks + concat, per-token store_prefill loop, packed decode metadata), op for op.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn.functional as F

from oracle import torch_ref


class ReferenceQwen3:
    """The reference model as functions of its weights (``config`` needs the Qwen3Config fields)."""

    def __init__(self, config, state_dict: dict[str, torch.Tensor], device: str | torch.device = "cpu",
                 exact: bool = False):
        """``exact``: RMSNorm and attention with exact sums at the reference's rounding points
        (``torch_ref.rms_norm_exact`` / ``attend_exact``) instead of ATen's fp32 sums -- the
        numerics of the HIP model; everything else is the same op chain."""
        self.config = config
        self.exact = exact
        self.w = {k: v.detach().to(device) for k, v in state_dict.items()}
        if "lm_head.weight" not in self.w:
            self.w["lm_head.weight"] = self.w["model.embed_tokens.weight"]
        self.device = torch.device(device)
        self.dtype = self.w["model.embed_tokens.weight"].dtype
        d = config.head_dim
        self.inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32, device=device) / d))

    # -- building blocks (qwen3.py:55-156) ---------------------------------------------------
    def _rms(self, x, weight):
        if self.exact:
            return torch_ref.rms_norm_exact(x, weight, self.config.rms_norm_eps)
        xf = x.float()
        normed = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.config.rms_norm_eps)
        return weight * normed.to(x.dtype)

    def _rope(self, position_ids):
        freqs = position_ids.float().unsqueeze(-1) * self.inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(self.dtype), emb.sin().to(self.dtype)

    @staticmethod
    def _rotate(x):
        half = x.shape[-1] // 2
        return torch.cat((-x[..., half:], x[..., :half]), dim=-1)

    def _qkv(self, layer, h, cos, sin):
        c = self.config
        p = f"model.layers.{layer}.self_attn."
        b, n, _ = h.shape
        q = F.linear(h, self.w[p + "q_proj.weight"]).view(b, n, c.num_attention_heads, c.head_dim)
        q = self._rms(q, self.w[p + "q_norm.weight"]).transpose(1, 2)
        k = F.linear(h, self.w[p + "k_proj.weight"]).view(b, n, c.num_key_value_heads, c.head_dim)
        k = self._rms(k, self.w[p + "k_norm.weight"]).transpose(1, 2)
        v = F.linear(h, self.w[p + "v_proj.weight"]).view(b, n, c.num_key_value_heads, c.head_dim).transpose(1, 2)
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
        return q * cos + self._rotate(q) * sin, k * cos + self._rotate(k) * sin, v

    def _mlp(self, layer, x):
        p = f"model.layers.{layer}.mlp."
        gate = F.silu(F.linear(x, self.w[p + "gate_proj.weight"]))
        return F.linear(gate * F.linear(x, self.w[p + "up_proj.weight"]), self.w[p + "down_proj.weight"])

    # -- forward (qwen3.py:438-625) ----------------------------------------------------------
    def forward(self, input_ids, attention_mask=None, position_ids=None, past_key_values=None, paged=None,
                last_only: bool = False):
        """Returns (logits ``[B, L, V]``, presents).  ``paged``: dict(slot_mapping, block_tables,
        context_lens, kv_pools) for the decode path; otherwise ``past_key_values`` (per layer dense
        ``[B, Hkv, past, D]``, or None) with ``attention_mask`` over ``past + L``.  ``last_only``:
        logits of the last position only (``[B, 1, V]``): the reference projects every position and
        samples the last (sampler.py:9-23); projecting that row alone is the same product, and the
        GEMM the HIP model issues."""
        c = self.config
        scaling = c.head_dim ** -0.5
        batch, length = input_ids.shape
        h = F.embedding(input_ids, self.w["model.embed_tokens.weight"])
        if paged is not None:
            bias = torch_ref.paged_bias(paged["block_tables"], paged["context_lens"],
                                        paged["kv_pools"][0][0].shape[1], self.dtype)
        else:
            past = 0 if past_key_values is None else past_key_values[0][0].shape[2]
            kv_len = past + length
            if attention_mask is None:
                attention_mask = torch.ones((batch, kv_len), dtype=torch.bool, device=self.device)
            if position_ids is None:
                position_ids = torch.arange(past, kv_len, device=self.device).unsqueeze(0).expand(batch, -1)
            qpos = torch.arange(past, kv_len, device=self.device)
            kpos = torch.arange(kv_len, device=self.device)
            allowed = (kpos.unsqueeze(0) <= qpos.unsqueeze(1)).view(1, 1, length, kv_len) \
                & attention_mask.bool().view(batch, 1, 1, kv_len)
            bias = torch.zeros(allowed.shape, dtype=self.dtype, device=self.device)
            bias.masked_fill_(~allowed, torch.finfo(self.dtype).min)
        cos, sin = self._rope(position_ids)
        presents = []
        for layer in range(c.num_hidden_layers):
            p = f"model.layers.{layer}."
            x = self._rms(h, self.w[p + "input_layernorm.weight"])
            q, k, v = self._qkv(layer, x, cos, sin)
            if paged is not None:
                k, v = torch_ref.apply_paged_kv_pool(k, v, paged["kv_pools"][layer], paged["slot_mapping"],
                                                     paged["block_tables"])
                presents.append(paged["kv_pools"][layer])
            else:
                if past_key_values is not None:
                    k = torch.cat((past_key_values[layer][0], k), dim=2)
                    v = torch.cat((past_key_values[layer][1], v), dim=2)
                presents.append((k, v))
            attn = (torch_ref.attend_exact if self.exact else torch_ref.attend)(q, k, v, bias, scaling)
            h = h + F.linear(attn, self.w[p + "self_attn.o_proj.weight"])
            h = h + self._mlp(layer, self._rms(h, self.w[p + "post_attention_layernorm.weight"]))
        if last_only:
            h = h[:, -1:]
        h = self._rms(h, self.w["model.norm.weight"])
        return F.linear(h, self.w["lm_head.weight"]), presents


def left_pad(prompts: Sequence[Sequence[int]], pad_token_id: int = 0, device="cpu"):
    """``_left_pad_sequences`` (src/mini_infra/worker/base_runner.py:26-60)."""
    width = max(len(p) for p in prompts)
    ids = torch.full((len(prompts), width), pad_token_id, dtype=torch.long, device=device)
    mask = torch.zeros((len(prompts), width), dtype=torch.bool, device=device)
    for i, p in enumerate(prompts):
        ids[i, width - len(p):] = torch.tensor(list(p), dtype=torch.long, device=device)
        mask[i, width - len(p):] = True
    pos = (mask.long().cumsum(-1) - 1).clamp_(min=0)
    return ids, mask, pos


def prefill(model: ReferenceQwen3, prompts, pad_token_id: int = 0):
    """Whole-prompt prefill (base_runner.py:63-79): (first tokens, per-layer K/V)."""
    ids, mask, pos = left_pad(prompts, pad_token_id, model.device)
    logits, presents = model.forward(ids, attention_mask=mask, position_ids=pos)
    return logits[:, -1].argmax(-1).tolist(), presents


def prefill_chunk_logits(model: ReferenceQwen3, chunk_token_ids, start_positions, block_tables, pools, block_size,
                         pad_token_id: int = 0, last_only: bool = False):
    """``run_prefill_chunk_step`` (paged_runner.py:32-102): gather history, mask, dense forward.
    Returns (last-position logits ``[B, V]``, per-layer K/V of history + chunk).  ``last_only``:
    project only the last position (see ``ReferenceQwen3.forward``)."""
    lens = [len(c) for c in chunk_token_ids]
    width = max(lens)
    hist = [-(-s // block_size) for s in start_positions]
    max_hist = max(hist)
    rows = [[pad_token_id] * (width - n) + list(ids) + [0] * (width - n) + list(range(s, s + n)) + [s, n]
            + list(t[:hb]) + [0] * (max_hist - hb)
            for ids, s, t, n, hb in zip(chunk_token_ids, start_positions, block_tables, lens, hist)]
    packed = torch.tensor(rows, dtype=torch.long, device=model.device)
    input_ids, position_ids = packed[:, :width], packed[:, width:2 * width]
    starts, chunk_len = packed[:, 2 * width:2 * width + 1], packed[:, 2 * width + 1:2 * width + 2]
    mask = torch.arange(width, device=model.device).unsqueeze(0) >= width - chunk_len
    past = None
    if max_hist:
        hpos = torch.arange(max_hist * block_size, device=model.device).unsqueeze(0)
        mask = torch.cat((hpos < starts, mask), dim=1)
        past = torch_ref.gather_blocks(pools, packed[:, 2 * width + 2:])
    logits, presents = model.forward(input_ids, attention_mask=mask, position_ids=position_ids, past_key_values=past,
                                     last_only=last_only)
    return logits[:, -1], presents


def prefill_chunk_step(model: ReferenceQwen3, chunk_token_ids, start_positions, block_tables, pools, block_size,
                       pad_token_id: int = 0):
    """``run_prefill_chunk_step``: (greedy tokens after each row's last position, per-layer K/V)."""
    logits, presents = prefill_chunk_logits(model, chunk_token_ids, start_positions, block_tables, pools, block_size,
                                            pad_token_id)
    return logits.argmax(-1).tolist(), presents


def store_prefill(pools, presents, block_tables, chunk_lens, start_positions, block_size):
    """``store_prefill`` (paged_runner.py:104-136): per-token slot loop, then write_prefill."""
    rows, positions, slots = torch_ref.store_prefill_indices(block_tables, chunk_lens, start_positions,
                                                             presents[0][0].shape[2], block_size)
    device = pools[0][0].device
    torch_ref.write_prefill(pools, presents, torch.tensor(rows, device=device), torch.tensor(positions, device=device),
                            torch.tensor(slots, device=device))


def decode_step(model: ReferenceQwen3, block_tables, last_tokens, positions, pools, block_size):
    """``prepare_decode_inputs`` + ``run_decode_step`` (paged_runner.py:138-189): logits ``[B, V]``."""
    packed = torch_ref.prepare_decode_rows(block_tables, last_tokens, positions, block_size).to(model.device)
    paged = {"slot_mapping": packed[:, 2], "block_tables": packed[:, 4:], "context_lens": packed[:, 3],
             "kv_pools": pools}
    logits, _ = model.forward(packed[:, 0:1], position_ids=packed[:, 1:2], paged=paged)
    return logits[:, -1]


def mixed_step_logits(model: ReferenceQwen3, chunk_token_ids, start_positions, chunk_tables, last_tokens, positions,
                      decode_tables, pools, block_size, pad_token_id: int = 0, chunk_tokens: int | None = None,
                      decode_rows: int | None = None):
    """A mixed step -- prompt chunks and decode tokens in one forward, the batching the reference
    plans next (src/mini_infra/core/scheduler.py:310-311) and does not define -- as the reference's
    ops over one flattened ``[1, C + D]`` batch: the P chunks' tokens back to back (ragged rows, no
    padding between them), then one token per decoding sequence as ``prepare_decode_inputs`` packs
    them.  Token-wise ops (embedding, norms, projections, MLP, lm_head) run once over all tokens;
    attention runs per segment: each chunk's as a chunk step's (history gathered from the pool,
    causal inside the chunk; the rows are laid out left-padded to the longest chunk L for it, the
    padding masked), the decode tokens' as a paged decode step's (append, then attend over the
    context), neither reading the other's blocks.  Returns (logits ``[P + D, V]`` of each chunk's
    last token then each decode token, the chunks' per-layer ``(K, V)`` ``[P, Hkv, L, D]``,
    left-padded as ``prefill_chunk_logits`` returns them).

    ``chunk_tokens`` / ``decode_rows`` (at least the chunks' tokens / the decode tokens) pad C and D:
    pad chunk tokens (token ``pad_token_id``, position 0) belong to no row; pad decode rows append
    nothing, attend to nothing (zero output) and return no logits; every op still runs over all
    C + D rows, so each GEMM has the padded M."""
    c = model.config
    dev = model.device
    scaling = c.head_dim ** -0.5
    rows, live = len(chunk_token_ids), len(last_tokens)
    lens = [len(t) for t in chunk_token_ids]
    width, total = max(lens), sum(lens)
    n = total if chunk_tokens is None else chunk_tokens
    decode_rows = live if decode_rows is None else decode_rows
    if n < total or decode_rows < live:
        raise ValueError(f"chunk_tokens {n} / decode_rows {decode_rows} below the step's {total} / {live}")
    first = [sum(lens[:r]) for r in range(rows)]
    ids = torch.full((n,), pad_token_id, dtype=torch.long)
    pos = torch.zeros((n,), dtype=torch.long)
    for toks, start, f in zip(chunk_token_ids, start_positions, first):
        ids[f:f + len(toks)] = torch.tensor(list(toks), dtype=torch.long)
        pos[f:f + len(toks)] = torch.arange(start, start + len(toks))
    # padded layout of the chunk rows: row r, position width - len + t <-> ragged token first[r] + t
    pad_rows = torch.tensor([r for r, l in enumerate(lens) for _ in range(l)], dtype=torch.long, device=dev)
    pad_cols = torch.tensor([width - l + t for l in lens for t in range(l)], dtype=torch.long, device=dev)
    hist = [-(-s // block_size) for s in start_positions]
    max_hist = max(hist)
    hist_ids = torch.zeros((rows, max_hist), dtype=torch.long)
    for r, (t, hb) in enumerate(zip(chunk_tables, hist)):
        hist_ids[r, :hb] = torch.tensor(list(t[:hb]), dtype=torch.long)
    dec = torch_ref.prepare_decode_rows(decode_tables, last_tokens, positions, block_size).to(dev)
    pad = torch.zeros(decode_rows - live, dtype=torch.long, device=dev)
    flat_ids = torch.cat((ids.to(dev), dec[:, 0], pad + pad_token_id)).unsqueeze(0)
    flat_pos = torch.cat((pos.to(dev), dec[:, 1], pad)).unsqueeze(0)
    # visibility of the chunk rows (history slots < start, causal inside the chunk, no left padding)
    allowed = torch_ref.chunk_allowed_mask(start_positions, lens, max_hist, block_size, width).to(dev)
    chunk_bias = torch.zeros(allowed.shape, dtype=model.dtype, device=dev)
    chunk_bias.masked_fill_(~allowed, torch.finfo(model.dtype).min)
    dec_bias = torch_ref.paged_bias(dec[:, 4:], dec[:, 3], block_size, model.dtype)
    attend = torch_ref.attend_exact if model.exact else torch_ref.attend

    def padded(x):  # [H, total, Dh] ragged -> [P, H, L, Dh] left-padded (zeros in the padding)
        out = torch.zeros((rows, width, x.shape[0], x.shape[2]), dtype=x.dtype, device=dev)
        out[pad_rows, pad_cols] = x.transpose(0, 1)
        return out.transpose(1, 2)

    h = F.embedding(flat_ids, model.w["model.embed_tokens.weight"])
    cos, sin = model._rope(flat_pos)
    presents = []
    for layer in range(c.num_hidden_layers):
        p = f"model.layers.{layer}."
        x = model._rms(h, model.w[p + "input_layernorm.weight"])
        q, k, v = model._qkv(layer, x, cos, sin)  # [1, H, T, D]
        qc, kc, vc = padded(q[0, :, :total]), padded(k[0, :, :total]), padded(v[0, :, :total])
        presents.append((kc, vc))
        if max_hist:
            (hk, hv), = torch_ref.gather_blocks([pools[layer]], hist_ids.to(dev))
            kc, vc = torch.cat((hk, kc), dim=2), torch.cat((hv, vc), dim=2)
        chunk_out = attend(qc.contiguous(), kc, vc, chunk_bias, scaling)  # [P, L, H D]
        qd = q[0, :, n:n + live].transpose(0, 1).unsqueeze(2)  # [D, H, 1, Dh]
        kd = k[0, :, n:n + live].transpose(0, 1).unsqueeze(2)
        vd = v[0, :, n:n + live].transpose(0, 1).unsqueeze(2)
        hk, hv = torch_ref.apply_paged_kv_pool(kd, vd, pools[layer], dec[:, 2], dec[:, 4:])
        dec_out = attend(qd.contiguous(), hk, hv, dec_bias, scaling)  # [D, 1, H D]
        zeros = torch.zeros((n - total + decode_rows - live, chunk_out.shape[-1]), dtype=chunk_out.dtype, device=dev)
        attn = torch.cat((chunk_out[pad_rows, pad_cols], zeros[:n - total], dec_out.reshape(live, -1),
                          zeros[n - total:])).unsqueeze(0)
        h = h + F.linear(attn, model.w[p + "self_attn.o_proj.weight"])
        h = h + model._mlp(layer, model._rms(h, model.w[p + "post_attention_layernorm.weight"]))
    ends = torch.tensor([f + l - 1 for f, l in zip(first, lens)], dtype=torch.long, device=dev)
    last = torch.cat((h[0].index_select(0, ends), h[0, n:])).unsqueeze(1)
    logits = F.linear(model._rms(last, model.w["model.norm.weight"]), model.w["lm_head.weight"])
    return logits[:rows + live, -1], presents


class ReferenceScheduleBackend:
    """The reference's PagedScheduleBackend over this restatement
    (src/mini_infra/engine/paged_schedule_backend.py:70-128), for the continuous-batching loop.

    Pools live on ``model.device``.  With ``forced_tokens`` (request_idx -> token list) every step
    returns those tokens instead of its own greedy choice -- the run follows another backend's
    sequences; with ``watch_tokens`` it keeps its own greedy choice and only compares.  Either way
    it records, per produced token, ``(request_idx, index, own argmax, other token, logit gap,
    row std)`` where the gap is ``max logit - logit[other]`` (0 when they agree, or tie exactly)
    and the row std is the standard deviation of the row's logits (the scale of the gap).
    """

    def __init__(self, model: ReferenceQwen3, requests, max_running_requests: int, block_size: int = 16,
                 num_blocks: int | None = None, forced_tokens: dict | None = None, watch_tokens: dict | None = None):
        from mini_infra_qwen3_amd.core import KVCacheManager, required_pool_blocks

        c = model.config
        self.model = model
        self.device = model.device
        self.block_size = block_size
        num_blocks = num_blocks or required_pool_blocks(requests, max_running_requests, block_size)
        self.pools = torch_ref.make_pools(c.num_hidden_layers, num_blocks, block_size, c.num_key_value_heads,
                                          c.head_dim, dtype=model.dtype, device=model.device)
        self.kv_cache_manager = KVCacheManager(block_size, num_blocks)
        if forced_tokens is not None and watch_tokens is not None:
            raise ValueError("forced_tokens and watch_tokens are exclusive")
        self.forced = forced_tokens
        self.watched = forced_tokens if forced_tokens is not None else watch_tokens
        self.records: list[tuple[int, int, int, int, float, float]] = []

    def _choose(self, request_ids, produced_index, logits):
        own = logits.argmax(-1).tolist()
        if self.watched is None:
            return own
        out = []
        for r, k, row, mine in zip(request_ids, produced_index, logits, own):
            seq = self.watched.get(r, [])
            other = seq[k] if k < len(seq) else -1
            gap = float(row.max() - row[other]) if other >= 0 else float("inf")
            self.records.append((r, k, mine, other, gap, float(row.std())))
            out.append(other if self.forced is not None else mine)
        return out

    def execute_prefill(self, chunks):
        from mini_infra_qwen3_amd.engine import ScheduleStepOutput

        tables = [self.kv_cache_manager.block_table(ch.state.request.request_idx) for ch in chunks]
        starts = [ch.start for ch in chunks]
        lens = [ch.num_tokens for ch in chunks]
        logits, presents = prefill_chunk_logits(self.model, [ch.state.request.token_ids[ch.start:ch.end] for ch in chunks],
                                                starts, tables, self.pools, self.block_size, last_only=True)
        store_prefill(self.pools, presents, tables, lens, starts, self.block_size)
        last = [i for i, ch in enumerate(chunks) if ch.is_last]
        tokens = self._choose([chunks[i].state.request.request_idx for i in last], [0] * len(last),
                              logits[last].float()) if last else []
        return ScheduleStepOutput(tokens, 0.0, 0.0, len(chunks), 0)

    def execute_decode(self, states):
        from mini_infra_qwen3_amd.engine import ScheduleStepOutput

        tables = [self.kv_cache_manager.block_table(s.request.request_idx) for s in states]
        logits = decode_step(self.model, tables, [s.generated[-1] for s in states],
                             [s.cache_length for s in states], self.pools, self.block_size).float()
        tokens = self._choose([s.request.request_idx for s in states], [len(s.generated) for s in states], logits)
        return ScheduleStepOutput(tokens, 0.0, 0.0, len(states), 0)

    def execute_mixed(self, states, chunks):
        """A mixed step (``mixed_step_logits``): the decode rows of ``states`` and the prompt chunks of
        ``chunks`` in one forward; tokens of the decode rows first, then those of the chunks that
        complete their prompt."""
        from mini_infra_qwen3_amd.engine import ScheduleStepOutput

        manager = self.kv_cache_manager
        tables = [manager.block_table(ch.state.request.request_idx) for ch in chunks]
        starts = [ch.start for ch in chunks]
        lens = [ch.num_tokens for ch in chunks]
        # With exact numerics a mixed step runs at a padded shape -- the chunks' tokens rounded up to
        # a multiple of 128, the decode rows to a power of two -- which fixes each GEMM's M.
        chunk_tokens = decode_rows = None
        if self.model.exact:
            chunk_tokens = -(-sum(lens) // 128) * 128
            decode_rows = 1 << (len(states) - 1).bit_length() if states else 0
        logits, presents = mixed_step_logits(
            self.model, [ch.state.request.token_ids[ch.start:ch.end] for ch in chunks], starts, tables,
            [s.generated[-1] for s in states], [s.cache_length for s in states],
            [manager.block_table(s.request.request_idx) for s in states], self.pools, self.block_size,
            chunk_tokens=chunk_tokens, decode_rows=decode_rows)
        store_prefill(self.pools, presents, tables, lens, starts, self.block_size)
        logits = logits.float()
        rows = len(chunks)
        dec = self._choose([s.request.request_idx for s in states], [len(s.generated) for s in states], logits[rows:])
        last = [i for i, ch in enumerate(chunks) if ch.is_last]
        pf = self._choose([chunks[i].state.request.request_idx for i in last], [0] * len(last),
                          logits[last]) if last else []
        return ScheduleStepOutput(dec + pf, 0.0, 0.0, len(states) + len(chunks), 0)
