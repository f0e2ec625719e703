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

    def __init__(self, config, state_dict: dict[str, torch.Tensor], device: str | torch.device = "cpu"):
        self.config = config
        self.w = {k: v.detach().to(device) for k, v in state_dict.items()}
        if "lm_head.weight" not in self.w:
            self.w["lm_head.weight"] = self.w["model.embed_tokens.weight"]
        self.device = torch.device(device)
        self.dtype = self.w["model.embed_tokens.weight"].dtype
        d = config.head_dim
        self.inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32, device=device) / d))

    # -- building blocks (qwen3.py:55-156) ---------------------------------------------------
    def _rms(self, x, weight):
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
    def forward(self, input_ids, attention_mask=None, position_ids=None, past_key_values=None, paged=None):
        """Returns (logits ``[B, L, V]``, presents).  ``paged``: dict(slot_mapping, block_tables,
        context_lens, kv_pools) for the decode path; otherwise ``past_key_values`` (per layer dense
        ``[B, Hkv, past, D]``, or None) with ``attention_mask`` over ``past + L``."""
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
            attn = torch_ref.attend(q, k, v, bias, scaling)
            h = h + F.linear(attn, self.w[p + "self_attn.o_proj.weight"])
            h = h + self._mlp(layer, self._rms(h, self.w[p + "post_attention_layernorm.weight"]))
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
                         pad_token_id: int = 0):
    """``run_prefill_chunk_step`` (paged_runner.py:32-102): gather history, mask, dense forward.
    Returns (last-position logits ``[B, V]``, per-layer K/V of history + chunk)."""
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
    logits, presents = model.forward(input_ids, attention_mask=mask, position_ids=position_ids, past_key_values=past)
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


class ReferenceScheduleBackend:
    """The reference's PagedScheduleBackend over this restatement
    (src/mini_infra/engine/paged_schedule_backend.py:70-128), for the continuous-batching loop.

    Pools live on ``model.device``.  With ``forced_tokens`` (request_idx -> token list) every step
    returns those tokens instead of its own greedy choice -- the run follows another backend's
    sequences -- and records, per produced token, ``(request_idx, forced, own argmax, logit gap,
    row std)`` where the gap is ``max logit - logit[forced]`` (0 when they agree) and the row std
    is the standard deviation of the row's logits (the scale of the gap).
    """

    def __init__(self, model: ReferenceQwen3, requests, max_running_requests: int, block_size: int = 16,
                 num_blocks: int | None = None, forced_tokens: dict | None = None):
        from mini_infra_qwen3_amd.core import KVCacheManager, required_pool_blocks

        c = model.config
        self.model = model
        self.device = model.device
        self.block_size = block_size
        num_blocks = num_blocks or required_pool_blocks(requests, max_running_requests, block_size)
        self.pools = torch_ref.make_pools(c.num_hidden_layers, num_blocks, block_size, c.num_key_value_heads,
                                          c.head_dim, dtype=model.dtype, device=model.device)
        self.kv_cache_manager = KVCacheManager(block_size, num_blocks)
        self.forced = forced_tokens
        self.records: list[tuple[int, int, int, float, float]] = []

    def _choose(self, request_ids, produced_index, logits):
        own = logits.argmax(-1).tolist()
        if self.forced is None:
            return own
        out = []
        for r, k, row, mine in zip(request_ids, produced_index, logits, own):
            token = self.forced[r][k]
            self.records.append((r, token, mine, float(row.max() - row[token]), float(row.std())))
            out.append(token)
        return out

    def execute_prefill(self, chunks):
        from mini_infra_qwen3_amd.engine import ScheduleStepOutput

        tables = [self.kv_cache_manager.block_table(ch.state.request.request_idx) for ch in chunks]
        starts = [ch.start for ch in chunks]
        lens = [ch.num_tokens for ch in chunks]
        logits, presents = prefill_chunk_logits(self.model, [ch.state.request.token_ids[ch.start:ch.end] for ch in chunks],
                                                starts, tables, self.pools, self.block_size)
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
        """A mixed step is, by definition, the decode step of ``states`` and the chunk step of
        ``chunks``: disjoint requests with disjoint blocks, so neither reads what the other writes.
        Runs both; tokens of the decode rows first, as the mixed step returns them."""
        from mini_infra_qwen3_amd.engine import ScheduleStepOutput

        decode = self.execute_decode(states)
        prefill = self.execute_prefill(chunks)
        return ScheduleStepOutput(decode.next_tokens + prefill.next_tokens, 0.0, 0.0, len(states) + len(chunks), 0)
