"""Writes golden vectors of the reference's bf16 torch path (run with the reference importable).

    python tests/golden/make_golden.py [reference src dir, default /root/reference/src]

What only running the reference pins: the bits of its bf16 attention (scores, bf16 scale product,
fp32 softmax cast back, bf16 PV: src/mini_infra/model/qwen3.py:219-255) and of its Qwen3 forward,
paged decode and chunked-prefill runner path (src/mini_infra/worker/paged_runner.py:32-189) on
this machine's torch, CPU.  Inputs come from tests/golden/recipe.py; outputs go to
reference_bf16.safetensors (tensors) and reference_bf16.json (tokens, pool digests, versions).
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import recipe  # noqa: E402


def pool_digest(pool) -> list[str]:
    return [hashlib.sha256(torch.stack([k, v]).view(torch.int16).numpy().tobytes()).hexdigest()
            for k, v in pool.kv_pools]


def main(src: str) -> None:
    sys.path.insert(0, src)
    from mini_infra.core import KVCacheManager
    from mini_infra.model import Qwen3Config, Qwen3ForCausalLM
    from mini_infra.worker import PagedKVCachePool, PagedRunner

    cfg = Qwen3Config(**recipe.CONFIG, torch_dtype="bfloat16", tie_word_embeddings=True)
    model = Qwen3ForCausalLM(cfg)
    shapes = {n: tuple(p.shape) for n, p in model.state_dict().items()}
    weights = recipe.state_dict(shapes)
    inv_freq = model.model.rotary_emb.inv_freq.clone()
    model = model.to(torch.bfloat16)
    model.model.rotary_emb.inv_freq = inv_freq  # fp32, as the reference loader keeps it
    model.lm_head.weight = torch.nn.Parameter(torch.empty_like(model.lm_head.weight))  # untie
    model.load_state_dict(weights)
    model.eval()
    tensors, meta = {}, {"torch": torch.__version__, "config": recipe.CONFIG}

    with torch.inference_mode():
        attn = model.model.layers[0].self_attn
        tensors["attend_decode_out"] = attn._attend(*recipe.attend_decode_inputs()).contiguous()
        tensors["attend_prefill_out"] = attn._attend(*recipe.attend_prefill_inputs()).contiguous()

        # whole-prompt prefill + paged decode
        runner = PagedRunner(model)
        prompts = recipe.prompts(recipe.PREFILL_PROMPT_LENS, "prefill_prompts")
        manager = KVCacheManager(recipe.BLOCK_SIZE, 24)
        pool = PagedKVCachePool(cfg.num_hidden_layers, 24, recipe.BLOCK_SIZE, cfg.num_key_value_heads, cfg.head_dim,
                                torch.bfloat16, torch.device("cpu"))
        for i, p in enumerate(prompts):
            manager.allocate_slots(i, len(p))
        tables = [manager.block_table(i) for i in range(len(prompts))]
        out = runner.run_prefill_step(prompts)
        runner.store_prefill(pool, out.prefill_cache, tables, [len(p) for p in prompts], [0] * len(prompts))
        meta["prefill_tokens"] = out.next_tokens
        meta["prefill_tables"] = tables
        tokens, lengths, logits = list(out.next_tokens), [len(p) for p in prompts], []
        meta["decode_tokens"] = []
        for _ in range(recipe.DECODE_STEPS):
            for i in range(len(prompts)):
                manager.allocate_slots(i, 1)
            tables = [manager.block_table(i) for i in range(len(prompts))]
            ids, pos, md = runner.prepare_decode_inputs(tables, tokens, lengths, recipe.BLOCK_SIZE)
            step_logits, _ = model(ids, position_ids=pos, attn_metadata=md._replace(kv_pools=tuple(pool.kv_pools)))
            logits.append(step_logits[:, -1])
            tokens = step_logits[:, -1].argmax(-1).tolist()
            lengths = [n + 1 for n in lengths]
            meta["decode_tokens"].append(tokens)
        meta["decode_tables"] = tables
        tensors["decode_logits"] = torch.stack(logits).contiguous()
        meta["decode_pool_sha256"] = pool_digest(pool)

        # chunked prefill with history, two rounds
        prompts = recipe.prompts(recipe.CHUNK_PROMPT_LENS, "chunk_prompts")
        manager = KVCacheManager(recipe.BLOCK_SIZE, 16)
        pool = PagedKVCachePool(cfg.num_hidden_layers, 16, recipe.BLOCK_SIZE, cfg.num_key_value_heads, cfg.head_dim,
                                torch.bfloat16, torch.device("cpu"))
        manager.allocate_slots(7, 20)  # another request's block first
        for i, p in enumerate(prompts):
            manager.allocate_slots(i, len(p))
        tables = [manager.block_table(i) for i in range(len(prompts))]
        meta["chunk_tables"] = tables
        meta["chunk_tokens"] = []
        for starts, ends in (([0, 0], recipe.CHUNK_CUTS), (recipe.CHUNK_CUTS, [len(p) for p in prompts])):
            chunks = [p[s:e] for p, s, e in zip(prompts, starts, ends)]
            out = runner.run_prefill_chunk_step(chunks, starts, tables, pool)
            runner.store_prefill(pool, out.prefill_cache, tables, [e - s for s, e in zip(starts, ends)], starts)
            meta["chunk_tokens"].append(out.next_tokens)
        meta["chunk_pool_sha256"] = pool_digest(pool)

    save_file(tensors, str(HERE / "reference_bf16.safetensors"))
    (HERE / "reference_bf16.json").write_text(json.dumps(meta, indent=1) + "\n")
    print({k: tuple(v.shape) for k, v in tensors.items()}, meta["prefill_tokens"], meta["chunk_tokens"])


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
