"""The oracle against golden vectors written by running the reference's own bf16 torch path
(tests/golden/make_golden.py): attention, whole-prompt prefill, paged decode and chunked prefill
with history, bit for bit on this machine's torch (CPU)."""

import hashlib
import json
import sys
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

from mini_infra_qwen3_amd.core import KVCacheManager
from mini_infra_qwen3_amd.model import Qwen3Config, Qwen3ForCausalLM
from oracle import qwen3_ref, torch_ref

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import recipe  # noqa: E402


@pytest.fixture(scope="module")
def golden():
    return load_file(str(GOLDEN / "reference_bf16.safetensors")), json.loads((GOLDEN / "reference_bf16.json").read_text())


@pytest.fixture(scope="module")
def model():
    cfg = Qwen3Config(**recipe.CONFIG, tie_word_embeddings=False)
    shapes = {n: tuple(p.shape) for n, p in Qwen3ForCausalLM(cfg).state_dict().items()}
    return qwen3_ref.ReferenceQwen3(cfg, recipe.state_dict(shapes))


def digest(pools):
    return [hashlib.sha256(torch.stack([k, v]).view(torch.int16).numpy().tobytes()).hexdigest() for k, v in pools]


def test_attention_bits(golden):
    tensors, _ = golden
    scale = 128 ** -0.5
    assert torch.equal(torch_ref.attend(*recipe.attend_decode_inputs(), scale), tensors["attend_decode_out"])
    assert torch.equal(torch_ref.attend(*recipe.attend_prefill_inputs(), scale), tensors["attend_prefill_out"])


def test_prefill_and_paged_decode_bits(golden, model):
    tensors, meta = golden
    prompts = recipe.prompts(recipe.PREFILL_PROMPT_LENS, "prefill_prompts")
    manager = KVCacheManager(recipe.BLOCK_SIZE, 24)
    for i, p in enumerate(prompts):
        manager.allocate_slots(i, len(p))
    tables = [manager.block_table(i) for i in range(len(prompts))]
    assert tables == meta["prefill_tables"]
    pools = torch_ref.make_pools(2, 24, recipe.BLOCK_SIZE, 8, 128)
    tokens, presents = qwen3_ref.prefill(model, prompts)
    assert tokens == meta["prefill_tokens"]
    qwen3_ref.store_prefill(pools, presents, tables, [len(p) for p in prompts], [0] * 3, recipe.BLOCK_SIZE)
    lengths = [len(p) for p in prompts]
    for step in range(recipe.DECODE_STEPS):
        for i in range(3):
            manager.allocate_slots(i, 1)
        tables = [manager.block_table(i) for i in range(3)]
        logits = qwen3_ref.decode_step(model, tables, tokens, lengths, pools, recipe.BLOCK_SIZE)
        assert torch.equal(logits, tensors["decode_logits"][step]), f"step {step}"
        tokens = logits.argmax(-1).tolist()
        assert tokens == meta["decode_tokens"][step]
        lengths = [n + 1 for n in lengths]
    assert digest(pools) == meta["decode_pool_sha256"]


def test_chunked_prefill_bits(golden, model):
    _, meta = golden
    prompts = recipe.prompts(recipe.CHUNK_PROMPT_LENS, "chunk_prompts")
    tables = meta["chunk_tables"]
    pools = torch_ref.make_pools(2, 16, recipe.BLOCK_SIZE, 8, 128)
    for k, (starts, ends) in enumerate((([0, 0], recipe.CHUNK_CUTS), (recipe.CHUNK_CUTS, [len(p) for p in prompts]))):
        chunks = [p[s:e] for p, s, e in zip(prompts, starts, ends)]
        tokens, presents = qwen3_ref.prefill_chunk_step(model, chunks, starts, tables, pools, recipe.BLOCK_SIZE)
        qwen3_ref.store_prefill(pools, presents, tables, [e - s for s, e in zip(starts, ends)], starts,
                                recipe.BLOCK_SIZE)
        assert tokens == meta["chunk_tokens"][k]
    assert digest(pools) == meta["chunk_pool_sha256"]


def test_a_planted_rounding_change_is_caught(golden):
    """Dropping the reference's bf16 rounding of the scores (fp32 scores instead) moves output bits."""
    tensors, _ = golden
    q, k, v, bias = recipe.attend_decode_inputs()
    kk = k.repeat_interleave(2, dim=1).float()
    scores = (q.float() @ kk.transpose(2, 3)) * 128 ** -0.5 + bias.float()
    probs = torch.softmax(scores, dim=-1).to(torch.bfloat16)
    out = (probs @ v.repeat_interleave(2, dim=1)).transpose(1, 2).reshape(2, 1, -1)
    assert not torch.equal(out, tensors["attend_decode_out"])
