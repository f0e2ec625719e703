"""Host-side model checks: config validation, parameter names, and the fp32 RoPE table."""

import pytest
import torch

from mini_infra_qwen3_amd.model import Qwen3Config, Qwen3ForCausalLM, qwen3_0_6b


def tiny():
    return Qwen3Config(vocab_size=100, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=32)


def test_rope_frequencies_stay_fp32_after_dtype_cast():
    """A bf16 inv_freq moves late-position angles by whole radians; the reference loader keeps it
    fp32 across model.to(dtype) (src/mini_infra/model/loader.py:65-68)."""
    model = Qwen3ForCausalLM(tiny()).to(torch.bfloat16)
    rope = model.model.rotary_emb
    assert rope.inv_freq.dtype == torch.float32
    want = 1.0 / (1e6 ** (torch.arange(0, 32, 2, dtype=torch.float32) / 32))  # rope_theta default 1e6
    torch.testing.assert_close(rope.inv_freq, want, rtol=0, atol=0)
    cos, _ = rope(torch.tensor([[40000]]), torch.bfloat16)
    angle = torch.tensor(40000.0) * want[1]
    assert abs(cos[0, 0, 1].float().item() - torch.cos(angle).item()) <= 8e-3


def test_parameter_names_match_reference_state_dict():
    """Same names as the reference Qwen3ForCausalLM (src/mini_infra/model/qwen3.py:295-625)."""
    names = set(Qwen3ForCausalLM(tiny()).state_dict())
    for want in ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight",
                 "model.layers.1.self_attn.q_proj.weight", "model.layers.1.self_attn.k_norm.weight",
                 "model.layers.0.mlp.down_proj.weight", "model.layers.0.post_attention_layernorm.weight"):
        assert want in names
    assert not any("inv_freq" in n or "_empty_pool" in n for n in names)


def test_qwen3_0_6b_shape():
    c = qwen3_0_6b()
    assert (c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads, c.head_dim) == (28, 16, 8, 128)
    assert (c.hidden_size, c.intermediate_size, c.vocab_size) == (1024, 3072, 151936)
    assert c.tie_word_embeddings


def test_config_rejects_indivisible_heads():
    with pytest.raises(ValueError):
        Qwen3Config(vocab_size=10, hidden_size=16, intermediate_size=16, num_hidden_layers=1,
                    num_attention_heads=3, num_key_value_heads=2, head_dim=8).validate()


def test_set_exact_switches_every_layer_and_fused_weights_follow_the_linears():
    """``set_exact`` flips both numerics flags of every layer; the bandwidth form's concatenated
    q/k/v weight is cached and rebuilt when a projection's weight changes in place."""
    from mini_infra_qwen3_amd.model.qwen3 import _concat_weight

    model = Qwen3ForCausalLM(tiny())
    assert model.exact
    assert model.set_exact(False) is model and not model.exact
    assert all(not layer.self_attn.exact and not layer.mlp.exact for layer in model.model.layers)
    attn = model.model.layers[0].self_attn
    linears = (attn.q_proj, attn.k_proj, attn.v_proj)
    fused = _concat_weight(attn, linears)
    assert _concat_weight(attn, linears) is fused
    assert torch.equal(fused, torch.cat([l.weight for l in linears]))
    with torch.no_grad():
        attn.k_proj.weight.add_(1.0)
    rebuilt = _concat_weight(attn, linears)
    nq = attn.q_proj.out_features
    assert rebuilt is not fused and torch.equal(rebuilt[nq:nq + attn.k_proj.out_features], attn.k_proj.weight)
    assert model.set_exact(True).exact
