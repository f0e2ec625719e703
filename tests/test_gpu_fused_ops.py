"""Fused layer ops (RMSNorm + residual add, q/k RMSNorm + RoPE + decode append, SwiGLU product)
against the reference's torch op chains on the same GPU (src/mini_infra/model/qwen3.py:55-78,
111-145, 182-217, 282-283, 347-355).

Everything elementwise is bit-exact.  The one freedom is the order of the fp32 sum of squares
inside RMSNorm, which can move a normalised value by one bf16 ulp when it sits on a rounding
boundary; those cases are bounded (one ulp) and rare."""

import pytest
import torch
import torch.nn.functional as F

from mini_infra_qwen3_amd import data_plane

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6


def ref_rms(x, w):  # qwen3.py:67-78
    xf = x.float()
    return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(x.dtype)


def ref_rope(x, cos, sin):  # qwen3.py:111-145, x [..., 128], cos / sin broadcast
    rot = torch.cat((-x[..., 64:], x[..., :64]), dim=-1)
    return x * cos + rot * sin


def within_one_ulp(got, want, max_fraction=1e-3, atol=0.0, ulps=1):
    """|got - want| <= ``ulps`` bf16 ulps of want (+ atol: after RoPE a one-ulp change of a
    normalised input can survive cancellation between the two products as one ulp at magnitude
    ~1).  A one-ulp change of the normalised value can become two after the weight product."""
    got, want = got.float(), want.float()
    diff = (got - want).abs()
    assert (diff <= want.abs() * ulps * 2.0 ** -7 + atol).all(), f"max diff {diff.max().item()}"
    assert (diff > 0).float().mean().item() <= max_fraction


def randn(*shape, seed, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("hidden", [128, 1024, 4096, 3072])
def test_rms_norm_with_and_without_residual(hidden):
    x, r = randn(37, 5, hidden, seed=1), randn(37, 5, hidden, seed=2, scale=3.0)
    w = randn(hidden, seed=3, scale=0.1) + 1
    out, res = data_plane.rms_norm(x, w, EPS)
    assert res is x or torch.equal(res, x)
    within_one_ulp(out, ref_rms(x, w), ulps=2)
    out, res = data_plane.rms_norm(x, w, EPS, residual=r)
    h = r + x  # the reference's `residual + output`
    assert torch.equal(res, h)
    within_one_ulp(out, ref_rms(h, w), ulps=2)


def test_qk_norm_rope_prefill_form():
    B, L, H, G = 3, 33, 16, 8
    q, k, v = randn(B, L, H * 128, seed=4), randn(B, L, G * 128, seed=5), randn(B, L, G * 128, seed=6)
    qw, kw = randn(128, seed=7, scale=0.1) + 1, randn(128, seed=8, scale=0.1) + 1
    pos = torch.randint(0, 40000, (B, L), device=DEV)
    inv = 1.0 / (1e6 ** (torch.arange(0, 128, 2, device=DEV, dtype=torch.float32) / 128))
    ang = torch.cat((pos.float()[..., None] * inv, pos.float()[..., None] * inv), -1)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    q_out, k_out, v_out = data_plane.qk_norm_rope(q, k, v, qw, kw, cos, sin, EPS)
    want_q = ref_rope(ref_rms(q.view(B, L, H, 128), qw), cos[:, :, None], sin[:, :, None])
    want_k = ref_rope(ref_rms(k.view(B, L, G, 128), kw), cos[:, :, None], sin[:, :, None])
    within_one_ulp(q_out.view(B, L, H, 128), want_q, max_fraction=2e-3, atol=2 ** -7)
    within_one_ulp(k_out.view(B, L, G, 128), want_k, max_fraction=2e-3, atol=2 ** -7)
    assert torch.equal(v_out.view(B, L, G * 128), v)


def test_qk_norm_rope_decode_form_appends_into_pool_slots():
    B, H, G, nb, bs = 6, 16, 8, 9, 16
    q, k, v = randn(B, 1, H * 128, seed=9), randn(B, 1, G * 128, seed=10), randn(B, 1, G * 128, seed=11)
    qw, kw = randn(128, seed=12, scale=0.1) + 1, randn(128, seed=13, scale=0.1) + 1
    cos, sin = randn(B, 1, 128, seed=14), randn(B, 1, 128, seed=15)
    key_pool = randn(nb, bs, G, 128, seed=16)
    value_pool = randn(nb, bs, G, 128, seed=17)
    kp0, vp0 = key_pool.clone(), value_pool.clone()
    slots = torch.tensor([5, 140, -1, 17, nb * bs, 2], device=DEV)  # -1 and one-past-the-end are skipped
    q_out, k_out, v_out = data_plane.qk_norm_rope(q, k, v, qw, kw, cos, sin, EPS, slot_mapping=slots,
                                                  key_pool=key_pool, value_pool=value_pool)
    assert k_out is None and v_out is None
    want_k = ref_rope(ref_rms(k.view(B, G, 128), kw), cos, sin)
    within_one_ulp(q_out, ref_rope(ref_rms(q.view(B, H, 128), qw), cos, sin), max_fraction=2e-3, atol=2 ** -7)
    kflat, vflat, k0, v0 = (t.view(-1, G, 128) for t in (key_pool, value_pool, kp0, vp0))
    written = [(i, s) for i, s in enumerate(slots.tolist()) if 0 <= s < nb * bs]
    for i, s in written:
        within_one_ulp(kflat[s], want_k[i], max_fraction=2e-2, atol=2 ** -7)
        assert torch.equal(vflat[s], v.view(B, G, 128)[i])
    untouched = torch.ones(nb * bs, dtype=torch.bool, device=DEV)
    untouched[[s for _, s in written]] = False
    assert torch.equal(kflat[untouched], k0[untouched]) and torch.equal(vflat[untouched], v0[untouched])


def test_qk_norm_rope_vector_and_scalar_forms_are_bit_identical():
    """16-byte aligned rows take the vector form (16 lanes per head), others one head per
    wavefront: the same bits, rows and pool slots alike (the sum of squares is exact in fp64)."""
    T, H, G, nb, bs = 300, 16, 8, 24, 16
    qk = randn(T, H * 128 + G * 128 + 1, seed=30)
    q_odd, k_odd = qk[:, 1:H * 128 + 1], qk[:, H * 128 + 1:]   # 2-byte offset: the scalar form
    v = randn(T, G * 128, seed=31)
    qw, kw = randn(128, seed=32, scale=0.1) + 1, randn(128, seed=33, scale=0.1) + 1
    cos, sin = randn(T, 128, seed=34), randn(T, 128, seed=35)
    slots = torch.randperm(nb * bs, device=DEV)[:T]
    slots[::7] = -1
    outs = []
    for q, k in ((q_odd, k_odd), (q_odd.contiguous(), k_odd.contiguous())):
        kp, vp = torch.zeros(nb, bs, G, 128, dtype=torch.bfloat16, device=DEV), \
            torch.zeros(nb, bs, G, 128, dtype=torch.bfloat16, device=DEV)
        q_out, k_out, v_out = data_plane.qk_norm_rope(q, k, v, qw, kw, cos, sin, EPS, slot_mapping=slots,
                                                      key_pool=kp, value_pool=vp, rows=True)
        outs.append((q_out, k_out, v_out, kp, vp))
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(outs[1][2].view(T, -1), v)


def test_silu_mul_and_strided_views():
    gu = randn(7, 3, 2 * 3072, seed=18, scale=3.0)
    gate, up = gu[..., :3072], gu[..., 3072:]
    out = data_plane.silu_mul(gate, up)
    within_one_ulp(out, F.silu(gate) * up, max_fraction=1e-3)


def test_fused_ops_reject_bad_input():
    x = randn(4, 1004, seed=19)
    with pytest.raises(ValueError):
        data_plane.rms_norm(x, randn(1004, seed=20), EPS)  # hidden not a multiple of 8
    with pytest.raises(ValueError):
        data_plane.silu_mul(randn(4, 8, seed=21), randn(4, 16, seed=22))
    with pytest.raises(RuntimeError):
        data_plane.rms_norm(x.cpu(), randn(1004, seed=20).cpu(), EPS)
