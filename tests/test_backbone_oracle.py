"""Pins of the K/V producer oracle (oracle/backbone.py) on the CPU.

Each oracle function is checked against torch's own library routines written
in the reference's (b, heads, t, head_dim) form (reference:
src/backbone.py:16-33: qkv_proj(x).view(b, t, 3, heads, hd).permute(2, 0, 3,
1, 4).unbind(0), F.scaled_dot_product_attention, transpose + reshape), against
closed forms, and against the reference's published parameter count.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import backbone as bb


def _params(cfg, rng, ln_random=True):
    p = {}
    for name, shape in bb.param_names(cfg):
        if name.endswith("norm.weight"):
            a = 1.0 + 0.1 * rng.standard_normal(shape) if ln_random else np.ones(shape)
        elif name.endswith("bias"):
            a = 0.05 * rng.standard_normal(shape)
        else:
            a = 0.02 * rng.standard_normal(shape)
        p[name] = a.astype(np.float32)
    return p


def test_param_count_matches_reference():
    """Default config: 283,421,184 (reference: tests/test_skeleton.py:28-32)."""
    cfg = bb.Config()
    assert bb.param_count(cfg) == 283_421_184
    assert sum(int(np.prod(s)) for _, s in bb.param_names(cfg)) == 283_421_184
    names = [n for n, _ in bb.param_names(cfg)]
    assert len(names) == len(set(names)) == 2 + 6 * 30 + 2
    assert names[0] == "token_embed.weight" and names[-1] == "final_norm.bias"
    assert "blocks.29.attn.qkv_proj.weight" in names


def test_layer_norm_matches_torch_and_closed_forms():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((37, 1536)) * 3 + rng.standard_normal((37, 1)) * 50
    g = rng.standard_normal(1536)
    b = rng.standard_normal(1536)
    want = F.layer_norm(torch.from_numpy(x), (1536,), torch.from_numpy(g), torch.from_numpy(b),
                        eps=1e-5).numpy()
    assert np.abs(bb.layer_norm(x, g, b) - want).max() < 1e-10
    # constant row -> beta exactly
    c = np.full((2, 1536), 7.25)
    assert np.array_equal(bb.layer_norm(c, g, b), np.broadcast_to(b, (2, 1536)))
    # invariance to a*x + c (a > 0) with eps = 0
    y0 = bb.layer_norm(x, g, b, eps=0.0)
    y1 = bb.layer_norm(2.5 * x - 11.0, g, b, eps=0.0)
    assert np.abs(y0 - y1).max() < 1e-9


def test_linear_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((9, 16))
    w = rng.standard_normal((40, 16))
    b = rng.standard_normal(40)
    want = F.linear(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b)).numpy()
    assert np.abs(bb.linear(x, w, b) - want).max() < 1e-12
    eye = np.eye(16)
    assert np.array_equal(bb.linear(x, eye), x)


def _torch_block(x_btd, p, layer, heads):
    """The reference block in its own tensor form, built from torch routines."""
    b, t, D = x_btd.shape
    hd = D // heads
    pre = f"blocks.{layer}."
    P = {k: torch.from_numpy(v).double() for k, v in p.items() if k.startswith(pre)}
    xn = F.layer_norm(x_btd, (D,), P[pre + "norm.weight"], P[pre + "norm.bias"], eps=1e-5)
    qkv = F.linear(xn, P[pre + "attn.qkv_proj.weight"], P[pre + "attn.qkv_proj.bias"])
    q, k, v = qkv.view(b, t, 3, heads, hd).permute(2, 0, 3, 1, 4).unbind(0)
    ctx = F.scaled_dot_product_attention(q, k, v)
    ctx = ctx.transpose(1, 2).reshape(b, t, heads * hd)
    h = F.linear(ctx, P[pre + "attn.out_proj.weight"], P[pre + "attn.out_proj.bias"])
    return x_btd + h, k, v


@pytest.mark.parametrize("frames,T,heads", [(2, 40, 2), (1, 7, 3)])
def test_block_matches_reference_form(frames, T, heads):
    cfg = bb.Config(num_layers=1, hidden_dim=heads * 128, num_heads=heads, tokens_per_frame=T)
    rng = np.random.default_rng(frames * 10 + T)
    p = _params(cfg, rng)
    D = cfg.hidden_dim
    x = rng.standard_normal((frames * T, D)).astype(np.float32)
    got_x, q, k, v = bb.block_forward(x, p, 0, frames, T, heads)
    want_x, k_ref, v_ref = _torch_block(torch.from_numpy(x).double().view(frames, T, D), p, 0,
                                        heads)
    assert np.abs(got_x - want_x.reshape(frames * T, D).numpy()).max() < 1e-5
    # token-major (b*T + t, h*128 + d) <-> reference (b, h, t, d)
    k_tm = torch.from_numpy(k).double().view(frames, T, heads, 128).permute(0, 2, 1, 3)
    v_tm = torch.from_numpy(v).double().view(frames, T, heads, 128).permute(0, 2, 1, 3)
    assert k_tm.shape == k_ref.shape == (frames, heads, T, 128)
    assert (k_tm - k_ref).abs().max() < 1e-5
    assert (v_tm - v_ref).abs().max() < 1e-5


def test_backbone_reshape_and_zero_out_proj_closed_form():
    """Zero out_proj weights and bias leave the residual stream at the token
    embedding, so hidden = final_norm(token_embed(latents.reshape(b, T, C)))
    for any depth, and every layer's k/v come from that same stream."""
    cfg = bb.Config(num_layers=3, hidden_dim=256, num_heads=2, tokens_per_frame=12)
    rng = np.random.default_rng(3)
    p = _params(cfg, rng)
    for i in range(3):
        p[f"blocks.{i}.attn.out_proj.weight"][:] = 0
        p[f"blocks.{i}.attn.out_proj.bias"][:] = 0
    frames = 2
    lat = rng.standard_normal((frames, 16, 3, 4)).astype(np.float32)
    hidden, per_layer = bb.backbone_forward(lat, p, cfg, frames)
    rows = torch.from_numpy(lat).reshape(frames, 12, 16)  # reference: src/backbone.py:61
    emb = F.linear(rows.double(), torch.from_numpy(p["token_embed.weight"]).double(),
                   torch.from_numpy(p["token_embed.bias"]).double())
    want = F.layer_norm(emb, (256,), torch.from_numpy(p["final_norm.weight"]).double(),
                        torch.from_numpy(p["final_norm.bias"]).double(), eps=1e-5)
    assert np.abs(hidden - want.reshape(frames * 12, 256).numpy()).max() < 1e-5
    x = emb.reshape(frames * 12, 256).numpy().astype(np.float32)
    for i, (q, k, v) in enumerate(per_layer):
        q2, k2, v2 = bb.qkv_project(x, p, i, 256)
        assert np.array_equal(k, k2) and np.array_equal(v, v2) and np.array_equal(q, q2)


def test_bf16_mode_rounds_storage_points():
    cfg = bb.Config(num_layers=1, hidden_dim=128, num_heads=1, tokens_per_frame=5)
    rng = np.random.default_rng(4)
    p = _params(cfg, rng)
    x = rng.standard_normal((5, 128)).astype(np.float32)
    _, q, k, v = bb.block_forward(x, p, 0, 1, 5, 1, bf16=True)
    for a in (q, k, v):
        assert np.array_equal(a, bb.round_bf16(a))
    _, q32, k32, _ = bb.block_forward(x, p, 0, 1, 5, 1, bf16=False)
    assert np.abs(k - k32).max() < 2e-2
