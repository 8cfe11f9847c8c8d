"""Upstream K/V producer oracle. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates the reference's random-init DiT self-attention stack
(reference: src/backbone.py:8-67, src/config.py:6-27) on the CPU:

  layer_norm      nn.LayerNorm over the last dim, float64 two-pass mean and
                  biased variance (backbone.py:28,48; eps 1e-5).
  linear          nn.Linear, x W^T + b in float64 (backbone.py:13-14,44).
  block_forward   DiTSelfAttentionBlock.forward (backbone.py:16-33): LN ->
                  qkv_proj -> q, k, v = the three [D]-column blocks of the
                  projection -> per-frame non-causal attention with scale
                  1/sqrt(head_dim) (oracle.attention.attention_keys, the
                  F.scaled_dot_product_attention of backbone.py:20) ->
                  out_proj -> residual add.
  backbone_forward  SelfAttentionBackbone.forward (backbone.py:58-67):
                  latents (b, C, rows, cols) reshaped without a permute to
                  (b, T, C) rows -> token_embed -> blocks -> final_norm.
  param_names / param_count  the module's state_dict names, shapes and the
                  closed-form parameter count (tests/test_skeleton.py:8-17).

Everything is token-major [frames*T, D]: the reference's per-layer k of shape
(b, heads, t, head_dim) has element (b, h, t, d) at (b*T + t, h*128 + d).

bf16 mode mirrors the library's storage points: the projection weights are
bf16 (the caller rounds them), and the normalised activations, q/k/v and the
attention output are rounded to bf16 where the library stores them; the
residual stream, the statistics and every accumulation stay wide.

Pinned by tests/test_backbone_oracle.py:
  * layer_norm / linear / attention against torch's own library routines
    (F.layer_norm, F.linear, F.scaled_dot_product_attention) written in the
    reference's (b, heads, t, head_dim) form with view/permute/unbind, so a
    wrong q/k/v block order, head interleave or residual fails;
  * closed forms: a constant row normalises to beta exactly; LN is invariant
    to x -> a*x + c (a > 0, eps = 0); zero out_proj leaves the residual
    stream unchanged, so hidden = final_norm(token_embed(latents));
  * the reference's published parameter count 283,421,184
    (reference: tests/test_skeleton.py:28-32).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import attention as at

HEAD_DIM = 128
LN_EPS = 1e-5


@dataclass(frozen=True)
class Config:
    """BackboneConfig fields used by the forward (reference: src/config.py:6-16)."""
    num_layers: int = 30
    hidden_dim: int = 1536
    num_heads: int = 12
    head_dim: int = 128
    latent_channels: int = 16
    tokens_per_frame: int = 1560


def param_names(cfg: Config) -> list[tuple[str, tuple[int, ...]]]:
    """(name, shape) in state_dict order (token_embed, blocks, final_norm)."""
    D, C = cfg.hidden_dim, cfg.latent_channels
    out = [("token_embed.weight", (D, C)), ("token_embed.bias", (D,))]
    for i in range(cfg.num_layers):
        b = f"blocks.{i}."
        out += [(b + "norm.weight", (D,)), (b + "norm.bias", (D,)),
                (b + "attn.qkv_proj.weight", (3 * D, D)), (b + "attn.qkv_proj.bias", (3 * D,)),
                (b + "attn.out_proj.weight", (D, D)), (b + "attn.out_proj.bias", (D,))]
    out += [("final_norm.weight", (D,)), ("final_norm.bias", (D,))]
    return out


def param_count(cfg: Config) -> int:
    """Closed form of the reference test (reference: tests/test_skeleton.py:8-17)."""
    D, C = cfg.hidden_dim, cfg.latent_channels
    per_block = D * 3 * D + 3 * D + D * D + D + 2 * D
    return cfg.num_layers * per_block + C * D + D + 2 * D


def round_bf16(x: np.ndarray) -> np.ndarray:
    return at.round_bf16(torch.from_numpy(np.asarray(x, dtype=np.float32))).numpy()


def layer_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = LN_EPS) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    c = x - mean
    var = (c * c).mean(axis=-1, keepdims=True)
    return c / np.sqrt(var + eps) * np.asarray(gamma, np.float64) + np.asarray(beta, np.float64)


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    y = np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T
    if b is not None:
        y = y + np.asarray(b, dtype=np.float64)
    return y


def _store(x: np.ndarray, bf16: bool) -> np.ndarray:
    """Value as the library stores it: fp32, or bf16 in bf16 mode."""
    x32 = np.asarray(x, dtype=np.float32)
    return round_bf16(x32) if bf16 else x32


def qkv_project(x: np.ndarray, p: dict, layer: int, D: int, bf16: bool = False):
    """LN + qkv_proj of one block -> (q, k, v), token-major [rows, D]."""
    b = f"blocks.{layer}."
    xn = _store(layer_norm(x, p[b + "norm.weight"], p[b + "norm.bias"]), bf16)
    w, bias = p[b + "attn.qkv_proj.weight"], p[b + "attn.qkv_proj.bias"]
    return tuple(_store(linear(xn, w[i * D:(i + 1) * D], bias[i * D:(i + 1) * D]), bf16)
                 for i in range(3))


def block_forward(x: np.ndarray, p: dict, layer: int, frames: int, T: int, heads: int,
                  bf16: bool = False):
    """One DiTSelfAttentionBlock on the fp32 residual stream x [frames*T, D].

    Returns (x_next, q, k, v) with x_next float64 and q/k/v as stored."""
    D = heads * HEAD_DIM
    q, k, v = qkv_project(x, p, layer, D, bf16)
    ctx = np.empty((frames * T, D), dtype=np.float32)
    for f in range(frames):
        sl = slice(f * T, (f + 1) * T)
        ctx[sl] = at.attention_keys(torch.from_numpy(q[sl]), torch.from_numpy(k[sl]),
                                    torch.from_numpy(v[sl]), heads).numpy()
    ctx = _store(ctx, bf16)
    b = f"blocks.{layer}."
    h = linear(ctx, p[b + "attn.out_proj.weight"], p[b + "attn.out_proj.bias"])
    x_next = np.asarray(x, np.float64) + h
    return x_next, q, k, v


def backbone_forward(latents: np.ndarray, p: dict, cfg: Config, frames: int, bf16: bool = False,
                     layers: int | None = None):
    """latents: frames * C * T values -> (hidden [frames*T, D], [(q, k, v)] per layer).

    The residual stream is carried in fp32 between blocks, as in the library."""
    T, C, D = cfg.tokens_per_frame, cfg.latent_channels, cfg.hidden_dim
    rows = np.asarray(latents, dtype=np.float32).reshape(frames * T, C)
    x = linear(rows, p["token_embed.weight"], p["token_embed.bias"]).astype(np.float32)
    per_layer = []
    for layer in range(cfg.num_layers if layers is None else layers):
        x64, q, k, v = block_forward(x, p, layer, frames, T, cfg.num_heads, bf16)
        x = x64.astype(np.float32)
        per_layer.append((q, k, v))
    hidden = layer_norm(x, p["final_norm.weight"], p["final_norm.bias"])
    return hidden, per_layer
