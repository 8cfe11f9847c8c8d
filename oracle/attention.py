"""Attention oracle. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates the reference golden (reference: traces/gen_golden.py:30-74): per
head, scores = Q K^T / sqrt(head_dim) in fp32, softmax over keys, then
softmax @ V, with explicit torch.matmul + torch.softmax on the CPU. The
causal / sliding-window forms only change which key rows take part; query
rows are processed in chunks of 128 so the score matrix stays bounded
(reference: traces/gen_golden.py:46-74).

bf16 cases: inputs are rounded to bf16 first, the golden is then computed in
fp32 from the rounded values.

Pinned by (tests/test_oracle_pins.py):
  * float64 brute force on tiny shapes (attention_f64 below, an independent
    numpy loop-free evaluation);
  * closed forms: a single key returns that key's V row; identical keys
    return the mean of V; softmax rows sum to 1 within 1e-5
    (reference: traces/gen_golden.py:116);
  * the reference's published per-frame output mean/std of the 8-frame
    seed-42 intra golden (reference: traces/golden_meta.json:14-54),
    regenerated from oracle.trace_synth.
"""

from __future__ import annotations

import math

import numpy as np
import torch

HEAD_DIM = 128


def round_bf16(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 (round to nearest even) -> fp32."""
    return x.to(torch.bfloat16).to(torch.float32)


def attention_intra(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int,
                    head_dim: int = HEAD_DIM) -> torch.Tensor:
    """q,k,v [T, D] fp32 -> [T, D]; frame attends to its own keys."""
    return attention_keys(q, k, v, heads, head_dim)


def attention_keys(q: torch.Tensor, k_all: torch.Tensor, v_all: torch.Tensor, heads: int,
                   head_dim: int = HEAD_DIM, chunk: int = 128,
                   return_rowsum_err: bool = False):
    """q [T, D] against every row of k_all / v_all [S, D] -> [T, D] fp32."""
    q = q.to(torch.float32)
    k_all = k_all.to(torch.float32)
    v_all = v_all.to(torch.float32)
    t = q.shape[0]
    s = k_all.shape[0]
    scale = 1.0 / math.sqrt(head_dim)
    out = torch.empty(t, heads * head_dim, dtype=torch.float32)
    worst = 0.0
    with torch.no_grad():
        kh = k_all.view(s, heads, head_dim)
        vh = v_all.view(s, heads, head_dim)
        qh = q.view(t, heads, head_dim)
        for h in range(heads):
            k_h = kh[:, h, :]
            v_h = vh[:, h, :]
            kt = k_h.transpose(0, 1).contiguous()
            for r0 in range(0, t, chunk):
                r1 = min(r0 + chunk, t)
                sc = torch.matmul(qh[r0:r1, h, :], kt) * scale
                p = torch.softmax(sc, dim=-1)
                if return_rowsum_err:
                    worst = max(worst, float((p.sum(dim=-1) - 1.0).abs().max()))
                out[r0:r1, h * head_dim:(h + 1) * head_dim] = torch.matmul(p, v_h)
    if return_rowsum_err:
        return out, worst
    return out


def key_range(mode: str, f: int, T: int, window_frames: int = 0) -> tuple[int, int]:
    """Absolute key rows [begin, end) attended by query frame f."""
    if mode == "intra":
        return f * T, (f + 1) * T
    end = (f + 1) * T
    begin = 0
    if window_frames and f + 1 > window_frames:
        begin = (f + 1 - window_frames) * T
    return begin, end


def attention_frames(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, frames: int, T: int,
                     heads: int, mode: str = "intra", window_frames: int = 0,
                     frame_list=None) -> torch.Tensor:
    """q/k/v [frames*T, D] -> out [frames*T, D] for intra / cross / window."""
    out = torch.zeros_like(q, dtype=torch.float32)
    for f in (range(frames) if frame_list is None else frame_list):
        b, e = key_range(mode, f, T, window_frames)
        out[f * T:(f + 1) * T] = attention_keys(q[f * T:(f + 1) * T], k[b:e], v[b:e], heads)
    return out


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, heads: int,
                  head_dim: int = HEAD_DIM) -> np.ndarray:
    """Float64 brute force, numpy only: q [T, D], k/v [S, D] -> [T, D]."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    t, s = q.shape[0], k.shape[0]
    qh = q.reshape(t, heads, head_dim)
    kh = k.reshape(s, heads, head_dim)
    vh = v.reshape(s, heads, head_dim)
    logits = np.einsum("thd,shd->hts", qh, kh) / math.sqrt(head_dim)
    logits -= logits.max(axis=-1, keepdims=True)
    w = np.exp(logits)
    w /= w.sum(axis=-1, keepdims=True)
    o = np.einsum("hts,shd->thd", w, vh)
    return o.reshape(t, heads * head_dim)
