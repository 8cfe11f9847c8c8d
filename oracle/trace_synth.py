"""Seeded synthetic motion trace. TEST INFRASTRUCTURE ONLY.

Regenerates the reference's synthetic trace (motion regimes + coupled Q/K/V
drift) so that the attention oracle can be checked against the golden
statistics the reference publishes for its 8-frame seed-42 trace
(reference: traces/trace_meta_8f.json, traces/golden_meta.json).

To reproduce the same numbers the draws must come from a CPU
torch.Generator seeded once, in the reference's order (reference:
traces/gen_synthetic_motion.py:52-89): static mask, static base, moving
start, then per frame (jitter, walk); then Q for all frames, K0, V0, then per
frame (K step, V step). Tile partition: 16-token row-major runs, the last
one shorter (reference: traces/gen_synthetic_motion.py:41-49).

Pinned by tests/test_oracle_pins.py against trace_meta_8f.json (59 static /
39 moving tiles, first-vs-last cosine statistics to 6 decimals).
"""

from __future__ import annotations

import torch

STATIC_BASE = (0.05, 0.02)       # mean, std
STATIC_JITTER_STD = 0.01
MOVING_START = (1.5, 0.4)        # mean, std
MOVING_WALK_STD = 0.25
MOVING_CLIP = (0.8, 4.0)
KV_DRIFT = 0.15


def tile_counts(tokens_per_frame: int, tile_tokens: int) -> torch.Tensor:
    full, rem = divmod(tokens_per_frame, tile_tokens)
    counts = [tile_tokens] * full + ([rem] if rem else [])
    return torch.tensor(counts, dtype=torch.long)


def motion_scores(gen: torch.Generator, num_tiles: int, frames: int, frac_static: float):
    static = torch.rand(num_tiles, generator=gen) < frac_static
    s_base = (STATIC_BASE[0] + STATIC_BASE[1] * torch.randn(num_tiles, generator=gen)).clamp(min=0.005)
    m_base = (MOVING_START[0] + MOVING_START[1] * torch.randn(num_tiles, generator=gen)).clamp(*MOVING_CLIP)
    scores = torch.empty(frames, num_tiles)
    scores[0] = torch.where(static, s_base, m_base)
    for f in range(1, frames):
        jit = STATIC_JITTER_STD * torch.randn(num_tiles, generator=gen)
        walk = MOVING_WALK_STD * torch.randn(num_tiles, generator=gen)
        scores[f] = torch.where(static, (scores[f - 1] + jit).clamp(min=0.0),
                                (scores[f - 1] + walk).clamp(*MOVING_CLIP))
    return scores, static


def synthetic_trace(frames: int = 8, seed: int = 42, tokens: int = 1560, hidden: int = 1536,
                    tile_tokens: int = 16, frac_static: float = 0.65):
    """-> dict(q, k, v [frames, tokens, hidden] fp32, scores [frames, tiles], static)."""
    gen = torch.Generator().manual_seed(seed)
    counts = tile_counts(tokens, tile_tokens)
    scores, static = motion_scores(gen, int(counts.numel()), frames, frac_static)
    per_token = torch.repeat_interleave(scores, counts, dim=1)
    q = torch.randn(frames, tokens, hidden, generator=gen)
    k = torch.empty(frames, tokens, hidden)
    v = torch.empty(frames, tokens, hidden)
    k[0] = torch.randn(tokens, hidden, generator=gen)
    v[0] = torch.randn(tokens, hidden, generator=gen)
    for f in range(1, frames):
        step = KV_DRIFT * per_token[f].unsqueeze(1)
        k[f] = k[f - 1] + step * torch.randn(tokens, hidden, generator=gen)
        v[f] = v[f - 1] + step * torch.randn(tokens, hidden, generator=gen)
    return dict(q=q, k=k, v=v, scores=scores, static=static, counts=counts)


def cosine_report(x: torch.Tensor, static_tok: torch.Tensor) -> dict:
    cos = torch.nn.functional.cosine_similarity(x[0], x[-1], dim=1)
    s, m = cos[static_tok], cos[~static_tok]
    return {"static": {"mean": round(s.mean().item(), 6), "min": round(s.min().item(), 6)},
            "moving": {"mean": round(m.mean().item(), 6), "max": round(m.max().item(), 6)}}
