"""Synthetic workloads of the five benchmark configurations.

C1  1 frame x 1560 tokens (30x52 grid), 12 x 128 heads, fp32 Q/K/V ~ N(0,1)
    (seed 42), policy none.
C2  C1 plus per-tile motion ~ U[0,1) (seed 43); motion-gated arena holding
    22 of the 98 tiles (budget 22 fp32 tiles = 4,325,376 B).
C3  8 frames causal cross-frame, 30 layers, bf16 N(0,1) (seed 42 + layer);
    motion from a smooth random field: per frame Gaussian-blurred N(0,1)
    noise on the 30x52 grid, AR(1) across frames (rho = 0.9), mapped to
    [0, 1) by the normal CDF, per-tile score = mean over the tile's 16
    row-major tokens.
C4  50 frames, sliding window of 8 frames, the C3 field plus an integer
    camera pan (the field rolls one column per frame), all five policies.
C5  45x80 grid = 3600 tokens (225 tiles), 21 frames causal, bf16; motion
    U[0,1) with 10% of the tiles of every frame forced to [0.9, 1).

Q/K/V for the benchmark are drawn on the device (torch generator) so that
multi-GB inputs never cross PCIe; tests draw small cases on the host.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

try:  # scipy provides the blur and the normal CDF; both are in this image
    from scipy.ndimage import gaussian_filter
    from scipy.special import ndtr
except ImportError:  # pragma: no cover - image always has scipy
    gaussian_filter = None
    ndtr = None

HEADS = 12
HEAD_DIM = 128
HIDDEN = HEADS * HEAD_DIM
TILE_TOKENS = 16
FP32_TILE_BYTES = TILE_TOKENS * HIDDEN * 4 * 2   # 196,608
BF16_TILE_BYTES = TILE_TOKENS * HIDDEN * 2 * 2   # 98,304


@dataclass(frozen=True)
class Config:
    name: str
    grid: tuple
    frames: int
    layers: int
    dtype: str          # "fp32" | "bf16"
    mode: str           # "intra" | "cross"
    window: int         # 0 = full causal prefix
    policies: tuple
    set_aside: int      # arena budget in bytes

    @property
    def tokens(self) -> int:
        return self.grid[0] * self.grid[1]

    @property
    def num_tiles(self) -> int:
        return (self.tokens + TILE_TOKENS - 1) // TILE_TOKENS

    @property
    def elem(self) -> int:
        return 4 if self.dtype == "fp32" else 2

    def frame_units(self) -> int:
        """Query-frame x key-frame pairs attended (work unit 4*T^2*dh*H)."""
        if self.mode == "intra":
            return self.frames
        w = self.window or self.frames
        return sum(min(f + 1, w) for f in range(self.frames))

    def flops_per_layer(self) -> float:
        return 4.0 * self.tokens ** 2 * HEAD_DIM * HEADS * self.frame_units()


# Arena budgets. C2: 22 fp32 tiles. C3-C5: 2,162,688 B = 22 bf16 tiles, about
# half of one XCD's 4 MB L2, so the arena of a layer can stay L2 resident.
C2_SET_ASIDE = 22 * FP32_TILE_BYTES
BF16_SET_ASIDE = 22 * BF16_TILE_BYTES

CONFIGS = {
    "c1": Config("c1", (30, 52), 1, 1, "fp32", "intra", 0, ("none",), 0),
    "c2": Config("c2", (30, 52), 1, 1, "fp32", "intra", 0, ("none", "motion"), C2_SET_ASIDE),
    "c3": Config("c3", (30, 52), 8, 30, "bf16", "cross", 0, ("none", "recency", "motion"),
                 BF16_SET_ASIDE),
    "c4": Config("c4", (30, 52), 50, 30, "bf16", "cross", 8,
                 ("none", "uniform", "recency", "motion", "reuse_weighted"), BF16_SET_ASIDE),
    "c5": Config("c5", (45, 80), 21, 30, "bf16", "cross", 0, ("none", "motion"),
                 BF16_SET_ASIDE),
}


def tile_means(field: np.ndarray, tile_tokens: int = TILE_TOKENS) -> np.ndarray:
    """[frames, rows, cols] -> [frames, tiles]: mean over each row-major tile."""
    f = field.reshape(field.shape[0], -1)
    n = f.shape[1]
    tiles = (n + tile_tokens - 1) // tile_tokens
    out = np.empty((f.shape[0], tiles), dtype=np.float64)
    for t in range(tiles):
        out[:, t] = f[:, t * tile_tokens:min(n, (t + 1) * tile_tokens)].mean(axis=1)
    return out


def smooth_motion(frames: int, grid=(30, 52), *, seed: int, rho: float = 0.9,
                  sigma: float = 2.0, pan: int = 0) -> np.ndarray:
    """Per-tile motion in [0, 1) from a blurred AR(1) field -> [frames, tiles] f32."""
    rng = np.random.default_rng(seed)
    field = np.empty((frames,) + tuple(grid))
    m = None
    for f in range(frames):
        eps = gaussian_filter(rng.standard_normal(grid), sigma=sigma, mode="wrap")
        eps /= eps.std() + 1e-12
        m = eps if m is None else rho * m + math.sqrt(1.0 - rho * rho) * eps
        field[f] = np.roll(m, shift=pan * f, axis=1) if pan else m
    u = ndtr(field)
    u = np.minimum(u, np.nextafter(1.0, 0.0))
    return tile_means(u).astype(np.float32)


def uniform_motion(frames: int, tiles: int, *, seed: int, forced_high: float = 0.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    s = rng.random((frames, tiles), dtype=np.float32)
    if forced_high > 0:
        k = int(round(forced_high * tiles))
        for f in range(frames):
            idx = rng.choice(tiles, size=k, replace=False)
            s[f, idx] = (0.9 + 0.1 * rng.random(k)).astype(np.float32)
    return np.minimum(s, np.float32(np.nextafter(np.float32(1.0), np.float32(0.0))))


def motion_for(cfg: Config, layer: int = 0) -> np.ndarray:
    """Motion scores [frames, tiles] (float32) of a configuration and layer."""
    if cfg.name in ("c1", "c2"):
        return uniform_motion(cfg.frames, cfg.num_tiles, seed=43)
    if cfg.name == "c3":
        return smooth_motion(cfg.frames, cfg.grid, seed=1000 + layer)
    if cfg.name == "c4":
        return smooth_motion(cfg.frames, cfg.grid, seed=2000 + layer, pan=1)
    if cfg.name == "c5":
        return uniform_motion(cfg.frames, cfg.num_tiles, seed=3000 + layer, forced_high=0.1)
    raise KeyError(cfg.name)


def qkv_host(frames: int, tokens: int, *, seed: int, hidden: int = HIDDEN):
    """Q, K, V float32 [frames*tokens, hidden] ~ N(0,1) from numpy PCG64."""
    rng = np.random.default_rng(seed)
    shape = (frames * tokens, hidden)
    q = rng.standard_normal(shape, dtype=np.float32)
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    return q, k, v


def qkv_device(frames: int, tokens: int, *, seed: int, dtype, device="cuda",
               hidden: int = HIDDEN):
    """Q, K, V ~ N(0,1) drawn on the device, cast to dtype (torch)."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    shape = (frames * tokens, hidden)
    out = []
    for _ in range(3):
        x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
        out.append(x.to(dtype))
    return tuple(out)


def synthetic_clip(frames: int, height: int = 480, width: int = 832, *, seed: int = 0,
                   max_shift: float = 2.0):
    """uint8 gray clip [frames, height, width] for the motion producer: a smooth
    random texture (Gaussian-filtered noise, sigma 2 px) whose content moves
    by a random-walk global shift (up to max_shift px per frame and axis)
    plus a drifting sinusoidal local warp of 1.5 px. Synthetic input only
    (the reference reads a DAVIS / mp4 clip through OpenCV)."""
    from scipy.ndimage import map_coordinates
    rng = np.random.default_rng(seed)
    pad = 48
    base = gaussian_filter(rng.standard_normal((height + 2 * pad, width + 2 * pad)), 2.0,
                           mode="wrap")
    base = (base - base.mean()) / (base.std() + 1e-12)
    yy, xx = np.mgrid[0:height, 0:width].astype(np.float64)
    out = np.empty((frames, height, width), dtype=np.uint8)
    ox = oy = 0.0
    for f in range(frames):
        warp = 1.5 * np.sin(2 * math.pi * (xx / width + 0.05 * f)) * np.cos(
            2 * math.pi * yy / height)
        img = map_coordinates(base, [yy + pad + oy, xx + pad + ox + warp], order=1, mode="wrap")
        out[f] = np.clip(np.rint(128 + 40 * img), 0, 255).astype(np.uint8)
        ox += rng.uniform(-max_shift, max_shift)
        oy += rng.uniform(-max_shift, max_shift)
    return out
