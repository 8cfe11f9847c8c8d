"""Upstream motion producer oracle. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference turns a video clip into per-tile motion scores with OpenCV's
dense Farneback optical flow (reference: traces/gen_motion_from_video.py:
104-135): cv2.calcOpticalFlowFarneback(prev, next, None, pyr_scale=0.5,
levels=3, winsize=15, iterations=3, poly_n=5, poly_sigma=1.2, flags=0)
between consecutive gray frames, the per-pixel flow magnitude, its mean over
16x16-pixel latent-grid cells (cell_map, :61-67), the mean over row-major
16-cell tiles (:113-121), then the reuse threshold tau = the given
percentile of the change rates of frames 1.. (:124-126).

OpenCV is a third-party dependency of the reference (the `cv2` module, no
version pinned in the reference; absent from this image). This module
restates the algorithm its 4.x CPU implementation publishes
(modules/video/src/optflowgf.cpp, modules/imgproc/src/smooth, resize):

  level count     k = 0..levels-1: scale *= pyr_scale, stop at the first k
                  where cols*scale or rows*scale < 32; levels = that k.
  per level k     (coarse to fine) scale = pyr_scale^k, sigma = (1/scale -
                  1)/2, ksize = max(round_half_even(5*sigma) | 1, 3); both
                  frames: uint8 -> float, GaussianBlur(ksize, sigma) with a
                  reflect-101 border (sigma 0 at full scale: the fixed 3-tap
                  [1/4, 1/2, 1/4]), bilinear resize to (round(cols*scale),
                  round(rows*scale)) with half-pixel centres and clamped
                  edges; then the polynomial expansion.
  poly_exp        Farneback (2003) quadratic fit per pixel under a separable
                  Gaussian applicability of 2n+1 taps (sigma poly_sigma),
                  replicated borders; channels [b_y, b_x, a_yy, a_xx, a_xy].
  update_matrices per pixel, R1 sampled bilinearly at x + flow, averaged
                  with R0 (the displaced-frame form of the paper's
                  A(x), delta-b(x)), outside samples fall back to R0, a
                  5-pixel border down-weighted by {0.14, 0.14, 0.4472,
                  0.4472, 0.4472}; M = [A^T A, A^T delta-b] (5 values).
  update_flow     M averaged over a winsize x winsize box (replicated
                  border, scale 1/winsize^2), then flow = (A^T A + 1e-3 I
                  in determinant form)^-1 A^T delta-b.
  iterations      M from the initial flow, then `iterations` times: flow from
                  box(M), and M from that flow except after the last.
  initial flow    zero at the coarsest level, else the coarser level's flow
                  resized bilinearly and multiplied by 1/pyr_scale.

Computation is float64 throughout except where OpenCV's float storage
changes the result's meaning: the Gaussian taps (float32 kernels) and the
flow (float32 between steps, x + dx formed in float32, which decides the
inside/outside branch of update_matrices at the far border). The library
computes in float32 with float64 solves, so parity is a tolerance; where
x + dx falls within rounding of the last row or column the two can take
different branches, a local jump the box filter spreads over one window.

Pinned by tests/test_motion_oracle.py:
  * gaussian_kernel / sep_filter against scipy.ndimage.correlate1d with
    mode "mirror" (= reflect-101) and the published sigma rule;
  * resize_linear against scipy.ndimage.zoom(order=1, grid_mode=True,
    mode="nearest") (half-pixel centres, clamped edges);
  * poly_exp recovers every coefficient of an exact quadratic image in the
    interior (closed form: a wrong channel order, tap, sign or inverse-Gram
    entry fails), and a constant image gives zero linear and quadratic terms;
  * box_mean against scipy.ndimage.uniform_filter(mode="nearest");
  * farneback: identical frames give exactly zero flow outside the band
    along the right and bottom edges where the bilinear sample of R1 needs a
    pixel past the last row or column (OpenCV's outside branch keeps R0's
    linear terms there; one level: a band of iterations*(winsize//2)+1
    pixels); a smooth texture shifted by a known sub-pixel (dx, dy)
    (including a shift that needs the pyramid) gives that flow in the
    interior; swapping the frames negates it;
  * change_rates / trace post-processing against the reference's numpy form
    (reshape-mean cells, np.add.reduceat tiles, np.percentile) and closed
    forms (constant magnitude, the short last tile).
Parity with cv2 itself is unpinned (no cv2 here): the OpenCV-specific
constants (border weights, 1e-3 regulariser, level-0 3-tap pre-blur, level
rule) follow its published source, and no vector from cv2 checks them.
"""

from __future__ import annotations

import numpy as np

MIN_SIZE = 32
BORDER_WEIGHTS = np.array([0.14, 0.14, 0.4472, 0.4472, 0.4472], dtype=np.float32)
_SMALL_GAUSSIAN = {1: [1.0], 3: [0.25, 0.5, 0.25], 5: [0.0625, 0.25, 0.375, 0.25, 0.0625],
                   7: [0.03125, 0.109375, 0.21875, 0.28125, 0.21875, 0.109375, 0.03125]}


def round_half_even(x: float) -> int:
    """cvRound: nearest integer, ties to even."""
    return int(np.rint(x))


def gaussian_kernel(ksize: int, sigma: float) -> np.ndarray:
    """getGaussianKernel(ksize, sigma) as float32 taps (returned as float64)."""
    if sigma <= 0 and ksize in _SMALL_GAUSSIAN:
        return np.array(_SMALL_GAUSSIAN[ksize], dtype=np.float64)
    if sigma <= 0:
        sigma = ((ksize - 1) * 0.5 - 1) * 0.3 + 0.8
    x = np.arange(ksize, dtype=np.float64) - (ksize - 1) * 0.5
    t = np.exp(-x * x / (2.0 * sigma * sigma))
    return (t / t.sum()).astype(np.float32).astype(np.float64)


def reflect101(idx: np.ndarray, n: int) -> np.ndarray:
    """Border index map "gfedcb|abcdefgh|gfedcba"."""
    if n == 1:
        return np.zeros_like(idx)
    period = 2 * (n - 1)
    i = np.abs(idx) % period
    return np.where(i >= n, period - i, i)


def sep_filter(img: np.ndarray, kx: np.ndarray, ky: np.ndarray) -> np.ndarray:
    """Separable correlation, rows (kx) then columns (ky), reflect-101 border."""
    H, W = img.shape
    hx, hy = len(kx) // 2, len(ky) // 2
    cols = reflect101(np.arange(-hx, W + hx), W)
    tmp = np.zeros((H, W))
    for j, w in enumerate(kx):
        tmp += w * img[:, cols[j:j + W]]
    rows = reflect101(np.arange(-hy, H + hy), H)
    out = np.zeros((H, W))
    for i, w in enumerate(ky):
        out += w * tmp[rows[i:i + H], :]
    return out


def gaussian_blur(img: np.ndarray, ksize: int, sigma: float) -> np.ndarray:
    k = gaussian_kernel(ksize, sigma)
    return sep_filter(img, k, k)


def linear_taps(src: int, dst: int):
    """resize INTER_LINEAR source index and weight of dst samples 0..dst-1."""
    scale = 1.0 / (dst / src)
    f = (np.arange(dst) + 0.5) * scale - 0.5
    s = np.floor(f).astype(np.int64)
    w = f - s
    low = s < 0
    s[low], w[low] = 0, 0.0
    high = s >= src - 1
    s[high], w[high] = src - 1, 0.0
    return s, np.minimum(s + 1, src - 1), w


def resize_linear(img: np.ndarray, width: int, height: int) -> np.ndarray:
    """resize(img, (width, height), INTER_LINEAR); same size is a copy. The
    last axes are (rows, cols); leading axes (channels) are carried."""
    H, W = img.shape[-2:]
    if (H, W) == (height, width):
        return img.astype(np.float64).copy()
    x0, x1, wx = linear_taps(W, width)
    y0, y1, wy = linear_taps(H, height)
    h = img[..., x0] * (1.0 - wx) + img[..., x1] * wx
    return h[..., y0, :] * (1.0 - wy)[:, None] + h[..., y1, :] * wy[:, None]


def prepare_gaussian(n: int, sigma: float):
    """Applicability taps g, x*g, x^2*g (float32) and the inverse-Gram entries
    ig11, ig03, ig33, ig55 of the 6-term quadratic basis [1, x, y, x^2, y^2, xy]."""
    if sigma < np.finfo(np.float32).eps:
        sigma = n * 0.3
    x = np.arange(-n, n + 1, dtype=np.float64)
    g = np.exp(-x * x / (2.0 * sigma * sigma)).astype(np.float32).astype(np.float64)
    g = (g / g.sum()).astype(np.float32).astype(np.float64)
    xg = (x * g).astype(np.float32).astype(np.float64)
    xxg = (x * x * g).astype(np.float32).astype(np.float64)
    gg = np.outer(g, g)                       # [y, x]
    X = np.broadcast_to(x[None, :], gg.shape)
    Y = np.broadcast_to(x[:, None], gg.shape)
    basis = [np.ones_like(gg), X, Y, X * X, Y * Y, X * Y]
    G = np.array([[np.sum(gg * a * b) for b in basis] for a in basis])
    iG = np.linalg.inv(G)
    return g, xg, xxg, iG[1, 1], iG[0, 3], iG[3, 3], iG[5, 5]


def poly_exp(img: np.ndarray, n: int, sigma: float) -> np.ndarray:
    """[H, W] -> [5, H, W]: per-pixel quadratic coefficients
    [b_y, b_x, a_yy, a_xx, a_xy] (f ~ c + b.(x, y) + a_xx x^2 + a_yy y^2 + a_xy xy)."""
    H, W = img.shape
    g, xg, xxg, ig11, ig03, ig33, ig55 = prepare_gaussian(n, sigma)
    img = img.astype(np.float64)
    rows = np.arange(H)
    v0 = g[n] * img
    v1 = np.zeros_like(img)
    v2 = np.zeros_like(img)
    for k in range(1, n + 1):
        lo = img[np.maximum(rows - k, 0)]
        hi = img[np.minimum(rows + k, H - 1)]
        v0 = v0 + g[n + k] * (lo + hi)
        v1 = v1 + xg[n + k] * (hi - lo)
        v2 = v2 + xxg[n + k] * (lo + hi)
    cols = np.arange(W)
    b1 = g[n] * v0
    b3 = g[n] * v1
    b5 = g[n] * v2
    b2 = np.zeros_like(img)
    b4 = np.zeros_like(img)
    b6 = np.zeros_like(img)
    for k in range(1, n + 1):
        l, r = np.maximum(cols - k, 0), np.minimum(cols + k, W - 1)
        t0 = v0[:, r] + v0[:, l]
        b1 += t0 * g[n + k]
        b4 += t0 * xxg[n + k]
        b2 += (v0[:, r] - v0[:, l]) * xg[n + k]
        b3 += (v1[:, r] + v1[:, l]) * g[n + k]
        b6 += (v1[:, r] - v1[:, l]) * xg[n + k]
        b5 += (v2[:, r] + v2[:, l]) * g[n + k]
    return np.stack([b3 * ig11, b2 * ig11, b1 * ig03 + b5 * ig33, b1 * ig03 + b4 * ig33,
                     b6 * ig55])


def _border_scale(H: int, W: int) -> np.ndarray:
    B = len(BORDER_WEIGHTS)
    bw = BORDER_WEIGHTS.astype(np.float64)
    sx = np.ones(W)
    sy = np.ones(H)
    for i in range(min(B, W)):
        sx[i] *= bw[i]
        sx[W - 1 - i] *= bw[i]
    for i in range(min(B, H)):
        sy[i] *= bw[i]
        sy[H - 1 - i] *= bw[i]
    return sy[:, None] * sx[None, :]


def update_matrices(R0: np.ndarray, R1: np.ndarray, flow: np.ndarray) -> np.ndarray:
    """R0, R1 [5, H, W], flow [H, W, 2] (x, y) -> M [5, H, W]."""
    _, H, W = R0.shape
    yy, xx = np.mgrid[0:H, 0:W].astype(np.float32)
    # the flow is stored as float32 and x + dx formed in float32, as OpenCV
    # does: the inside/outside choice below depends on it at the far border
    dx32 = flow[..., 0].astype(np.float32)
    dy32 = flow[..., 1].astype(np.float32)
    fx, fy = (xx + dx32).astype(np.float64), (yy + dy32).astype(np.float64)
    dx, dy = dx32.astype(np.float64), dy32.astype(np.float64)
    x1, y1 = np.floor(fx), np.floor(fy)
    fx, fy = fx - x1, fy - y1
    x1, y1 = x1.astype(np.int64), y1.astype(np.int64)
    inside = (x1 >= 0) & (x1 < W - 1) & (y1 >= 0) & (y1 < H - 1)
    xa, ya = np.clip(x1, 0, W - 2), np.clip(y1, 0, H - 2)
    a00, a01 = (1 - fx) * (1 - fy), fx * (1 - fy)
    a10, a11 = (1 - fx) * fy, fx * fy
    s = (a00 * R1[:, ya, xa] + a01 * R1[:, ya, xa + 1] + a10 * R1[:, ya + 1, xa]
         + a11 * R1[:, ya + 1, xa + 1])
    r2 = np.where(inside, s[0], 0.0)
    r3 = np.where(inside, s[1], 0.0)
    r4 = np.where(inside, (R0[2] + s[2]) * 0.5, R0[2])
    r5 = np.where(inside, (R0[3] + s[3]) * 0.5, R0[3])
    r6 = np.where(inside, (R0[4] + s[4]) * 0.25, R0[4] * 0.5)
    r2 = (R0[0] - r2) * 0.5 + r4 * dy + r6 * dx
    r3 = (R0[1] - r3) * 0.5 + r6 * dy + r5 * dx
    sc = _border_scale(H, W)
    r2, r3, r4, r5, r6 = (a * sc for a in (r2, r3, r4, r5, r6))
    return np.stack([r4 * r4 + r6 * r6, (r4 + r5) * r6, r5 * r5 + r6 * r6,
                     r4 * r2 + r6 * r3, r6 * r2 + r5 * r3])


def box_sum(a: np.ndarray, m: int) -> np.ndarray:
    """Sum over the (2m+1) x (2m+1) window of the last two axes, replicated border."""
    pad = [(0, 0)] * (a.ndim - 2) + [(m, m), (m, m)]
    p = np.pad(a.astype(np.float64), pad, mode="edge")
    c = np.cumsum(p, axis=-2)
    c = np.concatenate([np.zeros_like(c[..., :1, :]), c], axis=-2)
    v = c[..., 2 * m + 1:, :] - c[..., :-(2 * m + 1), :]
    c = np.cumsum(v, axis=-1)
    c = np.concatenate([np.zeros_like(c[..., :, :1]), c], axis=-1)
    return c[..., :, 2 * m + 1:] - c[..., :, :-(2 * m + 1)]


def box_mean(a: np.ndarray, winsize: int) -> np.ndarray:
    """OpenCV's FarnebackUpdateFlow_Blur window: sum over 2*(winsize//2)+1
    pixels per axis, scaled by 1/winsize^2."""
    return box_sum(a, winsize // 2) / float(winsize * winsize)


def solve_flow(Mb: np.ndarray) -> np.ndarray:
    g11, g12, g22, h1, h2 = Mb
    idet = 1.0 / (g11 * g22 - g12 * g12 + 1e-3)
    return np.stack([(g11 * h2 - g12 * h1) * idet, (g22 * h1 - g12 * h2) * idet], axis=-1)


def level_plan(width: int, height: int, pyr_scale: float, levels: int):
    """[(k, scale, sigma, ksize, w, h)] from the coarsest level down to 0."""
    scale = 1.0
    k = 0
    while k < levels:
        scale *= pyr_scale
        if width * scale < MIN_SIZE or height * scale < MIN_SIZE:
            break
        k += 1
    plan = []
    for lv in range(k, -1, -1):
        s = 1.0
        for _ in range(lv):
            s *= pyr_scale
        sigma = (1.0 / s - 1.0) * 0.5
        ksize = max(round_half_even(sigma * 5) | 1, 3)
        plan.append((lv, s, sigma, ksize, round_half_even(width * s), round_half_even(height * s)))
    return plan


def _level_image(frame: np.ndarray, sigma: float, ksize: int, w: int, h: int) -> np.ndarray:
    return resize_linear(gaussian_blur(frame.astype(np.float64), ksize, sigma), w, h)


def farneback_clip(frames: np.ndarray, pyr_scale=0.5, levels=3, winsize=15, iterations=3,
                   poly_n=5, poly_sigma=1.2, flags=0) -> np.ndarray:
    """uint8 [n, H, W] -> flows [n-1, H, W, 2] float32, flow p = (frames[p], frames[p+1]).

    Each frame's expansion is computed once per level and used by both pairs
    it belongs to (identical to recomputing it per pair)."""
    if flags != 0:
        raise NotImplementedError("flags other than 0")
    if not 0 < pyr_scale < 1:
        raise ValueError("pyr_scale must be in (0, 1)")
    n, H, W = frames.shape
    plan = level_plan(W, H, pyr_scale, levels)
    prev_flow = None
    for lv, s, sigma, ksize, w, h in plan:
        R = np.stack([poly_exp(_level_image(f, sigma, ksize, w, h), poly_n, poly_sigma)
                      for f in frames])
        if prev_flow is None:
            flow = np.zeros((n - 1, h, w, 2), dtype=np.float32)
        else:
            flow = resize_linear(np.moveaxis(prev_flow, -1, 1), w, h)
            flow = (np.moveaxis(flow, 1, -1) * (1.0 / pyr_scale)).astype(np.float32)
        out = np.empty_like(flow)
        for p in range(n - 1):
            fl = flow[p]
            M = update_matrices(R[p], R[p + 1], fl)
            for it in range(iterations):
                fl = solve_flow(box_mean(M, winsize)).astype(np.float32)
                if it < iterations - 1:
                    M = update_matrices(R[p], R[p + 1], fl)
            out[p] = fl
        prev_flow = out
    return prev_flow.astype(np.float32)


def calc_optical_flow_farneback(prev, nxt, pyr_scale=0.5, levels=3, winsize=15, iterations=3,
                                poly_n=5, poly_sigma=1.2, flags=0) -> np.ndarray:
    """cv2.calcOpticalFlowFarneback(prev, next, None, ...) -> [H, W, 2] float32."""
    return farneback_clip(np.stack([prev, nxt]), pyr_scale, levels, winsize, iterations,
                          poly_n, poly_sigma, flags)[0]


# ---- per-tile change rates and the trace (reference: gen_motion_from_video.py:61-67,110-149)


def cell_map(mag: np.ndarray, rows: int, cols: int) -> np.ndarray:
    h, w = mag.shape[-2:]
    ch, cw = h // rows, w // cols
    if ch * rows != h or cw * cols != w:
        raise ValueError(f"grid {rows}x{cols} does not divide {w}x{h}")
    return mag.reshape(mag.shape[:-2] + (rows, ch, cols, cw)).astype(np.float64).mean(axis=(-3, -1))


def change_rates(flows: np.ndarray, rows: int, cols: int, tile_tokens: int):
    """flows [P, H, W, 2] -> (cell maps [P, rows, cols], change [P, tiles] float64)."""
    mag = np.sqrt(np.square(flows.astype(np.float64)).sum(axis=-1))
    cm = cell_map(mag, rows, cols)
    flat = cm.reshape(cm.shape[0], -1)
    tokens = rows * cols
    tiles = -(-tokens // tile_tokens)
    counts = np.full(tiles, tile_tokens)
    counts[-1] = tokens - (tiles - 1) * tile_tokens
    sums = np.add.reduceat(flat, np.arange(0, tiles * tile_tokens, tile_tokens), axis=1)
    return cm, sums / counts


def trace_from_change(change_pairs: np.ndarray, reuse_percentile: float = 50.0):
    """Pair change rates [n-1, tiles] -> (change [n, tiles], tau, reuse [n, tiles]):
    row 0 repeats row 1, tau = percentile of rows 1.., reuse = change < tau with
    row 0 forced to 0 (reference: gen_motion_from_video.py:121-126)."""
    n = change_pairs.shape[0] + 1
    change = np.zeros((n, change_pairs.shape[1]))
    change[1:] = change_pairs
    change[0] = change[1]
    tau = float(np.percentile(change[1:], reuse_percentile))
    reuse = (change < tau).astype(np.int64)
    reuse[0] = 0
    return change, tau, reuse


def trace_rows(change: np.ndarray, tau: float, reuse: np.ndarray, tokens: int,
               tile_tokens: int):
    """CSV rows frame_id,tile_id,motion_score,is_static,token_start,token_count,reuse
    (reference: gen_motion_from_video.py:138-149)."""
    n, tiles = change.shape
    out = []
    for f in range(n):
        for t in range(tiles):
            cnt = tile_tokens if t < tiles - 1 else tokens - (tiles - 1) * tile_tokens
            out.append([f, t, f"{change[f, t]:.6f}", int(change[f, t] < tau), t * tile_tokens,
                        int(cnt), int(reuse[f, t])])
    return out
